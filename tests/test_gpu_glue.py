"""GPU parity of the decode step's small launches: the embedding lookup fused
with the first norm (hsmoe_embed_add_rms_norm), the MTP block's input
(hsmoe_mtp_input) and the step's emission record (hsmoe_decode_step_record).

Each replaces a sequence of launches the engine made before, and must equal
that sequence bit for bit: the torch lookup followed by hsmoe_add_rms_norm
(itself checked against the oracle elsewhere), the three norms and two bf16
adds of the MTP input, and the reference's emission rule (engine.py:2862-2922
at temperature 0) written out in torch on the same device tensors.
"""
import pytest
import torch

from home_seek_amd import ops, synthetic

pytestmark = pytest.mark.gpu

D, V, SEED, EPS = 4096, 1000, 99, 1e-6


def bf16_rows(dev, tag, m, d=D, scale=1.0, shift=0.0):
    return (synthetic.hidden(SEED, tag, m, d, dev).float() * scale + shift).to(torch.bfloat16).contiguous()


@pytest.mark.parametrize("d", [D, 512, 7168])
@pytest.mark.parametrize("with_res", [True, False])
def test_embed_add_rms_norm_bit_exact(dev, d, with_res):
    table = bf16_rows(dev, 1, V, d, 0.02)
    w = bf16_rows(dev, 2, 1, d, 0.05, 1.0).reshape(-1)
    res = bf16_rows(dev, 3, 1, d, 0.1).reshape(-1) if with_res else None
    ids = torch.tensor([[5, 0, V - 1, 731, 5, 42, 999, 1]], dtype=torch.int64, device=dev)
    h, out = ops.embed_add_rms_norm(ids, table, w, res, EPS)
    h_ref, out_ref = ops.add_rms_norm(table[ids], w, residual=res, eps=EPS, want_sum=True)
    torch.cuda.synchronize()
    assert h.shape == (1, 8, d) and out.shape == (1, 8, d)
    assert torch.equal(h, h_ref) and torch.equal(out, out_ref)


def test_embed_add_rms_norm_out_of_range_ids_read_zeros(dev):
    table = bf16_rows(dev, 4, V, D, 0.02)
    w = bf16_rows(dev, 5, 1, D, 0.05, 1.0).reshape(-1)
    res = bf16_rows(dev, 6, 1, D, 0.1).reshape(-1)
    ids = torch.tensor([-1, V, 3], dtype=torch.int64, device=dev)
    h, out = ops.embed_add_rms_norm(ids, table, w, res, EPS)
    x = torch.stack([torch.zeros(D, dtype=torch.bfloat16, device=dev)] * 2 + [table[3]])
    h_ref, out_ref = ops.add_rms_norm(x, w, residual=res, eps=EPS, want_sum=True)
    torch.cuda.synchronize()
    assert torch.equal(h, h_ref) and torch.equal(out, out_ref)


def _mtp_input_unfused(tok, embed, h_prev, enorm, hnorm, w, res):
    e = ops.rms_norm(embed[tok.reshape(-1)], enorm, EPS)
    h_in = ops.rms_norm(h_prev.reshape(1, -1), hnorm, EPS) + e
    return ops.add_rms_norm(h_in, w, residual=res, eps=EPS, want_sum=True)


@pytest.mark.parametrize("d,with_res", [(D, True), (D, False), (8192, True), (520, True)])
def test_mtp_input_bit_exact(dev, d, with_res):
    embed = bf16_rows(dev, 10, V, d, 0.02)
    h_prev = bf16_rows(dev, 11, 1, d, 300.0)  # a residual stream far larger than the embedding
    enorm, hnorm, w = (bf16_rows(dev, 12 + j, 1, d, 0.05, 1.0).reshape(-1) for j in range(3))
    res = bf16_rows(dev, 15, 1, d, 0.1).reshape(-1) if with_res else None
    for t in (0, 17, V - 1):
        tok = torch.tensor([[t]], dtype=torch.int64, device=dev)
        h, out = ops.mtp_input(tok, embed, h_prev, enorm, hnorm, w, res, EPS)
        h_ref, out_ref = _mtp_input_unfused(tok, embed, h_prev, enorm, hnorm, w, res)
        torch.cuda.synchronize()
        assert torch.equal(h, h_ref) and torch.equal(out, out_ref), t


def _record_ref(tokens, pred, result):
    """The emission rule of engine.py:2862-2922 at temperature 0, on the device values."""
    a = tokens[0]
    n = tokens.numel() - 1
    if n == 0:
        return tokens[:1].clone(), 1, int(a), 0
    n_acc = int(result[0])
    bonus = int(pred[min(max(int(result[1]), 0), n)])
    row = torch.cat([tokens, torch.tensor([bonus], dtype=torch.int64, device=tokens.device)])
    count = 1 + (n_acc > 0) * (n_acc + 1)
    return row, count, bonus if n_acc > 0 else int(a), n_acc


@pytest.mark.parametrize("n", [0, 1, 2, 3])
def test_decode_step_record_matches_rule(dev, n):
    cap = 6
    width = n + 2 if n > 0 else 1
    rows = torch.full((cap, width), -7, dtype=torch.int64, device=dev)
    counts = torch.full((cap,), -7, dtype=torch.int64, device=dev)
    naccs = torch.full((cap,), -7, dtype=torch.int64, device=dev)
    k = torch.zeros((), dtype=torch.int64, device=dev)
    cur = torch.zeros(1, 1, dtype=torch.int64, device=dev)
    cases = [(acc, acc) for acc in range(n + 1)] if n > 0 else [(0, 0)] * 3
    expect = []
    for step, (acc, brow) in enumerate(cases):
        tokens = torch.tensor([100 + step] + [200 + 10 * step + j for j in range(n)], dtype=torch.int64, device=dev)
        pred = torch.tensor([300 + 10 * step + j for j in range(n + 1)], dtype=torch.int64, device=dev)
        result = torch.tensor([acc, brow], dtype=torch.int64, device=dev)
        row, count, nxt, nacc = ops.decode_step_record(tokens, pred if n else None, result if n else None,
                                                       record=(rows, counts, naccs, k), cur=cur)
        r_ref, c_ref, n_ref, a_ref = _record_ref(tokens, pred, result)
        torch.cuda.synchronize()
        assert torch.equal(row, r_ref) and int(count) == c_ref and int(nxt) == n_ref and int(nacc) == a_ref
        assert int(cur) == n_ref and int(k) == step + 1
        expect.append((r_ref, c_ref, a_ref))
    for step, (r_ref, c_ref, a_ref) in enumerate(expect):
        assert torch.equal(rows[step], r_ref) and int(counts[step]) == c_ref and int(naccs[step]) == a_ref
    assert bool((rows[len(expect):] == -7).all()) and bool((counts[len(expect):] == -7).all())


def test_decode_step_record_past_capacity_writes_no_row(dev):
    rows = torch.full((1, 3), -7, dtype=torch.int64, device=dev)
    counts = torch.full((1,), -7, dtype=torch.int64, device=dev)
    naccs = torch.full((1,), -7, dtype=torch.int64, device=dev)
    k = torch.ones((), dtype=torch.int64, device=dev)  # already at capacity
    tokens = torch.tensor([1, 2], dtype=torch.int64, device=dev)
    pred = torch.tensor([2, 9], dtype=torch.int64, device=dev)
    result = torch.tensor([1, 1], dtype=torch.int64, device=dev)
    ops.decode_step_record(tokens, pred, result, record=(rows, counts, naccs, k))
    torch.cuda.synchronize()
    assert int(k) == 2 and bool((rows == -7).all()) and int(counts[0]) == -7 and int(naccs[0]) == -7
