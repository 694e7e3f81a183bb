"""GPU parity of the layer launch's norm tail (hsmoe_moe_layer_decode_norm,
hsmoe_moe_layer_decode_routed_norm).

A launch with a norm tail ends with the next layer's residual adds and
RMSNorm of its own output: h_out = bf16(bf16(h + out) + residual), norm_out =
RMSNorm(h_out) * weight.  It must equal the same launch's bf16 output followed
by hsmoe_add_rms_norm, bit for bit, whichever way the output rows are made:
row-group sums over several slots (with and without the shared expert), a
lone routed slot's down items, or no expert at all (a zero output).  The
add + norm kernel itself is checked against the oracle elsewhere.
"""
import pytest
import torch

from home_seek_amd import _lib, expert_store, ops, synthetic

pytestmark = pytest.mark.gpu

D, I, E, K, SEED, EPS = 4096, 2048, 256, 6, 4711, 1e-6


@pytest.fixture(scope="module")
def layer(dev):
    store = expert_store.HbmExpertStore(1, E, D, I, dev, with_shared=True)
    store.fill_synthetic(SEED)
    gate, bias = synthetic.router_weights(SEED, 0, E, D, dev)
    torch.cuda.synchronize()
    return store, gate, bias


def rows(dev, tag, m, scale=1.0):
    return (synthetic.hidden(SEED, tag, m, D, dev).float() * scale).to(torch.bfloat16).contiguous()


def reference(out_bf16, h, weight, residual):
    return ops.add_rms_norm(h, weight, add=out_bf16, residual=residual, eps=EPS, want_sum=True)


@pytest.mark.parametrize("m,with_res", [(1, True), (3, True), (8, True), (1, False), (3, False)])
def test_router_layer_norm_tail_bit_exact(layer, dev, m, with_res):
    store, gate, bias = layer
    x = rows(dev, 10 + m, m)
    h = rows(dev, 20 + m, m, 300.0)  # a residual stream larger than the FFN output
    res = rows(dev, 30, 1, 0.1).reshape(-1) if with_res else None
    w = (rows(dev, 31, 1, 0.05).float() + 1.0).to(torch.bfloat16).reshape(-1)
    out, _, idx, wt = ops.moe_layer_decode(x, gate, bias, store.table(0), ops.SCALE_E8M0, store.shared_entry(0), I,
                                           K, 1.5, 10.0)
    h_ref, n_ref = reference(out, h, w, res)
    tail = ops.NormTail(h, w, res, EPS)
    out2 = torch.empty_like(out)
    _, _, idx2, wt2 = ops.moe_layer_decode(x, gate, bias, store.table(0), ops.SCALE_E8M0, store.shared_entry(0), I,
                                           K, 1.5, 10.0, out_bf16=out2, norm=tail)
    torch.cuda.synchronize()
    assert ops.moe_layer_status(dev) == 0
    assert torch.equal(idx, idx2) and torch.equal(wt, wt2) and torch.equal(out, out2)
    assert torch.equal(tail.h_out, h_ref) and torch.equal(tail.norm_out, n_ref)


@pytest.mark.parametrize("ids,shared", [
    ([[17, 40, 3, 200, 9, 111]], True),                          # six slots + shared
    ([[17, 40, 3, 200, 9, 111], [5, 17, 6, 7, 8, 250]], False),  # several slots, no shared expert
    ([[17]], False),                                             # one lone slot: its down items write the rows
    ([[-1, -1]], True),                                          # the shared expert only
    ([[-1, -1], [-1, 300]], False),                              # no expert at all: a zero output
])
def test_routed_layer_norm_tail_bit_exact(layer, dev, ids, shared):
    store, _, _ = layer
    m = len(ids)
    idx = torch.tensor(ids, dtype=torch.int64, device=dev)
    x = rows(dev, 40 + m, m)
    h = rows(dev, 50 + m, m, 300.0)
    res = rows(dev, 60, 1, 0.1).reshape(-1)
    w = (rows(dev, 61, 1, 0.05).float() + 1.0).to(torch.bfloat16).reshape(-1)
    sh = store.shared_entry(0) if shared else None
    tw = torch.full(idx.shape, 0.25, dtype=torch.float32, device=dev)
    out, _ = ops.moe_layer_decode_routed(x, idx, store.table(0), ops.SCALE_E8M0, sh, I, topk_w=tw)
    h_ref, n_ref = reference(out, h, w, res)
    h_in = h.clone()
    tail = ops.NormTail(h_in, w, res, EPS, h_out=h_in)  # in place
    ops.moe_layer_decode_routed(x, idx, store.table(0), ops.SCALE_E8M0, sh, I, topk_w=tw, norm=tail)
    torch.cuda.synchronize()
    assert ops.moe_layer_status(dev) == 0
    assert tail.h_out.data_ptr() == h_in.data_ptr()
    assert torch.equal(h_in, h_ref) and torch.equal(tail.norm_out, n_ref)


def test_hash_table_layer_norm_tail_and_repeated_calls(layer, dev):
    """Token-table routing, calls of different m on one workspace, each checked."""
    store, _, _ = layer
    table = (torch.arange(64, device=dev, dtype=torch.int64)[:, None] * 7 +
             torch.arange(K, device=dev, dtype=torch.int64)[None, :] * 41) % E
    w = (rows(dev, 71, 1, 0.05).float() + 1.0).to(torch.bfloat16).reshape(-1)
    for m in (2, 1, 3, 1):
        tok = torch.arange(m, dtype=torch.int64, device=dev) * 5 + m
        x = rows(dev, 80 + m, m)
        h = rows(dev, 90 + m, m, 30.0)
        out, _ = ops.moe_layer_decode_routed(x, table, store.table(0), ops.SCALE_E8M0, store.shared_entry(0), I,
                                             weight_all=1.0 / K, token_ids=tok, top_k=K)
        h_ref, n_ref = reference(out, h, w, None)
        tail = ops.NormTail(h, w, None, EPS)
        ops.moe_layer_decode_routed(x, table, store.table(0), ops.SCALE_E8M0, store.shared_entry(0), I,
                                    weight_all=1.0 / K, token_ids=tok, top_k=K, norm=tail)
        torch.cuda.synchronize()
        assert torch.equal(tail.h_out, h_ref) and torch.equal(tail.norm_out, n_ref), m
    assert ops.moe_layer_status(dev) == 0


def test_norm_tail_rejects_overlaps_and_shapes(layer, dev):
    """Checked on the host: nothing is launched."""
    store, gate, bias = layer
    x = rows(dev, 1, 2)
    h = rows(dev, 2, 2)
    w = torch.ones(D, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.NormTail(h, w[:-8])
    with pytest.raises(ValueError):
        ops.moe_layer_decode(rows(dev, 3, 1), gate, bias, store.table(0), ops.SCALE_E8M0, None, I,
                             norm=ops.NormTail(h, w))
    with pytest.raises(_lib.HsmoeError, match="overlap"):
        ops.moe_layer_decode(x, gate, bias, store.table(0), ops.SCALE_E8M0, None, I, norm=ops.NormTail(h, w,
                             norm_out=x))
    big = torch.empty(3 * D, dtype=torch.bfloat16, device=dev)
    with pytest.raises(_lib.HsmoeError, match="overlap"):
        ops.moe_layer_decode(x, gate, bias, store.table(0), ops.SCALE_E8M0, None, I,
                             norm=ops.NormTail(big[:2 * D].view(2, D), w, h_out=big[D:].view(2, D)))
    torch.cuda.synchronize()
    assert ops.moe_layer_status(dev) == 0
