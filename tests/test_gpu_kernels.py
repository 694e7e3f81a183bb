"""GPU parity: dequant, generators, router, lm_head/acceptance, RMSNorm vs the CPU oracle."""
import numpy as np
import pytest
import torch

from home_seek_amd import ops, synthetic
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def bf16_same(a, b):
    na = (a & 0x7FFF) > 0x7F80
    nb = (b & 0x7FFF) > 0x7F80
    return np.array_equal(na, nb) and np.array_equal(a[~na], b[~nb])


def test_fp4_dequant_exhaustive_e8m0(dev):
    """All 256 packed bytes x all 256 exponents, bit-exact (torch-cast E8M0 semantics)."""
    packed = np.tile(np.repeat(np.arange(256, dtype=np.uint8), 1).reshape(16, 16), (256, 1))  # [4096, 16]
    e = np.repeat(np.arange(256, dtype=np.uint8), 16).reshape(4096, 1)
    got = ops.fp4_dequant_bf16(torch.from_numpy(packed).to(dev), torch.from_numpy(e).to(dev).view(torch.float8_e8m0fnu))
    ref = orc.dequant_fp4(packed, e, e8m0=True, semantics="cast")
    assert bf16_same(orc.to_np_bf16(got), ref)


def test_fp4_dequant_f32_scales_bit_exact(dev):
    rng = np.random.default_rng(0)
    packed = rng.integers(0, 256, (512, 256), dtype=np.uint8)
    sf = rng.uniform(-3.0, 3.0, (512, 16)).astype(np.float32) * np.float32(2.0) ** rng.integers(-20, 20, (512, 16)).astype(np.float32)
    sf[0, :4] = [0.0, -0.0, 1e-40, 3e38]
    got = ops.fp4_dequant_bf16(torch.from_numpy(packed).to(dev), torch.from_numpy(sf).to(dev))
    ref = orc.dequant_fp4(packed, sf, e8m0=False)
    assert bf16_same(orc.to_np_bf16(got), ref)


def test_fp4_dequant_full_expert(dev):
    ex = orc.gen_fp4_expert(11, 3, 77, 4096, 2048)
    for name in ("w1", "w3", "w2"):
        p = torch.from_numpy(ex[name]).to(dev).view(torch.int8)
        s = torch.from_numpy(ex[name + "_scale"]).to(dev).view(torch.float8_e8m0fnu)
        assert np.array_equal(orc.to_np_bf16(ops.fp4_dequant_bf16(p, s)), ex[name + "_bf16"])


def test_fp8_dequant_all_codes(dev):
    rng = np.random.default_rng(1)
    data = np.tile(np.arange(256, dtype=np.uint8), (256, 2))  # [256, 512], includes NaN codes
    sf = rng.uniform(0.5, 2.0, (2, 4)).astype(np.float32) / np.float32(448.0)
    got = ops.fp8_dequant_bf16(torch.from_numpy(data).to(dev).view(torch.float8_e4m3fn), torch.from_numpy(sf).to(dev))
    assert bf16_same(orc.to_np_bf16(got), orc.dequant_fp8(data, sf))


@pytest.mark.parametrize("kind", ["bytes", "e4m3", "e8m0", "normal_bf16", "normal_f32", "uniform", "index"])
def test_generators_match_host(dev, kind):
    k = orc.key(99, orc.tag(5, 1, 2, 3))
    n = 100003
    if kind in ("bytes", "e4m3"):
        t = ops.gen_bytes(k, torch.empty(n, dtype=torch.uint8, device=dev), e4m3=kind == "e4m3")
        ref = orc.gen_bytes(k, n) if kind == "bytes" else orc.gen_e4m3(k, n)
    elif kind == "e8m0":
        t = ops.gen_e8m0(k, torch.empty(n, dtype=torch.uint8, device=dev))
        ref = orc.gen_e8m0(k, n)
    elif kind == "normal_bf16":
        t = ops.gen_normal(k, torch.empty(n, dtype=torch.bfloat16, device=dev), 0.1, 0.02)
        assert np.array_equal(orc.to_np_bf16(t), orc.gen_normal_bf16(k, n, 0.1, 0.02))
        return
    elif kind == "normal_f32":
        t = ops.gen_normal(k, torch.empty(n, dtype=torch.float32, device=dev), 1.0, 0.05)
        ref = orc.gen_normal_f32(k, n, 1.0, 0.05)
    elif kind == "index":
        t = ops.gen_index(k, torch.empty(n, dtype=torch.int64, device=dev), 129280)
        ref = orc.gen_index(k, n, 129280)
    else:
        t = ops.gen_uniform(k, torch.empty(n, dtype=torch.float32, device=dev), 0.5, 2.0, 1.0 / 448.0)
        ref = orc.gen_uniform_f32(k, n, 0.5, 2.0, np.float32(1.0 / 448.0))
    assert np.array_equal(t.cpu().numpy().view(ref.dtype), ref)


@pytest.mark.parametrize("m", [1, 3, 8, 64])
def test_router_ids_bit_exact(dev, m):
    seed = 1000 + m
    gate, bias = synthetic.router_weights(seed, 0, 256, 4096, dev)
    x = synthetic.hidden(seed, 0, m, 4096, dev)
    idx, w, lg = ops.router_topk(x, gate, bias, 6, 1.5, want_logits=True)
    ridx, rw, _, rlg = orc.router(orc.to_np_bf16(x), orc.to_np_bf16(gate), bias.cpu().numpy(), 6, 1.5,
                                  return_scores=True)
    assert np.array_equal(orc.to_np_bf16(lg), rlg)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=2e-6, atol=0)


def test_router_ties_and_no_bias(dev):
    x = torch.ones(2, 512, dtype=torch.bfloat16, device=dev)
    gate = torch.full((64, 512), 0.5, dtype=torch.bfloat16, device=dev)
    idx, w = ops.router_topk(x, gate, None, 6, 1.5)
    assert idx.cpu().tolist() == [[0, 1, 2, 3, 4, 5]] * 2
    assert torch.allclose(w, torch.full_like(w, 0.25))


@pytest.mark.parametrize(
    "n_tok,vocab,d",
    [(1, 4096, 512), (3, 129280, 4096), (8, 1000, 512), (2, 70001, 4096), (4, 33333, 4096),
     # the MFMA form with one group per row, with groups that do not fill its load pipeline, and with fewer
     # 4-row tiles than waves
     (3, 3001, 512), (4, 20001, 1536), (2, 5, 1536),
     # six tokens of 4096: fp64 hidden states past the LDS budget, widened into the workspace by a launch of their own
     (6, 3001, 4096),
     # the largest hidden size the entry point takes: 64 KiB of bf16 hidden states in the MFMA form's LDS
     (2, 3001, 8192), (3, 1001, 8192), (4, 2049, 8192), (1, 1001, 8192),
     # one token, row per wave: the full head, a hidden size of 3 chunks per lane, fewer rows than waves
     (1, 129280, 4096), (1, 33333, 1536), (1, 5, 2048)])
def test_lm_head_logits_argmax_bit_exact(dev, n_tok, vocab, d):
    seed = 7 + n_tok
    lm = synthetic.normal_bf16(seed, synthetic.tag(synthetic.KIND_LM_HEAD), (vocab, d), 0.0, 0.02, dev)
    h = synthetic.hidden(seed, 1, n_tok, d, dev)
    ids = torch.randint(0, vocab, (n_tok,), device=dev)
    logits, pred, result = ops.lm_head_accept(h, lm, ids)
    rl = orc.logits_bf16(orc.to_np_bf16(h), orc.to_np_bf16(lm))
    assert np.array_equal(orc.to_np_bf16(logits), rl)
    rp = [orc.argmax_first(rl[t]) for t in range(n_tok)]
    assert pred.cpu().tolist() == rp
    n, bonus = orc.mtp_accept(rl, ids.cpu().tolist())
    assert result.cpu().tolist() == [n, bonus]


def test_lm_head_accept_kats_on_device(dev):
    """The reference's accept/reject KATs (tests/test_mtp.py:355-456) with one-hot lm_head rows."""
    d, vocab = 512, 128
    lm = torch.zeros(vocab, d, dtype=torch.bfloat16, device=dev)
    for tok, dim in ((10, 0), (20, 1), (30, 2), (99, 3)):
        lm[tok, dim] = 1.0
    h = torch.zeros(4, d, dtype=torch.bfloat16, device=dev)
    for t in range(4):
        h[t, t] = 1.0
    for drafts, want in (([10, 20, 30], 3), ([10, 21, 30], 1), ([11, 20, 30], 0)):
        ids = torch.tensor([5] + drafts, device=dev)
        _, pred, result = ops.lm_head_accept(h, lm, ids)
        assert pred.cpu().tolist() == [10, 20, 30, 99]
        assert result.cpu().tolist() == [want, want]
    # ties: all-zero logits -> first index
    _, pred, _ = ops.lm_head_accept(torch.zeros(1, d, dtype=torch.bfloat16, device=dev), lm)
    assert pred.item() == 0


def test_rms_norm_within_one_ulp(dev):
    seed = 5
    x = synthetic.hidden(seed, 2, 5, 4096, dev)
    w = synthetic.normal_bf16(seed, synthetic.tag(synthetic.KIND_NORM_W), (4096,), 1.0, 0.05, dev)
    got = orc.bf16_to_f32(orc.to_np_bf16(ops.rms_norm(x, w)))
    ref = orc.bf16_to_f32(orc.rms_norm(orc.to_np_bf16(x), orc.to_np_bf16(w)))
    ulp = np.abs(ref) * 2.0 ** -7
    assert np.all(np.abs(got - ref) <= ulp)
    assert np.mean(got == ref) > 0.98


@pytest.mark.parametrize("rows,d", [(1, 4096), (3, 4096), (5, 512), (2, 16384)])
def test_add_rms_norm_matches_torch_adds_and_oracle(dev, rows, d):
    """h = bf16(bf16(x + add) + res) bit-exact against torch's bf16 adds; the norm
    within one bf16 step of the oracle (and equal to hsmoe_rms_norm of h)."""
    seed = 11 + rows
    x = synthetic.hidden(seed, 1, rows, d, dev)
    add = synthetic.hidden(seed, 2, rows, d, dev)
    res = synthetic.normal_bf16(seed, synthetic.tag(synthetic.KIND_RESIDUAL), (d,), 0.0, 0.1, dev)
    w = synthetic.normal_bf16(seed, synthetic.tag(synthetic.KIND_NORM_W), (d,), 1.0, 0.05, dev)
    h, hn = ops.add_rms_norm(x, w, add=add, residual=res, want_sum=True)
    assert torch.equal(h, (x + add) + res)
    assert torch.equal(hn, ops.rms_norm(h, w))
    got = orc.bf16_to_f32(orc.to_np_bf16(hn))
    ref = orc.bf16_to_f32(orc.rms_norm(orc.to_np_bf16(h), orc.to_np_bf16(w)))
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -7)
    h2, hn2 = ops.add_rms_norm(x, w, residual=res, want_sum=True)
    assert torch.equal(h2, x + res) and torch.equal(hn2, ops.rms_norm(x + res, w))
