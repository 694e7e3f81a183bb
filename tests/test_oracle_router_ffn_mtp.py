"""Router / FFN / acceptance oracle vs the reference's KATs, closed forms and torch."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as orc

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def test_splitmix64_published_values():
    vals = [int(h, 16) for h in KATS["splitmix64_seed0"]["values_hex"]]
    assert [orc.lib().hso_rand(0, i) for i in range(3)] == vals


def test_generator_distributions():
    k = orc.key(1, orc.tag(orc.KIND_HIDDEN))
    x = orc.bf16_to_f32(orc.gen_normal_bf16(k, 200000, 0.0, 1.0))
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    e = orc.gen_e8m0(k, 60000)
    assert e.min() == 119 and e.max() == 124 and np.all(np.bincount(e)[119:] > 9000)
    b = orc.gen_bytes(k, 80000)
    codes = np.concatenate([b & 15, b >> 4])
    assert np.all(np.abs(np.bincount(codes, minlength=16) / codes.size - 1 / 16) < 0.003)
    q = orc.gen_e4m3(k, 100000)
    assert not np.any((q & 0x7F) == 0x7F)


def test_stable_topk_kat():
    kat = KATS["stable_topk"]
    got = orc.stable_topk(np.array(kat["scores"], dtype=np.float32), kat["k"])
    assert got.tolist() == kat["expected"]


def test_router_ties_pick_lower_index():
    x = orc.f32_to_bf16(np.ones((1, 32), dtype=np.float32))
    gate = orc.f32_to_bf16(np.ones((16, 32), dtype=np.float32) * np.float32(0.5))
    idx, w = orc.router(x, gate, None, 6, 1.5)
    assert idx.tolist() == [[0, 1, 2, 3, 4, 5]]
    assert np.allclose(w, 0.25)


@pytest.mark.parametrize("scaling", KATS["routing_scaling"]["scaling"])
def test_router_weights_sum_to_scaling(scaling):
    rng = np.random.default_rng(5)
    x = orc.f32_to_bf16(rng.standard_normal((4, 64)).astype(np.float32))
    gate = orc.f32_to_bf16(rng.standard_normal((16, 64)).astype(np.float32))
    _, w = orc.router(x, gate, None, 4, scaling)
    assert np.allclose(w.sum(-1), scaling, atol=KATS["routing_scaling"]["atol"])


def test_router_matches_torch_formula_when_sums_are_exact():
    """Small-integer inputs make every fp32 partial sum exact, so torch's bf16
    matmul and the oracle's exact-then-round logits must coincide."""
    rng = np.random.default_rng(6)
    xf = rng.integers(-4, 5, (3, 64)).astype(np.float32)
    gf = (rng.integers(-8, 9, (32, 64)) / 8.0).astype(np.float32)
    bias = (rng.integers(-16, 17, 32) / 64.0).astype(np.float32)
    x, g = orc.f32_to_bf16(xf), orc.f32_to_bf16(gf)
    xt = torch.from_numpy(xf).to(torch.bfloat16)
    gt = torch.from_numpy(gf).to(torch.bfloat16)
    logits = (xt @ gt.t()) + torch.from_numpy(bias).to(torch.bfloat16)
    scores = F.softplus(logits.float()).sqrt()
    _, order = torch.sort(scores, dim=1, descending=True, stable=True)
    ref_idx = order[:, :6]
    raw = scores.gather(1, ref_idx)
    ref_w = raw / raw.sum(-1, keepdim=True).clamp(min=1e-20) * 1.5
    idx, w, sc, lg = orc.router(x, g, bias, 6, 1.5, return_scores=True)
    assert np.array_equal(lg, logits.view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(idx, ref_idx.numpy())
    np.testing.assert_allclose(w, ref_w.numpy(), rtol=1e-6)


def test_logits_exact_vs_integer_brute_force():
    rng = np.random.default_rng(8)
    xi = rng.integers(-100, 101, (2, 512))
    wi = rng.integers(-100, 101, (7, 512))
    x = orc.f32_to_bf16(xi.astype(np.float32))
    w = orc.f32_to_bf16((wi / 64.0).astype(np.float32))
    exact = (xi @ wi.T) / 64.0  # exact in float64 (|sum| < 2^53)
    assert np.array_equal(orc.logits_bf16(x, w), orc.f32_to_bf16(exact.astype(np.float32)) * 0 +
                          np.vectorize(orc.lib().hso_f64_to_bf16)(exact).astype(np.uint16))


def test_swiglu_is_silu_and_clamps_asymmetrically():
    L = KATS["swiglu_clamp"]["limit"]
    g = np.array([-20.0, -1.0, 0.5, 3.0, 15.0], dtype=np.float32)
    u = np.array([-20.0, 2.0, -0.5, 15.0, 1.0], dtype=np.float32)
    got = orc._swiglu_f32(g, u, L)
    gt, ut = torch.from_numpy(g), torch.from_numpy(u)
    ref = F.silu(gt.clamp(max=L)) * ut.clamp(-L, L)
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-6, atol=1e-7)
    sigmoid_only = (gt.clamp(max=L).sigmoid() * ut.clamp(-L, L)).numpy()
    assert np.abs(got - sigmoid_only).max() > 1.0
    assert got[0] != 0.0  # gate -20 is NOT clamped from below; up -20 IS clamped to -10


def test_expert_ffn_fp32_matches_float64_torch():
    rng = np.random.default_rng(9)
    d, i = 64, 32
    x = orc.f32_to_bf16(rng.standard_normal((3, d)).astype(np.float32))
    w1, w3 = (orc.f32_to_bf16((rng.standard_normal((i, d)) * 0.3).astype(np.float32)) for _ in range(2))
    w2 = orc.f32_to_bf16((rng.standard_normal((d, i)) * 0.3).astype(np.float32))
    got = orc.expert_ffn_fp32(x, w1, w3, w2, 10.0)
    t = lambda a: torch.from_numpy(orc.bf16_to_f32(a)).double()
    gate, up = t(x) @ t(w1).T, t(x) @ t(w3).T
    ref = (F.silu(gate.clamp(max=10.0)) * up.clamp(-10.0, 10.0)) @ t(w2).T
    np.testing.assert_allclose(got, ref.numpy(), rtol=2e-5, atol=1e-5)


def test_moe_layer_is_weighted_sum_of_experts():
    rng = np.random.default_rng(10)
    d, i = 64, 32
    mk = lambda r, c: orc.f32_to_bf16((rng.standard_normal((r, c)) * 0.3).astype(np.float32))
    experts = {e: {"w1_bf16": mk(i, d), "w3_bf16": mk(i, d), "w2_bf16": mk(d, i)} for e in range(5)}
    x = mk(2, d)
    idx = np.array([[3, 1, -1], [0, 3, 4]])
    w = np.array([[0.5, 1.0, 9.0], [0.25, 0.75, 2.0]], dtype=np.float32)
    got = orc.moe_layer_fp32(x, idx, w, experts, None)
    for t in range(2):
        ref = np.zeros(d)
        for j in range(3):
            if idx[t, j] >= 0:
                ex = experts[idx[t, j]]
                ref += w[t, j] * orc.expert_ffn_fp32(x[t:t + 1], ex["w1_bf16"], ex["w3_bf16"], ex["w2_bf16"])[0]
        np.testing.assert_allclose(got[t], ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("case", KATS["mtp_accept"]["cases"], ids=lambda c: c["name"])
def test_mtp_accept_kats(case):
    combined = [case["main_pred"]] + case["drafts"]
    v = 128
    logits = np.full((len(combined), v), orc.f32_to_bf16(np.array([-1.0], np.float32))[0], dtype=np.uint16)
    for t, a in enumerate(case["position_argmax"]):
        logits[t, a] = orc.f32_to_bf16(np.array([1.0], np.float32))[0]
    n, bonus = orc.mtp_accept(logits, combined)
    assert n == case["n_accept"] and bonus == min(n, len(combined) - 1)


def test_argmax_first_index_on_ties():
    row = orc.f32_to_bf16(np.array([1.0, 3.0, 2.0, 3.0], dtype=np.float32))
    assert orc.argmax_first(row) == 1
    t = torch.from_numpy(orc.bf16_to_f32(row)).to(torch.bfloat16)
    assert int(torch.argmax(t)) == 1


def test_rms_norm_matches_reference_formula():
    """Every element within one bf16 step of the reference's formula
    (utils.py:6-9, torch fp32), nearly all of them equal: the two differ only
    in the fp32 summation order of the mean of squares."""
    rng = np.random.default_rng(11)
    for rows, d, scale in ((2, 64, 1.0), (16, 4096, 1.0), (8, 4096, 300.0), (4, 7168, 1e-3)):
        x = orc.f32_to_bf16((rng.standard_normal((rows, d)) * scale).astype(np.float32))
        w = orc.f32_to_bf16(rng.normal(1.0, 0.05, d).astype(np.float32))
        xt = torch.from_numpy(orc.bf16_to_f32(x)).to(torch.bfloat16)
        wt = torch.from_numpy(orc.bf16_to_f32(w)).to(torch.bfloat16)
        var = xt.float().pow(2).mean(-1, keepdim=True)
        ref = (wt.float() * (xt.float() * torch.rsqrt(var + 1e-6))).to(torch.bfloat16).float().numpy()
        got = orc.bf16_to_f32(orc.rms_norm(x, w))
        # one bf16 step of each element: 2^(floor(log2 |ref|) - 7)
        step = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
        assert np.all(np.abs(got - ref) <= step), (rows, d, scale)
        assert np.mean(got == ref) >= 0.99, (rows, d, scale, np.mean(got == ref))
