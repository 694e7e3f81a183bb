"""Pins of the oracle's FFN, layer and decode-loop functions (CPU only).

- expert_ffn_ref_bf16 and moe_layer_reference against torch's own bf16 ops,
  running the reference's formulas (fused_moe.py:383-395, the _forward_legacy
  torch branch fused_moe.py:458-551, the shared add engine.py:1530-1536), on
  inputs whose gate/up sums are exact in fp32: there the BLAS accumulation
  order cannot matter, so the gate/up rounding points and the routing weights
  must agree bit for bit; after the SwiGLU (torch's sigmoid vs numpy's exp)
  and the down sums (accumulation order) within one bf16 step.
- moe_layer_fp32 (the FFN bar of every GPU test) against an independent
  float64 evaluation of sum_j w_j FFN_j(x) + FFN_shared(x).
- The router's logit definition (exact sum rounded once) against the
  reference's fp32-accumulated bf16 matmul on config-1 distributions: every
  top-6 difference must be a near-tie.
- The decode loop's emission rule (StackOracle.generate) against a direct
  restatement of the reference's loop (engine.py:2809-2922 at temperature 0)
  on a toy model whose next token is known.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as orc
from oracle.stack import StackOracle

LIMIT = 10.0


def bf16_steps_apart(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in bf16 steps between two bf16 bit arrays of finite values."""
    def ordered(h):
        v = h.astype(np.int32)
        return np.where(v & 0x8000, 0x8000 - (v & 0x7FFF), 0x8000 + v)
    return np.abs(ordered(a) - ordered(b))


def torch_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def exact_sum_inputs(rng, m, d, i, n_experts=1):
    """x: integers in [-6, 6]; weights: integers in [-15, 15] / 16 (both exact
    in bf16) -- every fp32 partial sum of x . w is a multiple of 1/16 below
    2^10 (d <= 160), hence exact."""
    x = rng.integers(-6, 7, (m, d)).astype(np.float32)
    ws = []
    for _ in range(n_experts):
        w1 = (rng.integers(-15, 16, (i, d)) / 16.0).astype(np.float32)
        w3 = (rng.integers(-15, 16, (i, d)) / 16.0).astype(np.float32)
        w2 = (rng.integers(-15, 16, (d, i)) / 16.0).astype(np.float32)
        ws.append((w1, w3, w2))
    return x, ws


def torch_ffn_pt(h, w1, w3, w2, limit=LIMIT):
    """fused_expert_ffn_pt (fused_moe.py:383-395) in torch bf16 -> (gate, up, act, out)."""
    gate_out = h @ w1.t()
    up_out = h @ w3.t()
    g = gate_out.float().clamp(max=limit)
    u = up_out.float().clamp(min=-limit, max=limit)
    act = (g * g.sigmoid() * u).to(w1.dtype)
    return gate_out, up_out, act, act @ w2.t()


def bf16t(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)


@pytest.mark.parametrize("m,d,i", [(1, 64, 32), (3, 128, 64), (8, 96, 160)])
def test_expert_ffn_ref_bf16_matches_torch_bf16_ops(m, d, i):
    rng = np.random.default_rng(100 + m)
    x, [(w1, w3, w2)] = exact_sum_inputs(rng, m, d, i)
    tg, tu, ta, to = torch_ffn_pt(bf16t(x), bf16t(w1), bf16t(w3), bf16t(w2))
    st = orc.expert_ffn_ref_bf16(orc.f32_to_bf16(x), orc.f32_to_bf16(w1), orc.f32_to_bf16(w3), orc.f32_to_bf16(w2),
                                 LIMIT, steps=True)
    assert np.array_equal(st["gate"], torch_bits(tg))
    assert np.array_equal(st["up"], torch_bits(tu))
    assert bf16_steps_apart(st["act"], torch_bits(ta)).max() <= 1
    assert np.mean(st["act"] == torch_bits(ta)) >= 0.99
    assert bf16_steps_apart(orc.f32_to_bf16(st["out"]), torch_bits(to)).max() <= 1
    # the gate clamp and the up clamp both occur in these draws
    assert (orc.bf16_to_f32(st["gate"]) > LIMIT).any() and (orc.bf16_to_f32(st["up"]) < -LIMIT).any()


def torch_forward_legacy(h, topk_idx, topk_w, experts, limit=LIMIT):
    """The torch branch of _forward_legacy (fused_moe.py:458-551) on bf16 weights
    -> (expert_weights bf16 [B, n_union], routed out bf16 [B, D])."""
    B, D = h.shape
    eids = sorted({int(e) for e in topk_idx.reshape(-1).tolist() if int(e) >= 0 and int(e) in experts})
    w1 = torch.cat([experts[e][0] for e in eids], dim=0)
    w3 = torch.cat([experts[e][1] for e in eids], dim=0)
    w2 = torch.cat([experts[e][2] for e in eids], dim=1)
    I = experts[eids[0]][0].shape[0]
    gate = h @ w1.T
    up = h @ w3.T
    ew = torch.zeros(B, len(eids), dtype=torch.bfloat16)
    pos = {e: q for q, e in enumerate(eids)}
    for b in range(B):
        for k in range(topk_idx.shape[1]):
            e = int(topk_idx[b, k])
            if e in pos:
                ew[b, pos[e]] = topk_w[b, k].to(torch.bfloat16)
    g = gate.float().clamp(max=limit)
    u = up.float().clamp(min=-limit, max=limit)
    act = (g * g.sigmoid() * u).to(torch.bfloat16)
    weighted = act.view(B, len(eids), I) * ew.unsqueeze(-1)
    return ew, weighted.reshape(B, len(eids) * I) @ w2.T


@pytest.mark.parametrize("m", [2, 5])
def test_moe_layer_reference_matches_torch_union_route(m):
    rng = np.random.default_rng(200 + m)
    d, i, n_exp, k = 64, 32, 8, 3
    x, ws = exact_sum_inputs(rng, m, d, i, n_exp)
    idx = np.stack([rng.permutation(n_exp)[:k] for _ in range(m)]).astype(np.int64)
    idx[0, 1] = -1  # an invalid id is skipped
    w = rng.uniform(0.1, 1.0, (m, k)).astype(np.float32)
    experts = {e: {"w1_bf16": orc.f32_to_bf16(a), "w3_bf16": orc.f32_to_bf16(b), "w2_bf16": orc.f32_to_bf16(c)}
               for e, (a, b, c) in enumerate(ws) if e != 5}  # expert 5 absent (loader returned None)
    sx, [(s1, s3, s2)] = exact_sum_inputs(rng, 1, d, i)
    shared = {"w1_bf16": orc.f32_to_bf16(s1), "w3_bf16": orc.f32_to_bf16(s3), "w2_bf16": orc.f32_to_bf16(s2)}
    st = orc.moe_layer_reference(orc.f32_to_bf16(x), idx, w, experts, shared, LIMIT, steps=True)
    h = bf16t(x)
    tex = {e: (bf16t(a), bf16t(b), bf16t(c)) for e, (a, b, c) in enumerate(ws) if e != 5}
    ew, routed = torch_forward_legacy(h, torch.from_numpy(idx), torch.from_numpy(w), tex)
    assert st["union"] == sorted({int(e) for e in idx.reshape(-1) if e >= 0 and e != 5})
    assert np.array_equal(st["ew"], torch_bits(ew))
    assert bf16_steps_apart(st["routed"], torch_bits(routed)).max() <= 1
    _, _, _, sh = torch_ffn_pt(h, bf16t(s1), bf16t(s3), bf16t(s2))
    assert bf16_steps_apart(st["shared"], torch_bits(sh)).max() <= 1
    # the shared add of engine.py:1530-1536 (a bf16 tensor add), bit for bit on the same operands
    r_t = torch.from_numpy(st["routed"].view(np.int16)).view(torch.bfloat16)
    s_t = torch.from_numpy(st["shared"].view(np.int16)).view(torch.bfloat16)
    assert np.array_equal(st["out"], torch_bits(r_t + s_t))
    assert np.array_equal(orc.bf16_add_bits(st["routed"], st["shared"]), torch_bits(r_t + s_t))


def test_bf16_add_matches_torch_on_wide_exponent_gaps():
    rng = np.random.default_rng(7)
    a = orc.f32_to_bf16((rng.standard_normal(20000) * 2.0 ** rng.integers(-30, 30, 20000)).astype(np.float32))
    b = orc.f32_to_bf16((rng.standard_normal(20000) * 2.0 ** rng.integers(-30, 30, 20000)).astype(np.float32))
    ta = torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
    tb = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16)
    assert np.array_equal(orc.bf16_add_bits(a, b), torch_bits(ta + tb))


def test_moe_layer_fp32_against_float64():
    """out[t] = sum_j w[t, j] FFN_{idx[t, j]}(x[t]) + FFN_shared(x[t]), each FFN
    = (silu(min(x.W1, L)) * clamp(x.W3, -L, L)) . W2 -- evaluated in float64
    with explicit index sums; ids < 0 and absent experts skipped."""
    rng = np.random.default_rng(11)
    m, d, i, n_exp, k = 3, 96, 64, 6, 2
    xb = orc.f32_to_bf16(rng.standard_normal((m, d)).astype(np.float32))
    mats = {e: [orc.f32_to_bf16((rng.standard_normal(s) * 0.2).astype(np.float32))
                for s in ((i, d), (i, d), (d, i))] for e in range(n_exp + 1)}
    experts = {e: dict(zip(("w1_bf16", "w3_bf16", "w2_bf16"), mats[e])) for e in range(n_exp) if e != 2}
    shared = dict(zip(("w1_bf16", "w3_bf16", "w2_bf16"), mats[n_exp]))
    idx = np.array([[0, 2], [4, -1], [5, 1]], dtype=np.int64)
    w = np.array([[0.7, 0.3], [1.1, 0.5], [0.2, 0.9]], dtype=np.float32)
    got = orc.moe_layer_fp32(xb, idx, w, experts, shared, LIMIT).astype(np.float64)

    def ffn64(xr, w1, w3, w2):
        x64 = orc.bf16_to_f32(xr).astype(np.float64)
        a, b, c = (orc.bf16_to_f32(t).astype(np.float64) for t in (w1, w3, w2))
        g = np.array([sum(x64[c_] * a[r, c_] for c_ in range(d)) for r in range(i)])
        u = np.array([sum(x64[c_] * b[r, c_] for c_ in range(d)) for r in range(i)])
        g = np.minimum(g, LIMIT)
        u = np.clip(u, -LIMIT, LIMIT)
        act = g / (1.0 + np.exp(-g)) * u
        return np.array([sum(act[r] * c[o, r] for r in range(i)) for o in range(d)])

    ref = np.zeros((m, d))
    for t in range(m):
        for j in range(k):
            e = int(idx[t, j])
            if e >= 0 and e in experts:
                ref[t] += float(w[t, j]) * ffn64(xb[t], *mats[e])
        ref[t] += ffn64(xb[t], *mats[n_exp])
    err = np.abs(got - ref)
    assert err.max() <= 1e-5 * np.abs(ref).max(), err.max()


def test_router_logit_definition_divergence_is_only_near_ties():
    """Config-1 distributions (x ~ N(0,1), gate ~ N(0,0.02), bias ~ N(0,0.01),
    D = 4096, 256 experts, top-6), 10^4 tokens over 4 gates.  The oracle (and
    the device) round the exact dot product once; the reference rounds an
    fp32-accumulated sum (torch's bf16 matmul).  Where the two logits differ
    the top-6 may change only between experts whose biased logits are within
    two bf16 steps of each other (one from the sum, one from the bias add);
    the rate is printed."""
    rng = np.random.default_rng(2026)
    d, n_exp, k, per_gate = 4096, 256, 6, 2500
    n_tok = n_logit_diff = n_set_diff = n_order_diff = 0
    worst_w = 0.0
    for _ in range(4):
        gate = orc.f32_to_bf16((rng.standard_normal((n_exp, d)) * 0.02).astype(np.float32))
        bias = (rng.standard_normal(n_exp) * 0.01).astype(np.float32)
        x = orc.f32_to_bf16(rng.standard_normal((per_gate, d)).astype(np.float32))
        idx, w, _, lg = orc.router(x, gate, bias, k, 1.5, return_scores=True)
        xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
        gt = torch.from_numpy(gate.view(np.int16)).view(torch.bfloat16)
        logits = torch.matmul(xt, gt.t()) + torch.from_numpy(bias).to(torch.bfloat16)
        scores = F.softplus(logits.float()).sqrt()
        _, order = torch.sort(scores, dim=1, descending=True, stable=True)
        ridx = order[:, :k].numpy()
        raw = scores.gather(1, order[:, :k])
        rw = (raw / raw.sum(-1, keepdim=True).clamp(min=1e-20) * 1.5).numpy()
        tl = torch_bits(logits)
        n_tok += per_gate
        n_logit_diff += int(np.sum(tl != lg))
        # away from cancellation (|logit| >= 1/4; the top-6 sit near +3) the two
        # definitions differ by at most one bf16 step before the bias add, two after it
        big = np.abs(orc.bf16_to_f32(lg)) >= 0.25
        assert bf16_steps_apart(tl, lg)[big].max() <= 2
        if n_tok == per_gate:
            ub = orc.logits_bf16(x[:500], gate)
            tub = torch_bits(torch.matmul(xt[:500], gt.t()))
            assert bf16_steps_apart(tub, ub)[np.abs(orc.bf16_to_f32(ub)) >= 0.25].max() <= 1
        for t in np.nonzero(np.any(ridx != idx, axis=1))[0]:
            mine, theirs = set(idx[t].tolist()), set(ridx[t].tolist())
            if mine == theirs:
                n_order_diff += 1
            else:
                n_set_diff += 1
            # every expert that moved is within one bf16 step of one it swapped with
            moved = [e for j, e in enumerate(idx[t]) if ridx[t, j] != e]
            for e in moved:
                partners = [int(ridx[t, j]) for j in range(k) if ridx[t, j] != idx[t, j]]
                partners += [int(v) for v in (mine ^ theirs)]
                assert min(bf16_steps_apart(lg[t, [e]], lg[t, [p]])[0] for p in partners if p != e) <= 2, t
        same = np.all(ridx == idx, axis=1)
        worst_w = max(worst_w, float(np.max(np.abs(rw[same] - w[same]) / np.abs(w[same]))))
    print(f"[router divergence] {n_tok} tokens: logits differing {n_logit_diff} of {n_tok * n_exp} "
          f"({n_logit_diff / (n_tok * n_exp):.2e}); top-6 set differs {n_set_diff}, order only {n_order_diff}; "
          f"max weight rel diff where ids agree {worst_w:.2e}")
    assert (n_set_diff + n_order_diff) / n_tok < 0.01
    assert worst_w < 2e-2


class ToyStack(StackOracle):
    """A StackOracle whose stack is replaced by a known next-token function f and
    a known draft function: forward_stack returns the ids, logits a one-hot row
    at f(id).  Exercises decode_step / generate (the emission rule) only."""

    def __init__(self, vocab, f, draft):
        self.vocab, self.f, self.draft, self.final_norm = vocab, f, draft, None

    def forward_stack(self, ids):
        return np.asarray(ids, dtype=np.int64)

    def logits(self, h, norm_w):
        out = np.zeros((len(h), self.vocab), dtype=np.float32)
        out[np.arange(len(h)), [self.f(int(t)) for t in h]] = 1.0
        return orc.f32_to_bf16(out)

    def drafts(self, h_last, tok, n=2, margins=None):
        return self.draft(tok, n)


def reference_loop(first, steps, f, draft, n_draft):
    """engine.py:2809-2922 at temperature 0 without stop tokens or a length cap:
    generated gets A = argmax; then the drafts from A, one verify of [A, drafts]
    (accept while pred[i] == combined[i + 1], _mtp_verify_batched
    engine.py:2487-2497), the accepted drafts, and the bonus token, which is
    also the next token to forward; with none accepted the next token is A."""
    generated, accepted, next_id = [], [], first
    for _ in range(steps):
        a = f(next_id)
        generated.append(a)
        next_id = a
        if n_draft == 0:
            accepted.append(0)
            continue
        drafts = draft(a, n_draft)
        combined = [a] + drafts
        n_acc, bonus_row = 0, len(combined) - 1
        for pos in range(len(combined) - 1):
            if f(combined[pos]) == combined[pos + 1]:
                n_acc += 1
            else:
                bonus_row = pos
                break
        accepted.append(n_acc)
        if n_acc > 0:
            generated.extend(drafts[:n_acc])
            next_id = f(combined[bonus_row])
            generated.append(next_id)
    return generated, accepted


@pytest.mark.parametrize("n_draft", [0, 1, 2, 3])
def test_generate_emission_rule_matches_reference_loop(n_draft):
    V = 97
    f = lambda t: (t * 31 + 7) % V

    def draft(tok, n):  # right, right-then-wrong or wrong, by token
        out, t = [], tok
        for j in range(n):
            t = f(t)
            out.append((t + 1) % V if (tok + j) % 3 == 0 else t)
        return out

    so = ToyStack(V, f, draft)
    got = so.generate(5, 12, n_draft=n_draft)
    ref = reference_loop(5, 12, f, draft, n_draft)
    assert got == ref
    if n_draft:
        assert 0 in ref[1] and max(ref[1]) >= 1


def test_softplus_matches_torch_across_its_threshold():
    """F.softplus (beta 1, threshold 20: x itself above 20) as router.py:30 calls it."""
    x = np.concatenate([np.linspace(-90, 90, 20001), [19.99, 20.0, 20.01, -0.0, 0.0]]).astype(np.float32)
    ref = F.softplus(torch.from_numpy(x)).numpy()
    got = orc.softplus_f32(x)
    np.testing.assert_allclose(got, ref, rtol=4e-7, atol=1e-30)  # libm exp/log1p: within 3 ulp
    assert np.array_equal(got[x > 20], x[x > 20])


def test_cpu_ref_route_matches_oracle():
    """oracle/cpu_ref.py (the timed CPU baseline: the reference's torch route)
    against the numpy/C oracle: FP4 and FP8 dequant bit for bit, router ids
    and weights, the union route + shared add within one bf16 step of
    moe_layer_reference, and the greedy acceptance."""
    from oracle import cpu_ref
    rng = np.random.default_rng(31)
    n, k = 64, 256
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    e8 = rng.integers(119, 125, (n, k // 32), dtype=np.uint8)
    got = cpu_ref.dequant_fp4(torch.from_numpy(packed), torch.from_numpy(e8))
    assert np.array_equal(torch_bits(got), orc.dequant_fp4(packed, e8))
    q = orc.gen_e4m3(orc.key(3, 1), 256 * 384).reshape(256, 384)
    sc = rng.uniform(0.5, 2.0, (2, 3)).astype(np.float32) / 448
    got8 = cpu_ref.dequant_fp8(torch.from_numpy(q), torch.from_numpy(sc))
    assert np.array_equal(torch_bits(got8), orc.dequant_fp8(q, sc))
    # router on exact-sum inputs
    x, _ = exact_sum_inputs(rng, 3, 64, 8)
    gate = (rng.integers(-15, 16, (32, 64)) / 16.0).astype(np.float32)
    bias = (rng.integers(-16, 17, 32) / 64.0).astype(np.float32)
    idx, w = cpu_ref.router(bf16t(x), bf16t(gate), torch.from_numpy(bias), 6, 1.5)
    ridx, rw = orc.router(orc.f32_to_bf16(x), orc.f32_to_bf16(gate), bias, 6, 1.5)
    assert np.array_equal(idx.numpy(), ridx)
    np.testing.assert_allclose(w.numpy(), rw, rtol=1e-6)
    # union route + shared on FP4 experts (per-call dequant inside cpu_ref)
    d, i, n_exp = 128, 128, 6  # one 128 x 128 scale block per shared matrix
    xb = orc.f32_to_bf16(rng.integers(-6, 7, (3, d)).astype(np.float32))
    raw, experts = {}, {}
    for e in range(n_exp):
        mats = [(rng.integers(0, 256, (i, d // 2), dtype=np.uint8), rng.integers(119, 125, (i, d // 32), dtype=np.uint8)),
                (rng.integers(0, 256, (i, d // 2), dtype=np.uint8), rng.integers(119, 125, (i, d // 32), dtype=np.uint8)),
                (rng.integers(0, 256, (d, i // 2), dtype=np.uint8), rng.integers(119, 125, (d, i // 32), dtype=np.uint8))]
        raw[e] = tuple(torch.from_numpy(t) for pair in mats for t in pair)
        experts[e] = {nm: orc.dequant_fp4(p, s) for nm, (p, s) in zip(("w1_bf16", "w3_bf16", "w2_bf16"), mats)}
    sq = [orc.gen_e4m3(orc.key(4, j), 128 * 128).reshape(128, 128) for j in range(3)]
    ss = [np.array([[rng.uniform(0.5, 2.0) / 448]], dtype=np.float32) for _ in range(3)]
    shared_raw = (torch.from_numpy(sq[0]), torch.from_numpy(ss[0]), torch.from_numpy(sq[1]), torch.from_numpy(ss[1]),
                  torch.from_numpy(sq[2]), torch.from_numpy(ss[2]))
    shared = {nm: orc.dequant_fp8(q_, s_) for nm, q_, s_ in zip(("w1_bf16", "w3_bf16", "w2_bf16"), sq, ss)}
    tid = np.array([[0, 2, 5], [1, 2, -1], [4, 3, 0]], dtype=np.int64)
    tw = rng.uniform(0.1, 1.0, (3, 3)).astype(np.float32)
    xt = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16)
    y = cpu_ref.moe_ffn(xt, torch.from_numpy(tid), torch.from_numpy(tw), raw.get, shared_raw)
    ref = orc.moe_layer_reference(xb, tid, tw, experts, shared, LIMIT)
    assert bf16_steps_apart(torch_bits(y), ref).max() <= 1
    # acceptance
    lg = np.zeros((3, 10), dtype=np.float32)
    lg[0, 4], lg[1, 7], lg[2, 1] = 1, 1, 1
    for cid, want in (([9, 4, 7], (2, 2)), ([9, 4, 6], (1, 1)), ([9, 5, 7], (0, 0))):
        _, n_acc, row = cpu_ref.lm_head_accept(torch.eye(3, dtype=torch.bfloat16), bf16t(lg.T.copy()), cid)
        assert (n_acc, row) == want == orc.mtp_accept(orc.f32_to_bf16(lg), cid)
