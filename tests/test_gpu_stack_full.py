"""The decode stack at full size: 43 MoE layers x 256 FP4 experts + FP8 shared
experts, D = 4096, I = 2048, V = 129,280, 3 hash layers, MTP block (the
decode workload of the reference's DeepSeek-V4-class model with attention
replaced by a fixed residual).

- Weights: samples of the device's synthetic weights equal the oracle's
  generators (lm_head rows, gates, the hash table, one expert's bytes).
- Teacher-forced layers 0 (hash), 3 and 42 and the MTP block: from the device's
  own layer input, the residual add is bit-exact, RMSNorm within one bf16 step,
  expert ids bit-exact, the FFN within max-abs 2e-2 / rel-L2 1e-3 of the fp32
  oracle.
- Token streams: the next token is a function f of the current one (no
  attention), so 8 graph-replayed decode steps with MTP verify must emit the
  plain greedy chain f(f(...)), whatever the drafts; forced perfect, half-right
  and wrong drafts must be accepted 2 / 1 / 0 per step and keep the chain.
- _mtp_verify_batched at full vocabulary: empty drafts -> (0, None), all
  accepted, partial, rejected (the reference's cases, tests/test_mtp.py:342-456),
  bonus logits = the verify's own row.
- The layer kernels' status word stays 0.
"""
import numpy as np
import pytest
import torch

from home_seek_amd import ops, stack
from oracle import oracle as orc
from oracle.stack import StackOracle, bf16_add

pytestmark = pytest.mark.gpu

SEED, NL, E, D, I, V, K = 90210, 43, 256, 4096, 2048, 129280, 6


@pytest.fixture(scope="module")
def eng(dev):
    e = stack.build_stack(SEED, NL, E, D, I, V, K, device=dev)
    torch.cuda.synchronize()
    yield e
    del e
    torch.cuda.empty_cache()


@pytest.fixture(scope="module")
def so():
    return StackOracle(SEED, NL, E, D, I, V, K)


def np16(t: torch.Tensor) -> np.ndarray:
    return orc.to_np_bf16(t.reshape(-1, t.shape[-1]))


def check_ffn(got: np.ndarray, ref: np.ndarray, what: str):
    err = got.astype(np.float64) - ref.astype(np.float64)
    rel = np.linalg.norm(err) / np.linalg.norm(ref)
    mx = np.abs(err).max()
    print(f"[{what}] rel-L2 {rel:.3e} max-abs {mx:.3e}")
    assert rel <= 1e-3 and mx <= 2e-2, (what, rel, mx)


def within_one_step(got: np.ndarray, ref: np.ndarray) -> bool:
    g, r = orc.bf16_to_f32(got), orc.bf16_to_f32(ref)
    return bool(np.all(np.abs(g - r) <= np.abs(r) * 2.0 ** -7))


def device_next(eng, tok: int) -> int:
    _, hf = eng._forward_stack(torch.tensor([[tok]], dtype=torch.int64, device=eng.device))
    _, pred, _ = ops.lm_head_accept(hf, eng.lm_head, None, want_logits=False)
    return int(pred.item())


def chain(first: int, n: int, f) -> list:
    out, t = [], first
    for _ in range(n):
        t = f(t)
        out.append(t)
    return out


def test_full_size_weights_match_oracle(eng, so):
    rows = [0, 1, 77777, V - 1]
    assert np.array_equal(np16(eng.lm_head[rows]), so.lm_head[rows])
    for l in (0, 3, 42):
        lw = eng._get_layer_weights(l)
        assert np.array_equal(np16(lw["ffn.gate.weight"]), so.layers[l]["gate"]), l
        assert np.array_equal(np16(lw["attn.residual"])[0], so.layers[l]["residual"]), l
    assert np.array_equal(eng._get_layer_weights(0)["ffn.gate.tid2eid"].cpu().numpy(), so.layers[0]["tid2eid"])
    ex = so.expert(42, 255)
    views = eng.store.expert_views(42, 255)
    for name, t in zip(("w1", "w1_scale", "w3", "w3_scale", "w2", "w2_scale"), views):
        assert np.array_equal(t.view(torch.uint8).cpu().numpy(), ex[name]), name


def test_teacher_forced_layers_and_mtp(eng, so):
    tok = 4242
    ids = torch.tensor([[tok]], dtype=torch.int64, device=eng.device)
    h = eng._embed(ids)
    for l in range(NL):
        lw = eng._get_layer_weights(l)
        if l in (0, 3, 42):
            ref = so.layer(np16(h), so.layers[l], l, [tok])
            h1 = h + lw["attn.residual"]
            assert np.array_equal(np16(h1), ref["h1"]), l
            hn = ops.rms_norm(h1.reshape(-1, D), lw["ffn_norm.weight"]).reshape(h1.shape)
            assert within_one_step(np16(hn), ref["hn"]), l
            f32 = torch.empty(1, D, dtype=torch.float32, device=eng.device)
            eng._forward_ffn(hn, lw, l, ids, out_f32=f32)
            f_ref, idx_ref = so.ffn(np16(hn), so.layers[l], l, [tok])
            assert np.array_equal(eng._last_routed_idx.reshape(1, K).cpu().numpy(), idx_ref), l
            check_ffn(f32.cpu().numpy(), f_ref, f"layer {l}")
        h, _ = eng._forward_layer(h, lw, l, ids)
    assert ops.moe_layer_status(eng.device) == 0
    # the MTP block's layer, from the device's own input (engine.py:2251-2339 stand-in)
    a = device_next(eng, tok)
    mw = eng._mtp_weights
    at = torch.tensor([[a]], dtype=torch.int64, device=eng.device)
    e = ops.rms_norm(eng._embed(at).reshape(1, D), mw["enorm.weight"])
    h_in = (ops.rms_norm(h.reshape(1, D), mw["hnorm.weight"]) + e).reshape(1, 1, D)
    ref = so.layer(np16(h_in), so.mtp["layer"], NL, [a])
    lw = mw["layer"]
    h1 = h_in + lw["attn.residual"]
    assert np.array_equal(np16(h1), ref["h1"])
    hn = ops.rms_norm(h1.reshape(-1, D), lw["ffn_norm.weight"]).reshape(h1.shape)
    assert within_one_step(np16(hn), ref["hn"])
    f32 = torch.empty(1, D, dtype=torch.float32, device=eng.device)
    eng._forward_ffn(hn, lw, NL, at, out_f32=f32)
    f_ref, idx_ref = so.ffn(np16(hn), so.mtp["layer"], NL, [a])
    assert np.array_equal(eng._last_routed_idx.reshape(1, K).cpu().numpy(), idx_ref)
    check_ffn(f32.cpu().numpy(), f_ref, "MTP layer")


def test_graph_decode_emits_the_greedy_chain(eng):
    first = 31337
    tokens, accs = eng.generate_greedy(first, 8, graph=True)
    print(f"tokens {tokens}, accepted per step {accs}")
    assert len(tokens) == 8 + sum(a + 1 for a in accs if a > 0)
    assert eng.generate_greedy(first, 8, graph=False) == (tokens, accs)
    assert tokens == chain(first, len(tokens), lambda t: device_next(eng, t))
    assert ops.moe_layer_status(eng.device) == 0


@pytest.mark.parametrize("kind,want", [("perfect", 2), ("half", 1), ("wrong", 0)])
def test_forced_drafts_keep_the_greedy_chain(eng, kind, want):
    def drafts_on_device(last_hidden, num_draft=2, temperature=0.0, last_token_id=None):
        a = int(last_token_id.reshape(-1)[0].item())
        d0 = device_next(eng, a)
        d1 = device_next(eng, d0)
        if kind == "half":
            d1 = (d1 + 1) % V
        elif kind == "wrong":
            d0 = (d0 + 1) % V
        return torch.tensor([[d0, d1]], dtype=torch.int64, device=eng.device), 2

    eng._mtp_generate_draft = drafts_on_device
    try:
        tokens, accs = eng.generate_greedy(2024, 3, graph=False)
    finally:
        del eng._mtp_generate_draft
    assert accs == [want] * 3
    assert tokens == chain(2024, len(tokens), lambda t: device_next(eng, t))
    assert ops.moe_layer_status(eng.device) == 0


def test_mtp_verify_batched_at_full_vocab(eng):
    dev = eng.device
    assert eng._mtp_verify_batched(torch.zeros(1, 0, dtype=torch.int64, device=dev), 0.0) == (0, None)
    a = device_next(eng, 5)
    d0 = device_next(eng, a)
    d1 = device_next(eng, d0)
    pos0 = eng._global_pos
    for drafts, want, row in (([d0, d1], 2, 2), ([d0, (d1 + 1) % V], 1, 1), ([(d0 + 1) % V, d1], 0, 0)):
        n, bonus = eng._mtp_verify_batched(torch.tensor([drafts], dtype=torch.int64, device=dev), 0.0,
                                           main_pred_id=torch.tensor([[a]], dtype=torch.int64, device=dev))
        assert n == want and eng._global_pos == pos0 + n, drafts
        eng._global_pos = pos0
        combined = torch.tensor([[a] + drafts], dtype=torch.int64, device=dev)
        _, hf = eng._forward_stack(combined)
        logits, pred, _ = ops.lm_head_accept(hf, eng.lm_head, combined.reshape(-1))
        assert torch.equal(bonus, logits[row:row + 1]), drafts
        # the bonus token is the greedy continuation of the last accepted token
        want_tok = (d0, d1, device_next(eng, d1))[row]
        assert int(pred[row].item()) == want_tok
    assert ops.moe_layer_status(dev) == 0


def test_full_size_decode_step_teacher_forced(eng):
    """Every kernel call of one full-size decode step (the 43-layer M=1
    forward, the MTP block's two drafts, the T=3 verify of [A, d0, d1] and the
    four lm_head passes), checked against the oracle on the inputs the device
    gave it: each residual add + RMSNorm, in its own launch or at the end of a
    layer launch (sums bit-exact, norm within one bf16 step), each layer's FFN
    (the same layer run without its norm tail: expert ids bit-exact, output
    within one bf16
    step plus the 2e-2 bar), each lm_head pass (logits' argmax, accepted count
    and bonus row bit-exact), and the step's row built from those decisions.
    The synthetic stack cannot be compared free-running: its residual stream
    grows to ~1e5 and each layer's bf16 roundings of sums that agree to ~2e-6
    flip a few elements by a whole bf16 step, which the next layers amplify
    (relative difference 1e-4 after one layer, 1e-2 after seven, where the
    first top-6 changes); teacher forcing checks every computation of the
    step instead.  The oracle regenerates each expert on use (16 threads)."""
    import time
    from home_seek_amd.engine import GreedyDecoder
    calls = []
    inner_ffn, inner_norm, inner_head = eng._forward_ffn, ops.add_rms_norm, ops.lm_head_accept
    inner_ffn_norm = eng._forward_ffn_norm

    def ffn(hn, lw, layer_idx, input_ids=None, out_f32=None):
        out, used = inner_ffn(hn, lw, layer_idx, input_ids, out_f32)
        calls.append(("ffn", np16(hn), lw, layer_idx, None if input_ids is None else input_ids.reshape(-1).tolist(),
                      np16(out), eng._last_routed_idx.reshape(-1, K).cpu().numpy()))
        return out, used

    def norm(x, weight, add=None, residual=None, eps=1e-6, want_sum=False):
        h, hn = inner_norm(x, weight, add=add, residual=residual, eps=eps, want_sum=True)
        calls.append(("norm", np16(x), None if add is None else np16(add),
                      None if residual is None else np16(residual.reshape(1, -1))[0], np16(weight.reshape(1, -1))[0],
                      np16(h), np16(hn)))
        return (h if want_sum else None), hn

    def head(h, lm_head, ids=None, want_logits=True, pred=None):
        lg, pred, res = inner_head(h, lm_head, ids, want_logits, pred=pred)
        calls.append(("head", np16(h), None if ids is None else ids.reshape(-1).tolist(), pred.cpu().tolist(),
                      res.cpu().tolist()))
        return lg, pred, res

    def ffn_norm(hn, lw, layer_idx, input_ids, h, weight, residual=None, ids_owned=False):
        # the layer's FFN output from the same launch without its tail (the tail
        # variant's own output is the same, bit for bit), then the fused launch
        out, _ = ffn(hn, lw, layer_idx, input_ids)
        fused = inner_ffn_norm(hn, lw, layer_idx, input_ids, h, weight, residual, ids_owned=ids_owned)
        assert fused is not None
        calls.append(("norm", np16(h), np16(out), None if residual is None else np16(residual.reshape(1, -1))[0],
                      np16(weight.reshape(1, -1))[0], np16(fused[0]), np16(fused[1])))
        calls.append(("tail",))
        return fused

    eng._forward_ffn, eng._forward_ffn_norm = ffn, ffn_norm
    ops.add_rms_norm, ops.lm_head_accept = norm, head
    try:
        dec = GreedyDecoder(eng, 1, graph=False)
        dec.reset(31337)
        dec.run(1)
    finally:
        del eng._forward_ffn, eng._forward_ffn_norm
        ops.add_rms_norm, ops.lm_head_accept = inner_norm, inner_head
    row = dec.rows[0].cpu().tolist()
    assert ops.moe_layer_status(eng.device) == 0
    t0 = time.time()
    so = StackOracle(SEED, NL, E, D, I, V, K, cache=False, workers=16)
    kinds = [c[0] for c in calls]
    assert kinds.count("ffn") == 2 * NL + 2 and kinds.count("head") == 4, kinds
    assert kinds.count("tail") == 2 * NL + 2, kinds  # every layer launch ends with the next norm
    heads, worst = [], 0.0
    for c in calls:
        if c[0] == "norm":
            _, x, add, res, w, h, hn = c
            ref = x if add is None else bf16_add(x, add)
            ref = ref if res is None else bf16_add(ref, res[None, :])
            assert np.array_equal(h, ref)
            assert within_one_step(hn, orc.rms_norm(h, w))
        elif c[0] == "ffn":
            _, hn, lw, layer, ids, out, idx = c
            lwo = so.mtp["layer"] if layer == NL else so.layers[layer]
            f_ref, idx_ref = so.ffn(hn, lwo, layer, ids)
            assert np.array_equal(idx, idx_ref), layer
            g, r = orc.bf16_to_f32(out), orc.bf16_to_f32(orc.f32_to_bf16(f_ref))
            worst = max(worst, float(np.max(np.abs(g - r))))
            assert not np.any(np.abs(g - r) > np.abs(r) * 2.0 ** -7 + 2e-2), layer
        elif c[0] == "head":
            _, h, ids, pred, res = c
            lg = orc.logits_bf16(h, so.lm_head)
            assert pred == so.argmax(lg)
            if ids is not None and len(ids) > 1:
                assert res == list(orc.mtp_accept(lg, ids))
            heads.append((pred, res))
    # the row from the checked decisions: A, the drafts, the verify's bonus
    a, d0, d1 = heads[0][0][0], heads[1][0][0], heads[2][0][0]
    v_pred, (n_acc, bonus_row) = heads[3]
    assert row == [a, d0, d1, v_pred[bonus_row]]
    assert int(dec.n_accs[0].item()) == n_acc
    print(f"row {row}, accepted {n_acc}; {len(calls)} calls checked (FFN max-abs vs bf16(oracle) {worst:.3g}); "
          f"oracle {time.time() - t0:.0f} s")
