"""GPU parity of the MoE-only decode stack (layers, MTP drafts, verify, decode loop)
against the CPU stack oracle, at a small shape the oracle runs in seconds.

Per layer the device is teacher-forced: the oracle recomputes each layer from
the device's own input, so errors do not compound.  Bars: the residual add is
bit-exact (a bf16 add), RMSNorm within one bf16 step, router and hash expert
ids bit-exact, the FFN within max-abs 2e-2 / rel-L2 1e-3 of the fp32 oracle.

Token streams: with attention replaced by a fixed residual the next token is a
function f of the current one, so a greedy stream with MTP verify must equal
the plain chain f(f(...f(first))) whatever the drafts are (speculative
decoding only changes how many tokens a step emits).  That invariant is
checked with the MTP block's drafts, with perfect drafts (every step accepts
both), with a half-right draft (accepts one) and with wrong drafts (accepts
none), and the free-running stream is compared with the oracle's.
"""
import numpy as np
import pytest
import torch

from home_seek_amd import ops, stack
from oracle import oracle as orc
from oracle.stack import StackOracle

pytestmark = pytest.mark.gpu

SEED, NL, E, D, I, V, K, NH = 4242, 4, 16, 512, 512, 1024, 6, 1


@pytest.fixture(scope="module")
def model(dev):
    eng = stack.build_stack(SEED, n_layers=NL, n_experts=E, d=D, i=I, vocab=V, top_k=K, n_hash=NH, device=dev)
    torch.cuda.synchronize()
    return eng, StackOracle(SEED, NL, E, D, I, V, K, NH)


def np16(t: torch.Tensor) -> np.ndarray:
    return orc.to_np_bf16(t.reshape(-1, t.shape[-1]))


def within_one_step(got: np.ndarray, ref: np.ndarray) -> bool:
    g, r = orc.bf16_to_f32(got), orc.bf16_to_f32(ref)
    return bool(np.all(np.abs(g - r) <= np.abs(r) * 2.0 ** -7))


def check_ffn(got: np.ndarray, ref: np.ndarray, what: str):
    err = got.astype(np.float64) - ref.astype(np.float64)
    rel = np.linalg.norm(err) / np.linalg.norm(ref)
    mx = np.abs(err).max()
    print(f"[{what}] rel-L2 {rel:.3e} max-abs {mx:.3e}")
    assert rel <= 1e-3 and mx <= 2e-2, (what, rel, mx)


def device_next(eng, ids: torch.Tensor) -> torch.Tensor:
    """Greedy next token of each id in ids [1, T] (plain forward, no MTP) -> [T] int64."""
    _, hf = eng._forward_stack(ids.reshape(1, -1))
    _, pred, _ = ops.lm_head_accept(hf, eng.lm_head, None, want_logits=False)
    return pred


def test_synthetic_weights_match_oracle(model):
    eng, so = model
    lw = eng._get_layer_weights(0)
    assert np.array_equal(np16(lw["ffn.gate.weight"]), so.layers[0]["gate"])
    assert np.array_equal(lw["ffn.gate.tid2eid"].cpu().numpy(), so.layers[0]["tid2eid"])
    assert np.array_equal(np16(eng.lm_head), so.lm_head)
    for l in range(NL):
        assert np.array_equal(np16(eng._get_layer_weights(l)["attn.residual"])[0], so.layers[l]["residual"])
    # hash ids of one token are distinct (odd step, power-of-two E)
    t = so.layers[0]["tid2eid"]
    assert all(len(set(r)) == K for r in t.tolist())


@pytest.mark.parametrize("ids", [[7], [3, 900, 3], [1023, 0, 512]])
def test_layers_match_oracle_teacher_forced(model, ids):
    eng, so = model
    tid = torch.tensor([ids], dtype=torch.int64, device=eng.device)
    h = eng._embed(tid)
    assert np.array_equal(np16(h), so.embed(ids))
    for l in range(NL):
        lw = eng._get_layer_weights(l)
        ref = so.layer(np16(h), so.layers[l], l, ids)
        h1 = h + lw["attn.residual"]
        assert np.array_equal(np16(h1), ref["h1"]), l
        hn = ops.rms_norm(h1.reshape(-1, D), lw["ffn_norm.weight"]).reshape(h1.shape)
        assert within_one_step(np16(hn), ref["hn"]), l
        f32 = torch.empty(len(ids), D, dtype=torch.float32, device=eng.device)
        ffn, _ = eng._forward_ffn(hn, lw, l, tid, out_f32=f32)
        # the FFN from the device's own normed input
        f_ref, idx_ref = so.ffn(np16(hn), so.layers[l], l, ids)
        assert np.array_equal(eng._last_routed_idx.reshape(len(ids), K).cpu().numpy(), idx_ref), l
        check_ffn(f32.cpu().numpy(), f_ref, f"layer {l} T={len(ids)}")
        assert np.array_equal(np16(ffn), orc.f32_to_bf16(f32.cpu().numpy()))
        h_next, _ = eng._forward_layer(h, lw, l, tid)
        assert np.array_equal(np16(h_next), np16(h1 + ffn)), l
        h = h_next


def test_verify_rows_equal_single_token_forwards(model):
    """No attention: row t of a T=3 verify is the M=1 forward of token t, bit for bit."""
    eng, _ = model
    ids = torch.tensor([[5, 77, 5]], dtype=torch.int64, device=eng.device)
    h3, f3 = eng._forward_stack(ids)
    for t in range(3):
        h1, f1 = eng._forward_stack(ids[:, t:t + 1])
        assert torch.equal(h3[0, t], h1[0, 0]) and torch.equal(f3[t], f1[0]), t


def test_fused_stack_equals_layer_loop(model, monkeypatch):
    """The fused chain (the embedding lookup in the first add + norm launch,
    each layer launch ending with the next layer's adds + RMSNorm) gives the
    values of the plain layer loop, bit for bit."""
    eng, _ = model
    ids = torch.tensor([[9, 400, 1000]], dtype=torch.int64, device=eng.device)
    h = eng._embed(ids)
    for l in range(NL):
        h, _ = eng._forward_layer(h, eng._get_layer_weights(l), l, ids)
    hf = eng._final_hidden(h)
    calls = []
    for name in ("add_rms_norm", "embed_add_rms_norm"):
        inner = getattr(ops, name)
        monkeypatch.setattr(ops, name, lambda *a, _n=name, _f=inner, **kw: calls.append(_n) or _f(*a, **kw))
    h2, hf2 = eng._forward_stack(ids)
    assert calls == ["embed_add_rms_norm"]  # the norm tails did the rest
    assert torch.equal(h, h2) and torch.equal(hf, hf2)


def test_mtp_drafts_match_oracle(model):
    eng, so = model
    cur = torch.tensor([[42]], dtype=torch.int64, device=eng.device)
    h, _ = eng._forward_stack(cur)
    a = device_next(eng, cur).reshape(1, 1)
    drafts, n = eng._mtp_generate_draft(h, 2, 0.0, last_token_id=a)
    assert n == 2 and tuple(drafts.shape) == (1, 2)
    assert a.item() == so.next_token(42)
    assert drafts.cpu().tolist()[0] == so.drafts(np16(h), a.item(), 2)


def chain(first: int, n: int, f) -> list:
    out, t = [], first
    for _ in range(n):
        t = f(t)
        out.append(t)
    return out


def test_decode_stream_matches_oracle_and_greedy_chain(model):
    eng, so = model
    steps = 5
    tokens, accs = eng.generate_greedy(11, steps, graph=False)
    margins = []
    ref_tokens, ref_accs = so.generate(11, steps, margins)
    print(f"tokens {tokens} accepted {accs}; smallest oracle top-2 logit gap {min(margins):.3e}")
    assert tokens == ref_tokens and accs == ref_accs
    assert all(0 <= a <= 2 for a in accs) and len(tokens) == steps + sum(a + 1 for a in accs if a > 0)
    f = lambda t: device_next(eng, torch.tensor([[t]], device=eng.device)).item()
    assert tokens == chain(11, len(tokens), f)


@pytest.mark.parametrize("kind,want", [("perfect", 2), ("half", 1), ("wrong", 0)])
def test_acceptance_paths_keep_the_greedy_chain(model, kind, want):
    eng, so = model

    def drafts_on_device(last_hidden, num_draft=2, temperature=0.0, last_token_id=None):
        d0 = device_next(eng, last_token_id.reshape(1, 1)).reshape(1, 1)
        d1 = device_next(eng, d0).reshape(1, 1)
        if kind == "half":
            d1 = (d1 + 1) % V
        elif kind == "wrong":
            d0 = (d0 + 1) % V
        return torch.cat([d0, d1], dim=-1), 2

    def drafts_oracle(h, a):
        d0 = so.next_token(a)
        d1 = so.next_token(d0)
        return [d0, (d1 + 1) % V] if kind == "half" else [(d0 + 1) % V, d1] if kind == "wrong" else [d0, d1]

    eng._mtp_generate_draft = drafts_on_device
    try:
        tokens, accs = eng.generate_greedy(300, 3, graph=False)
    finally:
        del eng._mtp_generate_draft
    assert accs == [want] * 3
    assert (tokens, accs) == so.generate(300, 3, draft_fn=drafts_oracle)
    assert tokens == chain(300, len(tokens), so.next_token)


def test_graph_replays_equal_eager(model):
    eng, _ = model
    eager = eng.generate_greedy(600, 6, graph=False)
    for _ in range(2):
        assert eng.generate_greedy(600, 6, graph=True) == eager


@pytest.mark.parametrize("n_draft", [0, 1, 3])
def test_draft_counts_match_oracle(model, n_draft):
    """config.mtp_num_draft = 0 is plain greedy decode (one token a step); 1 and
    3 drafts verify T = 2 and T = 4 rows.  Eager and graph streams equal the
    oracle's and the greedy chain; the layer status stays 0."""
    eng, so = model
    old = eng.config.mtp_num_draft
    eng.config.mtp_num_draft = n_draft
    try:
        assert eng.draft_count() == n_draft
        ref = so.generate(77, 4, n_draft=n_draft)
        for graph in (False, True):
            assert eng.generate_greedy(77, 4, graph=graph) == ref, graph
    finally:
        eng.config.mtp_num_draft = old
    tokens, accs = ref
    assert all(0 <= a <= n_draft for a in accs)
    if n_draft == 0:
        assert len(tokens) == 4 and accs == [0] * 4
    assert tokens == chain(77, len(tokens), so.next_token)
    assert ops.moe_layer_status(eng.device) == 0


def test_verify_reads_status_and_accepts(model):
    """_mtp_verify_batched: greedy acceptance of [A, drafts] against the oracle,
    bonus logits of the row the acceptance names, status words read at the
    same sync; no drafts -> (0, None)."""
    eng, so = model
    dev = eng.device
    assert eng._mtp_verify_batched(torch.zeros(1, 0, dtype=torch.int64, device=dev), 0.0) == (0, None)
    a = so.next_token(123)
    d0 = so.next_token(a)
    d1 = so.next_token(d0)
    for drafts, want in (([d0, d1], 2), ([d0, (d1 + 1) % V], 1), ([(d0 + 1) % V, d1], 0)):
        main = torch.tensor([[a]], dtype=torch.int64, device=dev)
        n, bonus = eng._mtp_verify_batched(torch.tensor([drafts], dtype=torch.int64, device=dev), 0.0,
                                           main_pred_id=main)
        assert n == want, drafts
        lv = so.logits(so.forward_stack([a] + drafts), so.final_norm)
        n_ref, row = orc.mtp_accept(lv, [a] + drafts)
        assert n_ref == want
        # the bonus row of the device's own verify logits; its greedy token is the oracle's
        combined = torch.tensor([[a] + drafts], dtype=torch.int64, device=dev)
        _, hf = eng._forward_stack(combined)
        logits, _, _ = ops.lm_head_accept(hf, eng.lm_head, combined.reshape(-1))
        assert torch.equal(bonus, logits[row:row + 1]), drafts
        assert so.argmax(np16(bonus)) == so.argmax(lv[row:row + 1])


def test_status_word_raises_once_and_restores_position(model):
    """A nonzero sticky status word (written from the host: no kernel gives up
    here) makes _mtp_verify_batched (with verify_fallback off) and
    GreedyDecoder.result() raise HsmoeError, restores _global_pos, and is
    cleared by the report, so the next verify runs clean."""
    from home_seek_amd._lib import HsmoeError
    from home_seek_amd.engine import GreedyDecoder
    eng, so = model
    dev = eng.device
    a = so.next_token(55)
    drafts = torch.tensor([[so.next_token(a), 3]], dtype=torch.int64, device=dev)
    main = torch.tensor([[a]], dtype=torch.int64, device=dev)
    assert eng._mtp_verify_batched(drafts, 0.0, main_pred_id=main)[0] == 1  # creates the layer workspaces
    words = ops.moe_layer_status_words(dev)
    assert words and all(int(w.item()) == 0 for w in words)
    pos = eng._global_pos
    words[0].fill_(1 + 4609)
    eng.verify_fallback = False
    try:
        with pytest.raises(HsmoeError):
            eng._mtp_verify_batched(drafts, 0.0, main_pred_id=main)
    finally:
        del eng.verify_fallback
    assert eng._global_pos == pos
    assert ops.moe_layer_status(dev) == 0
    assert eng._mtp_verify_batched(drafts, 0.0, main_pred_id=main)[0] == 1
    dec = GreedyDecoder(eng, 2, graph=False)
    dec.reset(9)
    dec.run(1)
    ops.moe_layer_status_words(dev)[-1].fill_(1 + 4611)
    with pytest.raises(HsmoeError):
        dec.result()
    assert ops.moe_layer_status(dev) == 0
    assert dec.result()[0][0] == so.next_token(9)


def test_loader_entries_match_oracle(model):
    """The reference-shaped loaders: _load_expert_weights gives int8 data and
    fp32 scales equal to the E8M0 values 2^(e-127); _load_bf16_deq and
    _get_shared_expert give the oracle's dequantisations bit for bit; the FP4
    FFN from the fp32-scale entry equals the one from the E8M0 bytes."""
    from home_seek_amd import fused_moe
    eng, so = model
    layer, eid = 1, 5
    ex = so.expert(layer, eid)
    ent = eng._load_expert_weights(layer, eid)
    assert [e[2] for e in ent] == ["fp4_gpu"] * 3
    for (w, s, _), name in zip(ent, ("w1", "w3", "w2")):
        assert w.dtype == torch.int8 and s.dtype == torch.float32
        assert np.array_equal(w.view(torch.uint8).cpu().numpy(), ex[name])
        want = np.ldexp(np.float32(1.0), ex[name + "_scale"].astype(np.int32) - 127).astype(np.float32)
        assert np.array_equal(s.cpu().numpy(), want), name
    for t, name in zip(eng._load_bf16_deq(layer, eid), ("w1", "w3", "w2")):
        assert np.array_equal(np16(t), ex[name + "_bf16"]), name
    sh = so.shared(layer)
    for t, name in zip(eng._get_shared_expert(layer), ("w1", "w3", "w2")):
        assert np.array_equal(np16(t), sh[name + "_bf16"]), name
    x = torch.from_numpy(orc.bf16_to_f32(so._normal(999, 3 * D, 0.0, 1.0).reshape(3, D))).to(
        eng.device, torch.bfloat16)
    (w1, s1, _), (w3, s3, _), (w2, s2, _) = ent
    raw = eng._load_expert_fp4_raw(layer, eid)
    y32 = fused_moe.fused_expert_ffn_triton(x, w1, w3, w2, w1_scale=s1, w3_scale=s3, w2_scale=s2)
    y8 = fused_moe.fused_expert_ffn_triton(x, raw[0], raw[2], raw[4], w1_scale=raw[1], w3_scale=raw[3],
                                           w2_scale=raw[5])
    assert torch.equal(y32, y8)
    ref = orc.expert_ffn_fp32(np16(x), ex["w1_bf16"], ex["w3_bf16"], ex["w2_bf16"], so.limit)
    # the bf16 output adds its own rounding (half a bf16 step) to the FFN bar
    y = y32.float().cpu().numpy().astype(np.float64)
    err = np.abs(y - ref)
    print(f"[fp4_gpu entry FFN] rel-L2 {np.linalg.norm(y - ref) / np.linalg.norm(ref):.3e}")
    assert np.all(err <= 2e-2 + np.abs(ref) * 2.0 ** -8)


def test_checkpoint_round_trip_through_the_loader(model, tmp_path):
    """The small stack written as a safetensors checkpoint in the reference's
    key layout and loaded back with home_seek_amd.checkpoint: every layer's
    FFN (hash layer included) and the MTP block's give the same outputs, bit
    for bit."""
    from safetensors.torch import save_file
    from home_seek_amd import checkpoint
    eng, _ = model
    t = {}
    for l in range(NL + 1):
        base = f"layers.{l}.ffn" if l < NL else "mtp.0.ffn"
        for e in range(E):
            for key, v in zip(checkpoint.expert_keys(f"{base}.experts.{e}"), eng.store.expert_views(l, e)):
                t[key] = v.cpu()
        for key, v in zip(checkpoint.expert_keys(f"{base}.shared_experts"), eng.store.shared_views(l)):
            t[key] = v.cpu()
        lw = eng._get_layer_weights(l) if l < NL else eng._mtp_weights["layer"]
        pre = f"layers.{l}" if l < NL else "mtp.0"
        for short in ("ffn.gate.weight", "ffn.gate.bias", "ffn.gate.tid2eid", "ffn_norm.weight"):
            if short in lw:
                t[f"{pre}.{short}"] = lw[short].cpu()
    for n in ("enorm", "hnorm", "norm"):
        t[f"mtp.0.{n}.weight"] = eng._mtp_weights[f"{n}.weight"].cpu()
    t["embed.weight"] = eng.embed.cpu()
    t["norm.weight"] = eng.norm_weight.cpu()
    save_file({k: v.contiguous() for k, v in t.items()}, str(tmp_path / "model.safetensors"))
    eng2 = checkpoint.load_engine(str(tmp_path), config=eng.config, device=eng.device)
    assert torch.equal(eng2.lm_head, eng.lm_head) and eng2._mtp_weights["layer_idx"] == NL
    ids = torch.tensor([[3, 900, 17]], dtype=torch.int64, device=eng.device)
    hn = torch.randn(1, 3, D, device=eng.device).to(torch.bfloat16)
    for l in range(NL + 1):
        lw = eng._get_layer_weights(l) if l < NL else eng._mtp_weights["layer"]
        lw2 = eng2._get_layer_weights(l) if l < NL else eng2._mtp_weights["layer"]
        a, _ = eng._forward_ffn(hn, lw, l, ids)
        b, _ = eng2._forward_ffn(hn, lw2, l, ids)
        assert torch.equal(a, b), l
    assert ops.moe_layer_status(eng.device) == 0


def test_layer_status_word_fails_the_verify_and_the_decoder(model):
    """A nonzero sticky status word in a layer workspace (written here from the
    host: no kernel gives up) makes _mtp_verify_batched run again on the
    staged kernels (a warning; the values of a clean verify), or raise with
    verify_fallback off, leaving _global_pos where it was; makes
    GreedyDecoder.result() raise; and is reported once (cleared)."""
    from home_seek_amd import _lib
    from home_seek_amd.engine import GreedyDecoder
    eng, _ = model
    dev = eng.device
    main = torch.tensor([[7]], dtype=torch.int64, device=dev)
    drafts = torch.tensor([[5, 6]], dtype=torch.int64, device=dev)
    n0, lg0 = eng._mtp_verify_batched(drafts, main_pred_id=main)  # the layer workspaces exist after this
    words = ops.moe_layer_status_words(dev)
    assert words and ops.moe_layer_status(dev) == 0
    pos = eng._global_pos
    words[0].fill_(1 + 4612)
    with pytest.warns(RuntimeWarning, match="gave up"):
        n1, lg1 = eng._mtp_verify_batched(drafts, main_pred_id=main)
    assert n1 == n0 and torch.equal(lg1, lg0) and eng._global_pos == pos + n0
    assert ops.moe_layer_status(dev) == 0 and eng.use_one_launch_layer
    eng._global_pos = pos
    eng.verify_fallback = False
    try:
        words[0].fill_(1 + 4612)
        with pytest.raises(_lib.HsmoeError, match="gave up"):
            eng._mtp_verify_batched(drafts, main_pred_id=main)
    finally:
        del eng.verify_fallback
    assert eng._global_pos == pos
    assert ops.moe_layer_status(dev) == 0
    n, logits = eng._mtp_verify_batched(drafts, main_pred_id=main)  # a clean verify works again
    assert logits is not None and 0 <= n <= 2
    dec = GreedyDecoder(eng, 2, graph=False)
    dec.reset(11)
    dec.run(1)
    ops.moe_layer_status_words(dev)[0].fill_(1 + 4609)
    with pytest.raises(_lib.HsmoeError, match="gave up"):
        dec.result()
    assert ops.moe_layer_status(dev) == 0
    dec.reset(11)
    dec.run(1)
    tokens, accs = dec.result()
    assert len(tokens) >= 1 and len(accs) == 1
