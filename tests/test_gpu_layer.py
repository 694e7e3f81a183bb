"""GPU parity of the fused one-launch MoE layer (hsmoe_moe_layer_decode).

The fused launch must reproduce router_topk followed by moe_decode bit for bit
(same tiles, same accumulation order), and through them the fp32 oracle within
the task's bar (rel-L2 <= 1e-3, max-abs <= 2e-2 on fp32 outputs).  Its
cross-workgroup handoffs are exercised with calls of every m in [1, 8] sharing
one workspace, absent experts, tables without a shared expert, and HIP graph
replays checked replay by replay.
"""
import numpy as np
import pytest
import torch

from home_seek_amd import expert_store, ops, synthetic
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

D, I, E, K, SEED = 4096, 2048, 256, 6, 31337


@pytest.fixture(scope="module")
def layer(dev):
    store = expert_store.HbmExpertStore(1, E, D, I, dev, with_shared=True)
    store.fill_synthetic(SEED)
    gate, bias = synthetic.router_weights(SEED, 0, E, D, dev)
    torch.cuda.synchronize()
    return store, gate, bias


def staged(x, gate, bias, table, shared, kind=ops.SCALE_E8M0):
    idx, w = ops.router_topk(x, gate, bias, K, 1.5)
    f32 = torch.empty(x.shape[0], D, dtype=torch.float32, device=x.device)
    out, _ = ops.moe_decode(x, idx, w, table, kind, shared, 10.0, out_f32=f32, d=D, i=I)
    return out, f32, idx, w


def fused(x, gate, bias, table, shared, kind=ops.SCALE_E8M0, **kw):
    """(out_bf16, out_f32, idx, w[, logits]) of the fused launch."""
    f32 = torch.empty(x.shape[0], D, dtype=torch.float32, device=x.device)
    res = ops.moe_layer_decode(x, gate, bias, table, kind, shared, I, K, 1.5, 10.0,
                               out_bf16=torch.empty(x.shape[0], D, dtype=torch.bfloat16, device=x.device),
                               out_f32=f32, **kw)
    return (res[0], f32) + tuple(res[2:])


@pytest.mark.parametrize("m", [1, 3, 8])
def test_fused_layer_equals_staged_and_oracle(layer, dev, m):
    store, gate, bias = layer
    x = synthetic.hidden(SEED, 10 + m, m, D, dev)
    a = fused(x, gate, bias, store.table(0), store.shared_entry(0))
    b = staged(x, gate, bias, store.table(0), store.shared_entry(0))
    torch.cuda.synchronize()
    assert ops.moe_layer_status(dev) == 0
    for got, ref, what in zip(a, b, ("bf16", "f32", "idx", "w")):
        assert torch.equal(got, ref), what
    xn = orc.to_np_bf16(x)
    ridx, rw = orc.router(xn, orc.to_np_bf16(gate), bias.cpu().numpy(), K, 1.5)
    assert np.array_equal(a[2].cpu().numpy(), ridx)
    experts = {int(e): orc.gen_fp4_expert(SEED, 0, int(e), D, I) for e in np.unique(ridx)}
    ref = orc.moe_layer_fp32(xn, ridx, a[3].cpu().numpy(), experts, orc.gen_shared_expert(SEED, 0, D, I), 10.0)
    got = a[1].cpu().numpy().astype(np.float64)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    mx = np.abs(got - ref).max()
    print(f"[fused layer M={m}] rel-L2 {rel:.3e} max-abs {mx:.3e}")
    assert rel <= 1e-3 and mx <= 2e-2


def test_fused_layer_logits_and_every_m_sharing_a_workspace(layer, dev):
    store, gate, bias = layer
    for m in (8, 1, 5, 2, 7, 3, 6, 4, 1):
        x = synthetic.hidden(SEED, 100 + m, m, D, dev)
        a = fused(x, gate, bias, store.table(0), store.shared_entry(0), want_logits=True)
        _, _, ref_logits = ops.router_topk(x, gate, bias, K, 1.5, want_logits=True)
        b = staged(x, gate, bias, store.table(0), store.shared_entry(0))
        torch.cuda.synchronize()
        assert torch.equal(a[4], ref_logits), m
        for got, ref, what in zip(a[:4], b, ("bf16", "f32", "idx", "w")):
            assert torch.equal(got, ref), (m, what)
    assert ops.moe_layer_status(dev) == 0


def test_fused_layer_absent_experts_no_shared_no_bias(layer, dev):
    """Absent table entries are skipped (a loader returning None), a layer
    without a shared expert, and a router without bias."""
    store, gate, bias = layer
    x = synthetic.hidden(SEED, 200, 3, D, dev)
    idx, _ = ops.router_topk(x, gate, None, K, 1.5)
    table = store.table(0).clone()
    drop = idx.reshape(-1)[::4]
    table[drop] = 0
    a = fused(x, gate, None, table, None)
    b = staged(x, gate, None, table, None)
    torch.cuda.synchronize()
    assert ops.moe_layer_status(dev) == 0
    for got, ref, what in zip(a, b, ("bf16", "f32", "idx", "w")):
        assert torch.equal(got, ref), what
    # every expert absent: the output is zero
    z = fused(x, gate, None, torch.zeros_like(table), None)
    zs = staged(x, gate, None, torch.zeros_like(table), None)
    torch.cuda.synchronize()
    assert torch.count_nonzero(z[1]) == 0 and torch.count_nonzero(z[0]) == 0
    assert torch.count_nonzero(zs[1]) == 0 and torch.count_nonzero(zs[0]) == 0


@pytest.mark.parametrize("m", [1, 3])
def test_fused_layer_fp32_scales_and_bf16_experts(layer, dev, m):
    """A table in the engine's GPU-tier layout (engine.py:1260-1271): FP4 experts
    with fp32 block scales, some experts as dequantised bf16 weights
    (_load_bf16_deq) and one absent.  Runs of FP4 slots stop at the bf16 ones, so
    the fp32-scale run path and the per-slot path both run in one launch."""
    store, gate, bias = layer
    x = synthetic.hidden(SEED, 500 + m, m, D, dev)
    idx, _ = ops.router_topk(x, gate, bias, K, 1.5)
    ids = sorted(set(idx.cpu().reshape(-1).tolist()))
    absent = ids[0]
    as_bf16 = set(ids[1::3])
    entries = [None] * E
    for eid in ids[1:]:
        w1, s1, w3, s3, w2, s2 = store.expert_views(0, eid)
        if eid in as_bf16:
            ent = (ops.fp4_dequant_bf16(w1, s1), ops.fp4_dequant_bf16(w3, s3), ops.fp4_dequant_bf16(w2, s2))
        else:
            ent = (w1, s1.to(torch.float32), w3, s3.to(torch.float32), w2, s2.to(torch.float32))
        entries[eid] = ent
    table = ops.expert_table(entries, dev)
    a = fused(x, gate, bias, table, store.shared_entry(0), kind=ops.SCALE_F32)
    b = staged(x, gate, bias, table, store.shared_entry(0), kind=ops.SCALE_F32)
    torch.cuda.synchronize()
    assert ops.moe_layer_status(dev) == 0
    for got, ref, what in zip(a, b, ("bf16", "f32", "idx", "w")):
        assert torch.equal(got, ref), what
    experts = {e: orc.gen_fp4_expert(SEED, 0, e, D, I) for e in ids if e != absent}
    ref = orc.moe_layer_fp32(orc.to_np_bf16(x), a[2].cpu().numpy(), a[3].cpu().numpy(), experts,
                             orc.gen_shared_expert(SEED, 0, D, I), 10.0)
    got = a[1].cpu().numpy().astype(np.float64)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    mx = np.abs(got - ref).max()
    print(f"[fused layer fp32 scales + bf16, M={m}] rel-L2 {rel:.3e} max-abs {mx:.3e}")
    assert rel <= 1e-3 and mx <= 2e-2
    # the fp32-scale FP4 experts alone equal the E8M0 table bit for bit
    e8 = store.table(0).clone()
    e8[[absent] + sorted(as_bf16)] = 0
    c = fused(x, gate, bias, e8, store.shared_entry(0))
    only_fp4 = [None if (e == absent or e in as_bf16) else entries[e] for e in range(E)]
    d = fused(x, gate, bias, ops.expert_table(only_fp4, dev), store.shared_entry(0), kind=ops.SCALE_F32)
    torch.cuda.synchronize()
    for got, ref, what in zip(d, c, ("bf16", "f32", "idx", "w")):
        assert torch.equal(got, ref), what


def test_fused_layer_graph_replays(layer, dev):
    """Captured in a HIP graph and replayed, with eager work and host syncs
    between replays; every replay must equal the eager result."""
    store, gate, bias = layer
    xs = [synthetic.hidden(SEED, 300 + j, 1, D, dev) for j in range(3)]
    outs = [torch.empty(1, D, dtype=torch.float32, device=dev) for _ in range(3)]
    idxs = [torch.empty(1, K, dtype=torch.int64, device=dev) for _ in range(3)]
    ws = [torch.empty(1, K, dtype=torch.float32, device=dev) for _ in range(3)]
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for j in range(3):
            ops.moe_layer_decode(xs[j], gate, bias, store.table(0), ops.SCALE_E8M0, store.shared_entry(0), I,
                                 out_f32=outs[j], idx_out=idxs[j], w_out=ws[j])
        torch.cuda.synchronize()
        eager = [o.clone() for o in outs]
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for j in range(3):
                ops.moe_layer_decode(xs[j], gate, bias, store.table(0), ops.SCALE_E8M0, store.shared_entry(0), I,
                                     out_f32=outs[j], idx_out=idxs[j], w_out=ws[j])
    for rep in range(4):
        for o in outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for j in range(3):
            assert torch.equal(outs[j], eager[j]), (rep, j)
        staged(xs[rep % 3], gate, bias, store.table(0), store.shared_entry(0))  # eager work in between
        torch.cuda.synchronize()
    with torch.cuda.stream(s):
        assert ops.moe_layer_status(dev) == 0


def test_fused_layer_rejects_bad_shapes(layer, dev):
    store, gate, bias = layer
    x = synthetic.hidden(SEED, 400, 9, D, dev)
    with pytest.raises(ValueError):
        ops.moe_layer_decode(x, gate, bias, store.table(0), ops.SCALE_E8M0, None, I)


def test_workspace_rearms_before_the_tags_wrap(layer, dev):
    """The launch whose tag reaches 2^31 zeroes the workspace after the control
    words and restarts the epoch at 0 (so tags never wrap onto old words);
    results stay bit-identical across it.  The epoch is set from the host to
    just below the re-arm point."""
    store, gate, bias = layer
    x = synthetic.hidden(SEED, 700, 3, D, dev)
    ref = staged(x, gate, bias, store.table(0), store.shared_entry(0))
    fused(x, gate, bias, store.table(0), store.shared_entry(0))
    ws = ops._workspaces[(dev.index, ops.stream_ptr(dev), "layer")]  # the current one (not the retired)
    epoch = ws[0:4].view(torch.int32)
    epoch.fill_(0x7FFFFFFE)
    ctl = 4096
    for want_epoch in (0x7FFFFFFF, 0, 1):
        a = fused(x, gate, bias, store.table(0), store.shared_entry(0))
        torch.cuda.synchronize()
        assert int(epoch.item()) & 0xFFFFFFFF == want_epoch
        if want_epoch == 0:
            assert int(torch.count_nonzero(ws[ctl:])) == 0
        for got, r, what in zip(a, ref, ("bf16", "f32", "idx", "w")):
            assert torch.equal(got, r), (want_epoch, what)
    assert ops.moe_layer_status(dev) == 0


def routed(x, idx, table, shared, w=None, weight_all=1.0, token_ids=None, k=K, kind=ops.SCALE_E8M0):
    f32 = torch.empty(x.shape[0], D, dtype=torch.float32, device=x.device)
    bf = torch.empty(x.shape[0], D, dtype=torch.bfloat16, device=x.device)
    out, _ = ops.moe_layer_decode_routed(x, idx, table, kind, shared, I, topk_w=w, weight_all=weight_all,
                                         token_ids=token_ids, top_k=k, out_f32=f32, out_bf16=bf)
    return out, f32


@pytest.mark.parametrize("m", [1, 3, 8])
def test_routed_layer_equals_staged_decode(layer, dev, m):
    """Given ids and weights (FusedMoEFFN.forward's contract): bit-identical to
    moe_decode, with an invalid id, an out-of-range id and, for m = 3, an id
    given twice for one token (its weights add, in k order)."""
    store, gate, bias = layer
    x = synthetic.hidden(SEED, 800 + m, m, D, dev)
    idx, w = ops.router_topk(x, gate, bias, K, 1.5)
    idx = idx.clone()
    idx[0, 1] = -1
    idx[-1, 2] = E + 5
    if m == 3:
        idx[1, 4] = idx[1, 0]
    a = routed(x, idx, store.table(0), store.shared_entry(0), w=w)
    f32 = torch.empty(m, D, dtype=torch.float32, device=dev)
    b = ops.moe_decode(x, idx, w, store.table(0), ops.SCALE_E8M0, store.shared_entry(0), 10.0, out_f32=f32, d=D, i=I)
    torch.cuda.synchronize()
    assert ops.moe_layer_status(dev) == 0
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], f32)


def test_routed_layer_token_table_is_hash_routing(layer, dev):
    """A token table (a hash layer's tid2eid): ids tid2eid[token], every weight
    1/k, a token id outside the table selects nothing; equals moe_decode on the
    looked-up ids; also one expert alone with no shared expert (one id, weight 1)."""
    store, _, _ = layer
    V = 1000
    g = torch.Generator().manual_seed(5)
    tid2eid = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(V)]).to(dev)
    tok = torch.tensor([7, 999, 123, V + 3], dtype=torch.int64, device=dev)
    x = synthetic.hidden(SEED, 900, 4, D, dev)
    a = routed(x, tid2eid, store.table(0), store.shared_entry(0), weight_all=1.0 / K, token_ids=tok)
    ids = tid2eid[tok.clamp(max=V - 1)].clone()
    ids[3] = -1
    w = torch.full((4, K), 1.0 / K, dtype=torch.float32, device=dev)
    f32 = torch.empty(4, D, dtype=torch.float32, device=dev)
    ops.moe_decode(x, ids, w, store.table(0), ops.SCALE_E8M0, store.shared_entry(0), 10.0, out_f32=f32, d=D, i=I)
    torch.cuda.synchronize()
    assert torch.equal(a[1], f32)
    one = routed(x[:1], torch.tensor([[17]], device=dev), store.table(0), None, k=1)
    f1 = torch.empty(1, D, dtype=torch.float32, device=dev)
    ops.moe_decode(x[:1], torch.tensor([[17]], device=dev), torch.ones(1, 1, device=dev), store.table(0),
                   ops.SCALE_E8M0, None, 10.0, out_f32=f1, d=D, i=I)
    torch.cuda.synchronize()
    assert torch.equal(one[1], f1)
    assert ops.moe_layer_status(dev) == 0


@pytest.mark.parametrize("ids", [[[17]], [[17], [17]], [[-1], [40]], [[40, -1, 40]]])
def test_routed_layer_one_slot_alone(layer, dev, ids):
    """One routed slot and no shared expert: the down items write their rows
    themselves (no row-group sum); bit-identical to moe_decode in fp32 and
    bf16, also with two tokens on the slot and with repeated / invalid ids."""
    store, _, _ = layer
    idx = torch.tensor(ids, dtype=torch.int64, device=dev)
    m, k = idx.shape
    x = synthetic.hidden(SEED, 950 + m * k, m, D, dev)
    w = torch.rand(m, k, generator=torch.Generator().manual_seed(m * k)).to(dev)
    a = routed(x, idx, store.table(0), None, w=w, k=k)
    f32 = torch.empty(m, D, dtype=torch.float32, device=dev)
    b16, _ = ops.moe_decode(x, idx, w, store.table(0), ops.SCALE_E8M0, None, 10.0, out_f32=f32, d=D, i=I)
    torch.cuda.synchronize()
    assert ops.moe_layer_status(dev) == 0
    assert torch.equal(a[1], f32) and torch.equal(a[0], b16)


@pytest.mark.parametrize("fmt", ["e8m0", "fp32", "bf16"])
def test_lone_slot_every_format(layer, dev, fmt):
    """One token, one routed slot and no shared expert (the down items write
    the rows themselves) in each routed weight format -- FP4 with E8M0 scales
    and with fp32 scales (the two gate/up run paths) and dequantised bf16 (the
    per-item path): bit-identical to moe_decode; an invalid id gives the zero
    output."""
    store, _, _ = layer
    eid = 77
    w1, s1, w3, s3, w2, s2 = store.expert_views(0, eid)
    if fmt == "e8m0":
        table, kind = store.table(0), ops.SCALE_E8M0
    else:
        if fmt == "bf16":
            ent = (ops.fp4_dequant_bf16(w1, s1), ops.fp4_dequant_bf16(w3, s3), ops.fp4_dequant_bf16(w2, s2))
        else:
            ent = (w1, s1.to(torch.float32), w3, s3.to(torch.float32), w2, s2.to(torch.float32))
        table, kind = ops.expert_table([ent if e == eid else None for e in range(E)], dev), ops.SCALE_F32
    x = synthetic.hidden(SEED, 970, 1, D, dev)
    idx = torch.tensor([[eid]], dtype=torch.int64, device=dev)
    w = torch.tensor([[0.75]], dtype=torch.float32, device=dev)
    a = routed(x, idx, table, None, w=w, k=1, kind=kind)
    f32 = torch.empty(1, D, dtype=torch.float32, device=dev)
    b16, _ = ops.moe_decode(x, idx, w, table, kind, None, 10.0, out_f32=f32, d=D, i=I)
    torch.cuda.synchronize()
    assert ops.moe_layer_status(dev) == 0
    assert torch.equal(a[1], f32) and torch.equal(a[0], b16)
    z = routed(x, torch.tensor([[-1]], dtype=torch.int64, device=dev), table, None, w=w, k=1, kind=kind)
    torch.cuda.synchronize()
    assert ops.moe_layer_status(dev) == 0
    assert torch.count_nonzero(z[1]) == 0 and torch.count_nonzero(z[0]) == 0
