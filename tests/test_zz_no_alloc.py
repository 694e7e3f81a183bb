"""hsmoe_moe_layer_decode_noalloc, called through the C-ABI: bit-identical to
hsmoe_moe_layer_decode (which takes a workspace) on consecutive calls, the
second with fewer tokens, with status 0; shapes beyond the library's scratch
are rejected before anything is launched."""
import pytest
import torch

from home_seek_amd import _lib, expert_store, ops, synthetic

pytestmark = pytest.mark.gpu

D, I, E, K, SEED = 4096, 2048, 256, 6, 4711


@pytest.fixture(scope="module")
def layer(dev):
    store = expert_store.HbmExpertStore(1, E, D, I, dev, with_shared=True)
    store.fill_synthetic(SEED)
    gate, bias = synthetic.router_weights(SEED, 0, E, D, dev)
    torch.cuda.synchronize()
    return store, gate, bias


def outputs(m, dev):
    return (torch.empty(m, D, dtype=torch.bfloat16, device=dev), torch.empty(m, D, dtype=torch.float32, device=dev),
            torch.empty(m, K, dtype=torch.int64, device=dev), torch.empty(m, K, dtype=torch.float32, device=dev),
            torch.empty(m, E, dtype=torch.bfloat16, device=dev))


def no_alloc(x, gate, bias, table, shared):
    """-> (out_bf16, out_f32, idx, w, logits, status)."""
    m = x.shape[0]
    bf, f32, idx, w, logits = outputs(m, x.device)
    status = torch.full((1,), 7, dtype=torch.int32, device=x.device)
    rc = _lib.lib().hsmoe_moe_layer_decode_noalloc(
        _lib.ptr(x), m, D, I, _lib.ptr(gate), _lib.ptr(bias), E, K, 1.5, _lib.ptr(table), ops.SCALE_E8M0,
        _lib.ptr(shared), 10.0, _lib.ptr(idx), _lib.ptr(w), _lib.ptr(logits), _lib.ptr(f32), _lib.ptr(bf),
        _lib.ptr(status), _lib.stream_ptr(x.device))
    _lib.check(rc, "hsmoe_moe_layer_decode_noalloc")
    return bf, f32, idx, w, logits, status


def with_workspace(x, gate, bias, table, shared):
    """-> (out_bf16, out_f32, idx, w, logits) of hsmoe_moe_layer_decode."""
    m = x.shape[0]
    bf, f32, idx, w, logits = outputs(m, x.device)
    ws = torch.zeros(_lib.lib().hsmoe_moe_layer_workspace_size(m, D, I, E, K), dtype=torch.uint8, device=x.device)
    rc = _lib.lib().hsmoe_moe_layer_decode(
        _lib.ptr(x), m, D, I, _lib.ptr(gate), _lib.ptr(bias), E, K, 1.5, _lib.ptr(table), ops.SCALE_E8M0,
        _lib.ptr(shared), 10.0, _lib.ptr(idx), _lib.ptr(w), _lib.ptr(logits), _lib.ptr(f32), _lib.ptr(bf),
        _lib.ptr(ws), ws.numel(), _lib.stream_ptr(x.device))
    _lib.check(rc, "hsmoe_moe_layer_decode")
    torch.cuda.synchronize()
    assert int(ws[_lib.lib().hsmoe_moe_layer_status_offset():][:4].view(torch.int32).item()) == 0
    return bf, f32, idx, w, logits


def test_no_alloc_equals_workspace_entry(layer, dev):
    store, gate, bias = layer
    for m in (4, 1, 3):  # the second call has fewer tokens than the first
        x = synthetic.hidden(SEED, 40 + m, m, D, dev)
        got = no_alloc(x, gate, bias, store.table(0), store.shared_entry(0))
        torch.cuda.synchronize()
        ref = with_workspace(x, gate, bias, store.table(0), store.shared_entry(0))
        assert int(got[5].item()) == 0, m
        for g, r, what in zip(got, ref, ("bf16", "f32", "idx", "w", "logits")):
            assert torch.equal(g, r), (m, what)


def test_no_alloc_without_shared_or_bias(layer, dev):
    store, gate, _ = layer
    x = synthetic.hidden(SEED, 60, 2, D, dev)
    got = no_alloc(x, gate, None, store.table(0), None)
    torch.cuda.synchronize()
    ref = with_workspace(x, gate, None, store.table(0), None)
    assert int(got[5].item()) == 0
    for g, r, what in zip(got, ref, ("bf16", "f32", "idx", "w", "logits")):
        assert torch.equal(g, r), what


def test_no_alloc_rejects_shapes_beyond_its_scratch(layer, dev):
    """m = 8 at this size needs more than the scratch: an error, nothing launched."""
    store, gate, bias = layer
    L = _lib.lib()
    assert L.hsmoe_moe_layer_workspace_size(8, D, I, E, K) > 8 << 20 >= L.hsmoe_moe_layer_workspace_size(4, D, I, E, K)
    x = synthetic.hidden(SEED, 80, 8, D, dev)
    bf, f32, idx, w, _ = outputs(8, dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    rc = L.hsmoe_moe_layer_decode_noalloc(
        _lib.ptr(x), 8, D, I, _lib.ptr(gate), _lib.ptr(bias), E, K, 1.5, _lib.ptr(store.table(0)), ops.SCALE_E8M0,
        None, 10.0, _lib.ptr(idx), _lib.ptr(w), None, _lib.ptr(f32), _lib.ptr(bf), _lib.ptr(status),
        _lib.stream_ptr(dev))
    assert rc == -4 and b"scratch" in L.hsmoe_last_error()
    rc = L.hsmoe_moe_layer_decode_noalloc(
        _lib.ptr(x), 1, D, I, _lib.ptr(gate), _lib.ptr(bias), E, K, 1.5, _lib.ptr(store.table(0)), ops.SCALE_E8M0,
        None, 10.0, _lib.ptr(idx), _lib.ptr(w), None, _lib.ptr(f32), _lib.ptr(bf), None, _lib.stream_ptr(dev))
    assert rc == -1 and b"status_out" in L.hsmoe_last_error()
