"""GPU parity of the drop-in boundary's codec and router functions, called by
their reference names, and of the store checksum, against the CPU oracle."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from home_seek_amd import _fp4, expert_store, ops, router, synthetic
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def same_f32(a: np.ndarray, b: np.ndarray) -> bool:
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def same_bf16(a: np.ndarray, b: np.ndarray) -> bool:
    na, nb = (a & 0x7FFF) > 0x7F80, (b & 0x7FFF) > 0x7F80
    return np.array_equal(na, nb) and np.array_equal(a[~na], b[~nb])


@pytest.mark.parametrize("shape", [(3, 7), (9,), (2, 5, 3), (256, 1), (4, 48), (1, 0)])
def test_unpack_from_e2m1fn_x2_any_length(dev, shape):
    """_fp4.py:72-95 for rows of any length (not only multiples of 16 bytes),
    every byte value, the low nibble as the even column, -0.0 kept."""
    n = int(np.prod(shape))
    data = (np.arange(n) * 37 % 256).astype(np.uint8).reshape(shape)
    got = _fp4.unpack_from_e2m1fn_x2(torch.from_numpy(data).to(dev).view(torch.int8))
    assert got.shape == (*shape[:-1], shape[-1] * 2) and got.dtype == torch.float32
    lut = np.array(KATS["fp4_lut"]["values"], dtype=np.float32)
    ref = np.stack([lut[data & 0xF], lut[data >> 4]], axis=-1).reshape(got.shape)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    if n:
        b16 = _fp4.unpack_from_e2m1fn_x2(torch.from_numpy(data).to(dev), torch.bfloat16)
        assert torch.equal(b16.float().cpu(), got.cpu())


@pytest.mark.parametrize("fmt", ["fp32", "bf16"])
@pytest.mark.parametrize("block", [(32, 32), (1, 32), (128, 128), (7, 10)])
def test_cast_back_fp4_blocks(dev, fmt, block):
    """cast_back (_fp4.py:98-110) of int8 FP4 with the reference's default
    (32, 32) block and others, ragged shapes, non-power-of-two fp32 scales."""
    rng = np.random.default_rng(sum(block))
    n, kb = 70, 45
    data = rng.integers(0, 256, (n, kb), dtype=np.uint8)
    k = 2 * kb
    sf = (rng.uniform(0.1, 3.0, (-(-n // block[0]), -(-k // block[1]))) * 2.0 ** rng.integers(-8, 8)).astype(np.float32)
    got = _fp4.cast_back((torch.from_numpy(data).to(dev).view(torch.int8), torch.from_numpy(sf).to(dev)), fmt, block)
    ref = orc.cast_back(data, True, sf, block, out_f32=fmt == "fp32")
    if fmt == "fp32":
        assert got.dtype == torch.float32 and same_f32(got.cpu().numpy(), ref)
    else:
        assert got.dtype == torch.bfloat16 and same_bf16(orc.to_np_bf16(got), ref)


def test_cast_back_fp4_int32_packed_e8m0_scales(dev):
    """Scales as the quantiser packs them (4 E8M0 bytes per int32, transform_sf)."""
    rng = np.random.default_rng(5)
    n, k = 64, 256
    data = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    e = rng.integers(100, 150, (n, k // 32), dtype=np.uint8)  # 8 bytes per row -> 2 int32
    sf_i32 = torch.from_numpy(e.copy()).view(torch.int32).to(dev)
    got = _fp4.cast_back((torch.from_numpy(data).to(dev).view(torch.int8), sf_i32), "bf16", (1, 32))
    assert same_bf16(orc.to_np_bf16(got), orc.dequant_fp4(data, e, e8m0=True, semantics="shift"))
    got32 = _fp4.cast_back((torch.from_numpy(data).to(dev).view(torch.int8), sf_i32), "fp32", (1, 32))
    ref32 = orc.cast_back(data, True, orc.e8m0_table("shift")[e], (1, 32), out_f32=True)
    assert same_f32(got32.cpu().numpy(), ref32)


@pytest.mark.parametrize("block", [(128, 128), (32, 32)])
def test_cast_back_e4m3(dev, block):
    rng = np.random.default_rng(6)
    n, k = 300, 260
    data = rng.integers(0, 256, (n, k), dtype=np.uint8)  # NaN codes included
    sf = rng.uniform(0.5, 2.0, (-(-n // block[0]), -(-k // block[1]))).astype(np.float32) / 448
    t = torch.from_numpy(data).to(dev).view(torch.float8_e4m3fn)
    for fmt in ("fp32", "bf16"):
        got = _fp4.cast_back((t, torch.from_numpy(sf).to(dev)), fmt, block)
        ref = orc.cast_back(data, False, sf, block, out_f32=fmt == "fp32")
        ok = same_f32(got.cpu().numpy(), ref) if fmt == "fp32" else same_bf16(orc.to_np_bf16(got), ref)
        assert ok, fmt


@pytest.mark.parametrize("bt", [(1, 1), (1, 3), (2, 4), (1, 64)])
def test_router_functions_by_name(dev, bt):
    """compute_expert_affinity_with_bias / compute_expert_affinity (router.py:10-36)
    on [B, T, D] hidden states: ids bit-exact, weights to 2e-6."""
    B, T = bt
    seed = 77 + B * T
    gate, bias = synthetic.router_weights(seed, 0, 256, 4096, dev)
    h = synthetic.hidden(seed, 5, B * T, 4096, dev).reshape(B, T, 4096)
    idx, w = router.compute_expert_affinity_with_bias(h, gate, bias, top_k=6, routed_scaling_factor=1.5)
    ridx, rw = orc.router(orc.to_np_bf16(h.reshape(-1, 4096)), orc.to_np_bf16(gate), bias.cpu().numpy(), 6, 1.5)
    assert idx.shape == (B * T, 6) and idx.dtype == torch.int64 and w.dtype == torch.float32
    assert np.array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=2e-6, atol=0)
    idx0, w0 = router.compute_expert_affinity(h, gate, top_k=6, routed_scaling_factor=2.0)
    ridx0, rw0 = orc.router(orc.to_np_bf16(h.reshape(-1, 4096)), orc.to_np_bf16(gate), None, 6, 2.0)
    assert np.array_equal(idx0.cpu().numpy(), ridx0)
    np.testing.assert_allclose(w0.cpu().numpy(), rw0, rtol=2e-6, atol=0)
    # weights sum to the scaling factor (tests/test_fixes.py:338-370)
    np.testing.assert_allclose(w0.sum(-1).cpu().numpy(), 2.0, atol=KATS["routing_scaling"]["atol"])


def test_stable_topk_by_name(dev):
    """stable_topk (router.py:5-7): the reference's KAT (tests/test_tile_ops.py:30-37) and ties to the lower index."""
    kat = KATS["stable_topk"]
    got = router.stable_topk(torch.tensor(kat["scores"], device=dev), kat["k"])
    assert got.cpu().tolist() == kat["expected"]
    s = torch.tensor([[1.0, 3.0, 3.0, 0.5, 3.0]], device=dev)
    assert router.stable_topk(s, 3).cpu().tolist() == [[1, 2, 4]]


@pytest.mark.parametrize("nbytes", [0, 16, 48, (64 << 10) + 48, (3 << 20) + 16, (256 << 15) + 16, 100 << 20])
def test_xor_checksum_matches_host(dev, nbytes):
    g = torch.Generator(device="cpu").manual_seed(nbytes % 1000)
    host = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, generator=g)
    got = ops.xor_checksum(host.to(dev))
    assert np.array_equal(got.cpu().numpy(), orc.xor_checksum(host.numpy()))


def test_store_checksum_expert_record_and_linearity(dev):
    """A full-size expert record's checksum equals the XOR of the oracle
    generator's parts; a layer's checksum equals the XOR of its records'."""
    seed, d, i, n_exp = 21, 4096, 2048, 4
    st = expert_store.HbmExpertStore(1, n_exp, d, i, dev, with_shared=False)
    st.fill_synthetic(seed)
    acc = np.zeros(16, dtype=np.uint8)
    for e in range(n_exp):
        ex = orc.gen_fp4_expert(seed, 0, e, d, i)
        want = np.zeros(16, dtype=np.uint8)
        for part in ("w1", "w3", "w2", "w1_scale", "w3_scale", "w2_scale"):
            want ^= orc.xor_checksum(ex[part])
        got = st.checksum(st.expert_record(0, e)).cpu().numpy()
        assert np.array_equal(got, want), e
        acc ^= want
    assert np.array_equal(st.checksum(st.layer_region(0)).cpu().numpy(), acc)
    assert np.array_equal(st.checksum().cpu().numpy(), acc)
