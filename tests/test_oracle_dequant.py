"""Dequant oracle vs the reference's KATs and torch's own arithmetic."""
import json
from pathlib import Path

import numpy as np
import torch

from oracle import oracle as orc

def bf16_same(a, b):
    """Bit equality, with any NaN equal to any NaN (torch keeps NaN payloads/signs)."""
    na = (a & 0x7FFF) > 0x7F80
    nb = (b & 0x7FFF) > 0x7F80
    return np.array_equal(na, nb) and np.array_equal(a[~na], b[~nb])


KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
LUT = np.array(KATS["fp4_lut"]["values"], dtype=np.float32)


def test_interleave_lo_nibble_is_even_column():
    packed = np.array([[0x2A, 0xF1, 0x70, 0x08] * 4], dtype=np.uint8)  # 16 bytes = 32 columns
    out = orc.bf16_to_f32(orc.dequant_fp4(packed, np.array([[1.0]], dtype=np.float32), e8m0=False))
    for j, b in enumerate(packed[0]):
        assert out[0, 2 * j] == LUT[b & 15] and np.signbit(out[0, 2 * j]) == np.signbit(LUT[b & 15])
        assert out[0, 2 * j + 1] == LUT[b >> 4]


def test_per_group_scale_isolated():
    kat = KATS["per_group_scale"]
    n, k = kat["rows"], kat["cols"]
    rng = np.random.default_rng(7)
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = np.tile(np.array(kat["group_scales"], dtype=np.float32), (n, 1))
    out = orc.bf16_to_f32(orc.dequant_fp4(packed, scales, e8m0=False))
    codes = np.stack([packed & 15, packed >> 4], axis=-1).reshape(n, k)
    for g, s in enumerate(kat["group_scales"]):
        exp = (LUT[codes[:, 32 * g:32 * g + 32]] * np.float32(s))
        assert np.array_equal(out[:, 32 * g:32 * g + 32], orc.bf16_to_f32(orc.f32_to_bf16(exp)))


def test_fp4_dequant_matches_torch_formula():
    """(decoded.float() * sf.float()).to(bf16) evaluated by torch with the reference LUT."""
    rng = np.random.default_rng(3)
    n, k = 64, 256
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    sf = rng.uniform(1e-3, 4.0, (n, k // 32)).astype(np.float32)
    codes = torch.from_numpy(np.stack([packed & 15, packed >> 4], axis=-1).reshape(n, k).astype(np.int64))
    dec = torch.from_numpy(LUT)[codes]
    ref = (dec.float() * torch.from_numpy(sf).repeat_interleave(32, dim=1)).to(torch.bfloat16)
    got = orc.dequant_fp4(packed, sf, e8m0=False)
    assert np.array_equal(got, ref.view(torch.int16).numpy().view(np.uint16))
    # E8M0 bytes through torch's float8_e8m0fnu cast, all exponents
    e = rng.integers(0, 256, (n, k // 32), dtype=np.uint8)
    sfe = torch.from_numpy(e).view(torch.float8_e8m0fnu).to(torch.float32)
    ref = (dec.float() * sfe.repeat_interleave(32, dim=1)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = orc.dequant_fp4(packed, e, e8m0=True, semantics="cast")
    assert bf16_same(got, ref)


def test_fp8_block_dequant_matches_torch():
    rng = np.random.default_rng(4)
    n, k = 256, 384
    data = rng.integers(0, 256, (n, k), dtype=np.uint8)
    data[(data & 0x7F) == 0x7F] ^= 1
    sf = rng.uniform(0.5, 2.0, (2, 3)).astype(np.float32) / np.float32(448.0)
    ref = (torch.from_numpy(data).view(torch.float8_e4m3fn).to(torch.float32)
           * torch.from_numpy(sf).repeat_interleave(128, 0).repeat_interleave(128, 1)).to(torch.bfloat16)
    assert np.array_equal(orc.dequant_fp8(data, sf), ref.view(torch.int16).numpy().view(np.uint16))
