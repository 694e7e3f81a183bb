"""Pins the oracle's number formats: reference tables/KATs and torch's own casts
(the library routines the reference path runs on)."""
import json
import math
import random
from fractions import Fraction
from pathlib import Path

import numpy as np
import torch

from oracle import oracle as orc

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def test_e2m1_matches_reference_lut():
    lut = np.array(KATS["fp4_lut"]["values"], dtype=np.float32)
    got = orc.e2m1_table()
    assert np.array_equal(got, lut)
    # code 8 is -0.0 (sign kept)
    assert np.signbit(got[8]) and got[8] == 0.0


def test_e8m0_shift_kat_and_edges():
    t = orc.e8m0_table("shift")
    for e, v in KATS["ue8m0"]["pairs"]:
        assert t[e] == v
    assert t[0] == 0.0 and math.isinf(t[255])


def test_e8m0_cast_matches_torch_all_256():
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e8m0fnu).to(torch.float32).numpy()
    got = orc.e8m0_table("cast")
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all(), np.nonzero(~same)


def test_e4m3_matches_torch_all_256():
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    got = orc.e4m3_table()
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all(), np.nonzero(~same)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    pats = [0x3F808000, 0x3F818000, 0x3F808001, 0x3F80FFFF, 0x7F7FFFFF, 0x7F7F8000, 0x00008000, 0x00018000,
            0x80008000, 0x7F800000, 0xFF800000, 0x00000000, 0x80000000, 0x007FFFFF, 0x3F7FFF80]
    u = np.concatenate([np.array(pats, dtype=np.uint32), rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)])
    u = u[(u & 0x7FFFFFFF) <= 0x7F800000]  # NaN payloads: torch returns a canonical NaN, checked below
    f = u.view(np.float32)
    ref = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.f32_to_bf16(f), ref)
    assert np.array_equal(np.array([orc.lib().hso_f32_to_bf16(float(x)) for x in f[:2000]], dtype=np.uint16), ref[:2000])
    assert orc.f32_to_bf16(np.array([np.nan], dtype=np.float32))[0] == 0x7FC0


def _bf16_exact_round(x: Fraction) -> int:
    """Brute-force reference: nearest bf16 (ties to even) of an exact rational."""
    if x == 0:
        return 0
    sign = 0x8000 if x < 0 else 0
    a = abs(x)
    e = math.floor(math.log2(a))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp_e = max(e - 7, -133)
    q = a / Fraction(2) ** ulp_e
    fl = math.floor(q)
    rem = q - fl
    r = fl + (1 if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1) else 0)
    v = Fraction(r) * Fraction(2) ** ulp_e
    if v >= Fraction(2) ** 128:
        return sign | 0x7F80
    bits = np.array([float(v)], dtype=np.float32).view(np.uint32)[0] >> 16
    return sign | int(bits)


def test_f64_to_bf16_single_rounding_brute_force():
    rnd = random.Random(1)
    vals = []
    for _ in range(3000):
        m = rnd.getrandbits(53) | (1 << 52)
        e = rnd.randint(-140, 130)
        vals.append(math.ldexp(m, e - 52) * rnd.choice([-1, 1]))
    # exact ties and near-ties of bf16 midpoints (where double rounding via fp32 would fail)
    for k in range(200):
        base = 1.0 + k / 128.0
        vals += [base + 2.0**-8, base + 2.0**-8 + 2.0**-30, base + 2.0**-8 - 2.0**-40]
    for v in vals:
        assert orc.lib().hso_f64_to_bf16(v) == _bf16_exact_round(Fraction(v)), v
