"""Host-side pieces of the drop-in boundary (no GPU): the oracle's cast_back and
checksum pinned, transform_sf / _mtp_verify_batched / the checkpoint's lm_head
choice and scale conversion called by name, the workspace registry."""
import json
import weakref
from pathlib import Path

import numpy as np
import pytest
import torch

from home_seek_amd import _fp4, checkpoint, ops
from home_seek_amd.engine import HomeSeekMoEEngine
from home_seek_amd.model_config import MoEConfig
from oracle import oracle as orc

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


# ------------------------------------------------------------------ oracle cast_back

def test_oracle_cast_back_1x32_equals_pinned_dequant():
    rng = np.random.default_rng(1)
    packed = rng.integers(0, 256, (40, 64), dtype=np.uint8)
    e = rng.integers(110, 140, (40, 4), dtype=np.uint8)
    sf = orc.e8m0_table("cast")[e]
    got = orc.cast_back(packed, True, sf, (1, 32), out_f32=False)
    assert np.array_equal(got, orc.dequant_fp4(packed, e))


def test_oracle_cast_back_e4m3_128_equals_pinned_dequant():
    rng = np.random.default_rng(2)
    data = rng.integers(0, 256, (200, 300), dtype=np.uint8)
    data[(data & 0x7F) == 0x7F] = 0  # NaN codes aside
    sf = rng.uniform(0.5, 2.0, (2, 3)).astype(np.float32) / 448
    assert np.array_equal(orc.cast_back(data, False, sf, (128, 128), out_f32=False), orc.dequant_fp8(data, sf))


@pytest.mark.parametrize("block", [(32, 32), (1, 32), (128, 128), (3, 5), (1, 1)])
@pytest.mark.parametrize("fp4", [True, False])
def test_oracle_cast_back_matches_torch_formula(block, fp4):
    """The reference's steps run by torch's own routines (LUT decode from the
    reference's table, repeat_interleave along both axes, the fp32 product,
    .to(bf16)) on ragged shapes and non-power-of-two scales."""
    g = torch.Generator().manual_seed(3)
    n, kb = 37, 23
    if fp4:
        data = torch.randint(0, 256, (n, kb), generator=g, dtype=torch.uint8)
        lut = torch.tensor(KATS["fp4_lut"]["values"], dtype=torch.float32)
        vals = torch.stack([lut[(data & 0xF).long()], lut[(data >> 4).long()]], dim=-1).reshape(n, 2 * kb)
    else:
        data = torch.randint(0, 256, (n, kb), generator=g, dtype=torch.uint8)
        data[(data & 0x7F) == 0x7F] = 1
        vals = data.view(torch.float8_e4m3fn).to(torch.float32)
    k = vals.shape[1]
    sf = torch.rand(-(-n // block[0]), -(-k // block[1]), generator=g) * 3 + 0.1
    ref = vals * sf.repeat_interleave(block[0], dim=0).repeat_interleave(block[1], dim=1)[:n, :k]
    got32 = orc.cast_back(data.numpy(), fp4, sf.numpy(), block, out_f32=True)
    assert np.array_equal(got32.view(np.uint32), ref.numpy().view(np.uint32))
    got16 = orc.cast_back(data.numpy(), fp4, sf.numpy(), block, out_f32=False)
    assert np.array_equal(got16, ref.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))


# ------------------------------------------------------------------ oracle checksum

def test_oracle_xor_checksum_brute_force_and_linearity():
    rng = np.random.default_rng(4)
    buf = rng.integers(0, 256, 16 * 37, dtype=np.uint8)
    acc = 0
    for w in range(37):
        acc ^= int.from_bytes(buf[16 * w:16 * w + 16].tobytes(), "little")
    assert orc.xor_checksum(buf).tobytes() == acc.to_bytes(16, "little")
    a, b = buf[:16 * 20], buf[16 * 20:]
    assert np.array_equal(orc.xor_checksum(buf), orc.xor_checksum(a) ^ orc.xor_checksum(b))
    assert not orc.xor_checksum(np.concatenate([a, a])).any()
    assert not orc.xor_checksum(np.zeros(0, dtype=np.uint8)).any()


# ------------------------------------------------------------------ boundary functions by name

def test_transform_sf_by_name_matches_e8m0_shift():
    """transform_sf (_fp4.py:59-69): int32-packed E8M0 bytes -> 2^(e-127) by e << 23."""
    e = torch.arange(256, dtype=torch.uint8).reshape(4, 64)
    packed = e.view(torch.int32)  # [4, 16]: 4 scale bytes per int32
    got = _fp4.transform_sf(packed)
    assert got.shape == (4, 64) and got.dtype == torch.float32
    ref = orc.e8m0_table("shift")[e.numpy()]
    assert np.array_equal(got.numpy().view(np.uint32), ref.view(np.uint32))
    for ev, v in KATS["ue8m0"]["pairs"]:
        assert float(_fp4.transform_sf(torch.tensor([ev, 0, 0, 0], dtype=torch.uint8).view(torch.int32))[0]) == v
    f = torch.rand(3, 5)
    assert _fp4.transform_sf(f) is f
    with pytest.raises(TypeError):
        _fp4.transform_sf(torch.zeros(2, dtype=torch.int16))


def test_mtp_verify_batched_without_drafts_returns_zero_none():
    """ref tests/test_mtp.py:342-353: None or empty draft_ids -> (0, None), no forward."""
    eng = HomeSeekMoEEngine.__new__(HomeSeekMoEEngine)
    assert eng._mtp_verify_batched(None) == (0, None)
    assert eng._mtp_verify_batched(torch.empty(1, 0, dtype=torch.int64)) == (0, None)


class _FakeIndex:
    def __init__(self, tensors):
        self.t = tensors

    def get_weight(self, key):
        return self.t.get(key)


@pytest.mark.parametrize("have,tie,want", [
    (("embed", "head", "output"), False, "head"),
    (("embed", "output"), False, "output"),
    (("embed",), False, "embed"),
    (("embed", "head", "output"), True, "embed"),
    (("head",), True, "head"),          # tied but no embedding: the reference falls through
    ((), False, None),
])
def test_lm_head_choice_follows_reference_order(have, tie, want):
    """engine.py:431-443: tie_word_embeddings -> embed; else head.weight, else
    output.weight, else embed."""
    vals = {"embed": 1.0, "head": 2.0, "output": 3.0}
    idx = _FakeIndex({f"{k}.weight": torch.full((2, 4), vals[k]) for k in have})
    embed = checkpoint._bf16_weight(idx, "embed.weight", "cpu")
    cfg = MoEConfig(tie_word_embeddings=tie)
    got = checkpoint.select_lm_head(idx, cfg, embed, "cpu")
    if want is None:
        assert got is None
    else:
        assert got.dtype == torch.bfloat16 and float(got[0, 0]) == vals[want]


def test_fp4_scales_other_than_e8m0_are_taken_by_value():
    """The reference converts non-float8_e8m0fnu FP4 scales by value
    (scale.to(float32), engine.py:1066-1080): 64 is 2^6 -> exponent 133; 127 is
    no power of two -> refused; float8_e8m0fnu bytes stay bytes."""
    e = torch.tensor([[127, 3]], dtype=torch.uint8)
    assert torch.equal(checkpoint._e8m0_bytes(e.view(torch.float8_e8m0fnu)), e)
    assert torch.equal(checkpoint._e8m0_bytes(torch.tensor([[64, 1]], dtype=torch.uint8)),
                       torch.tensor([[133, 127]], dtype=torch.uint8))
    assert torch.equal(checkpoint._e8m0_bytes(torch.tensor([[0.25]], dtype=torch.float32)),
                       torch.tensor([[125]], dtype=torch.uint8))
    with pytest.raises(ValueError):
        checkpoint._e8m0_bytes(torch.tensor([[127]], dtype=torch.uint8))
    with pytest.raises(ValueError):
        checkpoint._e8m0_bytes(torch.tensor([[1.5]], dtype=torch.float32))


def test_grown_workspace_keeps_the_old_one_alive(monkeypatch):
    """A graph captured against a workspace still holds its address after the
    workspace grows: the replaced tensor must stay allocated."""
    monkeypatch.setattr(ops, "stream_ptr", lambda dev=None: 12345)
    monkeypatch.setattr(ops, "_workspaces", {})
    monkeypatch.setattr(ops, "_retired_workspaces", [])
    dev = torch.device("cpu")
    small = ops._workspace(dev, "router", 512)
    ref = weakref.ref(small)
    del small
    big = ops._workspace(dev, "router", 4096)
    assert big.numel() >= 4096
    assert ref() is not None and ref().numel() == 512
    assert ops._workspace(dev, "router", 100) is big
