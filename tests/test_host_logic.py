"""Host-side logic of the package that runs without a GPU."""
import numpy as np
import pytest
import torch

from home_seek_amd import expert_store, fused_moe, synthetic
from oracle import oracle as orc


def test_store_layout_checkpoint_shapes():
    s = expert_store.HbmExpertStore(1, 2, 4096, 2048, device="cpu", with_shared=True)
    assert s.payload_bytes == 13_369_344
    w1, s1, w3, s3, w2, s2 = s.expert_views(0, 1)
    assert w1.shape == (2048, 2048) and w1.dtype == torch.int8
    assert s1.shape == (2048, 128) and s1.dtype == torch.float8_e8m0fnu
    assert w2.shape == (4096, 1024) and s2.shape == (4096, 64)
    sh = s.shared_views(0)
    assert sh[0].dtype == torch.float8_e4m3fn and sh[0].shape == (2048, 4096)
    assert sh[1].shape == (16, 32) and sh[5].shape == (32, 16)
    t = s.table(0)
    assert t.shape == (2, 6) and int(t[1, 0]) == w1.data_ptr() and int(t[1, 5]) == s2.data_ptr()
    with pytest.raises(IndexError):
        s.expert_views(0, 2)


def test_tags_and_keys_match_oracle():
    for kind, layer, eid, sub in [(1, 0, 0, 0), (2, 42, 255, 2), (8, 0, 0, 0), (6, 17, 0, 1)]:
        t = synthetic.tag(kind, layer, eid, sub)
        assert t == orc.tag(kind, layer, eid, sub)
        assert synthetic.key(1234, t) == orc.key(1234, t)


def test_forward_without_valid_ids_returns_zeros():
    moe = fused_moe.FusedMoEFFN(hidden_size=512, intermediate_size=512)
    h = torch.randn(2, 512).to(torch.bfloat16)
    idx = torch.full((2, 6), -1, dtype=torch.int64)
    out = moe.forward(h, idx, torch.ones(2, 6), lambda l, e: pytest.fail("loader called"), 0)
    assert torch.equal(out, torch.zeros_like(h))
    out = moe.forward(h, torch.zeros(2, 6, dtype=torch.int64), torch.ones(2, 6), lambda l, e: None, 0)
    assert torch.equal(out, torch.zeros_like(h))


def test_cpu_tensors_are_rejected_not_computed():
    from home_seek_amd import ops, _lib
    with pytest.raises(_lib.HsmoeError):
        ops.fp4_dequant_bf16(torch.zeros(4, 16, dtype=torch.int8), torch.ones(4, 1))
