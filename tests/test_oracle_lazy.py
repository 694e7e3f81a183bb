"""The oracle's on-demand expert evaluation (moe_layer_fp32_lazy, and the
stack oracle's non-caching, threaded mode) equals the pinned moe_layer_fp32
bit for bit."""
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from oracle import oracle as orc
from oracle.stack import StackOracle


def test_lazy_layer_equals_moe_layer_fp32():
    seed, d, i, E = 5, 512, 512, 12
    rng = np.random.default_rng(0)
    x = orc.gen_normal_bf16(orc.key(seed, 1), 3 * d, 0.0, 1.0).reshape(3, d)
    idx = np.array([[0, 5, 7, -1], [5, 11, 2, 3], [7, 0, 9, 4]], dtype=np.int64)
    w = rng.uniform(0.1, 1.0, idx.shape).astype(np.float32)
    experts = {e: orc.gen_fp4_expert(seed, 0, e, d, i) for e in range(E) if e != 9}  # expert 9 absent
    shared = orc.gen_shared_expert(seed, 0, d, i)
    ref = orc.moe_layer_fp32(x, idx, w, experts, shared)
    fn = experts.get
    for pool in (None, ThreadPoolExecutor(4)):
        got = orc.moe_layer_fp32_lazy(x, idx, w, fn, lambda: shared, pool=pool)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(orc.moe_layer_fp32_lazy(x, idx, w, fn, None), orc.moe_layer_fp32(x, idx, w, experts, None))


def test_stack_oracle_modes_agree():
    args = (31, 2, 8, 512, 512, 600)
    a = StackOracle(*args, top_k=4, n_hash=1)
    b = StackOracle(*args, top_k=4, n_hash=1, cache=False, workers=4)
    assert a.decode_step(17) == b.decode_step(17)
    h = a.forward_stack([3, 4, 5])
    assert np.array_equal(h, b.forward_stack([3, 4, 5]))
    assert np.array_equal(a.logits(h, a.final_norm), b.logits(h, b.final_norm))
