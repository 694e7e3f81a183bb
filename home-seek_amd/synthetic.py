"""Seeded synthetic weights and inputs for the benchmark workloads.

Value i of a tensor is derived from rand64(key, i) (splitmix64), with
key = rand64(seed, tag) and the tag naming what the tensor is, so any slice
can be regenerated on the host.  Distributions (per workload definitions):
  FP4 expert codes   uniform over the 16 e2m1 codes, two per byte
  E8M0 scales        exponent uniform in [-8, -3] (bytes 119..124)
  gate weight        ~N(0, 0.02) bf16;  gate bias ~N(0, 0.01) fp32
  hidden x           ~N(0, 1) bf16
  shared expert      e4m3 codes uniform over the 254 finite codes, fp32 block
                     scales U(0.5, 2) / 448
  lm_head            ~N(0, 0.02) bf16; RMSNorm weight ~N(1, 0.05) bf16;
  attention stand-in residual ~N(0, 0.1) bf16
"Normal" is the Irwin-Hall sum of four 16-bit uniforms scaled to unit
variance (exactly reproducible on host and device; tails bounded at 3.46 sigma).
"""
from __future__ import annotations

import torch

from . import ops

MASK64 = (1 << 64) - 1

KIND_FP4_DATA = 1
KIND_FP4_SCALE = 2
KIND_GATE_W = 3
KIND_GATE_BIAS = 4
KIND_HIDDEN = 5
KIND_SHARED_DATA = 6
KIND_SHARED_SCALE = 7
KIND_LM_HEAD = 8
KIND_NORM_W = 9
KIND_RESIDUAL = 10
KIND_DRAFT = 11
KIND_TID2EID = 12

E8M0_LO, E8M0_SPAN = 119, 6


def tag(kind: int, layer: int = 0, eid: int = 0, sub: int = 0) -> int:
    kind, layer, eid, sub = int(kind), int(layer), int(eid), int(sub)
    return ((kind & 0xFF) << 56) | ((layer & 0xFFFF) << 40) | ((eid & 0xFFFFFFFF) << 8) | (sub & 0xFF)


def _mix64(z: int) -> int:
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def rand64(key: int, i: int) -> int:
    return _mix64((key + (i + 1) * 0x9E3779B97F4A7C15) & MASK64)


def key(seed: int, t: int) -> int:
    return rand64(seed & MASK64, t)


# ---------------------------------------------------------------- device fills

def fill_fp4_expert(seed: int, layer: int, eid: int, views) -> None:
    """views = (w1, s1, w3, s3, w2, s2) device tensors of one FP4 expert."""
    w1, s1, w3, s3, w2, s2 = views
    for sub, (w, s) in enumerate(((w1, s1), (w3, s3), (w2, s2))):
        ops.gen_bytes(key(seed, tag(KIND_FP4_DATA, layer, eid, sub)), w)
        ops.gen_e8m0(key(seed, tag(KIND_FP4_SCALE, layer, eid, sub)), s.view(torch.uint8), E8M0_LO, E8M0_SPAN)


def fill_shared_expert(seed: int, layer: int, views) -> None:
    """views = (w1, s1, w3, s3, w2, s2): e4m3 data + fp32 block scales."""
    w1, s1, w3, s3, w2, s2 = views
    for sub, (w, s) in enumerate(((w1, s1), (w3, s3), (w2, s2))):
        ops.gen_bytes(key(seed, tag(KIND_SHARED_DATA, layer, 0, sub)), w.view(torch.uint8), e4m3=True)
        ops.gen_uniform(key(seed, tag(KIND_SHARED_SCALE, layer, 0, sub)), s, 0.5, 2.0, 1.0 / 448.0)


def normal_bf16(seed: int, t: int, shape, mean: float, std: float, device) -> torch.Tensor:
    out = torch.empty(shape, dtype=torch.bfloat16, device=device)
    return ops.gen_normal(key(seed, t), out, mean, std)


def normal_f32(seed: int, t: int, shape, mean: float, std: float, device) -> torch.Tensor:
    out = torch.empty(shape, dtype=torch.float32, device=device)
    return ops.gen_normal(key(seed, t), out, mean, std)


def router_weights(seed: int, layer: int, n_experts: int, d: int, device):
    gate = normal_bf16(seed, tag(KIND_GATE_W, layer), (n_experts, d), 0.0, 0.02, device)
    bias = normal_f32(seed, tag(KIND_GATE_BIAS, layer), (n_experts,), 0.0, 0.01, device)
    return gate, bias


def hidden(seed: int, case: int, m: int, d: int, device) -> torch.Tensor:
    return normal_bf16(seed, tag(KIND_HIDDEN, 0, case), (m, d), 0.0, 1.0, device)


def zipf_routing(seed: int, m: int, n_experts: int, top_k: int = 6, s: float = 1.1, scaling: float = 1.5):
    """Prefill routing with Zipf(s)-skewed expert popularity, drawn without
    replacement per token (Gumbel-top-k over log p_e), on the host (numpy PCG64):
    expert of popularity rank r has p ~ 1/(r+1)^s, ranks assigned to ids by a
    seeded permutation; weights are the chosen p renormalised to `scaling`.
    -> (idx int64 [m, top_k], w fp32 [m, top_k]) numpy arrays."""
    import numpy as np

    rng = np.random.Generator(np.random.PCG64(seed))
    logp = -s * np.log(np.arange(1, n_experts + 1, dtype=np.float64))
    logp = logp[np.argsort(rng.permutation(n_experts))]  # id -> popularity
    g = logp[None, :] + rng.gumbel(size=(m, n_experts))
    idx = np.argsort(-g, axis=1, kind="stable")[:, :top_k].astype(np.int64)
    p = np.exp(logp[idx])
    w = (p / p.sum(axis=1, keepdims=True) * scaling).astype(np.float32)
    return idx, w
