"""Router of the reference (src/home_seek/router.py:5-36) on the HIP kernels."""
from __future__ import annotations

import torch

from . import ops


def stable_topk(scores: torch.Tensor, k: int) -> torch.Tensor:
    """Indices of the k largest scores per row, ties to the lower index (router.py:5-7)."""
    _, idx = torch.sort(scores, dim=1, descending=True, stable=True)
    return idx[:, :k].contiguous()


def compute_expert_affinity_with_bias(hidden_states: torch.Tensor, gate_weight: torch.Tensor,
                                      gate_bias: torch.Tensor | None, top_k: int = 6,
                                      routed_scaling_factor: float = 1.5):
    """(topk_indices int64 [N, k], topk_weights fp32 [N, k]); bias enters before
    softplus and both bf16 roundings of router.py:27-29 are kept."""
    x = hidden_states.reshape(-1, hidden_states.shape[-1])
    return ops.router_topk(x, gate_weight, gate_bias, top_k, routed_scaling_factor)


def compute_expert_affinity(hidden_states: torch.Tensor, gate_weight: torch.Tensor, top_k: int = 6,
                            routed_scaling_factor: float = 1.5):
    """router.py:10-19 (no bias)."""
    return compute_expert_affinity_with_bias(hidden_states, gate_weight, None, top_k, routed_scaling_factor)
