"""Synthetic MoE-only decode stack (the 43-layer decode + MTP-verify workload).

Every layer is (attention stand-in residual -> RMSNorm -> MoE FFN), the MoE
FFN being router or hash routing + routed FP4 experts + FP8 shared expert on
the HBM store; then the final RMSNorm and lm_head.  Seeded weights, generated
on the device by the same counter-based generators the CPU oracle uses:
  routed experts  FP4 codes uniform, E8M0 exponents in [-8, -3]
  shared expert   e4m3 + fp32 128x128 block scales U(0.5, 2)/448
  router          gate bf16 ~N(0, 0.02), bias fp32 ~N(0, 0.01)
  norms           bf16 ~N(1, 0.05); attention stand-in residual bf16 ~N(0, 0.1)
  lm_head         bf16 ~N(0, 0.02); the embedding is tied to it (embed[v] =
                  lm_head[v]), so no second vocab-sized table is stored
  hash layers     layers < n_hash route token v to experts
                  (b(v) + j * step) mod E, j < top_k, weight 1/top_k
                  (b(v) uniform; step odd, so the ids of a token are distinct)
  MTP block       one more store layer (its experts), its own router, norms
                  and residual
"""
from __future__ import annotations

import torch

from . import synthetic as syn
from .engine import HomeSeekMoEEngine
from .expert_store import HbmExpertStore
from .model_config import MoEConfig

HASH_STEP = 41  # odd: j * HASH_STEP mod E is distinct for j < E when E is a power of two


def hash_table(seed: int, layer: int, vocab: int, n_experts: int, top_k: int, device) -> torch.Tensor:
    """tid2eid [vocab, top_k] int64 of a hash-routed layer."""
    base = torch.empty(vocab, dtype=torch.int64, device=device)
    from . import ops
    ops.gen_index(syn.key(seed, syn.tag(syn.KIND_TID2EID, layer)), base, n_experts)
    j = torch.arange(top_k, dtype=torch.int64, device=device) * HASH_STEP
    return (base[:, None] + j[None, :]) % n_experts


def layer_weights(seed: int, layer: int, n_experts: int, d: int, device, vocab: int = 0, top_k: int = 0,
                  hashed: bool = False) -> dict:
    gate, bias = syn.router_weights(seed, layer, n_experts, d, device)
    lw = {
        "ffn.gate.weight": gate,
        "ffn.gate.bias": bias,
        "ffn_norm.weight": syn.normal_bf16(seed, syn.tag(syn.KIND_NORM_W, layer), (d,), 1.0, 0.05, device),
        "attn.residual": syn.normal_bf16(seed, syn.tag(syn.KIND_RESIDUAL, layer), (d,), 0.0, 0.1, device),
    }
    if hashed:
        lw["ffn.gate.tid2eid"] = hash_table(seed, layer, vocab, n_experts, top_k, device)
    return lw


def build_stack(seed: int, n_layers: int = 43, n_experts: int = 256, d: int = 4096, i: int = 2048,
                vocab: int = 129280, top_k: int = 6, n_hash: int = 3, device="cuda", log=None) -> HomeSeekMoEEngine:
    """The synthetic stack as a HomeSeekMoEEngine (store layer n_layers holds the MTP experts).
    log(str), if given, hears about fill progress every 8 layers."""
    device = torch.device(device)
    cfg = MoEConfig(num_hidden_layers=n_layers, hidden_size=d, moe_intermediate_size=i, vocab_size=vocab,
                    n_routed_experts=n_experts, num_experts_per_tok=top_k, num_hash_layers=n_hash)
    store = HbmExpertStore(n_layers + 1, n_experts, d, i, device, with_shared=True)
    for l0 in range(0, n_layers + 1, 8):
        store.fill_synthetic(seed, range(l0, min(n_layers + 1, l0 + 8)))
        if log is not None:
            torch.cuda.synchronize(device)
            log(f"store layers < {min(n_layers + 1, l0 + 8)} filled")
    lws = {l: layer_weights(seed, l, n_experts, d, device, vocab, top_k, hashed=l < n_hash)
           for l in range(n_layers)}
    lm_head = syn.normal_bf16(seed, syn.tag(syn.KIND_LM_HEAD), (vocab, d), 0.0, 0.02, device)
    final_norm = syn.normal_bf16(seed, syn.tag(syn.KIND_NORM_W, 0xFFFF), (d,), 1.0, 0.05, device)
    mtp = {
        "layer": layer_weights(seed, n_layers, n_experts, d, device),
        "layer_idx": n_layers,
        "hnorm.weight": syn.normal_bf16(seed, syn.tag(syn.KIND_NORM_W, 0xFFFF, 1), (d,), 1.0, 0.05, device),
        "enorm.weight": syn.normal_bf16(seed, syn.tag(syn.KIND_NORM_W, 0xFFFF, 2), (d,), 1.0, 0.05, device),
        "norm.weight": syn.normal_bf16(seed, syn.tag(syn.KIND_NORM_W, 0xFFFF, 3), (d,), 1.0, 0.05, device),
    }
    return HomeSeekMoEEngine(cfg, store, lws, lm_head=lm_head, norm_weight=final_norm, embed=lm_head,
                             mtp_weights=mtp)
