"""The reference's CPU PyTorch route, restated op for op in torch -- TEST
INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg times it (multi-threaded
torch on the host's cores), and the tests check it against the numpy/C
oracle.  The product package never imports it.

Each function follows the reference lines it cites; weights arrive in the
checkpoint's formats (packed e2m1 uint8 + E8M0 bytes, e4m3 + fp32 block
scales) and are dequantised per call, as the reference's loaders do.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

_E2M1 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
                     dtype=torch.float32)


def dequant_fp4(packed: torch.Tensor, scale_e8m0: torch.Tensor) -> torch.Tensor:
    """_dequantize_fp4_to_bf16._deq_one (fused_moe.py:22-26): e2m1 codes (low
    nibble = even column, unpack_from_e2m1fn_x2 _fp4.py:72-90) as fp32 times
    the per-32-column E8M0 scale (scale.float()), one bf16 rounding.
    packed uint8 [N, K/2], scale uint8 [N, K/32] -> bf16 [N, K]."""
    n = packed.shape[0]
    codes = torch.stack([packed & 0x0F, packed >> 4], dim=-1).reshape(n, -1)
    deq = _E2M1[codes.long()]
    sf = scale_e8m0.view(torch.float8_e8m0fnu).float().repeat_interleave(32, dim=1)
    return (deq * sf).to(torch.bfloat16)


def dequant_fp8(data_e4m3: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """load_fp8_weight -> cast_back(.., 'bf16', (128, 128)) (weight_loader.py:22-32,
    _fp4.py:98-110): e4m3 as fp32 times the fp32 block scale, one bf16 rounding."""
    x = data_e4m3.view(torch.float8_e4m3fn).to(torch.float32)
    sf = scale.repeat_interleave(128, dim=0).repeat_interleave(128, dim=1)[: x.shape[0], : x.shape[1]]
    return (x * sf).to(torch.bfloat16)


def ffn_pt(h: torch.Tensor, w1: torch.Tensor, w3: torch.Tensor, w2: torch.Tensor, limit: float = 10.0):
    """fused_expert_ffn_pt (fused_moe.py:383-395)."""
    gate_out = h @ w1.t()
    up_out = h @ w3.t()
    g = gate_out.float().clamp(max=limit)
    u = up_out.float().clamp(min=-limit, max=limit)
    activated = (g * g.sigmoid() * u).to(w1.dtype)
    return activated @ w2.t()


def router(x: torch.Tensor, gate_w: torch.Tensor, gate_bias: torch.Tensor | None, top_k: int = 6,
           scaling: float = 1.5):
    """compute_expert_affinity_with_bias (router.py:22-36)."""
    logits = torch.matmul(x.to(gate_w.dtype), gate_w.t())
    if gate_bias is not None:
        logits = logits + gate_bias.to(logits.dtype)
    scores = F.softplus(logits.float()).sqrt()
    _, order = torch.sort(scores, dim=1, descending=True, stable=True)
    idx = order[:, :top_k].contiguous()
    raw = scores.gather(1, idx)
    return idx, raw / raw.sum(dim=-1, keepdim=True).clamp(min=1e-20) * scaling


def forward_legacy(h: torch.Tensor, topk_idx: torch.Tensor, topk_w: torch.Tensor, load_expert, limit: float = 10.0):
    """FusedMoEFFN._forward_legacy, torch branch (fused_moe.py:458-551): the
    union of the selected experts, each loaded and dequantised per call
    (load_expert(eid) -> 6-tuple of checkpoint tensors or None), one gate/up
    GEMM over the concatenated weights, bf16 routing weights, one down GEMM."""
    B, D = h.shape
    eids = sorted({int(e) for e in topk_idx.reshape(-1).tolist() if int(e) >= 0})
    loaded = {}
    for eid in eids:
        raw = load_expert(eid)
        if raw is None:
            continue
        w1d, w1s, w3d, w3s, w2d, w2s = raw
        loaded[eid] = (dequant_fp4(w1d, w1s), dequant_fp4(w3d, w3s), dequant_fp4(w2d, w2s))
    if not loaded:
        return torch.zeros_like(h)
    ids = sorted(loaded)
    inter = loaded[ids[0]][0].shape[0]
    w1 = torch.cat([loaded[e][0] for e in ids], dim=0)
    w3 = torch.cat([loaded[e][1] for e in ids], dim=0)
    w2 = torch.cat([loaded[e][2] for e in ids], dim=1)
    gate = h @ w1.T
    up = h @ w3.T
    ew = torch.zeros(B, len(ids), dtype=torch.bfloat16)
    pos = torch.full((max(ids) + 1,), -1, dtype=torch.int64)
    for q, e in enumerate(ids):
        pos[e] = q
    valid = topk_idx >= 0
    mapped = pos[topk_idx.clamp(min=0, max=max(ids))]
    valid = valid & (topk_idx <= max(ids)) & (mapped >= 0)
    b_idx = torch.arange(B).unsqueeze(1).expand(-1, topk_idx.shape[1])
    ew[b_idx[valid], mapped[valid]] = topk_w[valid].to(torch.bfloat16)
    g = gate.float().clamp(max=limit)
    u = up.float().clamp(min=-limit, max=limit)
    activated = (g * g.sigmoid() * u).to(torch.bfloat16)
    weighted = activated.view(B, len(ids), inter) * ew.unsqueeze(-1)
    return weighted.reshape(B, len(ids) * inter) @ w2.T


def moe_ffn(x: torch.Tensor, idx: torch.Tensor, w: torch.Tensor, load_expert, shared_raw, limit: float = 10.0):
    """_forward_ffn's routed + shared part (engine.py:1410-1541): FusedMoEFFN.forward
    (= _forward_legacy) plus the FP8 shared expert through fused_expert_ffn_pt
    (SharedExpertFFN.forward at M = 1, fused_moe.py:585-598), added in bf16."""
    out = forward_legacy(x, idx, w, load_expert, limit)
    if shared_raw is not None:
        s1, ss1, s3, ss3, s2, ss2 = shared_raw
        sh = ffn_pt(x, dequant_fp8(s1, ss1), dequant_fp8(s3, ss3), dequant_fp8(s2, ss2), limit)
        out = out + sh.to(torch.bfloat16)
    return out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """utils.py:6-9."""
    xf = x.float()
    var = xf.pow(2).mean(-1, keepdim=True)
    return (weight.float() * (xf * torch.rsqrt(var + eps))).to(x.dtype)


def lm_head_accept(h: torch.Tensor, lm_head: torch.Tensor, combined_ids: list[int]):
    """The verify's logits and greedy acceptance (engine.py:2480-2497) ->
    (logits [T, V], n_accept, bonus_row)."""
    logits = torch.matmul(h.to(lm_head.dtype), lm_head.t())
    n_accept, t_total = 0, logits.shape[0]
    for i in range(t_total):
        pred = int(logits[i].argmax(dim=-1))
        if i == t_total - 1:
            return logits, n_accept, i
        if pred == int(combined_ids[i + 1]):
            n_accept += 1
        else:
            return logits, n_accept, i
    return logits, n_accept, t_total - 1
