"""MoE operators of the reference (src/home_seek/fused_moe.py) on the HIP kernels.

Same class and function names, constructor arguments and call signatures as
the reference, so HomeSeekInferenceEngine code that builds and calls them runs
unchanged:
  FusedMoEFFN.forward(hidden [B, D], topk_idx [B, k], topk_weights [B, k],
                      load_expert_fn(layer, eid) -> 6-tuple | 3-tuple | None,
                      layer_idx)                                   fused_moe.py:447-456
  FusedMoEFFN.forward_m1_fp4(hidden [1, D], {eid: 6-tuple}, {eid: weight})
                                                                   fused_moe.py:553-563
  SharedExpertFFN.forward(hidden [B, T, D], w1, w3, w2, dtype)     fused_moe.py:585-598
  fused_expert_ffn_pt / fused_expert_ffn_triton, triton_dequantize_fp4_to_bf16(_all)
The Triton/cuBLAS knobs (use_triton, triton_blocks, cublas_max_tokens) are
accepted and ignored: there is one HIP path and no dispatch between backends.
Numerics: fp32 accumulation and fp32 intermediates throughout (the reference
rounds gate/up/activations to bf16 on some routes); outputs are bf16.
Extra fast path for an engine that owns an HBM expert store:
  FusedMoEFFN.forward_table(hidden, topk_idx, topk_weights, table, scale_kind, shared)
which takes the ids on the device and never synchronises with the host.
"""
from __future__ import annotations

from typing import Callable, Optional

import torch

from . import ops
from ._lib import SCALE_E8M0, SCALE_F32


def _as_device(t: torch.Tensor, dev: torch.device) -> torch.Tensor:
    return t if t.device == dev else t.to(dev, non_blocking=True)


def _fp4_entry(w: tuple, dev: torch.device):
    """Normalises a reference 6-tuple; returns (entry tuple, scale_kind)."""
    w1, s1, w3, s3, w2, s2 = (_as_device(t, dev) for t in w)
    kinds = set()
    out = []
    for data, sc in ((w1, s1), (w3, s3), (w2, s2)):
        if data.dtype not in (torch.int8, torch.uint8):
            raise TypeError(f"FP4 expert weight must be int8, got {data.dtype}")
        kind, sc2 = ops.scale_kind_of(sc)
        kinds.add(kind)
        out += [data.contiguous(), sc2.contiguous()]
    if len(kinds) != 1:
        raise TypeError("all three scales of one expert must share one dtype")
    return tuple(out), kinds.pop()


def _bf16_entry(w: tuple, dev: torch.device):
    return tuple(_as_device(t, dev).to(torch.bfloat16).contiguous() for t in w)


def _run_decode_chunks(x: torch.Tensor, topk_idx: torch.Tensor, topk_w: torch.Tensor, table: torch.Tensor,
                       scale_kind: int, shared: Optional[torch.Tensor], limit: float, d: int, i: int,
                       out_f32: Optional[torch.Tensor] = None) -> torch.Tensor:
    """M <= 8: the decode kernel; more tokens: the prefill grouped GEMM (or, for
    hidden sizes it does not tile, the decode kernel over chunks of 8 tokens)."""
    m = x.shape[0]
    out = torch.empty(m, d, dtype=torch.bfloat16, device=x.device)
    if m > ops.MAX_DECODE_TOKENS and d % 1024 == 0:
        ops.moe_prefill(x, topk_idx, topk_w, table, scale_kind, shared, limit, out_bf16=out, out_f32=out_f32, i=i)
        return out
    step = ops.MAX_DECODE_TOKENS
    k = topk_idx.shape[-1]
    for a in range(0, m, step):
        b = min(m, a + step)
        o32 = None if out_f32 is None else out_f32[a:b]
        if _layer_kernel_fits(b - a, d, i, table.shape[0], k):
            # one persistent launch (hsmoe_moe_layer_decode_routed), bit-identical to moe_decode
            ops.moe_layer_decode_routed(x[a:b], topk_idx[a:b], table, scale_kind, shared, i, topk_w=topk_w[a:b],
                                        top_k=k, swiglu_limit=limit, out_bf16=out[a:b], out_f32=o32)
        else:
            ops.moe_decode(x[a:b], topk_idx[a:b], topk_w[a:b], table, scale_kind, shared, limit,
                           out_bf16=out[a:b], out_f32=o32, d=d, i=i)
    return out


def _layer_kernel_fits(m: int, d: int, i: int, n_experts: int, top_k: int) -> bool:
    """The shapes the one-launch layer kernel takes (else the two-launch decode kernels)."""
    return (m <= ops.MAX_DECODE_TOKENS and n_experts <= ops.MAX_LAYER_EXPERTS and top_k <= 16 and d % 512 == 0
            and i % 512 == 0 and d <= 8192 and max(m * d, 2 * m * i) * 2 <= 65536)


class FusedMoEFFN:
    def __init__(self, num_experts: int = 256, intermediate_size: int = 2048, hidden_size: int = 4096,
                 swiglu_limit: float = 10.0, use_triton: bool = True,
                 triton_blocks: tuple[int, int, int] = (16, 32, 64), cublas_max_tokens: int = 8):
        self.num_experts = num_experts
        self.intermediate_size = intermediate_size
        self.hidden_size = hidden_size
        self.swiglu_limit = swiglu_limit
        # the reference reads this flag to pick its M=1 route (engine.py:1458)
        self.use_triton = torch.cuda.is_available()
        self._triton_blocks = triton_blocks
        self._cublas_max_tokens = cublas_max_tokens

    # -------------------------------------------------------------- reference API
    def forward(self, hidden_states: torch.Tensor, topk_idx: torch.Tensor, topk_weights: torch.Tensor,
                load_expert_fn: Callable, layer_idx: int) -> torch.Tensor:
        """Routed FFN over the union of selected experts (fused_moe.py:458-551).

        Like the reference, the loader is called once per distinct valid id
        (which needs the ids on the host), None entries are skipped, and the
        output is zeros when no expert remains.  Exceptions propagate."""
        B, D = hidden_states.shape
        dev = hidden_states.device
        ids = sorted({int(e) for e in topk_idx.reshape(-1).tolist() if int(e) >= 0})
        if not ids:
            return torch.zeros_like(hidden_states)
        entries: list = [None] * (max(ids) + 1)
        kinds = set()
        inter = None
        for eid in ids:
            w = load_expert_fn(layer_idx, eid)
            if w is None:
                continue
            if len(w) == 6:
                ent, kind = _fp4_entry(w, dev)
                kinds.add(kind)
                inter = ent[0].shape[0]
            elif len(w) == 3:
                ent = _bf16_entry(w, dev)
                inter = ent[0].shape[0]
            else:
                continue
            entries[eid] = ent
        if inter is None:
            return torch.zeros_like(hidden_states)
        if len(kinds) > 1:
            raise TypeError("experts of one call mix E8M0 and fp32 scales")
        kind = kinds.pop() if kinds else SCALE_E8M0
        table = ops.expert_table(entries, dev)
        x = hidden_states.to(torch.bfloat16)
        out = _run_decode_chunks(x, topk_idx, topk_weights, table, kind, None, self.swiglu_limit, D, inter)
        return out.to(hidden_states.dtype)

    def forward_m1_fp4(self, hidden_states: torch.Tensor, fp4_data: dict, routing_w: dict) -> torch.Tensor:
        """M=1 FP4 route (fused_moe.py:553-563, 1147-1227): experts with weight
        0.0 are skipped; output [1, D] bf16."""
        dev = hidden_states.device
        eids = [e for e in sorted(fp4_data) if routing_w.get(e, 0.0) != 0.0]
        D = hidden_states.shape[1]
        if not eids:
            return torch.zeros(1, D, dtype=torch.bfloat16, device=dev)
        entries = []
        kinds = set()
        for e in eids:
            ent, kind = _fp4_entry(fp4_data[e], dev)
            entries.append(ent)
            kinds.add(kind)
        if len(kinds) > 1:
            raise TypeError("experts of one call mix E8M0 and fp32 scales")
        table = ops.expert_table(entries, dev)
        idx = torch.arange(len(eids), dtype=torch.int64).reshape(1, -1).to(dev)
        w = torch.tensor([[float(routing_w[e]) for e in eids]], dtype=torch.float32).to(dev)
        out, _ = ops.moe_decode(hidden_states.to(torch.bfloat16), idx, w, table, kinds.pop(), None,
                                self.swiglu_limit, d=D, i=entries[0][0].shape[0])
        return out

    def _swiglu(self, h, w1, w3):
        """fused_moe.py:565-570 (only reached by reference tests)."""
        gate = (h.float() @ w1.float().t())
        up = (h.float() @ w3.float().t())
        g = gate.clamp(max=self.swiglu_limit)
        u = up.clamp(min=-self.swiglu_limit, max=self.swiglu_limit)
        return (g * g.sigmoid() * u).to(w1.dtype)

    # -------------------------------------------------------------- device-id fast path
    def forward_table(self, hidden_states: torch.Tensor, topk_idx: torch.Tensor, topk_weights: torch.Tensor,
                      table: torch.Tensor, scale_kind: int = SCALE_E8M0, shared: Optional[torch.Tensor] = None,
                      out_f32: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Routed (+ shared) FFN with ids/weights on the device and experts given
        by an address table (HbmExpertStore.table): no host synchronisation."""
        x = hidden_states.reshape(-1, self.hidden_size).to(torch.bfloat16)
        out = _run_decode_chunks(x, topk_idx.reshape(x.shape[0], -1), topk_weights.reshape(x.shape[0], -1),
                                 table, scale_kind, shared, self.swiglu_limit, self.hidden_size,
                                 self.intermediate_size, out_f32)
        return out


class SharedExpertFFN:
    def __init__(self, hidden_size: int = 4096, intermediate_size: int = 2048, swiglu_limit: float = 10.0,
                 use_triton: bool = True, triton_blocks: tuple[int, int, int] = (16, 32, 64),
                 cublas_max_tokens: int = 8):
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.swiglu_limit = swiglu_limit
        self.use_triton = torch.cuda.is_available()
        self._triton_blocks = triton_blocks
        self._cublas_max_tokens = cublas_max_tokens

    def forward(self, hidden_states: torch.Tensor, w1, w3, w2, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
        """fused_moe.py:585-598: [B, T, D] -> [B, T, D] with bf16 weights."""
        B, T, D = hidden_states.shape
        out = fused_expert_ffn_pt(hidden_states.reshape(-1, D), w1, w3, w2, self.swiglu_limit)
        return out.reshape(B, T, D).to(dtype)


def fused_expert_ffn_pt(hidden: torch.Tensor, w1: torch.Tensor, w3: torch.Tensor, w2: torch.Tensor,
                        swiglu_limit: float = 10.0) -> torch.Tensor:
    """One bf16 expert (fused_moe.py:383-395) as a weight-1 slot of the HIP FFN."""
    dev = hidden.device
    w1, w3, w2 = _bf16_entry((w1, w3, w2), dev)
    table = ops.expert_table([(w1, w3, w2)], dev)
    m = hidden.shape[0]
    idx = torch.zeros(m, 1, dtype=torch.int64, device=dev)
    w = torch.ones(m, 1, dtype=torch.float32, device=dev)
    return _run_decode_chunks(hidden.to(torch.bfloat16), idx, w, table, SCALE_E8M0, None, swiglu_limit,
                              w1.shape[1], w1.shape[0])


def fused_expert_ffn_triton(hidden: torch.Tensor, w1: torch.Tensor, w3: torch.Tensor, w2: torch.Tensor,
                            swiglu_limit: float = 10.0, w1_scale: Optional[torch.Tensor] = None,
                            w3_scale: Optional[torch.Tensor] = None, w2_scale: Optional[torch.Tensor] = None,
                            triton_blocks=None, cublas_max_tokens=None) -> torch.Tensor:
    """fused_moe.py:269-380 (name kept for drop-in): FP4 weights with scales or bf16 weights."""
    dev = hidden.device
    if w1.dtype in (torch.int8, torch.uint8):
        if w1_scale is None or w3_scale is None or w2_scale is None:
            raise ValueError("FP4 weights need all three scales")
        ent, kind = _fp4_entry((w1, w1_scale, w3, w3_scale, w2, w2_scale), dev)
        inter = ent[0].shape[0]
    else:
        ent, kind = _bf16_entry((w1, w3, w2), dev), SCALE_E8M0
        inter = ent[0].shape[0]
    table = ops.expert_table([ent], dev)
    m = hidden.shape[0]
    idx = torch.zeros(m, 1, dtype=torch.int64, device=dev)
    w = torch.ones(m, 1, dtype=torch.float32, device=dev)
    return _run_decode_chunks(hidden.to(torch.bfloat16), idx, w, table, kind, None, swiglu_limit,
                              hidden.shape[1], inter)


def triton_dequantize_fp4_to_bf16(w_packed: torch.Tensor, w_scale: torch.Tensor) -> torch.Tensor:
    """fused_moe.py:672-710 (name kept for drop-in): [N, K/2] int8 + [N, K/32] scale -> bf16 [N, K]."""
    return ops.fp4_dequant_bf16(w_packed, w_scale)


def triton_dequantize_fp4_all(w1_packed, w1_scale, w3_packed, w3_scale, w2_packed, w2_scale):
    """fused_moe.py:713-723."""
    return (ops.fp4_dequant_bf16(w1_packed, w1_scale), ops.fp4_dequant_bf16(w3_packed, w3_scale),
            ops.fp4_dequant_bf16(w2_packed, w2_scale))


def clear_deq_cache() -> None:
    """fused_moe.py:156-162: there is no BF16 cache to clear (weights are decoded in registers)."""


def deq_cache_stats() -> tuple[int, int]:
    """fused_moe.py:164-166: always (0, 0) -- no BF16 cache exists."""
    return 0, 0
