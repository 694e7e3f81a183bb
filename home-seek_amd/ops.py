"""Torch-facing wrappers of the libhsmoe entry points.

Each function takes device tensors, checks shapes on the host, and enqueues
the HIP kernels on the current torch stream.  Workspaces are zero-filled once
per (device, stream, purpose) and reused; kernels leave their counters at
zero, so stream-ordered calls can share them.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import SCALE_E8M0, SCALE_F32, check, lib, ptr, require_cuda, stream_ptr

__all__ = [
    "SCALE_E8M0", "SCALE_F32", "scale_kind_of", "fp4_dequant_bf16", "fp8_dequant_bf16", "router_topk",
    "moe_decode", "moe_layer_decode", "moe_layer_decode_routed", "NormTail", "moe_layer_status", "moe_layer_status_words",
    "clear_moe_layer_status", "check_moe_layer_status", "lm_head_accept", "expert_table", "shared_entry",
    "dequant_blocked", "xor_checksum", "MAX_DECODE_TOKENS", "MAX_LAYER_EXPERTS", "embed_add_rms_norm", "mtp_input",
    "decode_step_record",
]

MAX_DECODE_TOKENS = 8
MAX_LAYER_EXPERTS = 256  # expert count the one-launch layer kernel handles

_workspaces: dict[tuple, torch.Tensor] = {}
# Workspaces replaced by larger ones.  A HIP graph captured before the growth
# still holds the old address, so the old tensor stays allocated for the life
# of the process (a graph replay must never touch freed memory).
_retired_workspaces: list[tuple[tuple, torch.Tensor]] = []


def _workspace(device: torch.device, purpose: str, nbytes: int) -> torch.Tensor:
    """Zero-filled device workspace of at least nbytes, one per (device,
    stream, purpose), grown when a call needs more.  A grown layer workspace
    keeps the sticky status word of the one it replaces; the replaced one is
    kept alive (graphs captured against it may still replay)."""
    key = (device.index, stream_ptr(device), purpose)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        new = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
        if ws is not None:
            if purpose == "layer":
                off = lib().hsmoe_moe_layer_status_offset()
                new[off:off + 4].copy_(ws[off:off + 4])
            _retired_workspaces.append((key, ws))
        ws = new
        _workspaces[key] = ws
    return ws


def scale_kind_of(scale: torch.Tensor) -> tuple[int, torch.Tensor]:
    """E8M0 bytes stay bytes; every other dtype is taken by value as fp32 (as
    `sf.float()` does in fused_moe.py:25)."""
    if scale.dtype == torch.float8_e8m0fnu:
        return SCALE_E8M0, scale.view(torch.uint8)
    if scale.dtype != torch.float32:
        scale = scale.to(torch.float32)
    return SCALE_F32, scale


def fp4_dequant_bf16(packed: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """bf16 [N, K] from packed e2m1 [N, K/2] and per-32-column scales [N, K/32]."""
    dev = require_cuda(packed, scale)
    if packed.dtype not in (torch.int8, torch.uint8):
        raise TypeError(f"packed FP4 must be int8/uint8, got {packed.dtype}")
    if packed.dim() != 2:
        raise ValueError("packed FP4 must be 2-D [N, K/2]")
    n, kh = packed.shape
    k = kh * 2
    kind, sc = scale_kind_of(scale)
    if sc.numel() == 1:
        sc = sc.reshape(1, 1).expand(n, k // 32)
    if tuple(sc.shape) != (n, k // 32):
        raise ValueError(f"scale shape {tuple(scale.shape)} does not match [{n}, {k // 32}]")
    packed = packed.contiguous()
    sc = sc.contiguous()
    out = torch.empty(n, k, dtype=torch.bfloat16, device=dev)
    rc = lib().hsmoe_fp4_dequant_bf16(ptr(packed), ptr(sc), kind, n, k, kh, k // 32, ptr(out), k, stream_ptr(dev))
    check(rc, "hsmoe_fp4_dequant_bf16")
    return out


def fp8_dequant_bf16(data: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """bf16 [N, K] from e4m3 [N, K] and fp32 (or E8M0) 128x128 block scales."""
    dev = require_cuda(data, scale)
    if data.dtype not in (torch.float8_e4m3fn, torch.uint8, torch.int8):
        raise TypeError(f"FP8 weight must be float8_e4m3fn, got {data.dtype}")
    n, k = data.shape
    if scale.dtype == torch.float8_e8m0fnu or scale.element_size() == 1:
        # _ue8m0_to_f32 (weight_loader.py:14-19): bits = e << 23
        scale = (scale.view(torch.uint8).to(torch.int32) << 23).view(torch.float32)
    scale = scale.to(torch.float32).contiguous()
    if tuple(scale.shape) != ((n + 127) // 128, (k + 127) // 128):
        raise ValueError(f"block scale shape {tuple(scale.shape)} does not match {n}x{k} / 128")
    data = data.contiguous().view(torch.uint8)
    out = torch.empty(n, k, dtype=torch.bfloat16, device=dev)
    check(lib().hsmoe_fp8_dequant_bf16(ptr(data), ptr(scale), n, k, ptr(out), stream_ptr(dev)),
          "hsmoe_fp8_dequant_bf16")
    return out


def dequant_blocked(data: torch.Tensor, scale: torch.Tensor, block: tuple[int, int],
                    out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """[N, K] fp32 or bf16 from FP4 (int8/uint8 packed [N, K/2]) or e4m3 ([N, K])
    data with fp32 scales, one per (block[0] x block[1]) block (hsmoe_dequant_blocked)."""
    dev = require_cuda(data, scale)
    if data.dim() != 2:
        raise ValueError("dequant_blocked takes 2-D data")
    if data.dtype in (torch.int8, torch.uint8):
        kind, k = _lib.DATA_FP4, data.shape[1] * 2
    elif data.dtype == torch.float8_e4m3fn:
        kind, k = _lib.DATA_E4M3, data.shape[1]
    else:
        raise TypeError(f"dequant_blocked takes packed FP4 (int8) or float8_e4m3fn data, got {data.dtype}")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("dequant_blocked writes fp32 or bf16")
    br, bc = int(block[0]), int(block[1])
    n = data.shape[0]
    scale = scale.to(torch.float32)
    if scale.dim() != 2 or br < 1 or bc < 1 or scale.shape[0] * br < n or scale.shape[1] * bc < k:
        raise ValueError(f"scale {tuple(scale.shape)} with block {tuple(block)} does not cover [{n}, {k}]")
    scale = scale.contiguous()
    data = data.contiguous().view(torch.uint8)
    out = torch.empty(n, k, dtype=out_dtype, device=dev)
    check(lib().hsmoe_dequant_blocked(ptr(data), kind, ptr(scale), n, k, br, bc, scale.shape[1], ptr(out),
                                      _lib.OUT_F32 if out_dtype == torch.float32 else _lib.OUT_BF16,
                                      stream_ptr(dev)), "hsmoe_dequant_blocked")
    return out


def router_topk(x: torch.Tensor, gate_w: torch.Tensor, bias: torch.Tensor | None, top_k: int = 6,
                scaling: float = 1.5, want_logits: bool = False, out: tuple | None = None):
    """(idx int64 [M, k], w fp32 [M, k][, logits bf16 [M, E]]) -- see hsmoe_router_topk.
    `out` = (idx, w) preallocated outputs to fill."""
    dev = require_cuda(x, gate_w, bias)
    x = x.to(torch.bfloat16).contiguous()
    gate_w = gate_w.to(torch.bfloat16).contiguous()
    m, d = x.shape
    e = gate_w.shape[0]
    if gate_w.shape[1] != d:
        raise ValueError(f"gate weight {tuple(gate_w.shape)} does not match hidden size {d}")
    if bias is not None:
        bias = bias.to(torch.float32).contiguous()
    if out is not None:
        idx, w = out
        if idx.shape != (m, top_k) or w.shape != (m, top_k) or idx.dtype != torch.int64 or w.dtype != torch.float32:
            raise ValueError("router_topk out tensors must be int64 / fp32 [M, top_k]")
    else:
        idx = torch.empty(m, top_k, dtype=torch.int64, device=dev)
        w = torch.empty(m, top_k, dtype=torch.float32, device=dev)
    logits = torch.empty(m, e, dtype=torch.bfloat16, device=dev) if want_logits else None
    nbytes = lib().hsmoe_router_workspace_size(m, e)
    ws = _workspace(dev, "router", nbytes)
    rc = lib().hsmoe_router_topk(ptr(x), ptr(gate_w), ptr(bias), m, d, e, top_k, scaling, ptr(idx), ptr(w),
                                 ptr(logits), ptr(ws), ws.numel(), stream_ptr(dev))
    check(rc, "hsmoe_router_topk")
    return (idx, w, logits) if want_logits else (idx, w)


def expert_table(entries: list, device: torch.device) -> torch.Tensor:
    """uint64 [n][6] device table from per-expert tuples.

    An entry is None (absent expert), a 6-tuple (w1, s1, w3, s3, w2, s2) of FP4
    tensors, or a 3-tuple (w1, w3, w2) of bf16 tensors."""
    rows = []
    for ent in entries:
        if ent is None:
            rows.append([0] * 6)
        elif len(ent) == 6:
            rows.append([t.data_ptr() for t in ent])
        elif len(ent) == 3:
            w1, w3, w2 = ent
            rows.append([w1.data_ptr(), 0, w3.data_ptr(), 0, w2.data_ptr(), 0])
        else:
            raise ValueError(f"expert entry of length {len(ent)}")
    host = torch.tensor(rows, dtype=torch.int64)
    return host.to(device, non_blocking=False)


def shared_entry(w1, s1, w3, s3, w2, s2, device: torch.device) -> torch.Tensor:
    """uint64 [6] device entry of the shared expert (e4m3 + fp32 block scales,
    or bf16 weights with s1 = s3 = s2 = None)."""
    vals = [t.data_ptr() if t is not None else 0 for t in (w1, s1, w3, s3, w2, s2)]
    return torch.tensor(vals, dtype=torch.int64).to(device)


def moe_decode(x: torch.Tensor, topk_idx: torch.Tensor, topk_w: torch.Tensor, table: torch.Tensor,
               scale_kind: int, shared: torch.Tensor | None = None, swiglu_limit: float = 10.0,
               out_bf16: torch.Tensor | None = None, out_f32: torch.Tensor | None = None,
               d: int | None = None, i: int | None = None):
    """Routed (+ shared) SwiGLU FFN for M <= 8 tokens; returns (out_bf16, out_f32)."""
    dev = require_cuda(x, topk_idx, topk_w, table, shared)
    if x.dtype != torch.bfloat16:
        raise TypeError(f"hidden states must be bf16, got {x.dtype}")
    x = x.contiguous()
    m, dd = x.shape
    d = dd if d is None else d
    if i is None:
        raise ValueError("intermediate size i is required")
    if m > MAX_DECODE_TOKENS:
        raise ValueError(f"moe_decode handles at most {MAX_DECODE_TOKENS} tokens, got {m}")
    topk_idx = topk_idx.to(torch.int64).contiguous()
    topk_w = topk_w.to(torch.float32).contiguous()
    k = topk_idx.shape[1]
    if out_bf16 is None:
        out_bf16 = torch.empty(m, d, dtype=torch.bfloat16, device=dev)
    nbytes = lib().hsmoe_moe_decode_workspace_size(m, d, i, k)
    ws = _workspace(dev, "decode", nbytes)
    rc = lib().hsmoe_moe_decode(ptr(x), m, d, i, ptr(topk_idx), ptr(topk_w), k, ptr(table), table.shape[0],
                                scale_kind, ptr(shared), swiglu_limit, ptr(out_f32), ptr(out_bf16), ptr(ws),
                                ws.numel(), stream_ptr(dev))
    check(rc, "hsmoe_moe_decode")
    return out_bf16, out_f32


MAX_PREFILL_PAIRS = 12288  # m * top_k per hsmoe_moe_prefill call


def moe_prefill(x: torch.Tensor, topk_idx: torch.Tensor, topk_w: torch.Tensor, table: torch.Tensor,
                scale_kind: int, shared: torch.Tensor | None = None, swiglu_limit: float = 10.0,
                out_bf16: torch.Tensor | None = None, out_f32: torch.Tensor | None = None, i: int | None = None):
    """Routed (+ shared) SwiGLU FFN for any number of tokens as a grouped GEMM
    (hsmoe_moe_prefill); returns (out_bf16, out_f32).  Token blocks of at most
    MAX_PREFILL_PAIRS // top_k rows go to one call each."""
    dev = require_cuda(x, topk_idx, topk_w, table, shared)
    if x.dtype != torch.bfloat16:
        raise TypeError(f"hidden states must be bf16, got {x.dtype}")
    if i is None:
        raise ValueError("intermediate size i is required")
    x = x.contiguous()
    m, d = x.shape
    topk_idx = topk_idx.to(torch.int64).reshape(m, -1).contiguous()
    topk_w = topk_w.to(torch.float32).reshape(m, -1).contiguous()
    k = topk_idx.shape[1]
    if out_bf16 is None:
        out_bf16 = torch.empty(m, d, dtype=torch.bfloat16, device=dev)
    step = max(1, MAX_PREFILL_PAIRS // k)
    for a in range(0, m, step):
        b = min(m, a + step)
        nbytes = lib().hsmoe_moe_prefill_workspace_size(b - a, d, i, table.shape[0], k)
        ws = _workspace(dev, "prefill", nbytes)
        rc = lib().hsmoe_moe_prefill(ptr(x[a:b]), b - a, d, i, ptr(topk_idx[a:b]), ptr(topk_w[a:b]), k, ptr(table),
                                     table.shape[0], scale_kind, ptr(shared), swiglu_limit,
                                     None if out_f32 is None else ptr(out_f32[a:b]), ptr(out_bf16[a:b]), ptr(ws),
                                     ws.numel(), stream_ptr(dev))
        check(rc, "hsmoe_moe_prefill")
    return out_bf16, out_f32


def moe_decode_stage(stage: int, x: torch.Tensor, topk_idx: torch.Tensor, topk_w: torch.Tensor,
                     table: torch.Tensor, scale_kind: int, shared: torch.Tensor | None, swiglu_limit: float,
                     d: int, i: int, out_bf16: torch.Tensor | None = None, out_f32: torch.Tensor | None = None):
    """Launches stage 1 (gate/up) or stage 2 (down) of moe_decode alone; inputs
    must already be contiguous bf16 / int64 / fp32 device tensors."""
    dev = x.device
    m = x.shape[0]
    k = topk_idx.shape[1]
    ws = _workspace(dev, "decode", lib().hsmoe_moe_decode_workspace_size(m, d, i, k))
    if stage == 1:
        rc = lib().hsmoe_moe_gate_up(ptr(x), m, d, i, ptr(topk_idx), ptr(topk_w), k, ptr(table), table.shape[0],
                                     scale_kind, ptr(shared), swiglu_limit, ptr(ws), ws.numel(), stream_ptr(dev))
    else:
        rc = lib().hsmoe_moe_down(ptr(x), m, d, i, ptr(topk_idx), ptr(topk_w), k, ptr(table), table.shape[0],
                                  scale_kind, ptr(shared), ptr(out_f32), ptr(out_bf16), ptr(ws), ws.numel(),
                                  stream_ptr(dev))
    check(rc, f"moe_decode stage {stage}")


class NormTail:
    """The next layer's residual adds and RMSNorm, done at the end of a layer
    launch (the _norm entry points): with out = the layer's output in bf16,
    h_out = bf16(bf16(h + out) + residual) and norm_out = RMSNorm(h_out) *
    weight, bit-identical to add_rms_norm(h, weight, add=out, residual=...).
    h [M, D] bf16; residual [D] or None; weight [D]; the outputs are
    allocated when not given (h_out may be h)."""

    def __init__(self, h: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor | None = None,
                 eps: float = 1e-6, h_out: torch.Tensor | None = None, norm_out: torch.Tensor | None = None):
        require_cuda(h, weight, residual, h_out, norm_out)
        if h.dtype != torch.bfloat16 or h.dim() != 2 or not h.is_contiguous():
            raise ValueError("norm tail h must be a contiguous bf16 [M, D] tensor")
        d = h.shape[1]
        self.h = h
        self.weight = weight.to(torch.bfloat16).reshape(-1).contiguous()
        self.residual = None if residual is None else residual.to(torch.bfloat16).reshape(-1).contiguous()
        if self.weight.numel() != d or (self.residual is not None and self.residual.numel() != d):
            raise ValueError("norm tail weight and residual must be one row of the hidden size")
        self.eps = float(eps)
        self.h_out = torch.empty_like(h) if h_out is None else h_out
        self.norm_out = torch.empty_like(h) if norm_out is None else norm_out
        for t in (self.h_out, self.norm_out):
            if t.shape != h.shape or t.dtype != torch.bfloat16 or not t.is_contiguous():
                raise ValueError("norm tail outputs must be contiguous bf16 tensors shaped like h")

    def struct(self, x: torch.Tensor) -> "_lib.NormTail":
        if tuple(self.h.shape) != tuple(x.shape):
            raise ValueError(f"norm tail rows {tuple(self.h.shape)} do not match the layer's {tuple(x.shape)}")
        return _lib.NormTail(ptr(self.h), ptr(self.residual), ptr(self.weight), self.eps, ptr(self.h_out),
                             ptr(self.norm_out))


def moe_layer_decode(x: torch.Tensor, gate_w: torch.Tensor, gate_bias: torch.Tensor | None, table: torch.Tensor,
                     scale_kind: int, shared: torch.Tensor | None, i: int, top_k: int = 6, scaling: float = 1.5,
                     swiglu_limit: float = 10.0, out_bf16: torch.Tensor | None = None,
                     out_f32: torch.Tensor | None = None, idx_out: torch.Tensor | None = None,
                     w_out: torch.Tensor | None = None, want_logits: bool = False, norm: NormTail | None = None):
    """Router + routed experts + shared expert of one layer for M <= 8 tokens in
    one launch; returns (out_bf16, out_f32, idx, w[, logits]).  With `norm`
    the launch ends with its norm tail (norm.h_out, norm.norm_out receive
    it) and no output is allocated unless asked for.

    Same results as router_topk followed by moe_decode.  Inputs must already be
    contiguous device tensors of the right dtypes when called inside a graph
    capture (no conversions are enqueued then)."""
    dev = require_cuda(x, gate_w, gate_bias, table, shared)
    if x.dtype != torch.bfloat16 or gate_w.dtype != torch.bfloat16:
        raise TypeError("hidden states and gate weight must be bf16")
    x = x.contiguous()
    gate_w = gate_w.contiguous()
    m, d = x.shape
    n_exp = gate_w.shape[0]
    if gate_w.shape[1] != d:
        raise ValueError(f"gate weight {tuple(gate_w.shape)} does not match hidden size {d}")
    if m > MAX_DECODE_TOKENS:
        raise ValueError(f"moe_layer_decode handles at most {MAX_DECODE_TOKENS} tokens, got {m}")
    if gate_bias is not None:
        gate_bias = gate_bias.to(torch.float32).contiguous()
    if idx_out is None:
        idx_out = torch.empty(m, top_k, dtype=torch.int64, device=dev)
    if w_out is None:
        w_out = torch.empty(m, top_k, dtype=torch.float32, device=dev)
    if tuple(idx_out.shape) != (m, top_k) or tuple(w_out.shape) != (m, top_k):
        raise ValueError("idx_out / w_out must be [M, top_k]")
    if out_bf16 is None and out_f32 is None and norm is None:
        out_bf16 = torch.empty(m, d, dtype=torch.bfloat16, device=dev)
    logits = torch.empty(m, n_exp, dtype=torch.bfloat16, device=dev) if want_logits else None
    nbytes = lib().hsmoe_moe_layer_workspace_size(m, d, i, n_exp, top_k)
    ws = _workspace(dev, "layer", nbytes)
    args = (ptr(x), m, d, i, ptr(gate_w), ptr(gate_bias), n_exp, top_k, scaling, ptr(table), scale_kind, ptr(shared),
            swiglu_limit, ptr(idx_out), ptr(w_out), ptr(logits), ptr(out_f32), ptr(out_bf16))
    if norm is None:
        rc = lib().hsmoe_moe_layer_decode(*args, ptr(ws), ws.numel(), stream_ptr(dev))
        check(rc, "hsmoe_moe_layer_decode")
    else:
        tail = norm.struct(x)
        rc = lib().hsmoe_moe_layer_decode_norm(*args, ctypes.addressof(tail), ptr(ws), ws.numel(), stream_ptr(dev))
        check(rc, "hsmoe_moe_layer_decode_norm")
    res = (out_bf16, out_f32, idx_out, w_out)
    return res + (logits,) if want_logits else res


def moe_layer_decode_routed(x: torch.Tensor, topk_idx: torch.Tensor, table: torch.Tensor, scale_kind: int,
                            shared: torch.Tensor | None, i: int, topk_w: torch.Tensor | None = None,
                            weight_all: float = 1.0, token_ids: torch.Tensor | None = None, top_k: int | None = None,
                            swiglu_limit: float = 10.0, out_bf16: torch.Tensor | None = None,
                            out_f32: torch.Tensor | None = None, norm: NormTail | None = None):
    """Routed + shared experts of M <= 8 tokens in one launch with the routing
    given (hsmoe_moe_layer_decode_routed); returns (out_bf16, out_f32).  With
    `norm` the launch ends with its norm tail, as in moe_layer_decode.

    token_ids None: topk_idx [M, k] are the ids.  Otherwise topk_idx is a
    token table [V, k] (a hash layer's tid2eid) and token t's ids are row
    token_ids[t].  topk_w [M, k] or None (every weight weight_all).  Same
    results as moe_decode on the same ids and weights.  Inside a graph capture
    the inputs must already be contiguous device tensors of the right dtypes."""
    dev = require_cuda(x, topk_idx, table, shared, topk_w, token_ids)
    if x.dtype != torch.bfloat16:
        raise TypeError("hidden states must be bf16")
    x = x.contiguous()
    m, d = x.shape
    if m > MAX_DECODE_TOKENS:
        raise ValueError(f"moe_layer_decode_routed handles at most {MAX_DECODE_TOKENS} tokens, got {m}")
    topk_idx = topk_idx.to(torch.int64).contiguous()
    k = topk_idx.shape[-1] if top_k is None else top_k
    rows = 0
    if token_ids is not None:
        token_ids = token_ids.reshape(-1).to(torch.int64).contiguous()
        if token_ids.numel() != m:
            raise ValueError("token_ids must hold one id per token")
        rows = topk_idx.shape[0]
        if topk_idx.dim() != 2 or topk_idx.shape[1] != k:
            raise ValueError("a token table must be [V, top_k]")
    elif topk_idx.numel() != m * k:
        raise ValueError("topk_idx must be [M, top_k]")
    if topk_w is not None:
        topk_w = topk_w.to(torch.float32).contiguous()
        if topk_w.numel() != m * k:
            raise ValueError("topk_w must be [M, top_k]")
    if out_bf16 is None and out_f32 is None and norm is None:
        out_bf16 = torch.empty(m, d, dtype=torch.bfloat16, device=dev)
    n_exp = table.shape[0]
    ws = _workspace(dev, "layer", lib().hsmoe_moe_layer_workspace_size(m, d, i, n_exp, k))
    args = (ptr(x), m, d, i, ptr(topk_idx), ptr(token_ids), rows, ptr(topk_w), float(weight_all), k, ptr(table),
            n_exp, scale_kind, ptr(shared), swiglu_limit, ptr(out_f32), ptr(out_bf16))
    if norm is None:
        rc = lib().hsmoe_moe_layer_decode_routed(*args, ptr(ws), ws.numel(), stream_ptr(dev))
        check(rc, "hsmoe_moe_layer_decode_routed")
    else:
        tail = norm.struct(x)
        rc = lib().hsmoe_moe_layer_decode_routed_norm(*args, ctypes.addressof(tail), ptr(ws), ws.numel(),
                                                      stream_ptr(dev))
        check(rc, "hsmoe_moe_layer_decode_routed_norm")
    return out_bf16, out_f32


def _layer_workspaces(device: torch.device, stream: int | None = None) -> list[torch.Tensor]:
    """The layer workspaces of `stream` (or of every stream) on the device,
    the retired ones included (a graph captured against one still writes it)."""
    return [ws for (d, st, purpose), ws in list(_workspaces.items()) + _retired_workspaces
            if purpose == "layer" and d == device.index and (stream is None or st == stream)]


def moe_layer_status_words(device: torch.device | None = None, stream: int | None = None) -> list[torch.Tensor]:
    """int32 [1] device views of the layer kernel's sticky status word in the
    layer workspaces of `stream` (a raw stream handle), or of every stream of
    the device (a decode graph's capture stream included) when None."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    off = lib().hsmoe_moe_layer_status_offset()
    return [ws[off:off + 4].view(torch.int32) for ws in _layer_workspaces(device, stream)]


def moe_layer_status(device: torch.device | None = None, stream: int | None = None) -> int:
    """The layer kernel's sticky status word: 0 when every cross-workgroup wait
    of every launch completed, else 1 + the code of a wait that gave up (the
    outputs of that launch are not valid).  Reads the workspaces of `stream`,
    or of every stream of the device when None.  Synchronises the device."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    status = 0
    for w in moe_layer_status_words(device, stream):
        status = status or int(w.item())
    return status


def clear_moe_layer_status(device: torch.device | None = None, stream: int | None = None) -> None:
    """Zeroes the sticky status words (of `stream`'s layer workspaces, or of
    every stream of the device), stream-ordered on the current stream, so that
    a reported give-up does not fail every later launch's check."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    for w in moe_layer_status_words(device, stream):
        w.zero_()


def check_moe_layer_status(device: torch.device | None = None, stream: int | None = None) -> None:
    """Raises HsmoeError when moe_layer_status is not 0; the status words are
    cleared first, so the error is reported once."""
    st = moe_layer_status(device, stream)
    if st:
        clear_moe_layer_status(device, stream)
        raise _lib.HsmoeError(f"moe_layer_kernel: a cross-workgroup wait gave up (status {st}); "
                              "the outputs of that launch are not valid")


def lm_head_accept(h: torch.Tensor, lm_head: torch.Tensor, ids: torch.Tensor | None = None,
                   want_logits: bool = True, pred: torch.Tensor | None = None):
    """(logits bf16 [T, V] | None, pred int64 [T], result int64 [2] = (n_accept, bonus_row)).
    pred, if given, is where the argmax goes (contiguous int64 [T], e.g. a
    slice of the next call's id buffer)."""
    dev = require_cuda(h, lm_head, ids, pred)
    h = h.to(torch.bfloat16).contiguous()
    n, d = h.shape
    vocab = lm_head.shape[0]
    if lm_head.dtype != torch.bfloat16 or not lm_head.is_contiguous():
        raise TypeError("lm_head must be a contiguous bf16 [V, D] tensor")
    if ids is not None:
        ids = ids.reshape(-1).to(torch.int64).contiguous()
        if ids.numel() != n:
            raise ValueError("ids must have one entry per hidden row")
    logits = torch.empty(n, vocab, dtype=torch.bfloat16, device=dev) if want_logits else None
    if pred is None:
        pred = torch.empty(n, dtype=torch.int64, device=dev)
    elif pred.dtype != torch.int64 or not pred.is_contiguous() or pred.numel() != n:
        raise ValueError("pred must be a contiguous int64 tensor of one entry per hidden row")
    result = torch.empty(2, dtype=torch.int64, device=dev)
    nbytes = lib().hsmoe_lm_head_workspace_size(n, vocab)
    ws = _workspace(dev, "lm_head", nbytes)
    rc = lib().hsmoe_lm_head_accept(ptr(h), ptr(lm_head), n, d, vocab, ptr(ids), ptr(logits), ptr(pred),
                                    ptr(result), ptr(ws), ws.numel(), stream_ptr(dev))
    check(rc, "hsmoe_lm_head_accept")
    return logits, pred, result


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """bf16 RMSNorm over the last dimension (utils.py:6-9)."""
    return add_rms_norm(x, weight, eps=eps)[1]


def add_rms_norm(x: torch.Tensor, weight: torch.Tensor, add: torch.Tensor | None = None,
                 residual: torch.Tensor | None = None, eps: float = 1e-6, want_sum: bool = False):
    """h = x (+ add) (+ residual), as torch bf16 adds; -> (h if want_sum else None, RMSNorm(h)).
    x, add: [..., D] bf16 of one shape; residual: [D] bf16, added to every row."""
    dev = require_cuda(x, weight, add, residual)
    if x.dtype != torch.bfloat16 or (add is not None and add.dtype != torch.bfloat16):
        raise TypeError("add_rms_norm takes bf16 rows")
    shape = x.shape
    d = shape[-1]
    x2 = x.reshape(-1, d).contiguous()
    if add is not None:
        if add.shape != shape:
            raise ValueError(f"add {tuple(add.shape)} does not match x {tuple(shape)}")
        add = add.reshape(-1, d).contiguous()
    if residual is not None:
        residual = residual.to(torch.bfloat16).reshape(-1).contiguous()
        if residual.numel() != d:
            raise ValueError("residual must be one row of the hidden size")
    w = weight.to(torch.bfloat16).reshape(-1).contiguous()
    if w.numel() != d:
        raise ValueError("norm weight must be one row of the hidden size")
    out = torch.empty_like(x2)
    h = torch.empty_like(x2) if want_sum else None
    check(lib().hsmoe_add_rms_norm(ptr(x2), ptr(add), ptr(residual), ptr(w), x2.shape[0], d, eps, ptr(h), ptr(out),
                                   stream_ptr(dev)), "hsmoe_add_rms_norm")
    return (None if h is None else h.reshape(shape)), out.reshape(shape)


def _bf16_row(t: torch.Tensor, d: int, what: str) -> torch.Tensor:
    t = t.to(torch.bfloat16).reshape(-1).contiguous()
    if t.numel() != d:
        raise ValueError(f"{what} must be one row of the hidden size")
    return t


def embed_add_rms_norm(ids: torch.Tensor, table: torch.Tensor, weight: torch.Tensor,
                       residual: torch.Tensor | None = None, eps: float = 1e-6):
    """The embedding lookup table[ids] followed by add_rms_norm(x, weight,
    residual=residual, want_sum=True), in one launch -> (h, RMSNorm(h)), each
    bf16 [*ids.shape, D]; an id outside [0, V) reads a row of zeros."""
    dev = require_cuda(ids, table, weight, residual)
    if table.dtype != torch.bfloat16 or table.dim() != 2 or not table.is_contiguous():
        raise TypeError("the embedding table must be a contiguous bf16 [V, D] tensor")
    vocab, d = table.shape
    ids_flat = ids.reshape(-1).to(torch.int64).contiguous()
    w = _bf16_row(weight, d, "norm weight")
    res = None if residual is None else _bf16_row(residual, d, "residual")
    rows = ids_flat.numel()
    h = torch.empty(rows, d, dtype=torch.bfloat16, device=dev)
    out = torch.empty_like(h)
    check(lib().hsmoe_embed_add_rms_norm(ptr(ids_flat), rows, ptr(table), vocab, ptr(res), ptr(w), d, eps, ptr(h),
                                         ptr(out), stream_ptr(dev)), "hsmoe_embed_add_rms_norm")
    shape = tuple(ids.shape) + (d,)
    return h.reshape(shape), out.reshape(shape)


def mtp_input(tok: torch.Tensor, embed: torch.Tensor, h_prev: torch.Tensor, enorm: torch.Tensor,
              hnorm: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor | None = None, eps: float = 1e-6):
    """The MTP block's input for one draft token (tok: one int64 on the device):
    h = RMSNorm(h_prev) * hnorm + RMSNorm(embed[tok]) * enorm (+ residual), as
    bf16 adds -> (h [1, D], RMSNorm(h) * weight [1, D]), in one launch."""
    dev = require_cuda(tok, embed, h_prev, enorm, hnorm, weight, residual)
    if embed.dtype != torch.bfloat16 or embed.dim() != 2 or not embed.is_contiguous():
        raise TypeError("the embedding table must be a contiguous bf16 [V, D] tensor")
    vocab, d = embed.shape
    tok = tok.reshape(-1).to(torch.int64).contiguous()
    if tok.numel() != 1:
        raise ValueError("mtp_input takes one token")
    hp = _bf16_row(h_prev, d, "h_prev")
    en, hn, w = (_bf16_row(t, d, "norm weight") for t in (enorm, hnorm, weight))
    res = None if residual is None else _bf16_row(residual, d, "residual")
    h = torch.empty(1, d, dtype=torch.bfloat16, device=dev)
    out = torch.empty_like(h)
    check(lib().hsmoe_mtp_input(ptr(tok), ptr(embed), vocab, ptr(hp), ptr(en), ptr(hn), ptr(res), ptr(w), d, eps,
                                ptr(h), ptr(out), stream_ptr(dev)), "hsmoe_mtp_input")
    return h, out


def decode_step_record(tokens: torch.Tensor, pred: torch.Tensor | None = None, result: torch.Tensor | None = None,
                       record: tuple | None = None, cur: torch.Tensor | None = None):
    """A greedy step's emission from the verify's outputs, in one launch.
    tokens int64 [1 + n] = [a, drafts]; pred int64 [1 + n] and result int64 [2]
    (n_accept, bonus_row) of lm_head_accept (unused when n == 0).  -> (row
    [n + 2] (or [1]), count, next, n_accept) device int64 tensors.  record =
    (rows [cap, width], counts [cap], n_accepts [cap], k []) also writes row
    k and advances k on the device; cur (one int64) receives next."""
    dev = require_cuda(tokens, pred, result, cur)
    tokens = tokens.reshape(-1)
    n = tokens.numel() - 1
    for t in (tokens, pred, result, cur) + (tuple(record) if record else ()):
        if t is not None and (t.dtype != torch.int64 or not t.is_contiguous()):
            raise TypeError("decode_step_record takes contiguous int64 tensors")
    width = n + 2 if n > 0 else 1
    outs = torch.empty(width + 3, dtype=torch.int64, device=dev)
    rows = counts = naccs = k = None
    cap = 0
    if record is not None:
        rows, counts, naccs, k = record
        cap = rows.shape[0]
        if rows.shape[1] != width or counts.numel() < cap or naccs.numel() < cap or k.numel() != 1:
            raise ValueError("record buffers do not match the step's row width and capacity")
    check(lib().hsmoe_decode_step_record(ptr(tokens), n, ptr(pred), ptr(result), ptr(outs),
                                         outs.data_ptr() + 8 * width, outs.data_ptr() + 8 * (width + 1),
                                         outs.data_ptr() + 8 * (width + 2), ptr(rows), ptr(counts), ptr(naccs),
                                         ptr(k), cap, ptr(cur), stream_ptr(dev)), "hsmoe_decode_step_record")
    return outs[:width], outs[width], outs[width + 1], outs[width + 2]


def xor_checksum(data: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """uint8 [16] device tensor: the XOR of the 16-byte words of `data`'s bytes
    (a contiguous device tensor whose byte size is a multiple of 16)."""
    dev = require_cuda(data, out)
    if not data.is_contiguous():
        raise ValueError("xor_checksum needs a contiguous tensor")
    nbytes = data.numel() * data.element_size()
    if out is None:
        out = torch.empty(16, dtype=torch.uint8, device=dev)
    elif out.numel() * out.element_size() != 16 or not out.is_contiguous():
        raise ValueError("xor_checksum out must be 16 contiguous bytes")
    ws = _workspace(dev, "checksum", lib().hsmoe_xor_checksum_workspace_size())
    check(lib().hsmoe_xor_checksum(ptr(data) if nbytes else None, nbytes, ptr(out), ptr(ws), ws.numel(),
                                   stream_ptr(dev)), "hsmoe_xor_checksum")
    return out


# ---------------------------------------------------------------- generators

def gen_bytes(key: int, out: torch.Tensor, e4m3: bool = False) -> torch.Tensor:
    dev = require_cuda(out)
    fn = lib().hsmoe_gen_e4m3 if e4m3 else lib().hsmoe_gen_bytes
    check(fn(key, out.numel() * out.element_size(), ptr(out), stream_ptr(dev)), "hsmoe_gen_bytes")
    return out


def gen_e8m0(key: int, out: torch.Tensor, lo: int = 119, span: int = 6) -> torch.Tensor:
    dev = require_cuda(out)
    check(lib().hsmoe_gen_e8m0(key, out.numel(), lo, span, ptr(out), stream_ptr(dev)), "hsmoe_gen_e8m0")
    return out


def gen_normal(key: int, out: torch.Tensor, mean: float, std: float) -> torch.Tensor:
    dev = require_cuda(out)
    if out.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("gen_normal fills bf16 or fp32 tensors")
    check(lib().hsmoe_gen_normal(key, out.numel(), mean, std, int(out.dtype == torch.bfloat16), ptr(out),
                                 stream_ptr(dev)), "hsmoe_gen_normal")
    return out


def gen_uniform(key: int, out: torch.Tensor, lo: float, hi: float, mul: float = 1.0) -> torch.Tensor:
    dev = require_cuda(out)
    if out.dtype != torch.float32:
        raise TypeError("gen_uniform fills fp32 tensors")
    check(lib().hsmoe_gen_uniform(key, out.numel(), lo, hi, mul, ptr(out), stream_ptr(dev)), "hsmoe_gen_uniform")
    return out


def gen_index(key: int, out: torch.Tensor, n_values: int) -> torch.Tensor:
    dev = require_cuda(out)
    if out.dtype != torch.int64:
        raise TypeError("gen_index fills int64 tensors")
    check(lib().hsmoe_gen_index(key, out.numel(), n_values, ptr(out), stream_ptr(dev)), "hsmoe_gen_index")
    return out


def key(seed: int, tag: int) -> int:
    """Stream key = splitmix64 output number tag+1 for `seed` (same as the device's rand64)."""
    from .synthetic import rand64
    return rand64(seed, tag)
