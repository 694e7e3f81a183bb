"""ctypes binding of libhsmoe.so (the HIP kernels behind the C ABI in include/hsmoe.h).

There is no fallback: if the library is missing or cannot be loaded, every
operator raises.  Tensors cross the boundary as raw device pointers
(``tensor.data_ptr()``) and the current torch stream.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libhsmoe.so"

SCALE_E8M0 = 0
SCALE_F32 = 1
DATA_FP4 = 0
DATA_E4M3 = 1
OUT_F32 = 0
OUT_BF16 = 1

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float
_u64 = ctypes.c_uint64
_size = ctypes.c_size_t



class NormTail(ctypes.Structure):
    """hsmoe_norm_tail: the next layer's residual adds + RMSNorm ending a layer launch."""
    _fields_ = [("h_dev", _c_void_p), ("residual_dev", _c_void_p), ("weight_dev", _c_void_p), ("eps", _f32),
                ("h_out_dev", _c_void_p), ("norm_out_dev", _c_void_p)]


# name -> (restype, argtypes); mirrors include/hsmoe.h
_SIGNATURES = {
    "hsmoe_version": (_int, []),
    "hsmoe_last_error": (ctypes.c_char_p, []),
    "hsmoe_clear_error": (None, []),
    "hsmoe_fp4_dequant_bf16": (_int, [_c_void_p, _c_void_p, _int, _i64, _i64, _i64, _i64, _c_void_p, _i64, _c_void_p]),
    "hsmoe_fp8_dequant_bf16": (_int, [_c_void_p, _c_void_p, _i64, _i64, _c_void_p, _c_void_p]),
    "hsmoe_dequant_blocked": (_int, [_c_void_p, _int, _c_void_p, _i64, _i64, _i64, _i64, _i64, _c_void_p, _int,
                                     _c_void_p]),
    "hsmoe_router_workspace_size": (_size, [_i64, _i64]),
    "hsmoe_router_topk": (_int, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _int, _f32, _c_void_p, _c_void_p,
                                 _c_void_p, _c_void_p, _size, _c_void_p]),
    "hsmoe_moe_decode_workspace_size": (_size, [_i64, _i64, _i64, _int]),
    "hsmoe_moe_decode": (_int, [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _int, _c_void_p, _i64, _int,
                                _c_void_p, _f32, _c_void_p, _c_void_p, _c_void_p, _size, _c_void_p]),
    "hsmoe_moe_gate_up": (_int, [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _int, _c_void_p, _i64, _int,
                                 _c_void_p, _f32, _c_void_p, _size, _c_void_p]),
    "hsmoe_moe_down": (_int, [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _int, _c_void_p, _i64, _int,
                              _c_void_p, _c_void_p, _c_void_p, _c_void_p, _size, _c_void_p]),
    "hsmoe_moe_layer_workspace_size": (_size, [_i64, _i64, _i64, _i64, _int]),
    "hsmoe_moe_layer_decode": (_int, [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _i64, _int, _f32, _c_void_p,
                                      _int, _c_void_p, _f32, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                      _c_void_p, _size, _c_void_p]),
    "hsmoe_moe_layer_status_offset": (_size, []),
    "hsmoe_moe_layer_decode_routed": (_int, [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _i64, _c_void_p, _f32,
                                             _int, _c_void_p, _i64, _int, _c_void_p, _f32, _c_void_p, _c_void_p,
                                             _c_void_p, _size, _c_void_p]),
    "hsmoe_moe_layer_decode_norm": (_int, [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _i64, _int, _f32,
                                           _c_void_p, _int, _c_void_p, _f32, _c_void_p, _c_void_p, _c_void_p,
                                           _c_void_p, _c_void_p, _c_void_p, _c_void_p, _size, _c_void_p]),
    "hsmoe_moe_layer_decode_routed_norm": (_int, [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _i64,
                                                  _c_void_p, _f32, _int, _c_void_p, _i64, _int, _c_void_p, _f32,
                                                  _c_void_p, _c_void_p, _c_void_p, _c_void_p, _size, _c_void_p]),
    "hsmoe_moe_layer_decode_noalloc": (_int, [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _i64, _int, _f32,
                                              _c_void_p, _int, _c_void_p, _f32, _c_void_p, _c_void_p, _c_void_p,
                                              _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "hsmoe_moe_prefill_workspace_size": (_size, [_i64, _i64, _i64, _i64, _int]),
    "hsmoe_moe_prefill": (_int, [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _int, _c_void_p, _i64, _int,
                                 _c_void_p, _f32, _c_void_p, _c_void_p, _c_void_p, _size, _c_void_p]),
    "hsmoe_lm_head_workspace_size": (_size, [_i64, _i64]),
    "hsmoe_lm_head_accept": (_int, [_c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _c_void_p,
                                    _c_void_p, _c_void_p, _size, _c_void_p]),
    "hsmoe_rms_norm": (_int, [_c_void_p, _c_void_p, _i64, _i64, _f32, _c_void_p, _c_void_p]),
    "hsmoe_add_rms_norm": (_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _f32, _c_void_p,
                                  _c_void_p, _c_void_p]),
    "hsmoe_embed_add_rms_norm": (_int, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _f32,
                                        _c_void_p, _c_void_p, _c_void_p]),
    "hsmoe_mtp_input": (_int, [_c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                               _i64, _f32, _c_void_p, _c_void_p, _c_void_p]),
    "hsmoe_decode_step_record": (_int, [_c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p,
                                        _c_void_p]),
    "hsmoe_xor_checksum_workspace_size": (_size, []),
    "hsmoe_xor_checksum": (_int, [_c_void_p, _i64, _c_void_p, _c_void_p, _size, _c_void_p]),
    "hsmoe_gen_bytes": (_int, [_u64, _i64, _c_void_p, _c_void_p]),
    "hsmoe_gen_e4m3": (_int, [_u64, _i64, _c_void_p, _c_void_p]),
    "hsmoe_gen_e8m0": (_int, [_u64, _i64, _int, _int, _c_void_p, _c_void_p]),
    "hsmoe_gen_normal": (_int, [_u64, _i64, _f32, _f32, _int, _c_void_p, _c_void_p]),
    "hsmoe_gen_uniform": (_int, [_u64, _i64, _f32, _f32, _f32, _c_void_p, _c_void_p]),
    "hsmoe_gen_index": (_int, [_u64, _i64, _i64, _c_void_p, _c_void_p]),
}

_lib = None


class HsmoeError(RuntimeError):
    """Raised when a libhsmoe entry point returns a negative status."""


def lib() -> ctypes.CDLL:
    """Loads libhsmoe.so once; raises if it is absent (build it with __graft_entry__.build())."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise HsmoeError(f"{LIB_PATH} is not built; run __graft_entry__.build() first")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().hsmoe_last_error().decode(errors="replace")
        raise HsmoeError(f"{what} failed ({rc}): {msg}")


def stream_ptr(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_cuda(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise HsmoeError(f"tensor on {t.device} passed to a GPU kernel; the HIP path has no CPU fallback")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise HsmoeError(f"tensors on different devices ({dev} and {t.device})")
    if dev is None:
        raise HsmoeError("no device tensor given")
    return dev
