"""FP4 / FP8 codec entry points of the reference's _fp4.py, on the HIP kernels.

unpack_from_e2m1fn_x2 (_fp4.py:72-95), transform_sf (_fp4.py:59-69) and
cast_back (_fp4.py:98-110) keep their names and argument meaning; the
quantiser `cast` is not part of the inference path and is not provided.
"""
from __future__ import annotations

import torch

from . import ops


def transform_sf(sf: torch.Tensor) -> torch.Tensor:
    """fp32 passes through; int32-packed E8M0 bytes become 2^(e-127) by `e << 23`."""
    if sf.dtype == torch.float32:
        return sf
    if sf.dtype != torch.int32:
        raise TypeError(f"transform_sf expects float32 or int32, got {sf.dtype}")
    sf = sf.contiguous().view(torch.uint8).to(torch.int32)
    return (sf << 23).view(torch.float32)


def unpack_from_e2m1fn_x2(x: torch.Tensor, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Decodes packed e2m1 (low nibble = even column) to [..., 2K] values."""
    if x.dtype not in (torch.int8, torch.uint8):
        raise TypeError("x must be int8 or uint8")
    if x.ndim == 0:
        raise ValueError("x must have at least 1 dimension so the last dim can be doubled")
    flat = x.reshape(-1, x.shape[-1])
    k = flat.shape[1] * 2
    if k % 32:
        raise ValueError("the HIP decoder needs a multiple of 16 packed bytes per row")
    ones = torch.ones(flat.shape[0], k // 32, dtype=torch.float32, device=x.device)
    out = ops.fp4_dequant_bf16(flat, ones)  # e2m1 values are exact in bf16
    return out.to(out_dtype).reshape(*x.shape[:-1], k)


def cast_back(x, fmt: str, block_size: tuple[int, int] = (32, 32)) -> torch.Tensor:
    """Dequantises (data, scale) as FP4 with (1, 32) blocks or e4m3 with (128, 128) blocks."""
    data, sf = x
    sf = transform_sf(sf) if sf.dtype in (torch.float32, torch.int32) else sf
    if data.dtype == torch.int8 and tuple(block_size) == (1, 32):
        out = ops.fp4_dequant_bf16(data, sf)
    elif data.dtype == torch.float8_e4m3fn and tuple(block_size) == (128, 128):
        out = ops.fp8_dequant_bf16(data, sf)
    else:
        raise NotImplementedError(f"cast_back for {data.dtype} with block {block_size}")
    return out.float() if fmt == "fp32" else out
