"""FP4 / FP8 codec entry points of the reference's _fp4.py, on the HIP kernels.

unpack_from_e2m1fn_x2 (_fp4.py:72-95), transform_sf (_fp4.py:59-69) and
cast_back (_fp4.py:98-110) keep their names and argument meaning; the
quantiser `cast` is not part of the inference path and is not provided.
"""
from __future__ import annotations

import torch

from . import ops


def transform_sf(sf: torch.Tensor) -> torch.Tensor:
    """fp32 passes through; int32-packed E8M0 bytes become 2^(e-127) by `e << 23`
    (each int32 holds 4 scale bytes, so the last dimension grows 4x)."""
    if sf.dtype == torch.float32:
        return sf
    if sf.dtype != torch.int32:
        raise TypeError(f"transform_sf expects float32 or int32, got {sf.dtype}")
    sf = sf.contiguous().view(torch.uint8).to(torch.int32)
    return (sf << 23).view(torch.float32)


def unpack_from_e2m1fn_x2(x: torch.Tensor, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Decodes packed e2m1 (low nibble = even column) to [..., 2K] values of any K."""
    if x.dtype not in (torch.int8, torch.uint8):
        raise TypeError("x must be int8 or uint8")
    if x.ndim == 0:
        raise ValueError("x must have at least 1 dimension so the last dim can be doubled")
    shape = (*x.shape[:-1], x.shape[-1] * 2)
    if x.numel() == 0:
        return torch.empty(shape, dtype=out_dtype, device=x.device)
    flat = x.reshape(-1, x.shape[-1])
    n, k = flat.shape[0], flat.shape[1] * 2
    one = torch.ones(1, 1, dtype=torch.float32, device=x.device)
    out = ops.dequant_blocked(flat, one, (n, k), torch.float32)  # e2m1 values are exact in every float dtype
    return out.to(out_dtype).reshape(shape)


def cast_back(x, fmt: str, block_size: tuple[int, int] = (32, 32)) -> torch.Tensor:
    """Dequantises (data, scale): int8 packed FP4 or float8_e4m3fn data, one
    scale per block_size block (fp32, int32-packed E8M0, or float8_e8m0fnu
    taken by value); the product in fp32, returned as fp32 (fmt == 'fp32')
    or bf16."""
    data, sf = x
    if data.dtype not in (torch.int8, torch.float8_e4m3fn):
        raise TypeError(f"cast_back takes int8 (FP4) or float8_e4m3fn data, got {data.dtype}")
    sf = transform_sf(sf) if sf.dtype in (torch.float32, torch.int32) else sf.to(torch.float32)
    out_dtype = torch.float32 if fmt == "fp32" else torch.bfloat16
    if data.dim() != 2 or sf.dim() != 2:
        raise ValueError("cast_back takes 2-D data and scales")
    br, bc = (int(b) for b in block_size)
    k = data.shape[1] * 2 if data.dtype == torch.int8 else data.shape[1]
    if data.shape[0] == 0 or k == 0:
        return torch.empty(data.shape[0], k, dtype=out_dtype, device=data.device)
    if data.dtype == torch.int8 and (br, bc) == (1, 32) and out_dtype == torch.bfloat16 and k % 32 == 0:
        return ops.fp4_dequant_bf16(data, sf[: data.shape[0], : k // 32])  # the vectorised kernel: same values
    return ops.dequant_blocked(data, sf, (br, bc), out_dtype)
