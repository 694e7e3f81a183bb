// RMSNorm arithmetic shared by hsmoe_add_rms_norm and the layer kernel's
// fused pre-norm, restating rms_norm (utils.py:6-9) with the residual adds of
// a layer (engine.py:2690): bf16 adds are the fp32 sum rounded once; a row's
// sum of squares runs per thread over its 8-column chunks t, t + 256, ... in
// column order (lo then hi of each packed pair), then across the wave by a
// fixed xor-butterfly (offsets 1, 2, ..., 32), then over the 4 waves in wave
// order; var = sum / d, inv = 1 / sqrt(var + eps), y = bf16(w * (x * inv)).
#pragma once
#include "hsmoe_common.h"

namespace hsmoe {

__device__ __forceinline__ uint32_t norm_add_bf16(uint32_t a, uint32_t b) {
  return f32_to_bf16_bits(__fadd_rn(bf16_bits_to_f32(a), bf16_bits_to_f32(b)));
}

// Elementwise bf16 add of two packed pairs.
__device__ __forceinline__ uint32_t norm_add_pair(uint32_t a, uint32_t b) {
  return norm_add_bf16(a & 0xffffu, b & 0xffffu) | (norm_add_bf16(a >> 16, b >> 16) << 16);
}

__device__ __forceinline__ uint4 norm_add_chunk(uint4 a, uint4 b) {
  return make_uint4(norm_add_pair(a.x, b.x), norm_add_pair(a.y, b.y), norm_add_pair(a.z, b.z), norm_add_pair(a.w, b.w));
}

__device__ __forceinline__ float norm_sumsq_pair(uint32_t p, float s) {
  const float lo = bf16_bits_to_f32(p & 0xffffu), hi = bf16_bits_to_f32(p >> 16);
  return __fmaf_rn(hi, hi, __fmaf_rn(lo, lo, s));
}

__device__ __forceinline__ float norm_sumsq_chunk(uint4 v, float s) {
  return norm_sumsq_pair(v.w, norm_sumsq_pair(v.z, norm_sumsq_pair(v.y, norm_sumsq_pair(v.x, s))));
}

// The wave's part of a row sum (fixed butterfly; every lane gets the sum).
__device__ __forceinline__ float norm_wave_sum(float s) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) s = __fadd_rn(s, __shfl_xor(s, off, 64));
  return s;
}

// inv = 1 / sqrt(mean + eps) from the 4 wave parts, added in wave order.
__device__ __forceinline__ float norm_inv(const float* part, int64_t d, float eps) {
  float tot = part[0];
#pragma unroll
  for (int q = 1; q < 4; ++q) tot = __fadd_rn(tot, part[q]);
  const float var = __fdiv_rn(tot, (float)d);
  return __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(var, eps)));
}

__device__ __forceinline__ uint32_t norm_scale_pair(uint32_t x, uint32_t w, float inv) {
  const float lo = __fmul_rn(bf16_bits_to_f32(w & 0xffffu), __fmul_rn(bf16_bits_to_f32(x & 0xffffu), inv));
  const float hi = __fmul_rn(bf16_bits_to_f32(w >> 16), __fmul_rn(bf16_bits_to_f32(x >> 16), inv));
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

__device__ __forceinline__ uint4 norm_scale_chunk(uint4 v, uint4 g, float inv) {
  return make_uint4(norm_scale_pair(v.x, g.x, inv), norm_scale_pair(v.y, g.y, inv), norm_scale_pair(v.z, g.z, inv),
                    norm_scale_pair(v.w, g.w, inv));
}

}  // namespace hsmoe
