// Shared device/host helpers for libhsmoe (gfx950 only).
//
// Number formats follow the reference's PyTorch path:
//   e2m1 codes      _fp4.py:72-95, fused_moe.py:604-608 (lo nibble = even column)
//   E8M0 scales     torch float8_e8m0fnu -> float32 (engine.py:1260-1271): 2^(e-127),
//                   e == 255 -> NaN.  v_cvt_scalef32_pk_*_fp4 applies exactly this.
//   fp32 scales     bf16(fp32(code) * scale), fused_moe.py:22-26
//   e4m3 + blocks   cast_back(..., (128, 128)), _fp4.py:98-110
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hsmoe {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2;

// Scale encodings accepted for FP4 weights.
enum ScaleKind : int {
  kScaleE8M0 = 0,  // one uint8 exponent per 32 columns
  kScaleF32 = 1,   // one fp32 value per 32 columns
};

// ------------------------------------------------------------------ loads
// A load through the global address space (global_load_*).  A pointer whose
// address space the compiler cannot see (an address read from a table or a
// parameter block) gives a flat load, which counts against lgkmcnt as well as
// vmcnt: every wait for an LDS access would then also wait for it.
template <typename T>
__device__ __forceinline__ T ldg(const void* p) {
  return *(const T __attribute__((address_space(1)))*)p;
}
// uint4 is a class (its copy would go through a generic reference): load the
// native 4 x u32 vector instead.
template <>
__device__ __forceinline__ uint4 ldg<uint4>(const void* p) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = *(const u32x4 __attribute__((address_space(1)))*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}

// A buffer resource (V#) over `bytes` bytes at `base`: loads through it take a
// 32-bit per-lane offset plus an immediate (one offset register serves a whole
// batch of loads), and a load past `bytes` returns zeros instead of touching
// memory.  base is made wave-uniform (it lives in scalar registers).
typedef __amdgpu_buffer_rsrc_t BufRsrc;
__device__ __forceinline__ BufRsrc make_buf(uint64_t base, uint32_t bytes) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)base);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
  const uint32_t n = __builtin_amdgcn_readfirstlane(bytes);
  // word 3 = 0x00020000: raw (unformatted) 32-bit data, the gfx9 setting
  return __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | lo), (short)0, (int)n, 0x00020000);
}
__device__ __forceinline__ uint4 bload128(BufRsrc r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint32_t bload32(BufRsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ __forceinline__ float bloadf(BufRsrc r, uint32_t off) { return __uint_as_float(bload32(r, off)); }
__device__ __forceinline__ uint2 bload64(BufRsrc r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
  return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint32_t bload8(BufRsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b8(r, (int)off, 0, 0);
}

// ------------------------------------------------------------------ bits
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Round-to-nearest-even fp32 -> bf16 (same as torch's .to(torch.bfloat16)).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  __bf16 h = (__bf16)f;
  return (uint32_t)__builtin_bit_cast(unsigned short, h);
}

// Correctly rounded fp64 -> bf16 (one rounding), NaN -> 0x7FC0.
__device__ __forceinline__ uint32_t f64_to_bf16_bits(double d) {
  if (__builtin_isnan(d)) return 0x7fc0u;
  uint64_t u = __double_as_longlong(d);
  uint32_t sign = (uint32_t)(u >> 48) & 0x8000u;
  uint64_t mag = u & 0x7fffffffffffffffull;
  int e = (int)(mag >> 52);  // biased fp64 exponent
  if (mag == 0) return sign;
  // bf16 keeps 7 fraction bits; for normal bf16 results (unbiased exponent
  // >= -126) drop 45 fraction bits of the fp64 with RNE.
  int ue = e - 1023;
  if (ue >= -126) {
    uint64_t frac_keep_shift = 45;
    uint64_t rounded = mag + ((1ull << (frac_keep_shift - 1)) - 1) + ((mag >> frac_keep_shift) & 1);
    uint64_t r = rounded >> frac_keep_shift;  // fp64 exponent(11) | fraction(7)
    int re = (int)(r >> 7) - 1023;            // exponent after rounding carry
    if (re > 127) return sign | 0x7f80u;
    return sign | (uint32_t)(((re + 127) << 7) | (uint32_t)(r & 0x7f));
  }
  // subnormal bf16: value = q * 2^-133 with q in [0, 128]
  double q = __builtin_ldexp(__builtin_fabs(d), 133);
  double rq = __builtin_rint(q);
  return sign | (uint32_t)rq;  // q == 128 is the smallest normal 0x0080
}

// ------------------------------------------------------------------ RNG
// splitmix64: rand(key, i) is the (i+1)-th output of splitmix64(key).
__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__host__ __device__ __forceinline__ uint64_t rand64(uint64_t key, uint64_t i) {
  return mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull);
}

// ------------------------------------------------------------------ decode
// 4 packed bytes (8 e2m1 codes) -> 8 bf16, E8M0 scale given as fp32 bits e<<23.
__device__ __forceinline__ bf16x8 fp4x8_to_bf16_e8m0(uint32_t w, float s) {
  bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 0);
  bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 1);
  bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 2);
  bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 3);
  bf16x8 r = {a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
  return r;
}

// 4 packed bytes -> 8 bf16 with an arbitrary fp32 scale: exact fp32 code
// value (scale 1.0), one fp32 multiply, one RNE rounding -- the reference's
// (deq.float() * sf.float()).to(torch.bfloat16).
__device__ __forceinline__ bf16x8 fp4x8_to_bf16_f32(uint32_t w, float s) {
  f32x2 v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
  f32x2 v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
  f32x2 v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
  f32x2 v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
  bf16x8 r = {(__bf16)__fmul_rn(v0[0], s), (__bf16)__fmul_rn(v0[1], s), (__bf16)__fmul_rn(v1[0], s),
              (__bf16)__fmul_rn(v1[1], s), (__bf16)__fmul_rn(v2[0], s), (__bf16)__fmul_rn(v2[1], s),
              (__bf16)__fmul_rn(v3[0], s), (__bf16)__fmul_rn(v3[1], s)};
  return r;
}

// 4 e4m3 bytes -> 4 fp32 (exact), then * block scale -> bf16 RNE.
__device__ __forceinline__ void fp8x4_to_bf16(uint32_t w, float s, bf16x8& r, int half) {
  f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
  f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(w, true);
  r[4 * half + 0] = (__bf16)(lo[0] * s);
  r[4 * half + 1] = (__bf16)(lo[1] * s);
  r[4 * half + 2] = (__bf16)(hi[0] * s);
  r[4 * half + 3] = (__bf16)(hi[1] * s);
}

__device__ __forceinline__ float e8m0_as_f32(uint32_t e) { return __uint_as_float(e << 23); }

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

}  // namespace hsmoe
