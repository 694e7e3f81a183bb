// RMSNorm between MoE layers, restating rms_norm (utils.py:6-9):
//   var = mean(float(x)^2); y = float(w) * (float(x) * rsqrt(var + eps)); out = bf16(y)
// optionally preceded by the two residual adds of a layer (torch bf16 adds:
// fp32 sum rounded once):
//   h = bf16(x + add)      the previous layer's FFN output (engine.py:2690)
//   h = bf16(h + res)      the attention stand-in residual of this layer
// One workgroup (256 threads) per row.  Each thread owns 8-column chunks
// c, c + 256, ...; the row stays in LDS between the sum-of-squares pass and
// the scaling pass, so x is read from memory once.  The sum of squares is
// accumulated per thread in column order, then reduced across the wave by a
// fixed xor-butterfly and across the 4 waves in wave order: results are
// deterministic.
#include "hsmoe_common.h"
#include "hsmoe_internal.h"

namespace hsmoe {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxD = 16384;

__device__ __forceinline__ uint32_t add_bf16(uint32_t a, uint32_t b) {
  return f32_to_bf16_bits(__fadd_rn(bf16_bits_to_f32(a), bf16_bits_to_f32(b)));
}

// Elementwise bf16 add of two packed pairs.
__device__ __forceinline__ uint32_t add_pair(uint32_t a, uint32_t b) {
  return add_bf16(a & 0xffffu, b & 0xffffu) | (add_bf16(a >> 16, b >> 16) << 16);
}

__device__ __forceinline__ uint4 add_chunk(uint4 a, uint4 b) {
  return make_uint4(add_pair(a.x, b.x), add_pair(a.y, b.y), add_pair(a.z, b.z), add_pair(a.w, b.w));
}

__device__ __forceinline__ float sumsq_pair(uint32_t p, float s) {
  const float lo = bf16_bits_to_f32(p & 0xffffu), hi = bf16_bits_to_f32(p >> 16);
  return __fmaf_rn(hi, hi, __fmaf_rn(lo, lo, s));
}

__device__ __forceinline__ uint32_t scale_pair(uint32_t x, uint32_t w, float inv) {
  const float lo = __fmul_rn(bf16_bits_to_f32(w & 0xffffu), __fmul_rn(bf16_bits_to_f32(x & 0xffffu), inv));
  const float hi = __fmul_rn(bf16_bits_to_f32(w >> 16), __fmul_rn(bf16_bits_to_f32(x >> 16), inv));
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

template <bool kAdd, bool kRes>
__global__ void __launch_bounds__(kThreads)
    add_rms_norm_kernel(const uint4* __restrict__ x, const uint4* __restrict__ add, const uint4* __restrict__ res,
                        const uint4* __restrict__ w, int64_t d, float eps, uint4* __restrict__ h_out,
                        uint4* __restrict__ out) {
  __shared__ uint4 row[kMaxD / 8];
  __shared__ float part[kThreads / 64];
  const int chunks = (int)(d / 8);
  const int64_t base = (int64_t)blockIdx.x * chunks;
  float s = 0.0f;
  for (int c = threadIdx.x; c < chunks; c += kThreads) {
    uint4 v = x[base + c];
    if (kAdd) v = add_chunk(v, add[base + c]);
    if (kRes) v = add_chunk(v, res[c]);
    if (h_out) h_out[base + c] = v;
    row[c] = v;
    s = sumsq_pair(v.w, sumsq_pair(v.z, sumsq_pair(v.y, sumsq_pair(v.x, s))));
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) s = __fadd_rn(s, __shfl_xor(s, off, 64));
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  float tot = part[0];
#pragma unroll
  for (int q = 1; q < kThreads / 64; ++q) tot = __fadd_rn(tot, part[q]);
  const float var = __fdiv_rn(tot, (float)d);
  const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(var, eps)));
  for (int c = threadIdx.x; c < chunks; c += kThreads) {
    const uint4 v = row[c], g = w[c];
    out[base + c] = make_uint4(scale_pair(v.x, g.x, inv), scale_pair(v.y, g.y, inv), scale_pair(v.z, g.z, inv),
                               scale_pair(v.w, g.w, inv));
  }
}

}  // namespace
}  // namespace hsmoe

using namespace hsmoe;

extern "C" int hsmoe_add_rms_norm(const void* x, const void* add, const void* res, const void* w, int64_t rows,
                                  int64_t d, float eps, void* h_out, void* out, hsmoe_stream_t stream) {
  if (!x || !w || !out || rows < 0 || d < 1) return fail(HSMOE_ERR_ARG, "hsmoe_add_rms_norm: bad arguments");
  if (d % 8 != 0 || d > kMaxD)
    return fail(HSMOE_ERR_SHAPE, "hsmoe_add_rms_norm: d must be a multiple of 8 and at most %d", kMaxD);
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(out, 16) || (add && !aligned(add, 16)) ||
      (res && !aligned(res, 16)) || (h_out && !aligned(h_out, 16)))
    return fail(HSMOE_ERR_SHAPE, "hsmoe_add_rms_norm: rows must be 16-byte aligned");
  if (rows == 0) return HSMOE_OK;
  hipStream_t st = (hipStream_t)stream;
  const uint4 *xp = (const uint4*)x, *ap = (const uint4*)add, *rp = (const uint4*)res, *wp = (const uint4*)w;
  uint4 *hp = (uint4*)h_out, *op = (uint4*)out;
  const dim3 grid((unsigned)rows), block(kThreads);
  if (add && res)
    hipLaunchKernelGGL((add_rms_norm_kernel<true, true>), grid, block, 0, st, xp, ap, rp, wp, d, eps, hp, op);
  else if (add)
    hipLaunchKernelGGL((add_rms_norm_kernel<true, false>), grid, block, 0, st, xp, ap, rp, wp, d, eps, hp, op);
  else if (res)
    hipLaunchKernelGGL((add_rms_norm_kernel<false, true>), grid, block, 0, st, xp, ap, rp, wp, d, eps, hp, op);
  else
    hipLaunchKernelGGL((add_rms_norm_kernel<false, false>), grid, block, 0, st, xp, ap, rp, wp, d, eps, hp, op);
  return check_launch("hsmoe_add_rms_norm");
}

extern "C" int hsmoe_rms_norm(const void* x, const void* w, int64_t rows, int64_t d, float eps, void* out,
                              hsmoe_stream_t stream) {
  return hsmoe_add_rms_norm(x, nullptr, nullptr, w, rows, d, eps, nullptr, out, stream);
}
