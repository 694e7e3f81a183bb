// RMSNorm between MoE layers, restating rms_norm (utils.py:6-9):
//   var = mean(float(x)^2); y = float(w) * (float(x) * rsqrt(var + eps)); out = bf16(y)
// optionally preceded by the two residual adds of a layer (torch bf16 adds:
// fp32 sum rounded once):
//   h = bf16(x + add)      the previous layer's FFN output (engine.py:2690)
//   h = bf16(h + res)      the attention stand-in residual of this layer
// One workgroup (256 threads) per row.  Each thread owns 8-column chunks
// c, c + 256, ...; the row stays in LDS between the sum-of-squares pass and
// the scaling pass, so x is read from memory once; the weight row is loaded
// into LDS in the first pass too, so that the scaling pass waits on no memory.  The sum of squares is
// accumulated per thread in column order, then reduced across the wave by a
// fixed xor-butterfly and across the 4 waves in wave order: results are
// deterministic.
#include "hsmoe_common.h"
#include "hsmoe_internal.h"
#include "hsmoe_norm.h"

namespace hsmoe {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxD = 16384;

template <bool kAdd, bool kRes>
__global__ void __launch_bounds__(kThreads)
    add_rms_norm_kernel(const uint4* __restrict__ x, const uint4* __restrict__ add, const uint4* __restrict__ res,
                        const uint4* __restrict__ w, int64_t d, float eps, uint4* __restrict__ h_out,
                        uint4* __restrict__ out) {
  __shared__ uint4 row[kMaxD / 8];
  __shared__ uint4 wrow[kMaxD / 8];
  __shared__ float part[kThreads / 64];
  const int chunks = (int)(d / 8);
  const int64_t base = (int64_t)blockIdx.x * chunks;
  float s = 0.0f;
  // every load of kB chunks in flight at once (one memory round trip for d <= 8192), then the chunks in column order
  constexpr int kB = 4;
  for (int c0 = threadIdx.x; c0 < chunks; c0 += kB * kThreads) {
    uint4 v[kB], a[kB], r[kB], wv[kB];
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      const int c = c0 + b * kThreads;
      if (c < chunks) {
        v[b] = x[base + c];
        wv[b] = w[c];
        if (kAdd) a[b] = add[base + c];
        if (kRes) r[b] = res[c];
      }
    }
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      const int c = c0 + b * kThreads;
      if (c < chunks) {
        uint4 u = v[b];
        wrow[c] = wv[b];
        if (kAdd) u = norm_add_chunk(u, a[b]);
        if (kRes) u = norm_add_chunk(u, r[b]);
        if (h_out) h_out[base + c] = u;
        row[c] = u;
        s = norm_sumsq_chunk(u, s);
      }
    }
  }
  s = norm_wave_sum(s);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  const float inv = norm_inv(part, d, eps);
  for (int c = threadIdx.x; c < chunks; c += kThreads) out[base + c] = norm_scale_chunk(row[c], wrow[c], inv);
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
