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

// kGather: row r of x is row ids[r] of a [vocab, d] table (an embedding
// lookup); an id outside [0, vocab) reads a row of zeros.
template <bool kAdd, bool kRes, bool kGather = false>
__global__ void __launch_bounds__(kThreads)
    add_rms_norm_kernel(const uint4* __restrict__ x, const uint4* __restrict__ add, const uint4* __restrict__ res,
                        const uint4* __restrict__ w, int64_t d, float eps, uint4* __restrict__ h_out,
                        uint4* __restrict__ out, const int64_t* __restrict__ ids = nullptr, int64_t vocab = 0) {
  __shared__ uint4 row[kMaxD / 8];
  __shared__ uint4 wrow[kMaxD / 8];
  __shared__ float part[kThreads / 64];
  const int chunks = (int)(d / 8);
  const int64_t base = (int64_t)blockIdx.x * chunks;
  bool have_x = true;
  const uint4* xr = x + base;  // this row's chunks
  if (kGather) {
    const int64_t id = ids[blockIdx.x];
    have_x = id >= 0 && id < vocab;
    xr = x + (have_x ? id : 0) * chunks;
  }
  float s = 0.0f;
  // every load of kB chunks in flight at once (one memory round trip for d <= 8192), then the chunks in column order
  constexpr int kB = 4;
  for (int c0 = threadIdx.x; c0 < chunks; c0 += kB * kThreads) {
    uint4 v[kB], a[kB], r[kB], wv[kB];
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      const int c = c0 + b * kThreads;
      if (c < chunks) {
        v[b] = have_x ? xr[c] : make_uint4(0u, 0u, 0u, 0u);
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

// The MTP block's input for one token, the data flow of the reference's draft
// step (engine.py:2251-2339) with its projections left out:
//   e = RMSNorm(embed[tok]) * enorm;  g = RMSNorm(h_prev) * hnorm;
//   h = bf16(g + e);  h = bf16(h + res) (when res is given);
//   h_out = h;  out = RMSNorm(h) * w
// One workgroup (d <= 8192: at most 4 chunks per thread, held in registers);
// each RMSNorm has add_rms_norm_kernel's arithmetic and order, so the result
// equals the three norm launches and the bf16 add it replaces, bit for bit.
__global__ void __launch_bounds__(kThreads)
    mtp_input_kernel(const int64_t* __restrict__ tok, const uint4* __restrict__ embed, int64_t vocab,
                     const uint4* __restrict__ h_prev, const uint4* __restrict__ enorm,
                     const uint4* __restrict__ hnorm, const uint4* __restrict__ res, const uint4* __restrict__ w,
                     int64_t d, float eps, uint4* __restrict__ h_out, uint4* __restrict__ out) {
  __shared__ float part[3][kThreads / 64];
  const int chunks = (int)(d / 8), tid = (int)threadIdx.x;
  // the norm weights and the residual depend on nothing: their loads go out
  // with the token id's, not after the barriers that the sums need
  const uint4 zero = make_uint4(0u, 0u, 0u, 0u);
  uint4 env[4], hnv[4], rsv[4], wv[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int c = tid + kThreads * b;
    env[b] = hnv[b] = rsv[b] = wv[b] = zero;
    if (c < chunks) {
      env[b] = enorm[c];
      hnv[b] = hnorm[c];
      if (res) rsv[b] = res[c];
      wv[b] = w[c];
    }
  }
  const int64_t id = tok[0];
  const bool have = id >= 0 && id < vocab;
  const uint4* er = embed + (have ? id : 0) * chunks;
  uint4 ev[4], gv[4];
  float se = 0.0f, sg = 0.0f;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int c = tid + kThreads * b;
    ev[b] = gv[b] = zero;
    if (c < chunks) {
      ev[b] = have ? er[c] : zero;
      gv[b] = h_prev[c];
      se = norm_sumsq_chunk(ev[b], se);
      sg = norm_sumsq_chunk(gv[b], sg);
    }
  }
  se = norm_wave_sum(se);
  sg = norm_wave_sum(sg);
  if ((tid & 63) == 0) {
    part[0][tid >> 6] = se;
    part[1][tid >> 6] = sg;
  }
  __syncthreads();
  const float ie = norm_inv(part[0], d, eps), ig = norm_inv(part[1], d, eps);
  float sh = 0.0f;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int c = tid + kThreads * b;
    if (c < chunks) {
      const uint4 e = norm_scale_chunk(ev[b], env[b], ie);
      uint4 h = norm_add_chunk(norm_scale_chunk(gv[b], hnv[b], ig), e);
      if (res) h = norm_add_chunk(h, rsv[b]);
      ev[b] = h;
      h_out[c] = h;
      sh = norm_sumsq_chunk(h, sh);
    }
  }
  sh = norm_wave_sum(sh);
  if ((tid & 63) == 0) part[2][tid >> 6] = sh;
  __syncthreads();
  const float ih = norm_inv(part[2], d, eps);
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int c = tid + kThreads * b;
    if (c < chunks) out[c] = norm_scale_chunk(ev[b], wv[b], ih);
  }
}

}  // namespace
}  // namespace hsmoe

using namespace hsmoe;

extern "C" int hsmoe_mtp_input(const int64_t* tok, const void* embed, int64_t vocab, const void* h_prev,
                               const void* enorm_w, const void* hnorm_w, const void* res, const void* w, int64_t d,
                               float eps, void* h_out, void* out, hsmoe_stream_t stream) {
  if (!tok || !embed || !h_prev || !enorm_w || !hnorm_w || !w || !h_out || !out || d < 1 || vocab < 1)
    return fail(HSMOE_ERR_ARG, "hsmoe_mtp_input: bad arguments");
  if (d % 8 != 0 || d > 8192) return fail(HSMOE_ERR_SHAPE, "hsmoe_mtp_input: d must be a multiple of 8, <= 8192");
  const void* rows16[] = {embed, h_prev, enorm_w, hnorm_w, w, h_out, out};
  for (const void* q : rows16)
    if (!aligned(q, 16)) return fail(HSMOE_ERR_SHAPE, "hsmoe_mtp_input: rows must be 16-byte aligned");
  if ((res && !aligned(res, 16)) || !aligned(tok, 8))
    return fail(HSMOE_ERR_SHAPE, "hsmoe_mtp_input: rows must be 16-byte aligned");
  hipLaunchKernelGGL(mtp_input_kernel, dim3(1), dim3(kThreads), 0, (hipStream_t)stream, tok, (const uint4*)embed,
                     vocab, (const uint4*)h_prev, (const uint4*)enorm_w, (const uint4*)hnorm_w, (const uint4*)res,
                     (const uint4*)w, d, eps, (uint4*)h_out, (uint4*)out);
  return check_launch("hsmoe_mtp_input");
}

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

extern "C" int hsmoe_embed_add_rms_norm(const int64_t* ids, int64_t rows, const void* table, int64_t vocab,
                                        const void* res, const void* w, int64_t d, float eps, void* h_out, void* out,
                                        hsmoe_stream_t stream) {
  if (!ids || !table || !w || !out || rows < 0 || d < 1 || vocab < 1)
    return fail(HSMOE_ERR_ARG, "hsmoe_embed_add_rms_norm: bad arguments");
  if (d % 8 != 0 || d > kMaxD)
    return fail(HSMOE_ERR_SHAPE, "hsmoe_embed_add_rms_norm: d must be a multiple of 8 and at most %d", kMaxD);
  if (!aligned(table, 16) || !aligned(w, 16) || !aligned(out, 16) || (res && !aligned(res, 16)) ||
      (h_out && !aligned(h_out, 16)) || !aligned(ids, 8))
    return fail(HSMOE_ERR_SHAPE, "hsmoe_embed_add_rms_norm: rows must be 16-byte aligned");
  if (rows == 0) return HSMOE_OK;
  hipStream_t st = (hipStream_t)stream;
  const uint4 *tp = (const uint4*)table, *rp = (const uint4*)res, *wp = (const uint4*)w;
  uint4 *hp = (uint4*)h_out, *op = (uint4*)out;
  const dim3 grid((unsigned)rows), block(kThreads);
  if (res)
    hipLaunchKernelGGL((add_rms_norm_kernel<false, true, true>), grid, block, 0, st, tp, nullptr, rp, wp, d, eps, hp,
                       op, ids, vocab);
  else
    hipLaunchKernelGGL((add_rms_norm_kernel<false, false, true>), grid, block, 0, st, tp, nullptr, nullptr, wp, d, eps,
                       hp, op, ids, vocab);
  return check_launch("hsmoe_embed_add_rms_norm");
}

extern "C" int hsmoe_rms_norm(const void* x, const void* w, int64_t rows, int64_t d, float eps, void* out,
                              hsmoe_stream_t stream) {
  return hsmoe_add_rms_norm(x, nullptr, nullptr, w, rows, d, eps, nullptr, out, stream);
}
