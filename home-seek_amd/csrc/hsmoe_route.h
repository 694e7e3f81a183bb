// Router device helpers shared by hsmoe_router_topk and the fused layer kernel
// (restating compute_expert_affinity_with_bias, router.py:22-36).
#pragma once
#include <math.h>

#include "hsmoe_common.h"

namespace hsmoe {

constexpr int kRouterTok = 8;  // tokens per logits wave

__device__ __forceinline__ double wave_sum_f64(double v) {
  // fixed butterfly order: the same lanes combine on every call
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

constexpr int kMaxChunks = 16;  // d <= 8192: 16-byte chunks per lane
constexpr int kMaxPerLane = 16;  // n_experts <= 1024

// torch.nn.functional.softplus(x) with beta = 1, threshold = 20.
__device__ __forceinline__ float softplus_f32(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

// Sort key: larger score first, equal scores -> smaller index first.  The
// float map is monotone, so NaN (0x7FC00000) ranks above +inf, which is where
// torch.sort(descending=True) puts it.
__device__ __forceinline__ uint64_t score_key(float v, int e) {
  uint32_t b = __float_as_uint(v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)b << 32) | (uint64_t)(0xffffffffu - (uint32_t)e);
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint64_t o = __shfl_xor(k, off, 64);
    k = o > k ? o : k;
  }
  return k;
}

// Top-k of one token by one wave: lane l keys experts l, l+64, ...; each round
// retires the wave-wide maximum key.  `sc` holds the token's fp32 scores,
// written by other blocks and read with agent-scope loads.
__device__ __forceinline__ void wave_topk(const float* sc, int64_t n_exp, int top_k, float scaling, int64_t* idx_out,
                          float* w_out) {
  const int lane = threadIdx.x & 63;
  const int per = (int)((n_exp + 63) / 64);
  uint64_t key[kMaxPerLane];
#pragma unroll
  for (int q = 0; q < kMaxPerLane; ++q) {
    const int e = lane + 64 * q;
    key[q] = (q < per && e < n_exp)
                 ? score_key(__hip_atomic_load(sc + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), e)
                 : 0ull;
  }
  float my_v = 0.0f, sum = 0.0f;
  int my_e = 0;
  for (int r = 0; r < top_k; ++r) {
    uint64_t best = 0;
#pragma unroll
    for (int q = 0; q < kMaxPerLane; ++q)
      if (q < per) best = key[q] > best ? key[q] : best;
    best = wave_max_u64(best);
    const int e = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
#pragma unroll
    for (int q = 0; q < kMaxPerLane; ++q)
      if (q < per && lane + 64 * q == e) key[q] = 0ull;
    uint32_t b = (uint32_t)(best >> 32);
    b = (b & 0x80000000u) ? (b & 0x7fffffffu) : ~b;  // undo score_key's float map
    const float v = __uint_as_float(b);
    if (lane == r) {
      my_v = v;
      my_e = e;
    }
    sum = __fadd_rn(sum, v);
  }
  sum = fmaxf(sum, 1e-20f);
  if (lane < top_k) {
    idx_out[lane] = my_e;
    w_out[lane] = __fmul_rn(__fdiv_rn(my_v, sum), scaling);
  }
}


// One wave computes the router logit and score of expert row `e` for the nt
// (<= 8) token rows of xs ([nt][d] bf16 in LDS); `wv` holds the row's lane
// chunks (lane l: columns 8l + 512c .. +8), loaded by load_gate_row.
//   logit = bf16(exact x . w)   (fp64 sum of exact bf16 products, one rounding)
//   logit = bf16(logit + bf16(bias[e]))  when bias != NULL
//   score = sqrt(softplus(float(logit)))
// Lane 0 writes the logit (when logits_row != NULL: logits_row[t * n_exp]) and
// the score (scores[t * n_exp], agent-scope store).
__device__ __forceinline__ void load_gate_row(const uint16_t* w, int64_t e, int64_t d, uint4 (&wv)[kMaxChunks]) {
  const int lane = threadIdx.x & 63;
  const uint16_t* wr = w + e * d;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c)
    if (lane * 8 + 512 * c < d) wv[c] = *reinterpret_cast<const uint4*>(wr + lane * 8 + 512 * c);
}

__device__ __forceinline__ void router_row(const uint4 (&wv)[kMaxChunks], const uint16_t* xs, int nt, int64_t d,
                                           int64_t e, int64_t n_exp, const float* bias, uint16_t* logits_row,
                                           float* scores) {
  const int lane = threadIdx.x & 63;
  double acc[kRouterTok];
#pragma unroll
  for (int t = 0; t < kRouterTok; ++t) acc[t] = 0.0;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    if (lane * 8 + 512 * c < d) {
      const uint32_t ww[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
      double wd[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        wd[2 * q] = (double)__uint_as_float(ww[q] << 16);
        wd[2 * q + 1] = (double)__uint_as_float(ww[q] & 0xffff0000u);
      }
#pragma unroll
      for (int t = 0; t < kRouterTok; ++t) {
        if (t < nt) {
          const uint4 xv = *reinterpret_cast<const uint4*>(xs + t * d + lane * 8 + 512 * c);
          const uint32_t xx[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            acc[t] = __fma_rn((double)__uint_as_float(xx[q] << 16), wd[2 * q], acc[t]);
            acc[t] = __fma_rn((double)__uint_as_float(xx[q] & 0xffff0000u), wd[2 * q + 1], acc[t]);
          }
        }
      }
    }
  }
  float b = 0.0f;
  if (bias) b = bf16_bits_to_f32(f32_to_bf16_bits(bias[e]));
#pragma unroll
  for (int t = 0; t < kRouterTok; ++t) {
    if (t < nt) {
      const double sum = wave_sum_f64(acc[t]);
      if (lane == 0) {
        uint32_t l = f64_to_bf16_bits(sum);
        if (bias) l = f32_to_bf16_bits(__fadd_rn(bf16_bits_to_f32(l), b));
        if (logits_row) logits_row[t * n_exp] = (uint16_t)l;
        const float score = sqrtf(softplus_f32(bf16_bits_to_f32(l)));
        __hip_atomic_store(scores + t * n_exp, score, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

}  // namespace hsmoe
