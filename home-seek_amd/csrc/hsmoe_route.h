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

// One DPP step of a wave-wide 64-bit max: every lane enabled by kRowMask
// takes the larger of its key and the key of the lane kCtrl names.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint64_t dpp_max_step(uint64_t k) {
  const int lo = (int)(uint32_t)k, hi = (int)(uint32_t)(k >> 32);
  const uint32_t olo = (uint32_t)__builtin_amdgcn_update_dpp(lo, lo, kCtrl, kRowMask, 0xf, false);
  const uint32_t ohi = (uint32_t)__builtin_amdgcn_update_dpp(hi, hi, kCtrl, kRowMask, 0xf, false);
  const uint64_t o = ((uint64_t)ohi << 32) | olo;
  return o > k ? o : k;
}

// The same steps for a 32-bit key (one DPP-fed max per step).
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t dpp_max_step32(uint32_t k) {
  const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp((int)k, (int)k, kCtrl, kRowMask, 0xf, false);
  return o > k ? o : k;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t k) {
  k = dpp_max_step32<0xb1, 0xf>(k);
  k = dpp_max_step32<0x4e, 0xf>(k);
  k = dpp_max_step32<0x141, 0xf>(k);
  k = dpp_max_step32<0x140, 0xf>(k);
  k = dpp_max_step32<0x142, 0xa>(k);
  k = dpp_max_step32<0x143, 0xc>(k);
  return (uint32_t)__builtin_amdgcn_readlane((int)k, 63);
}

// Wave-wide maximum of a 64-bit key, returned to every lane: quad swaps,
// half-row and row mirrors, then the row broadcasts of lane 15 and lane 31
// leave the maximum in lane 63 (six dependent DPP steps instead of six
// LDS-crossbar shuffles).
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
  k = dpp_max_step<0xb1, 0xf>(k);   // quad_perm [1,0,3,2]
  k = dpp_max_step<0x4e, 0xf>(k);   // quad_perm [2,3,0,1]
  k = dpp_max_step<0x141, 0xf>(k);  // row_half_mirror
  k = dpp_max_step<0x140, 0xf>(k);  // row_mirror
  k = dpp_max_step<0x142, 0xa>(k);  // row_bcast:15 into rows 1, 3
  k = dpp_max_step<0x143, 0xc>(k);  // row_bcast:31 into rows 2, 3
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 63);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}

// Top-k of one token by one wave: lane l keys experts l, l+64, ... (kPer of
// them, v[q] = score of expert l + 64q, sorted descending once), and each
// round retires the wave-wide maximum key, popping it from the head of its
// lane's list.
template <int kPer>
__device__ __forceinline__ void wave_topk_vals(const float (&v)[kPer], int64_t n_exp, int top_k, float scaling,
                                               int64_t* idx_out, float* w_out) {
  const int lane = threadIdx.x & 63;
  uint64_t key[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int e = lane + 64 * q;
    key[q] = e < n_exp ? score_key(v[q], e) : 0ull;
  }
#pragma unroll
  for (int i = 1; i < kPer; ++i)  // insertion network, descending
#pragma unroll
    for (int j = i; j > 0; --j) {
      const uint64_t a = key[j - 1], b = key[j];
      key[j - 1] = a > b ? a : b;
      key[j] = a > b ? b : a;
    }
  float my_v = 0.0f, sum = 0.0f;
  int my_e = 0;
  for (int r = 0; r < top_k; ++r) {
    // The lane holding the largest key: when a single lane holds the largest
    // high half (the score), its key is the largest; otherwise (equal scores)
    // the full 64-bit maximum decides.  Keys are unique, so one lane wins.
    const uint32_t hi = (uint32_t)(key[0] >> 32);
    const uint32_t mhi = wave_max_u32(hi);
    uint64_t top = __ballot(hi == mhi);
    if (__popcll(top) != 1) top = __ballot(key[0] == wave_max_u64(key[0]));
    const int win = (int)__builtin_ctzll(top);
    const uint64_t best = ((uint64_t)mhi << 32) | (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key[0], win);
    const bool mine = lane == win;
#pragma unroll
    for (int q = 0; q + 1 < kPer; ++q) key[q] = mine ? key[q + 1] : key[q];
    key[kPer - 1] = mine ? 0ull : key[kPer - 1];
    const int e = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
    uint32_t b = (uint32_t)(best >> 32);
    b = (b & 0x80000000u) ? (b & 0x7fffffffu) : ~b;  // undo score_key's float map
    const float val = __uint_as_float(b);
    if (lane == r) {
      my_v = val;
      my_e = e;
    }
    sum = __fadd_rn(sum, val);
  }
  sum = fmaxf(sum, 1e-20f);
  if (lane < top_k) {
    idx_out[lane] = my_e;
    w_out[lane] = __fmul_rn(__fdiv_rn(my_v, sum), scaling);
  }
}

// wave_topk_vals over the token's fp32 scores `sc`, written by other
// workgroups and read with agent-scope loads.
template <int kPer>
__device__ __forceinline__ void wave_topk_n(const float* sc, int64_t n_exp, int top_k, float scaling,
                                            int64_t* idx_out, float* w_out) {
  const int lane = threadIdx.x & 63;
  float v[kPer];  // every load is issued before any is used (one memory round trip)
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int e = lane + 64 * q;
    v[q] = __hip_atomic_load(sc + (e < n_exp ? e : n_exp - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  wave_topk_vals<kPer>(v, n_exp, top_k, scaling, idx_out, w_out);
}

__device__ __forceinline__ void wave_topk(const float* sc, int64_t n_exp, int top_k, float scaling, int64_t* idx_out,
                                          float* w_out) {
  const int per = (int)((n_exp + 63) / 64);
  if (per <= 1) wave_topk_n<1>(sc, n_exp, top_k, scaling, idx_out, w_out);
  else if (per <= 2) wave_topk_n<2>(sc, n_exp, top_k, scaling, idx_out, w_out);
  else if (per <= 4) wave_topk_n<4>(sc, n_exp, top_k, scaling, idx_out, w_out);
  else if (per <= 8) wave_topk_n<8>(sc, n_exp, top_k, scaling, idx_out, w_out);
  else wave_topk_n<16>(sc, n_exp, top_k, scaling, idx_out, w_out);
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

// The score of expert e from its exact logit sum (fp64): logit =
// bf16(sum), then bf16(logit + bf16(bias[e])) with a bias; the bf16 logit goes
// to *logit_out when non-null; score = sqrt(softplus(float(logit))).
// (bias_v: bias[e], already loaded; used when has_bias)
__device__ __forceinline__ float router_score_v(double sum, bool has_bias, float bias_v, uint16_t* logit_out) {
  uint32_t l = f64_to_bf16_bits(sum);
  if (has_bias) l = f32_to_bf16_bits(__fadd_rn(bf16_bits_to_f32(l), bf16_bits_to_f32(f32_to_bf16_bits(bias_v))));
  if (logit_out) *logit_out = (uint16_t)l;
  return sqrtf(softplus_f32(bf16_bits_to_f32(l)));
}
__device__ __forceinline__ float router_score(double sum, const float* bias, int64_t e, uint16_t* logit_out) {
  return router_score_v(sum, bias != nullptr, bias ? bias[e] : 0.0f, logit_out);
}

// Exact products of 8 bf16 pairs (a packed uint4 each) added to acc in fp64,
// element order.
__device__ __forceinline__ double dot8_f64(uint4 xv, uint4 wv, double acc) {
  const uint32_t xx[4] = {xv.x, xv.y, xv.z, xv.w}, ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    acc = __fma_rn((double)__uint_as_float(xx[q] << 16), (double)__uint_as_float(ww[q] << 16), acc);
    acc = __fma_rn((double)__uint_as_float(xx[q] & 0xffff0000u), (double)__uint_as_float(ww[q] & 0xffff0000u), acc);
  }
  return acc;
}

__device__ __forceinline__ void router_row(const uint4 (&wv)[kMaxChunks], const uint16_t* xs, int nt, int64_t d,
                                           int64_t e, int64_t n_exp, const float* bias, uint16_t* logits_row,
                                           float* scores) {
  const int lane = threadIdx.x & 63;
  // One token at a time (a rolled loop: the unrolled token loop made this the
  // largest straight-line code of the layer kernel, fetched cold by every
  // router item); per token the sum runs over chunks, then words, in order.
#pragma unroll 1
  for (int t = 0; t < nt; ++t) {
    double acc = 0.0;
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
      if (lane * 8 + 512 * c < d) {
        uint32_t ww[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
        // opaque to the optimiser: the fp64 weights are rebuilt per token
        // instead of being hoisted out of the token loop (256 registers)
        asm volatile("" : "+v"(ww[0]), "+v"(ww[1]), "+v"(ww[2]), "+v"(ww[3]));
        const uint4 xv = *reinterpret_cast<const uint4*>(xs + t * d + lane * 8 + 512 * c);
        const uint32_t xx[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc = __fma_rn((double)__uint_as_float(xx[q] << 16), (double)__uint_as_float(ww[q] << 16), acc);
          acc = __fma_rn((double)__uint_as_float(xx[q] & 0xffff0000u), (double)__uint_as_float(ww[q] & 0xffff0000u),
                         acc);
        }
      }
    }
    const double sum = wave_sum_f64(acc);
    if (lane == 0) {
      const float score = router_score(sum, bias, e, logits_row ? logits_row + t * n_exp : nullptr);
      __hip_atomic_store(scores + t * n_exp, score, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace hsmoe
