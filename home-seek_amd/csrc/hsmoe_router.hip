// Router: logits GEMV (exact fp64 accumulation, one bf16 rounding), bias add in
// bf16, sqrt(softplus) scores, stable top-k and renormalised weights.
// Restates compute_expert_affinity_with_bias (router.py:22-36).
//
// One launch: block (expert group, chunk of 8 tokens) computes 4 expert rows
// of logits for the chunk (the 2 MiB gate matrix is read once per chunk,
// HBM-bound); the chunk's last block to finish selects the top-k of each of
// its tokens with (score desc, index asc) order == torch.sort(stable=True).
#include <math.h>

#include "hsmoe_common.h"
#include "hsmoe_internal.h"

namespace hsmoe {
namespace {

constexpr int kTok = 8;         // tokens per logits wave
constexpr int kLogitWaves = 4;  // expert rows per logits workgroup

__device__ __forceinline__ double wave_sum_f64(double v) {
  // fixed butterfly order: the same lanes combine on every call
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

constexpr int kMaxChunks = 16;  // d <= 8192: 16-byte chunks per lane
constexpr int kMaxPerLane = 16;  // n_experts <= 1024
constexpr size_t kCounterBytes = 4096;

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
__device__ void wave_topk(const float* sc, int64_t n_exp, int top_k, float scaling, int64_t* idx_out,
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

// Block (expert group bx, token chunk by): wave w computes the logits of
// expert 4*bx + w for the chunk's (<= 8) tokens -- lane l holds columns
// 8l + 512c .. +8 of the row for every c, all loads issued before the math.
// The last block of a chunk (agent-scope arrival counter) runs the top-k of
// the chunk's tokens, one token per wave, and re-arms the counter.
__global__ void __launch_bounds__(64 * kLogitWaves)
    router_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const float* __restrict__ bias,
                  int64_t m, int64_t d, int64_t n_exp, int top_k, float scaling, uint16_t* __restrict__ logits_out,
                  float* __restrict__ stage, unsigned* __restrict__ counters, int64_t* __restrict__ idx_out,
                  float* __restrict__ w_out) {
  extern __shared__ __align__(16) uint16_t xs[];  // [nt][d]
  __shared__ int s_last;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t e = (int64_t)blockIdx.x * kLogitWaves + wave;
  const int64_t t0 = (int64_t)blockIdx.y * kTok;
  const int nt = (int)((m - t0) < kTok ? (m - t0) : kTok);
  // the gate rows do not depend on x: issue their loads before staging x
  uint4 wv[kMaxChunks];
  if (e < n_exp) {
    const uint16_t* wr = w + e * d;
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c)
      if (lane * 8 + 512 * c < d) wv[c] = *reinterpret_cast<const uint4*>(wr + lane * 8 + 512 * c);
  }
  for (int64_t q = threadIdx.x; q < nt * d / 8; q += blockDim.x)
    reinterpret_cast<uint4*>(xs)[q] = reinterpret_cast<const uint4*>(x + t0 * d)[q];
  __syncthreads();
  if (e < n_exp) {
    double acc[kTok];
#pragma unroll
    for (int t = 0; t < kTok; ++t) acc[t] = 0.0;
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
        for (int t = 0; t < kTok; ++t) {
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
    for (int t = 0; t < kTok; ++t) {
      if (t < nt) {
        const double sum = wave_sum_f64(acc[t]);
        if (lane == 0) {
          uint32_t l = f64_to_bf16_bits(sum);
          if (bias) l = f32_to_bf16_bits(__fadd_rn(bf16_bits_to_f32(l), b));
          if (logits_out) logits_out[(t0 + t) * n_exp + e] = (uint16_t)l;
          const float score = sqrtf(softplus_f32(bf16_bits_to_f32(l)));
          __hip_atomic_store(stage + (t0 + t) * n_exp + e, score, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(&counters[blockIdx.y], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             gridDim.x - 1;
  __syncthreads();
  if (!s_last) return;
  for (int t = wave; t < nt; t += kLogitWaves)
    wave_topk(stage + (t0 + t) * n_exp, n_exp, top_k, scaling, idx_out + (t0 + t) * top_k, w_out + (t0 + t) * top_k);
  if (threadIdx.x == 0) __hip_atomic_store(&counters[blockIdx.y], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace
}  // namespace hsmoe

using namespace hsmoe;

extern "C" size_t hsmoe_router_workspace_size(int64_t m, int64_t n_experts) {
  if (m < 0 || n_experts < 0) return 0;
  // [chunk arrival counters, fixed 4 KiB | staged fp32 scores [m][n_experts]]
  return kCounterBytes + (size_t)(((m * n_experts * 4) + 255) / 256 * 256);
}

extern "C" int hsmoe_router_topk(const void* x, const void* gate_w, const float* bias, int64_t m, int64_t d,
                                 int64_t n_experts, int top_k, float scaling, int64_t* idx_out, float* w_out,
                                 void* logits_out, void* workspace, size_t workspace_bytes, hsmoe_stream_t stream) {
  if (!x || !gate_w || !idx_out || !w_out || m < 0 || d <= 0 || n_experts <= 0)
    return fail(HSMOE_ERR_ARG, "hsmoe_router_topk: null pointer or bad size");
  if (n_experts > 1024 || top_k < 1 || top_k > 16 || top_k > n_experts)
    return fail(HSMOE_ERR_SHAPE, "hsmoe_router_topk: need 1 <= top_k <= min(16, n_experts) and n_experts <= 1024");
  if (d % 512 != 0 || d > 8192 || !aligned(x, 16) || !aligned(gate_w, 16))
    return fail(HSMOE_ERR_SHAPE,
                "hsmoe_router_topk: d must be a multiple of 512 (<= 8192) and x/gate_w 16-byte aligned");
  const int64_t chunks = (m + kTok - 1) / kTok;
  if ((size_t)chunks * 4 > kCounterBytes) return fail(HSMOE_ERR_SHAPE, "hsmoe_router_topk: m must be <= 8192");
  if (!workspace || workspace_bytes < hsmoe_router_workspace_size(m, n_experts) || !aligned(workspace, 256))
    return fail(HSMOE_ERR_WORKSPACE, "hsmoe_router_topk: zero-filled 256-byte aligned workspace of %zu bytes needed",
                hsmoe_router_workspace_size(m, n_experts));
  if (m == 0) return HSMOE_OK;
  unsigned* counters = (unsigned*)workspace;
  float* stage = (float*)((char*)workspace + kCounterBytes);
  dim3 grid((unsigned)((n_experts + kLogitWaves - 1) / kLogitWaves), (unsigned)chunks);
  const size_t lds = (size_t)(m < kTok ? m : kTok) * d * 2;
  hipLaunchKernelGGL(router_kernel, grid, dim3(64 * kLogitWaves), lds, (hipStream_t)stream, (const uint16_t*)x,
                     (const uint16_t*)gate_w, bias, m, d, n_experts, top_k, scaling, (uint16_t*)logits_out, stage,
                     counters, idx_out, w_out);
  return check_launch("hsmoe_router_topk");
}
