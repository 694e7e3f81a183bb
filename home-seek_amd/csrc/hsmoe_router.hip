// Router: logits GEMV (exact fp64 accumulation, one bf16 rounding), bias add in
// bf16, sqrt(softplus) scores, stable top-k and renormalised weights.
// Restates compute_expert_affinity_with_bias (router.py:22-36).
//
// Kernel 1 (router_logits): one wave per (expert row, group of 8 tokens); the
//   2 MiB gate matrix is read once per token group.  HBM-bound.
// Kernel 2 (router_topk): one workgroup per token; k rounds of a block argmax
//   with (score desc, index asc) order == torch.sort(stable=True) descending.
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

__global__ void __launch_bounds__(64 * kLogitWaves)
    router_logits_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const float* __restrict__ bias,
                         int64_t m, int64_t d, int64_t n_exp, uint16_t* __restrict__ logits) {
  const int lane = threadIdx.x & 63;
  const int64_t e = (int64_t)blockIdx.x * kLogitWaves + (threadIdx.x >> 6);
  const int64_t t0 = (int64_t)blockIdx.y * kTok;
  if (e >= n_exp) return;
  const int nt = (int)((m - t0) < kTok ? (m - t0) : kTok);
  double acc[kTok];
#pragma unroll
  for (int t = 0; t < kTok; ++t) acc[t] = 0.0;
  const uint16_t* wr = w + e * d;
  for (int64_t c = (int64_t)lane * 8; c < d; c += 512) {
    uint4 wv = *reinterpret_cast<const uint4*>(wr + c);
    double wd[8];
    uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      wd[2 * q] = (double)__uint_as_float(ww[q] << 16);
      wd[2 * q + 1] = (double)__uint_as_float(ww[q] & 0xffff0000u);
    }
#pragma unroll
    for (int t = 0; t < kTok; ++t) {
      if (t < nt) {
        uint4 xv = *reinterpret_cast<const uint4*>(x + (t0 + t) * d + c);
        uint32_t xx[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[t] = __fma_rn((double)__uint_as_float(xx[q] << 16), wd[2 * q], acc[t]);
          acc[t] = __fma_rn((double)__uint_as_float(xx[q] & 0xffff0000u), wd[2 * q + 1], acc[t]);
        }
      }
    }
  }
  float b = 0.0f;
  if (bias) b = bf16_bits_to_f32(f32_to_bf16_bits(bias[e]));
#pragma unroll
  for (int t = 0; t < kTok; ++t) {
    double s = wave_sum_f64(acc[t]);
    if (t < nt && lane == 0) {
      uint32_t l = f64_to_bf16_bits(s);
      if (bias) l = f32_to_bf16_bits(__fadd_rn(bf16_bits_to_f32(l), b));
      logits[(t0 + t) * n_exp + e] = (uint16_t)l;
    }
  }
}

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

__global__ void __launch_bounds__(256)
    router_topk_kernel(const uint16_t* __restrict__ logits, int64_t n_exp, int top_k, float scaling,
                       int64_t* __restrict__ idx_out, float* __restrict__ w_out) {
  __shared__ float s_score[1024];
  __shared__ uint64_t s_key[256];
  __shared__ int sel_idx[16];
  const int64_t t = blockIdx.x;
  const uint16_t* lr = logits + t * n_exp;
  for (int e = threadIdx.x; e < n_exp; e += blockDim.x) s_score[e] = sqrtf(softplus_f32(bf16_bits_to_f32(lr[e])));
  __syncthreads();
  for (int r = 0; r < top_k; ++r) {
    uint64_t best = 0;  // key 0 is below every real candidate
    for (int e = threadIdx.x; e < n_exp; e += blockDim.x) {
      bool taken = false;
      for (int q = 0; q < r; ++q) taken |= (sel_idx[q] == e);
      uint64_t k = taken ? 0 : score_key(s_score[e], e);
      best = k > best ? k : best;
    }
    s_key[threadIdx.x] = best;
    __syncthreads();
    for (int off = 128; off >= 1; off >>= 1) {
      if (threadIdx.x < off) {
        uint64_t o = s_key[threadIdx.x + off];
        if (o > s_key[threadIdx.x]) s_key[threadIdx.x] = o;
      }
      __syncthreads();
    }
    if (threadIdx.x == 0) sel_idx[r] = (int)(0xffffffffu - (uint32_t)(s_key[0] & 0xffffffffu));
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    float sum = 0.0f;
    for (int r = 0; r < top_k; ++r) sum = __fadd_rn(sum, s_score[sel_idx[r]]);
    sum = fmaxf(sum, 1e-20f);
    for (int r = 0; r < top_k; ++r) {
      idx_out[t * top_k + r] = sel_idx[r];
      w_out[t * top_k + r] = __fmul_rn(__fdiv_rn(s_score[sel_idx[r]], sum), scaling);
    }
  }
}

}  // namespace
}  // namespace hsmoe

using namespace hsmoe;

extern "C" size_t hsmoe_router_workspace_size(int64_t m, int64_t n_experts) {
  if (m < 0 || n_experts < 0) return 0;
  return (size_t)(((m * n_experts * 2) + 255) / 256 * 256);
}

extern "C" int hsmoe_router_topk(const void* x, const void* gate_w, const float* bias, int64_t m, int64_t d,
                                 int64_t n_experts, int top_k, float scaling, int64_t* idx_out, float* w_out,
                                 void* logits_out, void* workspace, size_t workspace_bytes, hsmoe_stream_t stream) {
  if (!x || !gate_w || !idx_out || !w_out || m < 0 || d <= 0 || n_experts <= 0)
    return fail(HSMOE_ERR_ARG, "hsmoe_router_topk: null pointer or bad size");
  if (n_experts > 1024 || top_k < 1 || top_k > 16 || top_k > n_experts)
    return fail(HSMOE_ERR_SHAPE, "hsmoe_router_topk: need 1 <= top_k <= min(16, n_experts) and n_experts <= 1024");
  if (d % 256 != 0 || !aligned(x, 16) || !aligned(gate_w, 16))
    return fail(HSMOE_ERR_SHAPE, "hsmoe_router_topk: d must be a multiple of 256 and x/gate_w 16-byte aligned");
  uint16_t* logits = (uint16_t*)logits_out;
  if (!logits) {
    if (!workspace || workspace_bytes < hsmoe_router_workspace_size(m, n_experts))
      return fail(HSMOE_ERR_WORKSPACE, "hsmoe_router_topk: workspace of %zu bytes needed",
                  hsmoe_router_workspace_size(m, n_experts));
    logits = (uint16_t*)workspace;
  }
  if (m == 0) return HSMOE_OK;
  dim3 g1((unsigned)((n_experts + kLogitWaves - 1) / kLogitWaves), (unsigned)((m + kTok - 1) / kTok));
  hipLaunchKernelGGL(router_logits_kernel, g1, dim3(64 * kLogitWaves), 0, (hipStream_t)stream, (const uint16_t*)x,
                     (const uint16_t*)gate_w, bias, m, d, n_experts, logits);
  int rc = check_launch("hsmoe_router_topk(logits)");
  if (rc) return rc;
  hipLaunchKernelGGL(router_topk_kernel, dim3((unsigned)m), dim3(256), 0, (hipStream_t)stream, logits, n_experts, top_k,
                     scaling, idx_out, w_out);
  return check_launch("hsmoe_router_topk(topk)");
}
