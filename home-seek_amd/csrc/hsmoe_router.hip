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
#include "hsmoe_route.h"

namespace hsmoe {
namespace {

constexpr int kTok = kRouterTok;
constexpr int kLogitWaves = 4;  // expert rows per logits workgroup
constexpr size_t kCounterBytes = 4096;

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
  const int wave = threadIdx.x >> 6;
  const int64_t e = (int64_t)blockIdx.x * kLogitWaves + wave;
  const int64_t t0 = (int64_t)blockIdx.y * kTok;
  const int nt = (int)((m - t0) < kTok ? (m - t0) : kTok);
  // the gate rows do not depend on x: issue their loads before staging x
  uint4 wv[kMaxChunks];
  if (e < n_exp) load_gate_row(w, e, d, wv);
  for (int64_t q = threadIdx.x; q < nt * d / 8; q += blockDim.x)
    reinterpret_cast<uint4*>(xs)[q] = reinterpret_cast<const uint4*>(x + t0 * d)[q];
  __syncthreads();
  if (e < n_exp)
    router_row(wv, xs, nt, d, e, n_exp, bias, logits_out ? logits_out + t0 * n_exp + e : nullptr,
               stage + t0 * n_exp + e);
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
