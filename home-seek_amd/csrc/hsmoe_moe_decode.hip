// Fused routed-expert SwiGLU FFN for m <= 8 tokens (decode M=1, MTP verify T=3).
//
// Restates, for the selected experts only, FusedMoEFFN._forward_legacy /
// _fused_moe_forward_m1_fp4 (fused_moe.py:458-551, 1147-1227) on top of
// fused_expert_ffn_pt (fused_moe.py:383-395), plus the shared expert add of
// _forward_ffn (engine.py:1530-1536):
//   gate = x W1^T, up = x W3^T                    fp32 accumulation
//   act  = min(gate,L) * sigmoid(min(gate,L)) * clamp(up,-L,L)
//   out  = sum_e w_e * act_e W2e^T  (+ shared FFN with weight 1)
// W = bf16(dequant(FP4)) exactly as hsmoe_fp4_dequant_bf16, decoded in
// registers (never written to memory).  Intermediates stay fp32; the weighted
// activation enters the down GEMM as a bf16 hi + lo pair (a = hi + lo + O(2^-17 a)),
// which the 16-column MFMA absorbs for free when m <= 8.
//
// Launch structure (both HBM-bound; see the DESIGN notes in the repo):
//   phase 1  grid (i/16, slots)  4 waves: wave w streams 16 rows x d/4 columns
//            of W1 and W3 of one expert; the 4 partials meet in LDS in fixed
//            order; SwiGLU, routing weight and the hi/lo split happen there.
//   phase 2  grid (d/16)  16 waves: wave w streams units (slot, 512 columns)
//            w, w+16, ... of W2 for 16 output rows; fixed-order LDS reduction.
// "Slots" are the distinct selected experts in ascending id order (the union
// of _forward_legacy, fused_moe.py:466-476) followed by the shared expert.
// Every workgroup derives the slot plan itself from topk_idx, so no host sync
// and no extra launch is needed.
#include <math.h>

#include "hsmoe_common.h"
#include "hsmoe_internal.h"
#include "hsmoe_tiles.h"

namespace hsmoe {
namespace {

constexpr int kMaxTok = 8;
constexpr int kMaxCand = 128;  // m * top_k
constexpr int kP1Waves = 4;
constexpr int kP2Waves = 4;

struct DecodeParams {
  const uint16_t* x;      // bf16 [m, d]
  const int64_t* idx;     // [m, top_k]
  const float* wts;       // [m, top_k]
  const uint64_t* table;  // [n_experts][6]
  const uint64_t* shared; // [6] or null
  uint16_t* act;          // bf16 [slots][2m][i]
  float* part;            // fp32 [slots][m][d] per-slot partial outputs
  unsigned* counters;     // [d / 64] arrival counters (zero between calls)
  float* out_f32;         // [m, d] or null
  uint16_t* out_bf16;     // [m, d] or null
  int64_t n_experts;
  int m, d, i, top_k;
  int scale_fmt;  // kFp4E8M0 or kFp4F32 for routed FP4 experts
  float limit;
};

struct Plan {
  int n_routed;
  int eid[kMaxCand];
};

// Distinct valid expert ids of topk_idx in ascending order (every thread of
// the block participates; ends with a barrier).
__device__ void build_plan(const DecodeParams& p, Plan& plan, int* s_cand, int* s_first) {
  const int n = p.m * p.top_k;
  for (int j = threadIdx.x; j < n; j += blockDim.x) {
    int64_t e = p.idx[j];
    bool ok = e >= 0 && e < p.n_experts && p.table[e * 6] != 0;
    s_cand[j] = ok ? (int)e : -1;
  }
  if (threadIdx.x == 0) plan.n_routed = 0;
  __syncthreads();
  for (int j = threadIdx.x; j < n; j += blockDim.x) {
    int e = s_cand[j];
    bool first = e >= 0;
    for (int q = 0; q < j && first; ++q) first = s_cand[q] != e;
    s_first[j] = first;
  }
  __syncthreads();
  for (int j = threadIdx.x; j < n; j += blockDim.x) {
    if (s_first[j]) {
      int e = s_cand[j], rank = 0;
      for (int q = 0; q < n; ++q) rank += (s_first[q] && s_cand[q] < e);
      plan.eid[rank] = e;
      atomicAdd(&plan.n_routed, 1);
    }
  }
  __syncthreads();
}

__global__ void __launch_bounds__(64 * kP1Waves) moe_gate_up_kernel(DecodeParams p) {
  extern __shared__ __align__(16) uint16_t xs[];  // [m][d] bf16
  __shared__ Plan plan;
  __shared__ int s_cand[kMaxCand];
  __shared__ int s_first[kMaxCand];
  __shared__ float s_wt[kMaxTok];
  __shared__ float red[kP1Waves][2][256];
  build_plan(p, plan, s_cand, s_first);
  const int n_slots = plan.n_routed + (p.shared ? 1 : 0);
  const int s = blockIdx.y;
  if (s >= n_slots) return;
  const bool is_shared = s == plan.n_routed;
  const uint64_t* ent = is_shared ? p.shared : p.table + (int64_t)plan.eid[s] * 6;
  const int r0 = blockIdx.x * 16;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // x -> LDS (16 bytes per thread per pass)
  const int n16 = p.m * p.d / 8;
  for (int q = threadIdx.x; q < n16; q += blockDim.x)
    reinterpret_cast<uint4*>(xs)[q] = reinterpret_cast<const uint4*>(p.x)[q];
  if (threadIdx.x < p.m) {
    float w = 0.0f;
    if (is_shared) {
      w = 1.0f;
    } else {
      const int e = plan.eid[s];
      for (int k = 0; k < p.top_k; ++k)
        if (p.idx[threadIdx.x * p.top_k + k] == e) w = __fadd_rn(w, p.wts[threadIdx.x * p.top_k + k]);
    }
    s_wt[threadIdx.x] = w;
  }
  __syncthreads();
  const int per = (p.d / 128) / kP1Waves;
  const int st0 = wave * per, st1 = st0 + per;
  f32x4 ag = {0, 0, 0, 0}, au = {0, 0, 0, 0};
  gate_up_slot(slot_format(p.scale_fmt, ent, is_shared), ent, xs, p.m, p.d, p.i, r0, st0, st1, ag, au);
  // D[4*(lane/16) + q][lane%16] lives in element q of lane
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = 4 * (lane >> 4) + q, col = lane & 15;
    red[wave][0][row * 16 + col] = ag[q];
    red[wave][1][row * 16 + col] = au[q];
  }
  __syncthreads();
  const int row = threadIdx.x >> 4, col = threadIdx.x & 15;
  if (col < p.m) {
    float gsum = 0.0f, usum = 0.0f;
#pragma unroll
    for (int w = 0; w < kP1Waves; ++w) {
      gsum = __fadd_rn(gsum, red[w][0][threadIdx.x]);
      usum = __fadd_rn(usum, red[w][1][threadIdx.x]);
    }
    const float act = swiglu(gsum, usum, p.limit);
    const float a = __fmul_rn(s_wt[col], act);
    const uint32_t hi = f32_to_bf16_bits(a);
    const uint32_t lo = f32_to_bf16_bits(__fadd_rn(a, -bf16_bits_to_f32(hi)));
    const int64_t base = ((int64_t)s * 2 * p.m) * p.i + r0 + row;
    p.act[base + (int64_t)col * p.i] = (uint16_t)hi;
    p.act[base + (int64_t)(p.m + col) * p.i] = (uint16_t)lo;
  }
}

// ---------------------------------------------------------------- phase 2
// Block (row group rg of 64 output rows, slot s): the slot's activation tile
// act[s] ([2m][i] bf16: hi then lo columns) is staged in LDS; wave w streams
// rows rg*64 + 16w .. +16 of W2 over all i/128 steps and writes the fp32
// partial sum of its rows for this slot.  The last block of a row group to
// finish (atomic arrival count) adds the slots' partials in slot order and
// writes the output, then re-arms the counter: deterministic, and nothing
// ever waits on another block.
__global__ void __launch_bounds__(64 * kP2Waves) moe_down_kernel(DecodeParams p) {
  extern __shared__ __align__(16) uint16_t as[];  // [2m][i] bf16
  __shared__ Plan plan;
  __shared__ int s_cand[kMaxCand];
  __shared__ int s_first[kMaxCand];
  __shared__ int s_last;
  build_plan(p, plan, s_cand, s_first);
  const int n_slots = plan.n_routed + (p.shared ? 1 : 0);
  const int s = blockIdx.y;
  if (n_slots == 0) {
    // no valid expert and no shared expert: the output is zero
    // (_forward_legacy returns zeros_like, fused_moe.py:473-474, 512-513)
    if (s == 0) {
      const int rows = 16 * kP2Waves;
      for (int q = threadIdx.x; q < rows * p.m; q += blockDim.x) {
        const int t = q / rows;
        const int64_t o = (int64_t)t * p.d + blockIdx.x * rows + (q - t * rows);
        if (p.out_f32) p.out_f32[o] = 0.0f;
        if (p.out_bf16) p.out_bf16[o] = 0;
      }
    }
    return;
  }
  if (s >= n_slots) return;  // not counted: the arrival target is n_slots
  const bool is_shared = s == plan.n_routed;
  const uint64_t* ent = is_shared ? p.shared : p.table + (int64_t)plan.eid[s] * 6;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r0 = blockIdx.x * (16 * kP2Waves) + 16 * wave;
  const int n16 = 2 * p.m * p.i / 8;
  const uint4* src = reinterpret_cast<const uint4*>(p.act + (int64_t)s * 2 * p.m * p.i);
  f32x4 acc = {0, 0, 0, 0};
  // the W2 rows do not depend on the activations: their first batch is in
  // flight while the tile is staged
  auto stage = [&]() {
    for (int q = threadIdx.x; q < n16; q += blockDim.x) reinterpret_cast<uint4*>(as)[q] = src[q];
    __syncthreads();
  };
  const int fmt = slot_format(p.scale_fmt, ent, is_shared);
  if (is_shared) {  // the shared expert's two step ranges, added
    const int half = shared_down_half(p.i);
    f32x4 acc1 = {0, 0, 0, 0};
    down_slot(fmt, ent, as, p.m, p.i, p.d, r0, 0, half, acc, stage);
    down_slot(fmt, ent, as, p.m, p.i, p.d, r0, half, p.i / 128, acc1, []() {});
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = __fadd_rn(acc[c], acc1[c]);
  } else {
    down_slot(fmt, ent, as, p.m, p.i, p.d, r0, acc, stage);
  }
  // lane (col = lane%16) holds rows 4*(lane/16)+q; column t (hi) + column m+t (lo)
  // of token t are combined through the lane that owns column t.
  // Cross-block handoff without cache flushes: partials are written with
  // agent-scope (L2-bypassing, sc1) stores, each wave waits for its stores to
  // complete before the barrier, and only then is the arrival counter bumped;
  // the last block reads the partials with agent-scope loads.
  float* part = p.part + (int64_t)s * p.m * p.d;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int col = lane & 15;
    const float lo = __shfl(acc[q], (lane & 48) | ((col + p.m) & 15), 64);
    if (col < p.m)
      __hip_atomic_store(part + (int64_t)col * p.d + r0 + 4 * (lane >> 4) + q, __fadd_rn(acc[q], lo), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(&p.counters[blockIdx.x], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             (unsigned)(n_slots - 1);
  __syncthreads();
  if (!s_last) return;
  const int rows = 16 * kP2Waves;
  for (int q = threadIdx.x; q < rows * p.m; q += blockDim.x) {
    const int t = q / rows, d = blockIdx.x * rows + (q - t * rows);
    const float v = sum_slots_agent(p.part + (int64_t)t * p.d + d, (int64_t)p.m * p.d, n_slots, nullptr);
    const int64_t o = (int64_t)t * p.d + d;
    if (p.out_f32) p.out_f32[o] = v;
    if (p.out_bf16) p.out_bf16[o] = (uint16_t)f32_to_bf16_bits(v);
  }
  if (threadIdx.x == 0) __hip_atomic_store(&p.counters[blockIdx.x], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }
// Workspace layout: [arrival counters, fixed 4 KiB at offset 0 | act | part].
// The counters sit at the same place for every shape and every call leaves
// them at zero, so calls of different shapes can share one workspace.
constexpr size_t kCounterBytes = 4096;  // d / 64 <= 1024 counters
size_t act_bytes(int64_t m, int64_t i, int top_k) { return align256((size_t)(m * top_k + 1) * 2 * m * i * 2); }
size_t part_bytes(int64_t m, int64_t d, int top_k) { return align256((size_t)(m * top_k + 1) * m * d * 4); }

}  // namespace
}  // namespace hsmoe

using namespace hsmoe;

extern "C" size_t hsmoe_moe_decode_workspace_size(int64_t m, int64_t d, int64_t i, int top_k) {
  if (m < 1 || i < 1 || d < 1 || top_k < 1) return 0;
  return kCounterBytes + act_bytes(m, i, top_k) + part_bytes(m, d, top_k);
}

static int moe_decode_launch(const void* x, int64_t m, int64_t d, int64_t i, const int64_t* topk_idx,
                             const float* topk_w, int top_k, const uint64_t* expert_table, int64_t n_experts,
                             int scale_kind, const uint64_t* shared, float swiglu_limit, float* out_f32,
                             void* out_bf16, void* workspace, size_t workspace_bytes, hsmoe_stream_t stream,
                             int stages, const char* name) {
  if (!x || !topk_idx || !topk_w || !expert_table || n_experts < 1 || ((stages & 2) && !out_f32 && !out_bf16))
    return fail(HSMOE_ERR_ARG, "%s: null pointer or no output", name);
  if (scale_kind != HSMOE_SCALE_E8M0 && scale_kind != HSMOE_SCALE_F32)
    return fail(HSMOE_ERR_ARG, "%s: unknown scale_kind %d", name, scale_kind);
  if (m < 1 || m > kMaxTok || top_k < 1 || top_k > 16 || m * top_k > kMaxCand)
    return fail(HSMOE_ERR_SHAPE, "%s: need 1 <= m <= 8 and 1 <= top_k <= 16 (got m=%lld top_k=%d)", name,
                (long long)m, top_k);
  if (d % 512 != 0 || i % 512 != 0 || d <= 0 || i <= 0 || (size_t)(d / 64) * 4 > kCounterBytes)
    return fail(HSMOE_ERR_SHAPE, "%s: d and i must be positive multiples of 512, d <= 65536 (d=%lld i=%lld)", name,
                (long long)d, (long long)i);
  if (!expert_fits(d, i))
    return fail(HSMOE_ERR_SHAPE, "%s: d*i too large (an expert matrix must stay below 4 GiB)", name);
  if (!aligned(x, 16)) return fail(HSMOE_ERR_SHAPE, "%s: x must be 16-byte aligned", name);
  const size_t need = hsmoe_moe_decode_workspace_size(m, d, i, top_k);
  if (!workspace || workspace_bytes < need || !aligned(workspace, 256))
    return fail(HSMOE_ERR_WORKSPACE, "%s: zero-filled workspace of %zu bytes (256-byte aligned) needed", name, need);
  if (m * d * 2 > 65536 || 2 * m * i * 2 > 65536)
    return fail(HSMOE_ERR_SHAPE, "%s: m*d and 2*m*i tiles must fit in 64 KiB of LDS", name);
  DecodeParams p;
  p.x = (const uint16_t*)x;
  p.idx = topk_idx;
  p.wts = topk_w;
  p.table = expert_table;
  p.shared = shared;
  p.counters = (unsigned*)workspace;
  p.act = (uint16_t*)((char*)workspace + kCounterBytes);
  p.part = (float*)((char*)workspace + kCounterBytes + act_bytes(m, i, top_k));
  p.out_f32 = out_f32;
  p.out_bf16 = (uint16_t*)out_bf16;
  p.n_experts = n_experts;
  p.m = (int)m;
  p.d = (int)d;
  p.i = (int)i;
  p.top_k = top_k;
  p.limit = swiglu_limit;
  p.scale_fmt = scale_kind == HSMOE_SCALE_E8M0 ? 0 : 1;
  const unsigned max_slots = (unsigned)(m * top_k + (shared ? 1 : 0));
  hipStream_t st = (hipStream_t)stream;
  if (stages & 1) {
    hipLaunchKernelGGL(moe_gate_up_kernel, dim3((unsigned)(i / 16), max_slots), dim3(64 * kP1Waves),
                       (size_t)(m * d * 2), st, p);
    int rc = check_launch(name);
    if (rc) return rc;
  }
  if (stages & 2) {
    hipLaunchKernelGGL(moe_down_kernel, dim3((unsigned)(d / (16 * kP2Waves)), max_slots), dim3(64 * kP2Waves),
                       (size_t)(2 * m * i * 2), st, p);
    return check_launch(name);
  }
  return HSMOE_OK;
}

extern "C" int hsmoe_moe_decode(const void* x, int64_t m, int64_t d, int64_t i, const int64_t* topk_idx,
                                const float* topk_w, int top_k, const uint64_t* expert_table, int64_t n_experts,
                                int scale_kind, const uint64_t* shared, float swiglu_limit, float* out_f32,
                                void* out_bf16, void* workspace, size_t workspace_bytes, hsmoe_stream_t stream) {
  return moe_decode_launch(x, m, d, i, topk_idx, topk_w, top_k, expert_table, n_experts, scale_kind, shared,
                           swiglu_limit, out_f32, out_bf16, workspace, workspace_bytes, stream, 3,
                           "hsmoe_moe_decode");
}

extern "C" int hsmoe_moe_gate_up(const void* x, int64_t m, int64_t d, int64_t i, const int64_t* topk_idx,
                                 const float* topk_w, int top_k, const uint64_t* expert_table, int64_t n_experts,
                                 int scale_kind, const uint64_t* shared, float swiglu_limit, void* workspace,
                                 size_t workspace_bytes, hsmoe_stream_t stream) {
  return moe_decode_launch(x, m, d, i, topk_idx, topk_w, top_k, expert_table, n_experts, scale_kind, shared,
                           swiglu_limit, nullptr, nullptr, workspace, workspace_bytes, stream, 1,
                           "hsmoe_moe_gate_up");
}

extern "C" int hsmoe_moe_down(const void* x, int64_t m, int64_t d, int64_t i, const int64_t* topk_idx,
                              const float* topk_w, int top_k, const uint64_t* expert_table, int64_t n_experts,
                              int scale_kind, const uint64_t* shared, float* out_f32, void* out_bf16,
                              void* workspace, size_t workspace_bytes, hsmoe_stream_t stream) {
  return moe_decode_launch(x, m, d, i, topk_idx, topk_w, top_k, expert_table, n_experts, scale_kind, shared, 0.0f,
                           out_f32, out_bf16, workspace, workspace_bytes, stream, 2, "hsmoe_moe_down");
}
