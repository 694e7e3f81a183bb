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

namespace hsmoe {
namespace {

constexpr int kMaxTok = 8;
constexpr int kMaxCand = 128;  // m * top_k
constexpr int kP1Waves = 4;
constexpr int kP2Waves = 16;

struct DecodeParams {
  const uint16_t* x;      // bf16 [m, d]
  const int64_t* idx;     // [m, top_k]
  const float* wts;       // [m, top_k]
  const uint64_t* table;  // [n_experts][6]
  const uint64_t* shared; // [6] or null
  uint16_t* act;          // bf16 [slots][2m][i]
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

// ---------------------------------------------------------------- weights
// Weight formats of a slot.  Routed experts are FP4 with the call's scale
// encoding, or bf16 when the table entry has no scale pointer; the shared
// expert is e4m3 with fp32 128x128 block scales, or bf16 likewise.
enum Fmt : int { kFp4E8M0 = 0, kFp4F32 = 1, kFp8Block = 2, kBf16 = 3 };

// One 128-column step of one matrix row as seen by lane (r, g): the columns
// 128*st + 32g .. +32 of row `row` (a K-column matrix).  MFMA j of the step
// uses columns +8j .. +8j+7, so the 4 lanes of a row cover 128 contiguous
// columns per step.
template <int F>
struct Raw;
template <>
struct Raw<kFp4E8M0> { uint4 a; uint32_t e; };
template <>
struct Raw<kFp4F32> { uint4 a; float s; };
template <>
struct Raw<kFp8Block> { uint4 a, b; float s; };
template <>
struct Raw<kBf16> { uint4 a, b, c, d; };

template <int F>
__device__ __forceinline__ Raw<F> load_step(const uint64_t w, const uint64_t sc, int64_t row, int64_t k, int64_t st,
                                            int g) {
  Raw<F> r;
  if constexpr (F == kFp4E8M0 || F == kFp4F32) {
    r.a = *reinterpret_cast<const uint4*>((const uint8_t*)w + row * (k / 2) + st * 64 + g * 16);
    const int64_t si = row * (k / 32) + st * 4 + g;
    if constexpr (F == kFp4E8M0)
      r.e = ((const uint8_t*)sc)[si];
    else
      r.s = ((const float*)sc)[si];
  } else if constexpr (F == kFp8Block) {
    const uint8_t* b = (const uint8_t*)w + row * k + st * 128 + g * 32;
    r.a = *reinterpret_cast<const uint4*>(b);
    r.b = *reinterpret_cast<const uint4*>(b + 16);
    r.s = ((const float*)sc)[(row / 128) * (k / 128) + st];
  } else {
    const uint4* b = reinterpret_cast<const uint4*>((const uint16_t*)w + row * k + st * 128 + g * 32);
    r.a = b[0];
    r.b = b[1];
    r.c = b[2];
    r.d = b[3];
  }
  return r;
}

template <int F>
__device__ __forceinline__ bf16x8 frag(const Raw<F>& r, int j) {
  if constexpr (F == kFp4E8M0 || F == kFp4F32) {
    const uint32_t dw = j == 0 ? r.a.x : j == 1 ? r.a.y : j == 2 ? r.a.z : r.a.w;
    if constexpr (F == kFp4E8M0)
      return fp4x8_to_bf16_e8m0(dw, e8m0_as_f32(r.e));
    else
      return fp4x8_to_bf16_f32(dw, r.s);
  } else if constexpr (F == kFp8Block) {
    const uint4& q = j < 2 ? r.a : r.b;
    const uint32_t d0 = (j & 1) ? q.z : q.x, d1 = (j & 1) ? q.w : q.y;
    bf16x8 f;
    fp8x4_to_bf16(d0, r.s, f, 0);
    fp8x4_to_bf16(d1, r.s, f, 1);
    return f;
  } else {
    const uint4& q = j == 0 ? r.a : j == 1 ? r.b : j == 2 ? r.c : r.d;
    return __builtin_bit_cast(bf16x8, q);
  }
}

template <int F>
constexpr int batch_steps() {
  return (F == kFp4E8M0 || F == kFp4F32) ? 4 : 2;
}

// ---------------------------------------------------------------- phase 1
// Streams rows r0..r0+15 of W1 and W3 over steps [st0, st1).  The B operand
// lane (c = token, g) holds x[c][128*st + 32g + 8j ..], matching frag().
template <int F>
__device__ __forceinline__ void gate_up(const DecodeParams& p, const uint64_t* ent, int r0, int st0, int st1,
                                        f32x4& ag, f32x4& au) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4, c = lane & 15;
  const int64_t row = r0 + r;
  const uint16_t* xr = p.x + (int64_t)c * p.d + g * 32;
  const bool xon = c < p.m;
  constexpr int kB = batch_steps<F>();
  for (int st = st0; st < st1; st += kB) {
    Raw<F> a1[kB], a3[kB];
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      if (st + b < st1) {
        a1[b] = load_step<F>(ent[0], ent[1], row, p.d, st + b, g);
        a3[b] = load_step<F>(ent[2], ent[3], row, p.d, st + b, g);
      }
    }
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      if (st + b < st1) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          bf16x8 xf = {};
          if (xon) xf = *reinterpret_cast<const bf16x8*>(xr + (int64_t)(st + b) * 128 + 8 * j);
          ag = mfma16x16x32(frag<F>(a1[b], j), xf, ag);
          au = mfma16x16x32(frag<F>(a3[b], j), xf, au);
        }
      }
    }
  }
}

__device__ __forceinline__ int slot_format(const DecodeParams& p, const uint64_t* ent, bool is_shared) {
  if (is_shared) return ent[1] ? kFp8Block : kBf16;
  return ent[1] ? p.scale_fmt : kBf16;
}

__global__ void __launch_bounds__(64 * kP1Waves) moe_gate_up_kernel(DecodeParams p) {
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
  const int per = (p.d / 128) / kP1Waves;
  const int st0 = wave * per, st1 = st0 + per;
  f32x4 ag = {0, 0, 0, 0}, au = {0, 0, 0, 0};
  switch (slot_format(p, ent, is_shared)) {
    case kFp4E8M0: gate_up<kFp4E8M0>(p, ent, r0, st0, st1, ag, au); break;
    case kFp4F32: gate_up<kFp4F32>(p, ent, r0, st0, st1, ag, au); break;
    case kFp8Block: gate_up<kFp8Block>(p, ent, r0, st0, st1, ag, au); break;
    default: gate_up<kBf16>(p, ent, r0, st0, st1, ag, au); break;
  }
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
    const float L = p.limit;
    const float gc = gsum > L ? L : gsum;                          // clamp(max=L), NaN passes
    const float uc = usum < -L ? -L : (usum > L ? L : usum);       // clamp(-L, L)
    const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-gc)));  // torch sigmoid
    const float act = __fmul_rn(__fmul_rn(gc, sig), uc);
    const float a = __fmul_rn(s_wt[col], act);
    const uint32_t hi = f32_to_bf16_bits(a);
    const uint32_t lo = f32_to_bf16_bits(__fadd_rn(a, -bf16_bits_to_f32(hi)));
    const int64_t base = ((int64_t)s * 2 * p.m) * p.i + r0 + row;
    p.act[base + (int64_t)col * p.i] = (uint16_t)hi;
    p.act[base + (int64_t)(p.m + col) * p.i] = (uint16_t)lo;
  }
}

// ---------------------------------------------------------------- phase 2
// Unit = (slot s, 512 columns from k0) of 16 rows of W2; the B operand lane
// (c, g) holds act[s][c][k0 + 128st + 32g + 8j ..] (c < m: hi, m <= c < 2m: lo).
template <int F>
__device__ __forceinline__ void down_unit(const DecodeParams& p, const uint64_t* ent, int s, int r0, int k0,
                                          f32x4& acc) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4, c = lane & 15;
  const int64_t row = r0 + r;
  const bool bon = c < 2 * p.m;
  const uint16_t* ar = p.act + ((int64_t)s * 2 * p.m + c) * p.i + k0 + g * 32;
  constexpr int kB = batch_steps<F>();
  const int st0 = k0 / 128;
#pragma unroll
  for (int sb = 0; sb < 4; sb += kB) {
    Raw<F> a[kB];
#pragma unroll
    for (int b = 0; b < kB; ++b) a[b] = load_step<F>(ent[4], ent[5], row, p.i, st0 + sb + b, g);
#pragma unroll
    for (int b = 0; b < kB; ++b) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bf16x8 bf = {};
        if (bon) bf = *reinterpret_cast<const bf16x8*>(ar + (sb + b) * 128 + 8 * j);
        acc = mfma16x16x32(frag<F>(a[b], j), bf, acc);
      }
    }
  }
}

__global__ void __launch_bounds__(64 * kP2Waves) moe_down_kernel(DecodeParams p) {
  __shared__ Plan plan;
  __shared__ int s_cand[kMaxCand];
  __shared__ int s_first[kMaxCand];
  __shared__ float red[kP2Waves][256];
  __shared__ float tot[256];
  build_plan(p, plan, s_cand, s_first);
  const int n_slots = plan.n_routed + (p.shared ? 1 : 0);
  const int r0 = blockIdx.x * 16;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int ups = p.i / 512;
  const int n_units = n_slots * ups;
  f32x4 acc = {0, 0, 0, 0};
  for (int u = wave; u < n_units; u += kP2Waves) {
    const int s = u / ups, k0 = (u - s * ups) * 512;
    const bool is_shared = s == plan.n_routed;
    const uint64_t* ent = is_shared ? p.shared : p.table + (int64_t)plan.eid[s] * 6;
    switch (slot_format(p, ent, is_shared)) {
      case kFp4E8M0: down_unit<kFp4E8M0>(p, ent, s, r0, k0, acc); break;
      case kFp4F32: down_unit<kFp4F32>(p, ent, s, r0, k0, acc); break;
      case kFp8Block: down_unit<kFp8Block>(p, ent, s, r0, k0, acc); break;
      default: down_unit<kBf16>(p, ent, s, r0, k0, acc); break;
    }
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) red[wave][(4 * (lane >> 4) + q) * 16 + (lane & 15)] = acc[q];
  __syncthreads();
  if (threadIdx.x < 256) {
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < kP2Waves; ++w) v = __fadd_rn(v, red[w][threadIdx.x]);
    tot[threadIdx.x] = v;
  }
  __syncthreads();
  if (threadIdx.x < 256) {
    const int row = threadIdx.x >> 4, t = threadIdx.x & 15;
    if (t < p.m) {
      const float v = __fadd_rn(tot[row * 16 + t], tot[row * 16 + p.m + t]);
      const int64_t o = (int64_t)t * p.d + r0 + row;
      if (p.out_f32) p.out_f32[o] = v;
      if (p.out_bf16) p.out_bf16[o] = (uint16_t)f32_to_bf16_bits(v);
    }
  }
}

size_t act_bytes(int64_t m, int64_t i, int top_k) { return (size_t)(m * top_k + 1) * 2 * m * i * 2; }

}  // namespace
}  // namespace hsmoe

using namespace hsmoe;

extern "C" size_t hsmoe_moe_decode_workspace_size(int64_t m, int64_t d, int64_t i, int top_k) {
  (void)d;
  if (m < 1 || i < 1 || top_k < 1) return 0;
  return (act_bytes(m, i, top_k) + 255) / 256 * 256;
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
  if (d % 512 != 0 || i % 512 != 0 || d <= 0 || i <= 0)
    return fail(HSMOE_ERR_SHAPE, "%s: d and i must be positive multiples of 512 (d=%lld i=%lld)", name,
                (long long)d, (long long)i);
  if (!aligned(x, 16)) return fail(HSMOE_ERR_SHAPE, "%s: x must be 16-byte aligned", name);
  const size_t need = hsmoe_moe_decode_workspace_size(m, d, i, top_k);
  if (!workspace || workspace_bytes < need || !aligned(workspace, 16))
    return fail(HSMOE_ERR_WORKSPACE, "%s: workspace of %zu bytes (16-byte aligned) needed", name, need);
  DecodeParams p;
  p.x = (const uint16_t*)x;
  p.idx = topk_idx;
  p.wts = topk_w;
  p.table = expert_table;
  p.shared = shared;
  p.act = (uint16_t*)workspace;
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
    hipLaunchKernelGGL(moe_gate_up_kernel, dim3((unsigned)(i / 16), max_slots), dim3(64 * kP1Waves), 0, st, p);
    int rc = check_launch(name);
    if (rc) return rc;
  }
  if (stages & 2) {
    hipLaunchKernelGGL(moe_down_kernel, dim3((unsigned)(d / 16)), dim3(64 * kP2Waves), 0, st, p);
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
