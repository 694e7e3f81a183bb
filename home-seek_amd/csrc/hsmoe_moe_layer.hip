// One MoE layer at decode (m <= 8 tokens) in a single persistent launch:
// router -> routed FP4 experts + FP8 shared expert -> fixed-order expert sum.
//
// Restates, for m <= 8, HomeSeekInferenceEngine._forward_ffn
// (engine.py:1410-1541): _compute_routing_experts / compute_expert_affinity_with_bias
// (engine.py:1025-1031, router.py:22-36), FusedMoEFFN.forward on the selected
// experts (fused_moe.py:447-563 over fused_expert_ffn_pt, fused_moe.py:383-395)
// and the SharedExpertFFN add (engine.py:1530-1536).  The arithmetic is that
// of hsmoe_router_topk followed by hsmoe_moe_decode (same tiles, same
// accumulation order), so the results are bit-identical to those two calls.
//
// Work items, in dependency order (item q only ever waits on items < q):
//   R    router rows: one expert row per item (its columns spread over the
//        workgroup's 256 threads), published as fp32 scores; the last R item
//        to finish also writes the routing outputs (top-k ids and weights)
//   SGU  shared-expert gate/up, 16 rows of W1 and W3 per item
//   SD   shared-expert down, 64 rows of W2 per item (ahead of the routed
//        items: its weights stream while the routing is still being decided)
//   GU   routed gate/up, (slot, 16 rows) per item; needs the slot plan
//   D    routed down, (slot, 64 rows) per item
// The last R item to finish builds the slot plan: top-k of every token from
// the scores, then the distinct valid expert ids ascending with their
// per-token weights.  It publishes the plan (expert id and weights per slot)
// in kFlagCopies copies and then the router flag; every other workgroup that
// runs a routed item (or the shared down) waits for the flag once per launch
// and copies its copy of the plan into LDS.  R items count their arrivals in
// groups of kRouterGroup (one counter per group, then one for the groups), so
// no counter takes more than 16 atomic increments.
// A down item issues its first W2 loads, then waits until every gate/up item
// of its slot has published the slot's activations, then stages them in LDS.
// The last down item of a row group adds the slots' partials in slot order
// (routed ascending, shared last) and writes the output rows.
// Workgroup b runs items b, b + G, b + 2G, ... with G no larger than the
// number of workgroups the GPU holds at once, so every item a workgroup waits
// for is held by a running workgroup.  Every wait is bounded; a wait that
// gives up records the waited-on control word in the workspace (sticky) and
// the workgroup carries on, so the launch always drains.
#include <mutex>

#include "hsmoe_common.h"
#include "hsmoe_internal.h"
#include "hsmoe_route.h"
#include "hsmoe_tiles.h"

namespace hsmoe {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxTok = 8;
constexpr int kMaxSlots = 128;  // m * top_k routed slots; slot kMaxSlots is never used as routed
constexpr int kMaxExperts = 256;
constexpr int kGuRows = 16;
constexpr int kDownRows = 16 * kWaves;
constexpr int kRtChunks = 8192 / 8 / kThreads;  // 16-byte gate-row chunks per thread (d <= 8192)
constexpr unsigned kSpinLimit = 1u << 16;
// Off: the launch faulted the GPU on MI355X (first with the parameters read
// through a null kernarg pointer in the item functions, then once more after
// that fix, cause not yet shown).  The entry point returns an error instead.
constexpr bool kLayerKernelEnabled = true;

// Control words (unsigned) at the start of the workspace.  Counters take the
// atomic increments; waiters never poll a counter.  The producer that
// completes a counter instead sets a flag, written in kFlagCopies copies 4 KiB
// apart (workgroup b polls copy b % kFlagCopies), so that polling spreads over
// several memory channels and never contends with the increments.
constexpr int kCtlRouter = 0;    // router items finished
constexpr int kCtlDone = 128;    // workgroups finished
constexpr int kCtlErr = 192;     // sticky: 1 + index of a control word whose wait gave up
constexpr int kCtlSlot = 256;    // + 16*s: gate/up items of slot s finished
constexpr int kCtlRowGroup = kCtlSlot + 16 * (kMaxSlots + 1);  // + g: down items of row group g finished
constexpr int kMaxRowGroups = 2048;
constexpr int kCtlRouterGrp = 4608;  // + 64*g: router items of group g finished
constexpr int kRouterGroup = 16;     // router items per group counter (at most 16 groups)
constexpr int kFlagCopies = 8;
constexpr int kFlagBase = 8192;      // word index of flag copy 0 (32 KiB)
constexpr int kFlagStride = 1024;    // words between copies (4 KiB)
constexpr int kFlagRouter = 0;       // + copy: the slot plan is published
constexpr int kFlagSlot = 16;        // + 4*s: every gate/up item of slot s finished
constexpr size_t kCtlBytes = 65536;
static_assert(kCtlRowGroup + kMaxRowGroups <= kCtlRouterGrp, "control block overflow");
static_assert(kCtlRouterGrp + 64 * (kMaxExperts / kRouterGroup) <= kFlagBase, "control block overflow");
// Published plan, one copy per flag copy: [0] slot count, [1 + s] expert id of
// slot s, [1 + S + s*m + t] weight of slot s for token t, [1 + S + S*m + 12s]
// the slot's table entry (6 pointers as 12 words) (S = m * top_k).
constexpr int kPlanStride = 4096;  // words between copies (16 KiB)
constexpr size_t kPlanBytes = (size_t)kFlagCopies * kPlanStride * 4;
static_assert(1 + kMaxSlots + kMaxSlots * kMaxTok + 12 * kMaxSlots <= kPlanStride, "plan copy overflow");
static_assert(kFlagSlot + 4 * (kMaxSlots + 1) <= kFlagStride, "flag block overflow");
static_assert((kFlagBase + kFlagCopies * kFlagStride) * 4 <= (int)kCtlBytes, "flag copies overflow");

struct LayerParams {
  const uint16_t* x;       // bf16 [m, d]
  const uint16_t* gate_w;  // bf16 [n_exp, d]
  const float* bias;       // [n_exp] or null
  const uint64_t* table;   // [n_exp][6]
  const uint64_t* shared;  // [6] or null
  int64_t n_exp;
  int m, d, i, top_k, scale_fmt, S;  // S = m * top_k routed slots
  float scaling, limit;
  int64_t* idx_out;    // [m, top_k]
  float* w_out;        // [m, top_k]
  uint16_t* logits;    // bf16 [m, n_exp] or null
  float* out_f32;      // [m, d] or null
  uint16_t* out_bf16;  // [m, d] or null
  unsigned* ctl;
  unsigned* plan;  // kFlagCopies published slot plans
  float* scores;  // [m][n_exp]
  float* act;   // fp32 [S + 1][m][i] weighted activations (slot S = shared)
  float* part;  // fp32 [S + 1][m][d] per-slot down partials
  int n_router, q_sgu, q_sd, q_gu, q_down, n_items;  // item ranges: R, SGU, SD, GU, D
};

// Waits (one thread) until this workgroup's copy of flag `flag` is set;
// polls with backoff.  Gives up after kSpinLimit polls, recording the flag.
__device__ bool wait_flag(unsigned* ctl, int flag) {
  const unsigned* f = ctl + kFlagBase + (int)(blockIdx.x % kFlagCopies) * kFlagStride + flag;
  int nap = 1;
  for (unsigned it = 0; it < kSpinLimit; ++it) {
    if (load_agent(f) != 0u) return true;
    if (nap == 1) __builtin_amdgcn_s_sleep(1);
    else if (nap == 2) __builtin_amdgcn_s_sleep(2);
    else if (nap == 4) __builtin_amdgcn_s_sleep(4);
    else if (nap == 8) __builtin_amdgcn_s_sleep(8);
    else __builtin_amdgcn_s_sleep(16);
    nap = nap < 16 ? 2 * nap : 16;
  }
  store_agent(ctl + kCtlErr, 1u + (unsigned)(kFlagBase + flag));
  return false;
}

// Sets every copy of flag `flag` (after the data it announces is complete).
__device__ __forceinline__ void set_flag(unsigned* ctl, int flag) {
  for (int c = 0; c < kFlagCopies; ++c) store_agent(ctl + kFlagBase + c * kFlagStride + flag, 1u);
}

struct Shared {
  uint64_t ent[kMaxSlots + 1][6];     // table entry of routed slot s (and of the shared expert at slot S)
  float red[kWaves][2][16 * kMaxTok];  // gate/up partials: [wave][gate|up][row * kMaxTok + token]
  double rpart[kWaves][kMaxTok];  // router: per-wave partial logit sums
  int64_t idx[kMaxSlots];  // top-k ids of every token
  float w[kMaxSlots];      // top-k weights of every token
  int eid[kMaxSlots];            // slot plan: expert id of routed slot s
  float wt[kMaxSlots][kMaxTok];  // slot plan: weight of routed slot s for token t
  float wt_item[kMaxTok];
  int flag;
  int n_routed;
  int have_plan;
  int wave_count[kWaves];
  unsigned char valid[kMaxExperts];  // expert e has a table entry (router items fill it)
  unsigned char used[kMaxExperts];   // expert e is selected by some token (plan build)
  short rank[kMaxExperts];           // slot of a selected expert (plan build)
};

// The slot plan of this launch in LDS, built by the last router item (every
// score is published): top-k of every token (one token per wave, ties to
// the lower index) and the distinct valid expert ids in ascending order with
// each token's weight for them (its top-k weights for that id, summed in k
// order; the union of _forward_legacy, fused_moe.py:466-476).
__device__ __forceinline__ void build_plan(const LayerParams& p, Shared& sh) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = p.m * p.top_k;
  // thread e holds expert e's table entry, loaded alongside the scores; the
  // selected ones go to sh.ent below (n_exp <= kThreads)
  uint64_t my_ent[6];
#pragma unroll
  for (int k = 0; k < 6; ++k)
    my_ent[k] = (int)threadIdx.x < p.n_exp ? ldg<uint64_t>(p.table + (int64_t)threadIdx.x * 6 + k) : 0ull;
  // (sh.valid was filled by this workgroup's router item)
  for (int e = threadIdx.x; e < p.n_exp; e += kThreads) sh.used[e] = 0;
  __syncthreads();
  // (n_exp <= kMaxExperts: at most 4 keys per lane)
  for (int t = wave; t < p.m; t += kWaves) {
    const float* sc = p.scores + (int64_t)t * p.n_exp;
    if (p.n_exp <= 64) wave_topk_n<1>(sc, p.n_exp, p.top_k, p.scaling, sh.idx + t * p.top_k, sh.w + t * p.top_k);
    else if (p.n_exp <= 128) wave_topk_n<2>(sc, p.n_exp, p.top_k, p.scaling, sh.idx + t * p.top_k, sh.w + t * p.top_k);
    else wave_topk_n<4>(sc, p.n_exp, p.top_k, p.scaling, sh.idx + t * p.top_k, sh.w + t * p.top_k);
  }
  __syncthreads();
  for (int j = threadIdx.x; j < n; j += kThreads) {
    const int64_t e = sh.idx[j];
    if (e >= 0 && e < p.n_exp && sh.valid[e]) sh.used[e] = 1;
  }
  __syncthreads();
  // slots = selected experts in ascending id order: ballot prefix ranks
  int base = 0;
  for (int e0 = 0; e0 < p.n_exp; e0 += kThreads) {
    const int e = e0 + threadIdx.x;
    const bool u = e < p.n_exp && sh.used[e];
    const uint64_t mask = __ballot(u);
    const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
    if (lane == 0) sh.wave_count[wave] = __popcll(mask);
    __syncthreads();
    int off = base;
    for (int w = 0; w < wave; ++w) off += sh.wave_count[w];
    if (u) {
      sh.rank[e] = (short)(off + below);
      sh.eid[off + below] = e;
      if (e0 == 0) {  // e == threadIdx.x: this thread holds the entry
#pragma unroll
        for (int k = 0; k < 6; ++k) sh.ent[off + below][k] = my_ent[k];
      }
    }
    for (int w = 0; w < kWaves; ++w) base += sh.wave_count[w];
    __syncthreads();
  }
  // each token's weight of each slot: its top-k weight for that expert (a
  // token's top-k ids are distinct, so at most one), else 0
  for (int c = threadIdx.x; c < base * p.m; c += kThreads) sh.wt[c / p.m][c % p.m] = 0.0f;
  __syncthreads();
  for (int j = threadIdx.x; j < n; j += kThreads) {
    const int64_t e = sh.idx[j];
    if (e >= 0 && e < p.n_exp && sh.valid[e]) sh.wt[sh.rank[e]][j / p.top_k] = __fadd_rn(0.0f, sh.w[j]);
  }
  if (threadIdx.x == 0) {
    sh.n_routed = base;
    sh.have_plan = 1;
  }
  __syncthreads();
}

// The routing outputs (and the zero output of a layer with no valid expert
// and no shared expert), written once by the last router item.
__device__ __forceinline__ void write_routing(const LayerParams& p, Shared& sh) {
  for (int j = threadIdx.x; j < p.m * p.top_k; j += kThreads) {
    p.idx_out[j] = sh.idx[j];
    p.w_out[j] = sh.w[j];
  }
  if (sh.n_routed == 0 && !p.shared) {
    // no down item will run, and the output is zero (_forward_legacy returns
    // zeros_like, fused_moe.py:473-474, 512-513)
    for (int c = threadIdx.x; c < p.m * p.d; c += kThreads) {
      if (p.out_f32) p.out_f32[c] = 0.0f;
      if (p.out_bf16) p.out_bf16[c] = 0;
    }
  }
}


// LDS of the layer kernel (file scope so the item functions below address it
// directly): x [m][d] or activations [2m][i] as bf16, and the block's scratch.
extern __shared__ __align__(16) uint16_t g_tile[];
__shared__ Shared g_sh;

// The streaming item functions are not inlined (each keeps its own register
// budget), so they read the launch parameters through the kernel's
// kernarg-segment address, which the kernel passes down: that builtin yields a
// valid address only in the kernel itself.  The router item is inlined: as a
// call it had to save a callee-saved register to scratch.
typedef const __attribute__((address_space(4))) LayerParams KernargParams;

__device__ __forceinline__ LayerParams params(uint64_t kernarg) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)kernarg);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(kernarg >> 32));
#if defined(__HIP_DEVICE_COMPILE__)
  return *(KernargParams*)(((uint64_t)hi << 32) | lo);
#else
  return LayerParams{};  // host pass: never called
#endif
}

// The slot plan in g_sh (a function of its own, called from the kernel's item
// loop, so its state adds to no streaming item's registers).  The last router
// item (publish) builds it, writes the routing outputs, publishes the plan
// copies and then sets the router flag; every other workgroup waits for the
// flag and copies the plan from copy blockIdx.x % kFlagCopies.
__device__ __noinline__ void plan_item(uint64_t kernarg, int publish) {
  const LayerParams p = params(kernarg);
  Shared& sh = g_sh;
  const int S = p.S, m = p.m, e0 = 1 + S + S * m, words = e0 + 12 * S;
  if (__builtin_amdgcn_readfirstlane(publish)) {
    build_plan(p, sh);
    for (int k = threadIdx.x; k < words; k += kThreads) {
      unsigned v;
      if (k == 0) v = (unsigned)sh.n_routed;
      else if (k <= S) v = (unsigned)sh.eid[k - 1];
      else if (k < e0) v = __float_as_uint(sh.wt[(k - 1 - S) / m][(k - 1 - S) % m]);
      else {
        const uint64_t ev = sh.ent[(k - e0) / 12][((k - e0) % 12) / 2];
        v = (k - e0) % 2 ? (unsigned)(ev >> 32) : (unsigned)ev;
      }
#pragma unroll
      for (int c = 0; c < kFlagCopies; ++c) store_agent(p.plan + c * kPlanStride + k, v);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) set_flag(p.ctl, kFlagRouter);
    write_routing(p, sh);  // read only after the launch
    return;
  }
  if (threadIdx.x == 0) wait_flag(p.ctl, kFlagRouter);
  __syncthreads();
  const unsigned* src = p.plan + (int)(blockIdx.x % kFlagCopies) * kPlanStride;
  for (int k = threadIdx.x; k < words; k += kThreads) {
    const unsigned v = load_agent(src + k);
    if (k == 0) sh.n_routed = (int)v;
    else if (k <= S) sh.eid[k - 1] = (int)v;
    else if (k < e0) sh.wt[(k - 1 - S) / m][(k - 1 - S) % m] = __uint_as_float(v);
    else reinterpret_cast<unsigned*>(sh.ent[(k - e0) / 12])[(k - e0) % 12] = v;
  }
  if (threadIdx.x == 0) sh.have_plan = 1;
  __syncthreads();
}

// Copies x into the LDS tile unless it is already there (state: 1 = x in LDS).
__device__ __forceinline__ void ensure_x(const LayerParams& p, int& state) {
  if (state == 1) return;
  const int n16 = p.m * p.d / 8;
  const uint4* src = reinterpret_cast<const uint4*>(p.x);
  for (int q0 = threadIdx.x; q0 < n16; q0 += 8 * kThreads) {
    uint4 v[8];  // every load of the pass in flight before the first LDS store
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = q0 + j * kThreads < n16 ? src[q0 + j * kThreads] : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (q0 + j * kThreads < n16) reinterpret_cast<uint4*>(g_tile)[q0 + j * kThreads] = v[j];
  }
  __syncthreads();
  state = 1;
}

// Router row e = q: thread t owns the row's 16-byte chunks t, t + 256, ...;
// per token it adds its exact products in fp64 (chunk then element order),
// the wave sums by a fixed butterfly and the 4 wave sums are added in wave
// order.  Every addition is of fp64 values holding exact bf16 products, so
// for the rows met in practice the sum is exact and equals the column-order
// sum; it is rounded to bf16 once.
__device__ __forceinline__ int router_item(uint64_t kernarg, int q_arg, int state_arg) {
  const int q = __builtin_amdgcn_readfirstlane(q_arg);
  int state = __builtin_amdgcn_readfirstlane(state_arg);
  const LayerParams p = params(kernarg);
  Shared& sh = g_sh;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t e = q;
  const int nch = p.d / 8;
  const uint4* wrow = reinterpret_cast<const uint4*>(p.gate_w + e * p.d);
  uint4 wv[kRtChunks];
#pragma unroll
  for (int j = 0; j < kRtChunks; ++j) {
    const int c = threadIdx.x + kThreads * j;
    wv[j] = c < nch ? ldg<uint4>(wrow + c) : make_uint4(0, 0, 0, 0);
  }
  // which experts the table holds (used if this item turns out to be the last)
  const bool has_entry = threadIdx.x < p.n_exp && ldg<uint64_t>(p.table + (int64_t)threadIdx.x * 6) != 0;
  ensure_x(p, state);
#pragma unroll 1
  for (int t = 0; t < p.m; ++t) {
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < kRtChunks; ++j) {
      const int c = threadIdx.x + kThreads * j;
      if (c < nch) acc = dot8_f64(reinterpret_cast<const uint4*>(g_tile + t * p.d)[c], wv[j], acc);
    }
    acc = wave_sum_f64(acc);
    if (lane == 0) sh.rpart[wave][t] = acc;
  }
  __syncthreads();
  if (threadIdx.x < p.n_exp) sh.valid[threadIdx.x] = has_entry;
  if (threadIdx.x < p.m) {
    const int t = threadIdx.x;
    double sum = sh.rpart[0][t];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) sum += sh.rpart[w][t];
    const float score = router_score(sum, p.bias, e, p.logits ? p.logits + t * p.n_exp + e : nullptr);
    store_agent(p.scores + t * p.n_exp + e, score);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int g = q / kRouterGroup;
    const int n_groups = (p.n_router + kRouterGroup - 1) / kRouterGroup;
    const int in_group = p.n_router - g * kRouterGroup < kRouterGroup ? p.n_router - g * kRouterGroup : kRouterGroup;
    bool last = add_agent(p.ctl + kCtlRouterGrp + 64 * g, 1u) == (unsigned)(in_group - 1);
    if (last) last = add_agent(p.ctl + kCtlRouter, 1u) == (unsigned)(n_groups - 1);
    sh.flag = last;
  }
  __syncthreads();
  return state;
}

__device__ __noinline__ int gate_up_item(uint64_t kernarg, int q_arg, int state_arg) {
  const int q = __builtin_amdgcn_readfirstlane(q_arg);
  int state = __builtin_amdgcn_readfirstlane(state_arg);
  const LayerParams p = params(kernarg);
  Shared& sh = g_sh;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int gu_per_slot = p.i / kGuRows;
  const bool is_shared = q < p.q_sd;
  const int qq = is_shared ? q - p.q_sgu : q - p.q_gu;
  const int s = is_shared ? p.S : qq / gu_per_slot;
  const int r0 = (qq % gu_per_slot) * kGuRows;
  if (!is_shared && s >= sh.n_routed) return state;
  if (threadIdx.x < p.m) sh.wt_item[threadIdx.x] = is_shared ? 1.0f : sh.wt[s][threadIdx.x];
  const uint64_t* ent = sh.ent[s];
  ensure_x(p, state);
  const int per = (p.d / 128) / kWaves;
  const int st0 = wave * per;
  f32x4 ag = {0, 0, 0, 0}, au = {0, 0, 0, 0};
  gate_up_slot(slot_format(p.scale_fmt, ent, is_shared), ent, g_tile, p.m, p.d, p.i, r0, st0, st0 + per, ag, au);
  if ((lane & 15) < kMaxTok) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int row = 4 * (lane >> 4) + c, col = lane & 15;
      sh.red[wave][0][row * kMaxTok + col] = ag[c];
      sh.red[wave][1][row * kMaxTok + col] = au[c];
    }
  }
  __syncthreads();
  const int row = threadIdx.x >> 4, col = threadIdx.x & 15;
  if (col < p.m) {
    float gsum = 0.0f, usum = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      gsum = __fadd_rn(gsum, sh.red[w][0][row * kMaxTok + col]);
      usum = __fadd_rn(usum, sh.red[w][1][row * kMaxTok + col]);
    }
    const float a = __fmul_rn(sh.wt_item[col], swiglu(gsum, usum, p.limit));
    store_agent(p.act + ((int64_t)s * p.m + col) * p.i + r0 + row, a);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0 && add_agent(p.ctl + kCtlSlot + 16 * s, 1u) == (unsigned)(gu_per_slot - 1))
    set_flag(p.ctl, kFlagSlot + 4 * s);
  return state;
}

// A run of routed gate/up items q, q + G, q + 2G, ... (G = grid) whose slots
// are in format F with whole batches (d / 512 a multiple of the batch): as
// soon as a wave has multiplied its last batch of item q it issues the first
// batch of item q + G into the same registers, so the cross-wave reduction,
// the publish and the wait for the stores of item q overlap the loads of the
// next item.  The slot arrival of item q is counted after its stores are
// complete; its result (is this the slot's last arrival?) is read one item
// later, when the loads of the next item have returned anyway, and for the
// run's last item at the end.  Same tiles and accumulation order as
// gate_up_item, so the results are identical.  Returns the last item run.
template <int F>
__device__ __noinline__ int gate_up_run(uint64_t kernarg, int q_arg, int state_arg) {
  constexpr int kB = gate_up_batch<F>();
  int q = __builtin_amdgcn_readfirstlane(q_arg);
  int state = __builtin_amdgcn_readfirstlane(state_arg);
  const LayerParams p = params(kernarg);
  Shared& sh = g_sh;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int G = (int)gridDim.x, gu_per_slot = p.i / kGuRows;
  const int per = (p.d / 128) / kWaves, nb = per / kB, st0 = wave * per;
  ensure_x(p, state);
  int s = (q - p.q_gu) / gu_per_slot, r0 = ((q - p.q_gu) % gu_per_slot) * kGuRows;
  Mat w1 = make_mat<F>(sh.ent[s][0], sh.ent[s][1], p.i, p.d), w3 = make_mat<F>(sh.ent[s][2], sh.ent[s][3], p.i, p.d);
  Batch<F, kB> b1, b3;
  b1.load(w1, r0 + r, p.d, st0, g);
  b3.load(w3, r0 + r, p.d, st0, g);
  unsigned pend = 0;  // thread 0: counter value before the previous item's arrival
  int pend_s = -1;
  for (;;) {
    if (threadIdx.x < p.m) sh.wt_item[threadIdx.x] = sh.wt[s][threadIdx.x];
    f32x4 ag = {0, 0, 0, 0}, au = {0, 0, 0, 0};
    for (int bt = 0; bt < nb; ++bt) {
      const int st = st0 + bt * kB;
#pragma unroll
      for (int b = 0; b < kB; ++b)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bf16x8 xf = lds_frag(g_tile, p.d, r, g, st + b, j, p.m);
          ag = mfma16x16x32(b1.frag(b, j, g), xf, ag);
          au = mfma16x16x32(b3.frag(b, j, g), xf, au);
        }
      if (bt + 1 < nb) {
        b1.load(w1, r0 + r, p.d, st + kB, g);
        b3.load(w3, r0 + r, p.d, st + kB, g);
      }
    }
    // the next item of this workgroup, if it continues the run
    const int q2 = q + G;
    const int s2 = (q2 - p.q_gu) / gu_per_slot, r02 = ((q2 - p.q_gu) % gu_per_slot) * kGuRows;
    const bool next = q2 < p.q_down && s2 < sh.n_routed && slot_format(p.scale_fmt, sh.ent[s2], false) == F;
    if (next) {
      w1 = make_mat<F>(sh.ent[s2][0], sh.ent[s2][1], p.i, p.d);
      w3 = make_mat<F>(sh.ent[s2][2], sh.ent[s2][3], p.i, p.d);
      b1.load(w1, r02 + r, p.d, st0, g);
      b3.load(w3, r02 + r, p.d, st0, g);
    }
    // epilogue of item q (as gate_up_item)
    if ((lane & 15) < kMaxTok) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int row = 4 * g + c, col = lane & 15;
        sh.red[wave][0][row * kMaxTok + col] = ag[c];
        sh.red[wave][1][row * kMaxTok + col] = au[c];
      }
    }
    __syncthreads();
    {
      const int row = threadIdx.x >> 4, col = threadIdx.x & 15;
      if (col < p.m) {
        float gsum = 0.0f, usum = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          gsum = __fadd_rn(gsum, sh.red[w][0][row * kMaxTok + col]);
          usum = __fadd_rn(usum, sh.red[w][1][row * kMaxTok + col]);
        }
        const float a = __fmul_rn(sh.wt_item[col], swiglu(gsum, usum, p.limit));
        store_agent(p.act + ((int64_t)s * p.m + col) * p.i + r0 + row, a);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);  // the stores of item q (and the next item's loads)
    __syncthreads();
    if (threadIdx.x == 0) {
      if (pend_s >= 0 && pend == (unsigned)(gu_per_slot - 1)) set_flag(p.ctl, kFlagSlot + 4 * pend_s);
      pend = add_agent(p.ctl + kCtlSlot + 16 * s, 1u);
      pend_s = s;
    }
    if (!next) break;
    q = q2;
    s = s2;
    r0 = r02;
  }
  if (threadIdx.x == 0 && pend == (unsigned)(gu_per_slot - 1)) set_flag(p.ctl, kFlagSlot + 4 * pend_s);
  return q;
}

// Slot and row group of down item q (shared down items first).
__device__ __forceinline__ void down_slot_of(const LayerParams& p, int q, bool& is_shared, int& s, int& g) {
  const int down_per_slot = p.d / kDownRows;
  is_shared = q < p.q_gu;
  const int qq = is_shared ? q - p.q_sd : q - p.q_down;
  s = is_shared ? p.S : qq / down_per_slot;
  g = qq % down_per_slot;
}

// Down item q, first part: W2 rows of the slot against its activations, the
// slot's fp32 partial sums written for the row group.  Needs the slot plan
// for a routed slot only (the shared slot runs before the plan exists).
__device__ __noinline__ int down_item(uint64_t kernarg, int q_arg, int state_arg) {
  const int q = __builtin_amdgcn_readfirstlane(q_arg);
  int state = __builtin_amdgcn_readfirstlane(state_arg);
  const LayerParams p = params(kernarg);
  Shared& sh = g_sh;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  bool is_shared;
  int s, g;
  down_slot_of(p, q, is_shared, s, g);
  if (!is_shared && s >= sh.n_routed) return state;
  const uint64_t* ent = sh.ent[s];
  const int r0 = g * kDownRows + 16 * wave;
  const int m = p.m, i = p.i;
  unsigned* const ctl = p.ctl;
  const float* const src = p.act + (int64_t)s * m * i;
  f32x4 acc = {0, 0, 0, 0};
  down_slot(slot_format(p.scale_fmt, ent, is_shared), ent, g_tile, m, i, p.d, r0, acc, [&]() __attribute__((always_inline)) {
    if (threadIdx.x == 0) wait_flag(ctl, kFlagSlot + 4 * s);
    __syncthreads();
    // fp32 activations -> bf16 hi rows [t][k] and lo rows [m + t][k]
    // (8 loads in flight per thread before any is used)
    const int n = m * i;
    for (int c0 = threadIdx.x; c0 < n; c0 += 8 * kThreads) {
      float a[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) a[j] = (c0 + j * kThreads < n) ? load_agent(src + c0 + j * kThreads) : 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int c = c0 + j * kThreads;
        if (c < n) {
          const uint32_t hi = f32_to_bf16_bits(a[j]);
          const uint32_t lo = f32_to_bf16_bits(__fadd_rn(a[j], -bf16_bits_to_f32(hi)));
          g_tile[c] = (uint16_t)hi;
          g_tile[n + c] = (uint16_t)lo;
        }
      }
    }
    __syncthreads();
  });
  state = 0;
  // lane (col = lane%16) holds rows 4*(lane/16)+c; column t (hi) + column m+t (lo)
  // of token t are combined through the lane that owns column t.
  float* part = p.part + (int64_t)s * m * p.d;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int col = lane & 15;
    const float lo = __shfl(acc[c], (lane & 48) | ((col + m) & 15), 64);
    if (col < m) store_agent(part + (int64_t)col * p.d + r0 + 4 * (lane >> 4) + c, __fadd_rn(acc[c], lo));
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  return state;
}

// Down item q, second part (the slot plan exists): arrival on the row group;
// the last slot to arrive adds the slots' partials in slot order (routed
// ascending, shared last) and writes the output rows.
__device__ __noinline__ void down_finish(uint64_t kernarg, int q_arg) {
  const int q = __builtin_amdgcn_readfirstlane(q_arg);
  const LayerParams p = params(kernarg);
  Shared& sh = g_sh;
  bool is_shared;
  int s, g;
  down_slot_of(p, q, is_shared, s, g);
  const int n_routed = sh.n_routed;
  if (!is_shared && s >= n_routed) return;
  const int m = p.m;
  const int n_slots = n_routed + (p.shared ? 1 : 0);
  if (threadIdx.x == 0) sh.flag = add_agent(p.ctl + kCtlRowGroup + g, 1u) == (unsigned)(n_slots - 1);
  __syncthreads();
  if (sh.flag) {
    for (int c = threadIdx.x; c < kDownRows * m; c += kThreads) {
      const int t = c / kDownRows, dd = g * kDownRows + (c - t * kDownRows);
      const float v = sum_slots_agent(p.part + (int64_t)t * p.d + dd, (int64_t)m * p.d, n_routed,
                                      p.shared ? p.part + ((int64_t)p.S * m + t) * p.d + dd : nullptr);
      const int64_t o = (int64_t)t * p.d + dd;
      if (p.out_f32) p.out_f32[o] = v;
      if (p.out_bf16) p.out_bf16[o] = (uint16_t)f32_to_bf16_bits(v);
    }
  }
}

__global__ void __launch_bounds__(kThreads) moe_layer_kernel(LayerParams p) {
  int state = 0;  // 1 while the LDS tile holds x
  if (threadIdx.x == 0) g_sh.have_plan = 0;
  if (p.shared && threadIdx.x < 6) g_sh.ent[p.S][threadIdx.x] = ldg<uint64_t>(p.shared + threadIdx.x);
  const uint64_t kernarg = (uint64_t)__builtin_amdgcn_kernarg_segment_ptr();  // &p
  const int n_items = p.n_items, q_sgu = p.q_sgu, q_sd = p.q_sd, q_gu = p.q_gu, q_down = p.q_down;
  for (int q = blockIdx.x; q < n_items; q += gridDim.x) {
    __syncthreads();  // the previous item's readers of the LDS scratch are done
    if (q < q_sgu) {
      state = router_item(kernarg, q, state);
      if (g_sh.flag) plan_item(kernarg, 1);  // the last router item
      continue;
    }
    if (q < q_sd) {  // shared gate/up
      state = gate_up_item(kernarg, q, state);
      continue;
    }
    if (q < q_gu) {  // shared down: the plan is needed only for its arrival
      state = down_item(kernarg, q, state);
      if (!g_sh.have_plan) plan_item(kernarg, 0);
      down_finish(kernarg, q);
      continue;
    }
    if (!g_sh.have_plan) plan_item(kernarg, 0);  // routed items need the slot plan
    if (q < q_down) {
      const int s = (q - q_gu) / (p.i / kGuRows);
      const int fmt = s < g_sh.n_routed ? slot_format(p.scale_fmt, g_sh.ent[s], false) : -1;
      const bool whole = ((p.d / 128) / kWaves) % gate_up_batch<kFp4E8M0>() == 0;
      if (fmt == kFp4E8M0 && whole) {
        q = gate_up_run<kFp4E8M0>(kernarg, q, state);
        state = 1;
      } else if (fmt == kFp4F32 && whole) {
        q = gate_up_run<kFp4F32>(kernarg, q, state);
        state = 1;
      } else {
        state = gate_up_item(kernarg, q, state);
      }
    } else {
      state = down_item(kernarg, q, state);
      down_finish(kernarg, q);
    }
  }
  // the last workgroup to finish re-arms every control word for the next call
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) g_sh.flag = add_agent(p.ctl + kCtlDone, 1u) == gridDim.x - 1;
  __syncthreads();
  if (!g_sh.flag) return;
  if (threadIdx.x == 0) {
    store_agent(p.ctl + kCtlRouter, 0u);
    store_agent(p.ctl + kCtlDone, 0u);
  }
  for (int s = threadIdx.x; s <= p.S; s += kThreads) store_agent(p.ctl + kCtlSlot + 16 * s, 0u);
  for (int g = threadIdx.x; g < p.d / kDownRows; g += kThreads) store_agent(p.ctl + kCtlRowGroup + g, 0u);
  for (int g = threadIdx.x; g < kMaxExperts / kRouterGroup; g += kThreads) store_agent(p.ctl + kCtlRouterGrp + 64 * g, 0u);
  for (int c = threadIdx.x; c < kFlagCopies * (p.S + 2); c += kThreads) {
    const int copy = c % kFlagCopies, f = c / kFlagCopies;  // f = 0: plan, f = 1 + s: slot s
    store_agent(p.ctl + kFlagBase + copy * kFlagStride + (f == 0 ? kFlagRouter : kFlagSlot + 4 * (f - 1)), 0u);
  }
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }
size_t scores_bytes(int64_t m, int64_t n_exp) { return align256((size_t)(m * n_exp * 4)); }
size_t act_bytes(int64_t m, int64_t i, int top_k) { return align256((size_t)(m * top_k + 1) * m * i * 4); }
size_t part_bytes(int64_t m, int64_t d, int top_k) { return align256((size_t)(m * top_k + 1) * m * d * 4); }

// Workgroups of moe_layer_kernel the device holds at once, for an LDS size.
int resident_workgroups(size_t lds, int* out) {
  static std::mutex mu;
  static int cache_dev = -1, cache_cus = 0;
  static size_t cache_lds[8] = {};
  static int cache_nb[8] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(HSMOE_ERR_LAUNCH, "hsmoe_moe_layer_decode: hipGetDevice failed");
  std::lock_guard<std::mutex> lock(mu);
  if (dev != cache_dev) {
    if (hipDeviceGetAttribute(&cache_cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return fail(HSMOE_ERR_LAUNCH, "hsmoe_moe_layer_decode: CU count query failed");
    cache_dev = dev;
    for (auto& c : cache_lds) c = 0;
  }
  for (int k = 0; k < 8; ++k)
    if (cache_lds[k] == lds + 1) {
      *out = cache_nb[k] * cache_cus;
      return HSMOE_OK;
    }
  int nb = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, moe_layer_kernel, kThreads, lds) != hipSuccess || nb < 1)
    return fail(HSMOE_ERR_LAUNCH, "hsmoe_moe_layer_decode: occupancy query failed (%d workgroups/CU)", nb);
  for (int k = 0; k < 8; ++k)
    if (cache_lds[k] == 0) {
      cache_lds[k] = lds + 1;
      cache_nb[k] = nb;
      break;
    }
  *out = nb * cache_cus;
  return HSMOE_OK;
}

}  // namespace
}  // namespace hsmoe

using namespace hsmoe;

extern "C" size_t hsmoe_moe_layer_workspace_size(int64_t m, int64_t d, int64_t i, int64_t n_experts, int top_k) {
  if (m < 1 || d < 1 || i < 1 || n_experts < 1 || top_k < 1) return 0;
  return kCtlBytes + kPlanBytes + scores_bytes(m, n_experts) + act_bytes(m, i, top_k) + part_bytes(m, d, top_k);
}

extern "C" int hsmoe_moe_layer_decode(const void* x, int64_t m, int64_t d, int64_t i, const void* gate_w,
                                      const float* gate_bias, int64_t n_experts, int top_k, float routed_scaling,
                                      const uint64_t* expert_table, int scale_kind, const uint64_t* shared,
                                      float swiglu_limit, int64_t* topk_idx_out, float* topk_w_out,
                                      void* logits_out, float* out_f32, void* out_bf16, void* workspace,
                                      size_t workspace_bytes, hsmoe_stream_t stream) {
  const char* name = "hsmoe_moe_layer_decode";
  if (!kLayerKernelEnabled)
    return fail(HSMOE_ERR_LAUNCH,
                "%s: disabled -- this persistent kernel faulted the GPU on its first runs and stays off until the "
                "cause is shown; use hsmoe_router_topk + hsmoe_moe_decode", name);
  if (!x || !gate_w || !expert_table || !topk_idx_out || !topk_w_out || (!out_f32 && !out_bf16))
    return fail(HSMOE_ERR_ARG, "%s: null pointer or no output", name);
  if (scale_kind != HSMOE_SCALE_E8M0 && scale_kind != HSMOE_SCALE_F32)
    return fail(HSMOE_ERR_ARG, "%s: unknown scale_kind %d", name, scale_kind);
  if (m < 1 || m > kMaxTok || n_experts < 1 || n_experts > kMaxExperts || top_k < 1 || top_k > 16 ||
      top_k > n_experts || m * top_k > kMaxSlots)
    return fail(HSMOE_ERR_SHAPE, "%s: need 1 <= m <= 8, n_experts <= 256, 1 <= top_k <= min(16, n_experts)", name);
  if (d % 512 != 0 || i % 512 != 0 || d <= 0 || i <= 0 || d > 8192 || d / kDownRows > kMaxRowGroups)
    return fail(HSMOE_ERR_SHAPE, "%s: d and i must be positive multiples of 512, d <= 8192 (d=%lld i=%lld)", name,
                (long long)d, (long long)i);
  if (!expert_fits(d, i))
    return fail(HSMOE_ERR_SHAPE, "%s: d*i too large (an expert matrix must stay below 4 GiB)", name);
  if (!aligned(x, 16) || !aligned(gate_w, 16)) return fail(HSMOE_ERR_SHAPE, "%s: x and gate_w must be 16-byte aligned", name);
  const size_t need = hsmoe_moe_layer_workspace_size(m, d, i, n_experts, top_k);
  if (!workspace || workspace_bytes < need || !aligned(workspace, 256))
    return fail(HSMOE_ERR_WORKSPACE, "%s: zero-filled workspace of %zu bytes (256-byte aligned) needed", name, need);
  const size_t lds = (size_t)(m * d > 2 * m * i ? m * d : 2 * m * i) * 2;
  if (lds > 65536) return fail(HSMOE_ERR_SHAPE, "%s: m*d and 2*m*i tiles must fit in 64 KiB of LDS", name);

  LayerParams p;
  p.x = (const uint16_t*)x;
  p.gate_w = (const uint16_t*)gate_w;
  p.bias = gate_bias;
  p.table = expert_table;
  p.shared = shared;
  p.n_exp = n_experts;
  p.m = (int)m;
  p.d = (int)d;
  p.i = (int)i;
  p.top_k = top_k;
  p.scale_fmt = scale_kind == HSMOE_SCALE_E8M0 ? kFp4E8M0 : kFp4F32;
  p.S = (int)(m * top_k);
  p.scaling = routed_scaling;
  p.limit = swiglu_limit;
  p.idx_out = topk_idx_out;
  p.w_out = topk_w_out;
  p.logits = (uint16_t*)logits_out;
  p.out_f32 = out_f32;
  p.out_bf16 = (uint16_t*)out_bf16;
  char* ws = (char*)workspace;
  p.ctl = (unsigned*)ws;
  ws += kCtlBytes;
  p.plan = (unsigned*)ws;
  ws += kPlanBytes;
  p.scores = (float*)ws;
  ws += scores_bytes(m, n_experts);
  p.act = (float*)ws;
  ws += act_bytes(m, i, top_k);
  p.part = (float*)ws;
  const int has_shared = shared ? 1 : 0;
  p.n_router = (int)n_experts;
  p.q_sgu = p.n_router;
  p.q_sd = p.q_sgu + has_shared * (int)(i / kGuRows);
  p.q_gu = p.q_sd + has_shared * (int)(d / kDownRows);
  p.q_down = p.q_gu + p.S * (int)(i / kGuRows);
  p.n_items = p.q_down + p.S * (int)(d / kDownRows);
  int resident = 0;
  int rc = resident_workgroups(lds, &resident);
  if (rc) return rc;
  const int grid = resident < p.n_items ? resident : p.n_items;
  hipLaunchKernelGGL(moe_layer_kernel, dim3((unsigned)grid), dim3(kThreads), lds, (hipStream_t)stream, p);
  return check_launch(name);
}

extern "C" size_t hsmoe_moe_layer_status_offset(void) { return (size_t)kCtlErr * 4; }
