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
//        workgroup's 256 threads), published as fp32 scores tagged with the
//        launch's tag, in kScoreCopies copies
//   SGU  shared-expert gate or up: 16 rows of W1 or of W3 per item, the rows'
//        fp32 sums published for the shared down
//   SD   shared-expert down, 32 rows of W2 per item, each over both halves of
//        the steps (two waves per half: an FP8 row is twice an FP4 one, so
//        an item streams what a routed down item does)
//   GU   routed gate/up, (slot, 16 rows) per item; needs the slot plan
//   D    routed down, (slot, 64 rows) per item
// Every workgroup that runs a routed item (or the shared down) builds the slot
// plan itself, once per launch: each wave polls one token's tagged scores (in
// copy blockIdx.x % kScoreCopies) until every one carries this launch's tag --
// no counters and no store acknowledgements on the way -- and takes that
// token's top-k from registers; then the distinct valid expert ids ascending
// become the slots, with their per-token weights and table entries.  The last
// workgroup of the grid also writes the routing outputs.  The launch's tag is
// the workspace's epoch word plus one; the last workgroup to finish stores it
// back, so consecutive launches never share a tag and nothing tagged needs
// clearing.
// A down item issues its first W2 loads, then waits until every gate/up item
// of its slot has published the slot's activations, then stages them in LDS.
// The last down item of a row group adds the slots' partials in slot order
// (routed ascending, shared last) and writes the output rows.
// With a norm tail (the _norm entry points) m more items come last, one per
// token row: the next layer's residual adds and RMSNorm of this layer's
// output, from the rows the row-group sums also publish as tagged words
// (see tail_item).
// Workgroup b runs items b, b + G, b + 2G, ... with G no larger than the
// number of workgroups the GPU holds at once, so every item a workgroup waits
// for is held by a running workgroup.  Every wait is bounded; a wait that
// gives up records the waited-on control word in the workspace (sticky) and
// the workgroup carries on, so the launch always drains.
#include <mutex>

#include "hsmoe_common.h"
#include "hsmoe_internal.h"
#include "hsmoe_norm.h"
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
static_assert(kMaxExperts == kThreads && kMaxExperts == 4 * 64, "plan build: one expert per thread, four per lane");

// Control words (unsigned) at the start of the workspace.  Every handoff
// between items is a tagged word (tag << 32 | fp32 bits, see read_launch_tag),
// polled until it carries this launch's tag; the only counter counts the
// workgroups that finished, so that the last one can advance the epoch.
constexpr int kCtlEpoch = 0;     // tag of the previous launch (0: none yet)
constexpr int kCtlDone = 128;    // workgroups finished
constexpr int kCtlErr = 192;     // sticky: 1 + the code of a wait that gave up:
constexpr int kWaitScores = 4608;  //   a plan's wait for the router scores
constexpr int kWaitAct = 4609;     //   a down item's wait for its slot's activations
constexpr int kWaitShared = 4610;  //   the shared down's wait for the shared activations
constexpr int kWaitPart = 4611;    //   a row group's wait for the slots' partials
constexpr int kWaitGate = 4612;    //   a shared up item's wait for its rows' gate sums
constexpr int kWaitTail = 4613;    //   a tail item's wait for its output row
constexpr int kMaxRowGroups = 2048;
constexpr size_t kCtlBytes = 4096;
// Once a launch's tag reaches kRearmTag its last workgroup zeroes the tagged
// words and restarts the epoch at 0, so tags never wrap onto words that old
// launches left in the workspace.
constexpr unsigned kRearmTag = 1u << 31;
// Router scores: kScoreCopies copies of [m][n_exp] tagged words, each copy
// 4 KiB aligned, so that the workgroups polling them spread over many memory
// channels.
constexpr int kScoreCopies = 16;

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
  uint64_t* scores;     // kScoreCopies copies of [m][n_exp] tagged fp32 scores
  int score_stride;     // 64-bit words between copies
  uint64_t* act;   // tagged [S][m][i] weighted activations of the routed slots
  uint64_t* sgh;   // tagged [2][m][i] shared expert gate row sums (0) and activations (1)
  uint64_t* part;  // tagged [S + 1][m][d] per-slot down partials (slot S: shared)
  uint64_t* fin;   // tagged [m][d] output rows for the tail items, or null (no tail)
  uint4* wipe;      // the workspace after the control words, zeroed at a re-arm
  int64_t wipe_n;   //   (16-byte units)
  unsigned* status_out;  // or null: receives this launch's status, the sticky word is cleared
  // given routing (no router items) when route_idx is set: token t's ids are
  // route_idx[route_tok[t]][:] (a token table of route_rows rows) or, without
  // route_tok, route_idx[t][:]; its weights route_w[t][:] or all route_wconst
  const int64_t* route_idx;
  const int64_t* route_tok;
  const float* route_w;
  float route_wconst;
  int64_t route_rows;
  // norm tail (tail_w set): h_out = bf16(bf16(h + bf16(out)) + res), norm_out = RMSNorm(h_out) * w
  const uint16_t* tail_h;    // bf16 [m, d]
  const uint16_t* tail_res;  // bf16 [d] or null
  const uint16_t* tail_w;    // bf16 [d] or null: no tail
  uint16_t* tail_h_out;      // bf16 [m, d] (may be tail_h)
  uint16_t* tail_out;        // bf16 [m, d]
  float tail_eps;
  // item ranges [start, end): R is [0, n_router); the others follow in an
  // order where every item's producers come before it
  int n_router, sgu0, sgu1, sd0, sd1, gu0, gu1, d0, d1, n_main, n_items;  // tail items: [n_main, n_items)
  // routed down items in pairs (drun = 2; else 1): in each block of 2 * dgrid
  // items, dk slots whose row groups a workgroup takes two at a time, so
  // that its second item reuses the staged activations of its first
  int drun, dgrid, dk;
};

// This launch's tag: the previous launch's plus one (never 0).  The epoch word
// changes only after every workgroup of the launch has finished its items.
// Read once per workgroup, at its start, into the workgroup's LDS (g_sh.tag):
// every wave of every item reading the one epoch word with agent-scope loads
// queued thousands of same-address reads at the coherence point.
__device__ __forceinline__ unsigned read_launch_tag(const unsigned* ctl) {
  const unsigned ep = load_agent(ctl + kCtlEpoch);
  return ep == 0xffffffffu ? 1u : ep + 1u;
}
__device__ __forceinline__ uint64_t tagged(unsigned tag, unsigned v) { return ((uint64_t)tag << 32) | v; }

// Reads the tagged words ubase[j * jstride + off] (j < min(cnt, kN); ubase
// and jstride the same in every lane, off the lane's own) into v once each
// carries `tag`: every load of a round in flight at once, a lane re-reading
// only the words it has not yet seen.  Gives up after kSpinLimit rounds,
// recording `code` (the values it has not seen stay 0).
template <int kN>
__device__ __forceinline__ void poll_tagged(const uint64_t* ubase, int64_t jstride, uint32_t off, int cnt,
                                            unsigned tag, float (&v)[kN], unsigned* ctl, int code) {
  unsigned need = 0;
#pragma unroll
  for (int j = 0; j < kN; ++j) {
    v[j] = 0.0f;
    if (j < cnt) need |= 1u << j;
  }
  for (unsigned it = 0; it < kSpinLimit; ++it) {
    const unsigned cur = need;
    uint64_t w[kN];
#pragma unroll
    for (int j = 0; j < kN; ++j) w[j] = (cur >> j) & 1u ? load_agent(ubase + (int64_t)j * jstride + off) : 0ull;
#pragma unroll
    for (int j = 0; j < kN; ++j)
      if (((cur >> j) & 1u) && (unsigned)(w[j] >> 32) == tag) {
        v[j] = __uint_as_float((unsigned)w[j]);
        need &= ~(1u << j);
      }
    if (__ballot(need != 0) == 0) return;
    __builtin_amdgcn_s_sleep(2);
  }
  if (need) store_agent(ctl + kCtlErr, 1u + (unsigned)code);
}

struct Shared {
  uint64_t ent[kMaxSlots + 1][6];     // table entry of routed slot s (and of the shared expert at slot S)
  float red[kWaves][2][16 * kMaxTok];  // gate/up partials: [wave][gate|up][row * kMaxTok + token]
  double rpart[kWaves][kMaxTok];  // router: per-wave partial logit sums
  float rscore[kMaxTok];          // router: the row's score per token
  int64_t idx[kMaxSlots];  // top-k ids of every token
  float w[kMaxSlots];      // top-k weights of every token
  int eid[kMaxSlots];            // slot plan: expert id of routed slot s
  float wt[kMaxSlots][kMaxTok];  // slot plan: weight of routed slot s for token t
  float wt_item[kMaxTok];
  unsigned tag;  // this launch's tag (read_launch_tag, once per workgroup)
  int flag;
  int n_routed;
  int have_plan;
  int last;  // this workgroup is the last of the launch to finish
  alignas(4) unsigned char valid[kMaxExperts];  // expert e has a table entry (plan build)
  alignas(4) unsigned char used[kMaxExperts];   // expert e is selected by some token (plan build)
  short rank[kMaxExperts];                      // slot of a selected expert (plan build)
};
static_assert(sizeof(Shared::red) >= 2 * 64 * 4 * sizeof(float), "shared down: two waves' accumulators");

// The router part of the slot plan: wave w takes the top-k of tokens w,
// w + kWaves (ties to the lower index) from the tokens' tagged scores, polled
// with agent-scope loads until all carry this launch's tag.
__device__ __forceinline__ void build_plan_scores(const LayerParams& p, Shared& sh, const uint64_t (&my_ent)[6]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // wave w holds tokens w and w + kWaves (m <= 2 * kWaves), 4 scores per lane
  // each (n_exp <= 256); a lane reloads only the words it has not yet seen
  static_assert(kMaxTok <= 2 * kWaves, "two tokens per wave");
  const uint64_t* copy = p.scores + (int64_t)(blockIdx.x % kScoreCopies) * p.score_stride;
  float v[2][4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
  unsigned need = 0;  // bit 4j + q: score of token wave + kWaves*j, expert lane + 64q
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (wave + kWaves * j < p.m && lane + 64 * q < p.n_exp) need |= 1u << (4 * j + q);
  // every load of a round in flight at once; the first round's go out
  // before the epoch load, so the table entries, the epoch and the first
  // round share one memory round trip
  uint64_t w[2][4];
  unsigned cur = need;
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      w[j][q] = (cur & (1u << (4 * j + q))) ? load_agent(copy + (wave + kWaves * j) * p.n_exp + lane + 64 * q) : 0ull;
  const unsigned tag = sh.tag;
  bool seen = false;
  for (unsigned it = 0; it < kSpinLimit; ++it) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if ((cur & (1u << (4 * j + q))) && (unsigned)(w[j][q] >> 32) == tag) {
          v[j][q] = __uint_as_float((unsigned)w[j][q]);
          need &= ~(1u << (4 * j + q));
        }
    if (__ballot(need != 0) == 0) {
      seen = true;
      break;
    }
    __builtin_amdgcn_s_sleep(2);
    cur = need;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        w[j][q] = (cur & (1u << (4 * j + q))) ? load_agent(copy + (wave + kWaves * j) * p.n_exp + lane + 64 * q) : 0ull;
  }
  if (!seen && lane == 0) store_agent(p.ctl + kCtlErr, 1u + (unsigned)kWaitScores);
  // (the table loads were in flight with the first poll)
  if ((int)threadIdx.x < p.n_exp) sh.valid[threadIdx.x] = my_ent[0] != 0ull;
  sh.used[threadIdx.x] = 0;  // all kMaxExperts == kThreads bytes: wave 0 reads them as words
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int t = wave + kWaves * j;
    if (t < p.m) wave_topk_vals<4>(v[j], p.n_exp, p.top_k, p.scaling, sh.idx + t * p.top_k, sh.w + t * p.top_k);
  }
}

// Slots from sh.idx / sh.w: the distinct valid ids ascending, each token's
// weight of each slot, the slots' table entries.
__device__ __forceinline__ void finish_plan(const LayerParams& p, Shared& sh, const uint64_t (&my_ent)[6]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = p.m * p.top_k;
  __syncthreads();
  // Wave 0 alone (LDS accesses of one wave take effect in program order):
  // mark the selected valid experts, rank them ascending (lane l counts
  // experts 4l .. 4l+3; exclusive prefix of the counts from three ballots),
  // then each token's weight of each slot (at most one top-k entry, as a
  // token's ids are distinct; else 0).
  if (wave == 0) {
    for (int j = lane; j < n; j += 64) {
      const int64_t e = sh.idx[j];
      if (e >= 0 && e < p.n_exp && sh.valid[e]) sh.used[e] = 1;
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const uint32_t u4 = reinterpret_cast<const uint32_t*>(sh.used)[lane];
    const uint32_t b0 = (u4 & 0xffu) != 0, b1 = (u4 & 0xff00u) != 0, b2 = (u4 & 0xff0000u) != 0,
                   b3 = (u4 & 0xff000000u) != 0;
    const uint32_t c = b0 + b1 + b2 + b3;
    const uint64_t m0 = __ballot(c & 1u), m1 = __ballot(c & 2u), m2 = __ballot(c & 4u);
    const int pre = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m0 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m0, 0)) +
                    2 * (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m1 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m1, 0)) +
                    4 * (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m2 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m2, 0));
    const int base = __popcll(m0) + 2 * __popcll(m1) + 4 * __popcll(m2);
    const int e4 = 4 * lane;
    if (b0) { sh.rank[e4] = (short)pre; sh.eid[pre] = e4; }
    if (b1) { sh.rank[e4 + 1] = (short)(pre + b0); sh.eid[pre + b0] = e4 + 1; }
    if (b2) { sh.rank[e4 + 2] = (short)(pre + b0 + b1); sh.eid[pre + b0 + b1] = e4 + 2; }
    if (b3) { sh.rank[e4 + 3] = (short)(pre + b0 + b1 + b2); sh.eid[pre + b0 + b1 + b2] = e4 + 3; }
    for (int s0 = 0; s0 < base; s0 += 64 / kMaxTok) {  // zero weights: (slot, token) per lane
      const int sl = s0 + lane / kMaxTok, t = lane % kMaxTok;
      if (sl < base && t < p.m) sh.wt[sl][t] = 0.0f;
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (!p.route_idx) {  // router ids: distinct per token
      for (int j = lane; j < n; j += 64) {
        const int64_t e = sh.idx[j];
        if (e >= 0 && e < p.n_exp && sh.valid[e]) sh.wt[sh.rank[e]][j / p.top_k] = __fadd_rn(0.0f, sh.w[j]);
      }
    } else {  // given ids may repeat within a token: their weights add, in k order
      for (int j = lane; j < n; j += 64) {
        const int64_t e = sh.idx[j];
        const int t = j / p.top_k, c0 = t * p.top_k;
        bool first = e >= 0 && e < p.n_exp && sh.valid[e];
        for (int c = c0; c < j && first; ++c) first = sh.idx[c] != e;
        if (first) {
          float w = 0.0f;
          for (int c = c0; c < c0 + p.top_k; ++c)
            if (sh.idx[c] == e) w = __fadd_rn(w, sh.w[c]);
          sh.wt[sh.rank[e]][t] = w;
        }
      }
    }
    if (lane == 0) sh.n_routed = base;
  }
  __syncthreads();
  // each selected expert's thread moves its table entry into its slot
  if ((int)threadIdx.x < p.n_exp && sh.used[threadIdx.x]) {
    const int sl = sh.rank[threadIdx.x];
#pragma unroll
    for (int k = 0; k < 6; ++k) sh.ent[sl][k] = my_ent[k];
  }
  if (threadIdx.x == 0) sh.have_plan = 1;
  __syncthreads();
}

// The slot plan of this launch in LDS (n_exp <= kThreads): thread e holds
// expert e's table entry.  The ids and weights come from the router's scores
// (build_plan_scores) or, with given routing, from the caller's arrays (a
// hash layer's token table, engine.py:1018-1023); then the distinct valid
// expert ids in ascending order become the slots, each token's weight for a
// slot being its weight for that id (a token's ids are distinct: at most
// one), else 0 -- the union of _forward_legacy, fused_moe.py:466-476.
__device__ __forceinline__ void build_plan(const LayerParams& p, Shared& sh, const uint64_t (&my_ent)[6]) {
  const int n = p.m * p.top_k;
  if (p.route_idx) {
    // given routing: nothing to wait for (ids of tokens outside the table: -1)
    for (int j = threadIdx.x; j < n; j += kThreads) {
      const int t = j / p.top_k, c = j - t * p.top_k;
      int64_t e = -1;
      if (p.route_tok) {
        const int64_t tok = ldg<int64_t>(p.route_tok + t);
        if (tok >= 0 && tok < p.route_rows) e = ldg<int64_t>(p.route_idx + tok * p.top_k + c);
      } else {
        e = ldg<int64_t>(p.route_idx + j);
      }
      sh.idx[j] = e;
      sh.w[j] = p.route_w ? ldg<float>(p.route_w + j) : p.route_wconst;
    }
    if ((int)threadIdx.x < p.n_exp) sh.valid[threadIdx.x] = my_ent[0] != 0ull;
    sh.used[threadIdx.x] = 0;
  } else {
    build_plan_scores(p, sh, my_ent);
  }
  finish_plan(p, sh, my_ent);
}

// The routing outputs (and the zero output of a layer with no valid expert
// and no shared expert), written once by the plan builder.
__device__ __forceinline__ void write_routing(const LayerParams& p, Shared& sh) {
  for (int j = threadIdx.x; j < p.m * p.top_k; j += kThreads) {
    if (p.idx_out) p.idx_out[j] = sh.idx[j];
    if (p.w_out) p.w_out[j] = sh.w[j];
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
#if defined(__HIP_DEVICE_COMPILE__)
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)kernarg);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(kernarg >> 32));
  return *(KernargParams*)(((uint64_t)hi << 32) | lo);
#else
  return LayerParams{};  // host pass: never called
#endif
}

// p.fin, loaded from the kernarg segment where it is used (a volatile load
// the compiler cannot hoist): held across down_finish's polls, the pointer
// made that function save a callee-saved register to scratch.
__device__ __forceinline__ uint64_t* fin_late(uint64_t kernarg) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)kernarg);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(kernarg >> 32));
  return ((const volatile KernargParams*)(((uint64_t)hi << 32) | lo))->fin;
#else
  return nullptr;
#endif
}

// The slot plan in g_sh (a function of its own, called from the kernel's item
// loop, so its state adds to no streaming item's registers); the last
// workgroup of the grid also writes the routing outputs.
__device__ __noinline__ void plan_item(uint64_t kernarg) {
  const LayerParams p = params(kernarg);
  Shared& sh = g_sh;
  uint64_t my_ent[6];  // expert threadIdx.x's table entry
#pragma unroll
  for (int k = 0; k < 6; ++k)
    my_ent[k] = (int)threadIdx.x < p.n_exp ? ldg<uint64_t>(p.table + (int64_t)threadIdx.x * 6 + k) : 0ull;
  build_plan(p, sh, my_ent);
  if (blockIdx.x == gridDim.x - 1) write_routing(p, sh);  // read only after the launch
}

// plan_item for given routing when a gate/up item comes next and the LDS
// tile does not hold x: it also copies x into the tile, by LDS-DMA loads
// (global_load_lds_dwordx4: lane l of a wave writes 16 bytes at the wave's
// base + 16 l, the tile's own layout) issued before the table entries and
// the ids, so that x and the plan's inputs share one memory round trip and
// no register holds x meanwhile.  The tile then holds x.
__device__ __noinline__ void plan_x_item(uint64_t kernarg) {
  const LayerParams p = params(kernarg);
  Shared& sh = g_sh;
  __syncthreads();  // the previous item's readers of the tile are done
  const int n16 = p.m * p.d / 8, wave = threadIdx.x >> 6;
  const uint4* src = reinterpret_cast<const uint4*>(p.x);
  typedef __attribute__((address_space(3))) char LdsByte;
  LdsByte* const tile = (LdsByte*)g_tile;
  for (int c0 = 0; c0 < n16; c0 += kThreads) {
    const int c = c0 + (int)threadIdx.x;
    LdsByte* const dst = tile + 16 * (c0 + 64 * wave);  // wave-uniform base
    if (c < n16) __builtin_amdgcn_global_load_lds((const void*)(src + c), (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
  }
  uint64_t my_ent[6];
#pragma unroll
  for (int k = 0; k < 6; ++k)
    my_ent[k] = (int)threadIdx.x < p.n_exp ? ldg<uint64_t>(p.table + (int64_t)threadIdx.x * 6 + k) : 0ull;
  build_plan(p, sh, my_ent);
  if (blockIdx.x == gridDim.x - 1) write_routing(p, sh);
  __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS-DMA loads have landed
  __syncthreads();                // and every wave's
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
  const unsigned tag = g_sh.tag;
  const float bias_v = p.bias && threadIdx.x < p.m ? ldg<float>(p.bias + e) : 0.0f;
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
  if (threadIdx.x < p.m) {
    const int t = threadIdx.x;
    double sum = sh.rpart[0][t];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) sum += sh.rpart[w][t];
    const float score = router_score_v(sum, p.bias != nullptr, bias_v, p.logits ? p.logits + t * p.n_exp + e : nullptr);
    sh.rscore[t] = score;
  }
  __syncthreads();
  for (int c = threadIdx.x; c < p.m * kScoreCopies; c += kThreads) {
    const int t = c % p.m, copy = c / p.m;
    store_agent(p.scores + (int64_t)copy * p.score_stride + t * p.n_exp + e, tagged(tag, __float_as_uint(sh.rscore[t])));
  }
  return state;
}

__device__ __noinline__ int gate_up_item(uint64_t kernarg, int q_arg, int state_arg) {
  const int q = __builtin_amdgcn_readfirstlane(q_arg);
  int state = __builtin_amdgcn_readfirstlane(state_arg);
  const LayerParams p = params(kernarg);
  Shared& sh = g_sh;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int gu_per_slot = p.i / kGuRows;
  const int qq = q - p.gu0;
  const int s = qq / gu_per_slot;
  const int r0 = (qq % gu_per_slot) * kGuRows;
  if (s >= sh.n_routed) return state;
  const unsigned tag = g_sh.tag;
  if (threadIdx.x < p.m) sh.wt_item[threadIdx.x] = sh.wt[s][threadIdx.x];
  const uint64_t* ent = sh.ent[s];
  ensure_x(p, state);
  const int per = (p.d / 128) / kWaves;
  const int st0 = wave * per;
  f32x4 ag = {0, 0, 0, 0}, au = {0, 0, 0, 0};
  gate_up_slot(slot_format(p.scale_fmt, ent, false), ent, g_tile, p.m, p.d, p.i, r0, st0, st0 + per, ag, au);
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
    store_agent(p.act + ((int64_t)s * p.m + col) * p.i + r0 + row, tagged(tag, __float_as_uint(a)));
  }
  return state;
}

// Shared gate/up, one matrix per item: item k streams the 16 rows of one row
// group of W1 or W3 -- one matrix, so twice the steps per batch of a routed
// gate/up item in the same registers -- and adds the four waves' K ranges in
// wave order, as gate_up_item does.  Items come in blocks of 8 row groups: W1
// of the 8 groups, then W3 of the same 8 (a short last block likewise).  The
// W1 item publishes its rows' gate sums to plane 0 of p.sgh; the W3 item (a
// larger item index, running beside it) waits for them and publishes the
// rows' activations SwiGLU(gate, up) (weight 1) to plane 1, which the shared
// down stages as a routed down stages its slot's.
__device__ __noinline__ int shared_half_item(uint64_t kernarg, int q_arg, int state_arg) {
  const int q = __builtin_amdgcn_readfirstlane(q_arg);
  int state = __builtin_amdgcn_readfirstlane(state_arg);
  const LayerParams p = params(kernarg);
  Shared& sh = g_sh;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // the W1 and W3 items of a row group are `span` (8) item indices apart, so
  // that they run on one XCD when workgroups are dealt to the 8 XCDs in turn
  const int k = q - p.sgu0, blk = k >> 4, span = min(8, p.i / kGuRows - 8 * blk);
  const int mat = (k & 15) >= span, r0 = (8 * blk + (k & 15) - mat * span) * kGuRows;
  const unsigned tag = g_sh.tag;
  const uint64_t* ent = sh.ent[p.S];
  ensure_x(p, state);
  const int per = (p.d / 128) / kWaves;
  const int st0 = wave * per;
  const uint64_t w = ent[2 * mat], sc = ent[2 * mat + 1];
  f32x4 acc = {0, 0, 0, 0};
  if (slot_format(p.scale_fmt, ent, true) == kFp8Block)
    gate_or_up_any<kFp8Block>(w, sc, g_tile, p.m, p.d, p.i, r0, st0, st0 + per, acc);
  else
    gate_or_up_any<kBf16>(w, sc, g_tile, p.m, p.d, p.i, r0, st0, st0 + per, acc);
  if ((lane & 15) < kMaxTok) {
#pragma unroll
    for (int c = 0; c < 4; ++c) sh.red[wave][0][(4 * (lane >> 4) + c) * kMaxTok + (lane & 15)] = acc[c];
  }
  __syncthreads();
  const int row = threadIdx.x >> 4, col = threadIdx.x & 15;
  if (col < p.m) {
    float sum = 0.0f;
#pragma unroll
    for (int w4 = 0; w4 < kWaves; ++w4) sum = __fadd_rn(sum, sh.red[w4][0][row * kMaxTok + col]);
    const uint32_t off = (uint32_t)(col * p.i + r0 + row);
    if (mat == 0) {
      store_agent(p.sgh + off, tagged(tag, __float_as_uint(sum)));
    } else {
      float gv[1];
      poll_tagged<1>(p.sgh, 0, off, 1, tag, gv, p.ctl, kWaitGate);
      const float a = __fmul_rn(1.0f, swiglu(gv[0], sum, p.limit));
      store_agent(p.sgh + (int64_t)p.m * p.i + off, tagged(tag, __float_as_uint(a)));
    }
  }
  return state;
}

// A run of routed gate/up items q, q + G, q + 2G, ... (G = grid) whose slots
// are in format F with whole batches (d / 512 a multiple of the batch): as
// soon as a wave has multiplied its last batch of item q it issues the first
// batch of item q + G into the same registers, so the cross-wave reduction
// and the tagged stores of item q overlap the loads of the next item.  Same
// tiles and accumulation order as gate_up_item, so the results are
// identical.  Returns the last item run.
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
  const unsigned tag = g_sh.tag;
  int s = (q - p.gu0) / gu_per_slot, r0 = ((q - p.gu0) % gu_per_slot) * kGuRows;
  Mat w1 = make_mat<F>(sh.ent[s][0], sh.ent[s][1], p.i, p.d), w3 = make_mat<F>(sh.ent[s][2], sh.ent[s][3], p.i, p.d);
  Batch<F, kB> b1, b3;
  b1.load(w1, r0 + r, p.d, st0, g);
  b3.load(w3, r0 + r, p.d, st0, g);
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
    const int s2 = (q2 - p.gu0) / gu_per_slot, r02 = ((q2 - p.gu0) % gu_per_slot) * kGuRows;
    const bool next = q2 < p.gu1 && s2 < sh.n_routed && slot_format(p.scale_fmt, sh.ent[s2], false) == F;
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
        store_agent(p.act + ((int64_t)s * p.m + col) * p.i + r0 + row, tagged(tag, __float_as_uint(a)));
      }
    }
    __syncthreads();  // sh.red and sh.wt_item are rewritten by the next item
    if (!next) break;
    q = q2;
    s = s2;
    r0 = r02;
  }
  return q;
}

// Slot, row group (kDownRows rows) and half of down item q: a routed down
// item covers its row group (h = 0); shared down items 2g + h cover rows
// 32h .. 32h + 31 of row group g, two waves per step range of the shared
// expert's split (shared_down_half).  Routed down items: with drun = 2,
// blocks of 2G items (G = dgrid) for dk slots each -- in a block, column c
// (item c and item c + G, which workgroup (d0 + c) % G runs one after the
// other) takes row groups c % half and half + c % half (half = groups per
// slot / 2) of slot c / half -- then the slots left, slot-major.
__device__ __forceinline__ void down_slot_of(const LayerParams& p, int q, bool& is_shared, int& s, int& g, int& h) {
  const int dps = p.d / kDownRows;
  is_shared = q >= p.sd0 && q < p.sd1;
  h = 0;
  if (is_shared) {
    s = p.S;
    g = (q - p.sd0) >> 1;
    h = (q - p.sd0) & 1;
    return;
  }
  int u = q - p.d0, s0 = 0;
  if (p.drun == 2) {
    const int G = p.dgrid, half = dps / 2, nb = p.S / p.dk;
    if (u < nb * 2 * G) {
      const int b = u / (2 * G), pp = u - b * 2 * G, r = pp >= G ? 1 : 0, c = pp - r * G;
      s = b * p.dk + c / half;
      g = r * half + c % half;
      return;
    }
    u -= nb * 2 * G;
    s0 = nb * p.dk;
  }
  s = s0 + u / dps;
  g = u % dps;
}

// Item index of routed down item (slot s, row group g): increasing in s.
__device__ __forceinline__ int down_index(const LayerParams& p, int s, int g) {
  const int dps = p.d / kDownRows;
  if (p.drun == 2) {
    const int G = p.dgrid, half = dps / 2, nb = p.S / p.dk;
    if (s < nb * p.dk) {
      const int b = s / p.dk;
      return p.d0 + b * 2 * G + (g / half) * G + (s - b * p.dk) * half + g % half;
    }
    return p.d0 + nb * 2 * G + (s - nb * p.dk) * dps + g;
  }
  return p.d0 + s * dps + g;
}

// Down item q, first part: W2 rows of the slot against its activations, the
// slot's fp32 partial sums published (tagged) for the row group.  Needs the
// slot plan for a routed slot only (the shared slot may run before the plan
// exists).  One instantiation per kind (routed or shared), so that each holds
// only its own formats' registers.
template <bool kShared>
__device__ __noinline__ int down_item(uint64_t kernarg, int q_arg, int state_arg) {
  const int q = __builtin_amdgcn_readfirstlane(q_arg);
  int state = __builtin_amdgcn_readfirstlane(state_arg);
  const LayerParams p = params(kernarg);
  Shared& sh = g_sh;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  bool is_shared_q;
  int s, g, h;
  down_slot_of(p, q, is_shared_q, s, g, h);
  constexpr bool is_shared = kShared;
  if (!is_shared && s >= sh.n_routed) return state;
  const unsigned tag = g_sh.tag;
  const uint64_t* ent = sh.ent[s];
  // shared: waves 0 and 2 (1 and 3) take rows r0 .. r0 + 15 over the first
  // (second) step range
  const int r0 = kShared ? g * kDownRows + 32 * h + 16 * (wave & 1) : g * kDownRows + 16 * wave;
  const int m = p.m, i = p.i;
  unsigned* const ctl = p.ctl;
  const uint64_t* const src = p.act + (int64_t)s * m * i;
  const uint64_t* const sgh = p.sgh;
  f32x4 acc = {0, 0, 0, 0};
  auto stage = [&]() __attribute__((always_inline)) {
    // fp32 activations (the shared slot's: plane 1 of p.sgh) -> bf16 hi
    // rows [t][k] and lo rows [m + t][k], each written once it carries this
    // launch's tag -- unless the tile holds them from this workgroup's
    // previous item
    if (!kShared && state == 2 + s) return;
    const int n = m * i;
    constexpr int kStageWords = 8;  // per thread and round (registers: the W2 batch is live)
    for (int u0 = 0; u0 < n; u0 += kStageWords * kThreads) {  // this thread's words u0 + threadIdx.x + kThreads * j
      const int c0 = u0 + (int)threadIdx.x;
      unsigned need = 0;
#pragma unroll
      for (int j = 0; j < kStageWords; ++j)
        if (c0 + kThreads * j < n) need |= 1u << j;
      for (unsigned it = 0; it < kSpinLimit; ++it) {
        const unsigned cur = need;  // every load of the round in flight at once
        uint64_t w[kStageWords];
#pragma unroll
        for (int j = 0; j < kStageWords; ++j) {
          const uint64_t* b = is_shared ? sgh + n : src;
          w[j] = (cur >> j) & 1u ? load_agent(b + u0 + kThreads * j + threadIdx.x) : 0ull;
        }
#pragma unroll
        for (int j = 0; j < kStageWords; ++j) {
          const bool fresh = (unsigned)(w[j] >> 32) == tag;
          if (((cur >> j) & 1u) && fresh) {
            const float a = __uint_as_float((unsigned)w[j]);
            const int c = c0 + kThreads * j;
            const uint32_t hi = f32_to_bf16_bits(a);
            const uint32_t lo = f32_to_bf16_bits(__fadd_rn(a, -bf16_bits_to_f32(hi)));
            g_tile[c] = (uint16_t)hi;
            g_tile[n + c] = (uint16_t)lo;
            need &= ~(1u << j);
          }
        }
        if (__ballot(need != 0) == 0) break;
        __builtin_amdgcn_s_sleep(2);
      }
      if (need) {  // gave up: zeros in the tile, the wait recorded
        store_agent(ctl + kCtlErr, 1u + (unsigned)(is_shared ? kWaitShared : kWaitAct));
#pragma unroll
        for (int j = 0; j < kStageWords; ++j)
          if ((need >> j) & 1u) {
            g_tile[c0 + kThreads * j] = 0;
            g_tile[n + c0 + kThreads * j] = 0;
          }
      }
    }
    __syncthreads();
  };
  const int fmt = slot_format(p.scale_fmt, ent, is_shared);
  if constexpr (kShared) {
    const int half = shared_down_half(i), st0 = wave < 2 ? 0 : half, st1 = wave < 2 ? half : i / 128;
    if (fmt == kFp8Block) down_any<kFp8Block, true>(ent, g_tile, m, i, p.d, r0, st0, st1, acc, stage);
    else down_any<kBf16, true>(ent, g_tile, m, i, p.d, r0, st0, st1, acc, stage);
    // first range + second range, in the waves of the first
    float* const xr = &sh.red[0][0][0];
    if (wave >= 2) {
#pragma unroll
      for (int c = 0; c < 4; ++c) xr[((wave - 2) * 64 + lane) * 4 + c] = acc[c];
    }
    __syncthreads();
    if (wave < 2) {
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = __fadd_rn(acc[c], xr[(wave * 64 + lane) * 4 + c]);
    }
  } else {
    // FP4 E8M0 at m >= 3: batches of 8 steps instead of 16 (measured at M=3:
    // 78.0 us against 78.8; at M=1 the 16-step batch is 0.2 us faster)
    if (fmt == kFp4E8M0 && m >= 3) down_any<kFp4E8M0, true, 8>(ent, g_tile, m, i, p.d, r0, 0, i / 128, acc, stage);
    else if (fmt == kFp4E8M0) down_any<kFp4E8M0, true>(ent, g_tile, m, i, p.d, r0, acc, stage);
    else if (fmt == kFp4F32) down_any<kFp4F32, true>(ent, g_tile, m, i, p.d, r0, acc, stage);
    else down_any<kBf16, true>(ent, g_tile, m, i, p.d, r0, acc, stage);
  }
  state = kShared ? 0 : 2 + s;
  // lane (col = lane%16) holds rows 4*(lane/16)+c; column t (hi) + column m+t (lo)
  // of token t are combined through the lane that owns column t.
  uint64_t* part = p.part + (int64_t)s * m * p.d;
  if (kShared && wave >= 2) return state;
  // one routed slot and no shared expert: this item is its row group's only
  // contributor and writes the rows itself (the value the row-group sum
  // would give: 0 + the partial), with no round trip through the partials
  const bool alone = !kShared && sh.n_routed == 1 && !p.shared;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int col = lane & 15;
    const float lo = __shfl(acc[c], (lane & 48) | ((col + m) & 15), 64);
    if (col < m) {
      const float v = __fadd_rn(acc[c], lo);
      const int row = r0 + 4 * (lane >> 4) + c;
      if (alone) {
        const float o = __fadd_rn(0.0f, v);
        if (p.out_f32) p.out_f32[(int64_t)col * p.d + row] = o;
        if (p.out_bf16) p.out_bf16[(int64_t)col * p.d + row] = (uint16_t)f32_to_bf16_bits(o);
        if (p.fin) store_agent(p.fin + (int64_t)col * p.d + row, tagged(tag, __float_as_uint(o)));
      } else {
        store_agent(part + (int64_t)col * p.d + row, tagged(tag, __float_as_uint(v)));
      }
    }
  }
  return state;
}

// Down item q, second part (the slot plan exists): of the row group's
// contributors (its down item of each routed slot, and the shared down), the
// one with the largest item index -- it waits only for smaller ones -- adds
// the slots' tagged partials in slot order (routed ascending, shared last)
// and writes the output rows.
__device__ __noinline__ void down_finish(uint64_t kernarg, int q_arg) {
  const int q = __builtin_amdgcn_readfirstlane(q_arg);
  const LayerParams p = params(kernarg);
  Shared& sh = g_sh;
  bool is_shared;
  int s, g, h;
  down_slot_of(p, q, is_shared, s, g, h);
  const int n_routed = sh.n_routed;
  if (!is_shared && s >= n_routed) return;
  if (n_routed == 1 && !p.shared) return;  // the down item wrote its rows itself
  int last = n_routed > 0 ? down_index(p, n_routed - 1, g) : -1;
  if (p.shared && p.sd0 + 2 * g + 1 > last) last = p.sd0 + 2 * g + 1;
  if (q != last) return;
  const unsigned tag = g_sh.tag;
  const int m = p.m;
  const int64_t stride = (int64_t)m * p.d;  // between slots
  for (int c0 = 0; c0 < kDownRows * m; c0 += kThreads) {
    const int c = c0 + (int)threadIdx.x;
    const bool mine = c < kDownRows * m;
    const int t = mine ? c / kDownRows : 0, dd = g * kDownRows + (mine ? c - t * kDownRows : 0);
    const uint32_t off = (uint32_t)(t * p.d + dd);
    float v = 0.0f;
    for (int s0 = 0; s0 < n_routed; s0 += 8) {
      float pv[8];
      poll_tagged<8>(p.part + (int64_t)s0 * stride, stride, off, mine ? n_routed - s0 : 0, tag, pv, p.ctl, kWaitPart);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (s0 + j < n_routed) v = __fadd_rn(v, pv[j]);
    }
    if (p.shared) {
      float pv[1];
      poll_tagged<1>(p.part + (int64_t)p.S * stride, stride, off, mine ? 1 : 0, tag, pv, p.ctl, kWaitPart);
      v = __fadd_rn(v, pv[0]);
    }
    if (mine) {
      const int64_t o = (int64_t)t * p.d + dd;
      if (p.out_f32) p.out_f32[o] = v;
      if (p.out_bf16) p.out_bf16[o] = (uint16_t)f32_to_bf16_bits(v);
      uint64_t* const fin = fin_late(kernarg);
      if (fin) store_agent(fin + o, tagged(tag, __float_as_uint(v)));
    }
  }
}

// Tail item of token row t (launches with a norm tail; the slot plan exists):
// the next layer's input from this layer's output row,
//   h_out = bf16(bf16(h + bf16(out)) + res),  norm_out = RMSNorm(h_out) * w,
// with the arithmetic and the order of hsmoe_add_rms_norm (hsmoe_norm.h):
// this thread's 8-column chunks c = tid, tid + 256, ... in turn, the wave's
// butterfly, the waves in order -- bit-identical to the layer's bf16 output
// followed by hsmoe_add_rms_norm.  The output row comes from the tagged words
// the row-group sums (or a lone slot's down items) publish; two chunks' 16
// words are polled with every load in flight at once.  A layer with no expert
// to run has a zero output and nothing to wait for.
__device__ __noinline__ void tail_item(uint64_t kernarg, int t_arg) {
  const int t = __builtin_amdgcn_readfirstlane(t_arg);
  const LayerParams p = params(kernarg);
  const unsigned tag = g_sh.tag;
  const bool zero = g_sh.n_routed == 0 && !p.shared;
  const int tid = (int)threadIdx.x;
  const int chunks = p.d / 8;  // d <= 8192: at most 4 chunks per thread
  const int64_t base = (int64_t)t * chunks;
  const uint4* h = (const uint4*)p.tail_h + base;
  const uint4* res = (const uint4*)p.tail_res;
  const uint4* w = (const uint4*)p.tail_w;
  const uint64_t* fin = p.fin + (int64_t)t * p.d;
  uint4 u[4], wv[4];
  float s = 0.0f;
#pragma unroll
  for (int b0 = 0; b0 < 4; b0 += 2) {
    uint4 hv[2], rv[2];
    unsigned need = 0;
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      const int c = tid + kThreads * (b0 + bb);
      hv[bb] = rv[bb] = wv[b0 + bb] = make_uint4(0u, 0u, 0u, 0u);
      if (c < chunks) {
        hv[bb] = h[c];
        if (res) rv[bb] = res[c];
        wv[b0 + bb] = w[c];
        if (!zero) need |= 0xffu << (8 * bb);
      }
    }
    float f[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) f[j] = 0.0f;
    for (unsigned it = 0; it < kSpinLimit; ++it) {
      const unsigned cur = need;
      uint64_t wd[16];
#pragma unroll
      for (int j = 0; j < 16; ++j)
        wd[j] = (cur >> j) & 1u ? load_agent(fin + 8 * (tid + kThreads * (b0 + (j >> 3))) + (j & 7)) : 0ull;
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (((cur >> j) & 1u) && (unsigned)(wd[j] >> 32) == tag) {
          f[j] = __uint_as_float((unsigned)wd[j]);
          need &= ~(1u << j);
        }
      if (__ballot(need != 0) == 0) break;
      __builtin_amdgcn_s_sleep(2);
    }
    if (need) store_agent(p.ctl + kCtlErr, 1u + (unsigned)kWaitTail);
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      const int c = tid + kThreads * (b0 + bb);
      const float* fb = f + 8 * bb;
      const uint4 a = make_uint4(f32_to_bf16_bits(fb[0]) | (f32_to_bf16_bits(fb[1]) << 16),
                                 f32_to_bf16_bits(fb[2]) | (f32_to_bf16_bits(fb[3]) << 16),
                                 f32_to_bf16_bits(fb[4]) | (f32_to_bf16_bits(fb[5]) << 16),
                                 f32_to_bf16_bits(fb[6]) | (f32_to_bf16_bits(fb[7]) << 16));
      uint4 x = norm_add_chunk(hv[bb], a);
      if (res) x = norm_add_chunk(x, rv[bb]);
      u[b0 + bb] = x;
      if (c < chunks) {
        ((uint4*)p.tail_h_out)[base + c] = x;
        s = norm_sumsq_chunk(x, s);
      }
    }
  }
  s = norm_wave_sum(s);
  float* const part = &g_sh.red[0][0][0];  // free: every item starts after a barrier
  if ((tid & 63) == 0) part[tid >> 6] = s;
  __syncthreads();
  const float inv = norm_inv(part, p.d, p.tail_eps);
  uint4* const out = (uint4*)p.tail_out + base;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int c = tid + kThreads * b;
    if (c < chunks) out[c] = norm_scale_chunk(u[b], wv[b], inv);
  }
}

__global__ void __launch_bounds__(kThreads, 2) moe_layer_kernel(LayerParams p) {
  int state = 0;  // 1 while the LDS tile holds x, 2 + s while routed slot s's activations
  if (threadIdx.x == 0) {
    g_sh.have_plan = 0;
    g_sh.tag = read_launch_tag(p.ctl);  // visible to every wave after the first item's barrier
  }
  if (p.shared && threadIdx.x < 6) g_sh.ent[p.S][threadIdx.x] = ldg<uint64_t>(p.shared + threadIdx.x);
  const uint64_t kernarg = (uint64_t)__builtin_amdgcn_kernarg_segment_ptr();  // &p
  const int n_main = p.n_main, n_router = p.n_router;
  // x comes with the slot plan only where the plan's inputs are in memory
  // (given routing); with the router, x in the plan's round trip measured
  // slower at M=3 (77.9 us against 77.6) and equal at M=1
  const bool given = p.route_idx != nullptr;
  int q = blockIdx.x;
  for (; q < n_main; q += gridDim.x) {
    __syncthreads();  // the previous item's readers of the LDS scratch are done
    if (q < n_router) {
      state = router_item(kernarg, q, state);
      continue;
    }
    if (q >= p.sgu0 && q < p.sgu1) {  // shared gate or up
      state = shared_half_item(kernarg, q, state);
      continue;
    }
    if (q >= p.sd0 && q < p.sd1) {  // shared down: the plan is needed only for its arrival
      state = down_item<true>(kernarg, q, state);
      if (!g_sh.have_plan) {
        const int qn = q + (int)gridDim.x;  // a gate/up item next: x comes with the plan
        if (given && qn >= p.gu0 && qn < p.gu1 && qn < n_main) {
          plan_x_item(kernarg);
          state = 1;
        } else {
          plan_item(kernarg);
        }
      }
      down_finish(kernarg, q);
      continue;
    }
    if (!g_sh.have_plan) {  // routed items need the slot plan (given routing: a gate/up item x too)
      if (given && state != 1 && q >= p.gu0 && q < p.gu1) {
        plan_x_item(kernarg);
        state = 1;
      } else {
        plan_item(kernarg);
      }
    }
    if (q >= p.gu0 && q < p.gu1) {
      const int s = (q - p.gu0) / (p.i / kGuRows);
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
      state = down_item<false>(kernarg, q, state);
      down_finish(kernarg, q);
    }
  }
  for (; q < p.n_items; q += gridDim.x) {  // norm tail items, last in the order
    __syncthreads();
    if (!g_sh.have_plan) plan_item(kernarg);
    tail_item(kernarg, q - p.n_main);
  }
  __syncthreads();
  // the routing outputs come from the last workgroup, also when it ran no item
  // that needs the plan (the plan waits only for R items, which wait for
  // nothing)
  if (blockIdx.x == gridDim.x - 1 && !g_sh.have_plan) plan_item(kernarg);
  // the last workgroup to finish (every workgroup has read the epoch and is
  // done with the workspace by then) advances the epoch to this launch's tag,
  // or at kRearmTag zeroes the tagged words and restarts the epoch at 0, and
  // re-arms the counter
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) g_sh.last = add_agent(p.ctl + kCtlDone, 1u) == gridDim.x - 1;
  __syncthreads();
  if (!g_sh.last) return;
  const unsigned tag = g_sh.tag;
  if (tag >= kRearmTag) {
    const uint4 zero = {0u, 0u, 0u, 0u};
    for (int64_t k = threadIdx.x; k < p.wipe_n; k += kThreads) p.wipe[k] = zero;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (p.status_out) {
      *p.status_out = load_agent(p.ctl + kCtlErr);
      store_agent(p.ctl + kCtlErr, 0u);
    }
    store_agent(p.ctl + kCtlEpoch, tag >= kRearmTag ? 0u : tag);
    store_agent(p.ctl + kCtlDone, 0u);
  }
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }
size_t layer_lds(int64_t m, int64_t d, int64_t i) { return (size_t)(m * d > 2 * m * i ? m * d : 2 * m * i) * 2; }
int64_t score_stride_words(int64_t m, int64_t n_exp) { return (m * n_exp * 8 + 4095) / 4096 * 512; }
size_t scores_bytes(int64_t m, int64_t n_exp) { return (size_t)kScoreCopies * score_stride_words(m, n_exp) * 8; }
size_t act_bytes(int64_t m, int64_t i, int top_k) { return align256((size_t)(m * top_k + 2) * m * i * 8); }
// partials of the m * top_k routed slots and the shared one, then the output rows (fin)
size_t part_bytes(int64_t m, int64_t d, int top_k) { return align256((size_t)(m * top_k + 2) * m * d * 8); }

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
  return kCtlBytes + scores_bytes(m, n_experts) + act_bytes(m, i, top_k) + part_bytes(m, d, top_k);
}

namespace {

// Checks the arguments of a layer launch (not the workspace) -> HSMOE_OK or an error.
int check_layer_args(const char* name, const void* x, int64_t m, int64_t d, int64_t i, const void* gate_w,
                     int64_t n_experts, int top_k, const uint64_t* expert_table, int scale_kind,
                     const int64_t* topk_idx_out, const float* topk_w_out, const float* out_f32,
                     const void* out_bf16, bool given_route = false, bool tail = false) {
  if (!x || !expert_table || (!tail && !out_f32 && !out_bf16) ||
      (!given_route && (!gate_w || !topk_idx_out || !topk_w_out)))
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
  if (!aligned(x, 16) || (!given_route && !aligned(gate_w, 16)))
    return fail(HSMOE_ERR_SHAPE, "%s: x and gate_w must be 16-byte aligned", name);
  if (layer_lds(m, d, i) > 65536) return fail(HSMOE_ERR_SHAPE, "%s: m*d and 2*m*i tiles must fit in 64 KiB of LDS", name);
  return HSMOE_OK;
}

// Launches moe_layer_kernel on checked arguments and a workspace of
// workspace_bytes >= hsmoe_moe_layer_workspace_size bytes (256-byte aligned).
struct GivenRoute {
  const int64_t* idx;
  const int64_t* tok;
  int64_t rows;
  const float* w;
  float wconst;
};

int launch_layer(const char* name, const void* x, int64_t m, int64_t d, int64_t i, const void* gate_w,
                 const float* gate_bias, int64_t n_experts, int top_k, float routed_scaling,
                 const uint64_t* expert_table, int scale_kind, const uint64_t* shared, float swiglu_limit,
                 int64_t* topk_idx_out, float* topk_w_out, void* logits_out, float* out_f32, void* out_bf16,
                 void* workspace, size_t workspace_bytes, unsigned* status_out, hipStream_t stream,
                 const GivenRoute* route = nullptr, const hsmoe_norm_tail* tail = nullptr) {
  const size_t lds = layer_lds(m, d, i);
  LayerParams p;
  p.tail_h = tail ? (const uint16_t*)tail->h_dev : nullptr;
  p.tail_res = tail ? (const uint16_t*)tail->residual_dev : nullptr;
  p.tail_w = tail ? (const uint16_t*)tail->weight_dev : nullptr;
  p.tail_h_out = tail ? (uint16_t*)tail->h_out_dev : nullptr;
  p.tail_out = tail ? (uint16_t*)tail->norm_out_dev : nullptr;
  p.tail_eps = tail ? tail->eps : 0.0f;
  p.route_idx = route ? route->idx : nullptr;
  p.route_tok = route ? route->tok : nullptr;
  p.route_rows = route ? route->rows : 0;
  p.route_w = route ? route->w : nullptr;
  p.route_wconst = route ? route->wconst : 0.0f;
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
  p.scores = (uint64_t*)ws;
  p.score_stride = (int)score_stride_words(m, n_experts);
  ws += scores_bytes(m, n_experts);
  p.act = (uint64_t*)ws;
  p.sgh = p.act + (size_t)p.S * m * i;
  ws += act_bytes(m, i, top_k);
  p.part = (uint64_t*)ws;
  p.fin = tail ? p.part + (size_t)(p.S + 1) * m * d : nullptr;
  p.wipe = (uint4*)((char*)workspace + kCtlBytes);
  p.wipe_n = (int64_t)((workspace_bytes - kCtlBytes) / 16);
  p.status_out = status_out;
  const int has_shared = shared ? 1 : 0;
  p.n_router = route ? 0 : (int)n_experts;
  // Item order after R (producers always before their consumers): SGU, SD,
  // GU, D -- the shared down streams while the routed work is still waiting
  // for the plan; for m <= 2 SGU, GU, D, SD -- there the routed work starts
  // early enough that the shared down, which nothing waits for but the
  // output sums, is better spent filling the last round (measured: M=1
  // 35.4 us against 36.2 with the shared down between GU and D and 38.9 with
  // it before GU; M=3 78.5 us in all three orders).
  const int n_sgu = has_shared * 2 * (int)(i / kGuRows), n_sd = has_shared * 2 * (int)(d / kDownRows);
  const int n_gu = p.S * (int)(i / kGuRows), n_d = p.S * (int)(d / kDownRows);
  p.sgu0 = p.n_router;
  p.sgu1 = p.sgu0 + n_sgu;
  if (m <= 2) {
    p.gu0 = p.sgu1;
    p.gu1 = p.gu0 + n_gu;
    p.d0 = p.gu1;
    p.d1 = p.d0 + n_d;
    p.sd0 = p.d1;
    p.sd1 = p.sd0 + n_sd;
  } else {
    p.sd0 = p.sgu1;
    p.sd1 = p.sd0 + n_sd;
    p.gu0 = p.sd1;
    p.gu1 = p.gu0 + n_gu;
    p.d0 = p.gu1;
    p.d1 = p.d0 + n_d;
  }
  p.n_main = p.sgu1 + n_sd + n_gu + n_d;
  p.n_items = p.n_main + (tail ? (int)m : 0);
  int resident = 0;
  int rc = resident_workgroups(lds, &resident);
  if (rc) return rc;
  const int grid = resident < p.n_items ? resident : p.n_items;
  // routed down items in pairs when two full rounds of them exist and the
  // grid splits into whole slots of half-slot columns
  const int dps = (int)(d / kDownRows);
  p.drun = 1;
  p.dgrid = grid;
  p.dk = 0;
  if (n_d >= 2 * grid && dps % 2 == 0 && grid % (dps / 2) == 0) {
    p.drun = 2;
    p.dk = 2 * grid / dps;
  }
  hipLaunchKernelGGL(moe_layer_kernel, dim3((unsigned)grid), dim3(kThreads), lds, stream, p);
  return check_launch(name);
}

__global__ void __launch_bounds__(256) clear_kernel(uint4* __restrict__ p, int64_t n) {
  const uint4 zero = {0u, 0u, 0u, 0u};
  for (int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x; k < n; k += (int64_t)gridDim.x * 256) p[k] = zero;
}

}  // namespace

extern "C" int hsmoe_moe_layer_decode(const void* x, int64_t m, int64_t d, int64_t i, const void* gate_w,
                                      const float* gate_bias, int64_t n_experts, int top_k, float routed_scaling,
                                      const uint64_t* expert_table, int scale_kind, const uint64_t* shared,
                                      float swiglu_limit, int64_t* topk_idx_out, float* topk_w_out,
                                      void* logits_out, float* out_f32, void* out_bf16, void* workspace,
                                      size_t workspace_bytes, hsmoe_stream_t stream) {
  const char* name = "hsmoe_moe_layer_decode";
  int rc = check_layer_args(name, x, m, d, i, gate_w, n_experts, top_k, expert_table, scale_kind, topk_idx_out,
                            topk_w_out, out_f32, out_bf16);
  if (rc) return rc;
  const size_t need = hsmoe_moe_layer_workspace_size(m, d, i, n_experts, top_k);
  if (!workspace || workspace_bytes < need || !aligned(workspace, 256))
    return fail(HSMOE_ERR_WORKSPACE, "%s: zero-filled workspace of %zu bytes (256-byte aligned) needed", name, need);
  return launch_layer(name, x, m, d, i, gate_w, gate_bias, n_experts, top_k, routed_scaling, expert_table,
                      scale_kind, shared, swiglu_limit, topk_idx_out, topk_w_out, logits_out, out_f32, out_bf16,
                      workspace, workspace_bytes, nullptr, (hipStream_t)stream);
}

extern "C" int hsmoe_moe_layer_decode_routed(const void* x, int64_t m, int64_t d, int64_t i, const int64_t* topk_idx,
                                             const int64_t* token_ids, int64_t table_rows, const float* topk_w,
                                             float weight_all, int top_k, const uint64_t* expert_table,
                                             int64_t n_experts, int scale_kind, const uint64_t* shared,
                                             float swiglu_limit, float* out_f32, void* out_bf16, void* workspace,
                                             size_t workspace_bytes, hsmoe_stream_t stream) {
  const char* name = "hsmoe_moe_layer_decode_routed";
  if (!topk_idx) return fail(HSMOE_ERR_ARG, "%s: null topk_idx", name);
  if (token_ids && table_rows < 1) return fail(HSMOE_ERR_ARG, "%s: a token table needs table_rows >= 1", name);
  int rc = check_layer_args(name, x, m, d, i, nullptr, n_experts, top_k, expert_table, scale_kind, nullptr, nullptr,
                            out_f32, out_bf16, true);
  if (rc) return rc;
  const size_t need = hsmoe_moe_layer_workspace_size(m, d, i, n_experts, top_k);
  if (!workspace || workspace_bytes < need || !aligned(workspace, 256))
    return fail(HSMOE_ERR_WORKSPACE, "%s: zero-filled workspace of %zu bytes (256-byte aligned) needed", name, need);
  const GivenRoute route{topk_idx, token_ids, token_ids ? table_rows : 0, topk_w, weight_all};
  return launch_layer(name, x, m, d, i, nullptr, nullptr, n_experts, top_k, 1.0f, expert_table, scale_kind, shared,
                      swiglu_limit, nullptr, nullptr, nullptr, out_f32, out_bf16, workspace, workspace_bytes, nullptr,
                      (hipStream_t)stream, &route);
}

namespace {

// Checks a norm tail of m rows of d (its h_out may be its h; norm_out must not
// overlap x, h, residual or weight).
int check_tail(const char* name, const hsmoe_norm_tail* tail, const void* x, int64_t m, int64_t d) {
  if (!tail || !tail->h_dev || !tail->weight_dev || !tail->h_out_dev || !tail->norm_out_dev)
    return fail(HSMOE_ERR_ARG, "%s: the norm tail needs h, weight, h_out and norm_out", name);
  if (!aligned(tail->h_dev, 16) || !aligned(tail->weight_dev, 16) || !aligned(tail->h_out_dev, 16) ||
      !aligned(tail->norm_out_dev, 16) || (tail->residual_dev && !aligned(tail->residual_dev, 16)))
    return fail(HSMOE_ERR_SHAPE, "%s: norm tail rows must be 16-byte aligned", name);
  if (!(tail->eps >= 0.0f)) return fail(HSMOE_ERR_ARG, "%s: norm tail eps must be >= 0", name);
  const size_t rows = (size_t)m * d * 2, row = (size_t)d * 2;
  auto overlap = [](const void* a, size_t na, const void* b, size_t nb) {
    const char *pa = (const char*)a, *pb = (const char*)b;
    return b && pa < pb + nb && pb < pa + na;
  };
  const void* out = tail->norm_out_dev;
  if (overlap(out, rows, x, rows) || overlap(out, rows, tail->h_dev, rows) ||
      overlap(out, rows, tail->h_out_dev, rows) || overlap(out, rows, tail->residual_dev, row) ||
      overlap(out, rows, tail->weight_dev, row) ||
      (tail->h_out_dev != tail->h_dev && overlap(tail->h_out_dev, rows, tail->h_dev, rows)))
    return fail(HSMOE_ERR_ARG, "%s: norm_out overlaps another operand (or h_out partly overlaps h)", name);
  return HSMOE_OK;
}

}  // namespace

extern "C" int hsmoe_moe_layer_decode_norm(const void* x, int64_t m, int64_t d, int64_t i, const void* gate_w,
                                           const float* gate_bias, int64_t n_experts, int top_k,
                                           float routed_scaling, const uint64_t* expert_table, int scale_kind,
                                           const uint64_t* shared, float swiglu_limit, int64_t* topk_idx_out,
                                           float* topk_w_out, void* logits_out, float* out_f32, void* out_bf16,
                                           const hsmoe_norm_tail* tail, void* workspace, size_t workspace_bytes,
                                           hsmoe_stream_t stream) {
  const char* name = "hsmoe_moe_layer_decode_norm";
  int rc = check_layer_args(name, x, m, d, i, gate_w, n_experts, top_k, expert_table, scale_kind, topk_idx_out,
                            topk_w_out, out_f32, out_bf16, false, true);
  if (rc) return rc;
  if ((rc = check_tail(name, tail, x, m, d))) return rc;
  const size_t need = hsmoe_moe_layer_workspace_size(m, d, i, n_experts, top_k);
  if (!workspace || workspace_bytes < need || !aligned(workspace, 256))
    return fail(HSMOE_ERR_WORKSPACE, "%s: zero-filled workspace of %zu bytes (256-byte aligned) needed", name, need);
  return launch_layer(name, x, m, d, i, gate_w, gate_bias, n_experts, top_k, routed_scaling, expert_table,
                      scale_kind, shared, swiglu_limit, topk_idx_out, topk_w_out, logits_out, out_f32, out_bf16,
                      workspace, workspace_bytes, nullptr, (hipStream_t)stream, nullptr, tail);
}

extern "C" int hsmoe_moe_layer_decode_routed_norm(const void* x, int64_t m, int64_t d, int64_t i,
                                                  const int64_t* topk_idx, const int64_t* token_ids,
                                                  int64_t table_rows, const float* topk_w, float weight_all,
                                                  int top_k, const uint64_t* expert_table, int64_t n_experts,
                                                  int scale_kind, const uint64_t* shared, float swiglu_limit,
                                                  float* out_f32, void* out_bf16, const hsmoe_norm_tail* tail,
                                                  void* workspace, size_t workspace_bytes, hsmoe_stream_t stream) {
  const char* name = "hsmoe_moe_layer_decode_routed_norm";
  if (!topk_idx) return fail(HSMOE_ERR_ARG, "%s: null topk_idx", name);
  if (token_ids && table_rows < 1) return fail(HSMOE_ERR_ARG, "%s: a token table needs table_rows >= 1", name);
  int rc = check_layer_args(name, x, m, d, i, nullptr, n_experts, top_k, expert_table, scale_kind, nullptr, nullptr,
                            out_f32, out_bf16, true, true);
  if (rc) return rc;
  if ((rc = check_tail(name, tail, x, m, d))) return rc;
  const size_t need = hsmoe_moe_layer_workspace_size(m, d, i, n_experts, top_k);
  if (!workspace || workspace_bytes < need || !aligned(workspace, 256))
    return fail(HSMOE_ERR_WORKSPACE, "%s: zero-filled workspace of %zu bytes (256-byte aligned) needed", name, need);
  const GivenRoute route{topk_idx, token_ids, token_ids ? table_rows : 0, topk_w, weight_all};
  return launch_layer(name, x, m, d, i, nullptr, nullptr, n_experts, top_k, 1.0f, expert_table, scale_kind, shared,
                      swiglu_limit, nullptr, nullptr, nullptr, out_f32, out_bf16, workspace, workspace_bytes, nullptr,
                      (hipStream_t)stream, &route, tail);
}

// Scratch of hsmoe_moe_layer_decode_noalloc: the workspace of every call of
// that entry point on one GPU.  Each GPU the library runs on holds its own
// copy, at its own address, until the process ends; it starts zeroed (static
// storage) and every launch leaves it ready for the next one.  In host code
// `scratch` names a host-side stand-in, not device memory: host code uses only
// the address hipGetSymbolAddress gives for the current device (g_scratch).
static __device__ __align__(256) unsigned char scratch[HSMOE_LAYER_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

// The current device's copy of `scratch`, looked up once per device (with the
// device current) and cleared on `stream` at that first call.
int device_scratch(const char* name, hipStream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(HSMOE_ERR_LAUNCH, "%s: no current device (or device index >= %d)", name, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(HSMOE_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", name, dev,
                  hipGetErrorString(e));
    const int64_t n = (int64_t)(HSMOE_LAYER_SCRATCH_BYTES / 16);
    hipLaunchKernelGGL(clear_kernel, dim3(1024), dim3(256), 0, stream, (uint4*)ptr, n);
    const int rc = check_launch(name);
    if (rc) return rc;
    g_scratch[dev] = ptr;
  }
  *out = g_scratch[dev];
  return HSMOE_OK;
}
}  // namespace

extern "C" int hsmoe_moe_layer_decode_noalloc(const void* x, int64_t m, int64_t d, int64_t i, const void* gate_w,
                                              const float* gate_bias, int64_t n_experts, int top_k,
                                              float routed_scaling, const uint64_t* expert_table, int scale_kind,
                                              const uint64_t* shared, float swiglu_limit, int64_t* topk_idx_out,
                                              float* topk_w_out, void* logits_out, float* out_f32, void* out_bf16,
                                              uint32_t* status_out, hsmoe_stream_t stream) {
  const char* name = "hsmoe_moe_layer_decode_noalloc";
  int rc = check_layer_args(name, x, m, d, i, gate_w, n_experts, top_k, expert_table, scale_kind, topk_idx_out,
                            topk_w_out, out_f32, out_bf16);
  if (rc) return rc;
  if (!status_out || !aligned(status_out, 4)) return fail(HSMOE_ERR_ARG, "%s: status_out must be a device uint32", name);
  const size_t need = hsmoe_moe_layer_workspace_size(m, d, i, n_experts, top_k);
  if (need > HSMOE_LAYER_SCRATCH_BYTES)
    return fail(HSMOE_ERR_WORKSPACE,
                "%s: this shape needs %zu bytes of scratch, more than the %zu the library holds per GPU "
                "(use hsmoe_moe_layer_decode with a workspace)", name, need, (size_t)HSMOE_LAYER_SCRATCH_BYTES);
  void* ws = nullptr;
  rc = device_scratch(name, (hipStream_t)stream, &ws);
  if (rc) return rc;
  return launch_layer(name, x, m, d, i, gate_w, gate_bias, n_experts, top_k, routed_scaling, expert_table,
                      scale_kind, shared, swiglu_limit, topk_idx_out, topk_w_out, logits_out, out_f32, out_bf16, ws,
                      HSMOE_LAYER_SCRATCH_BYTES, (unsigned*)status_out, (hipStream_t)stream);
}

extern "C" size_t hsmoe_moe_layer_status_offset(void) { return (size_t)kCtlErr * 4; }
