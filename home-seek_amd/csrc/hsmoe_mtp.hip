// lm_head logits + greedy argmax + longest-prefix draft acceptance.
//
// Restates the verify tail of _mtp_verify_batched (engine.py:2480-2497):
//   logits = bf16(h . lm_head^T); pred[t] = argmax(logits[t]) (first index
//   on ties, as torch.argmax); accept combined_ids[t+1] while it equals
//   pred[t]; the bonus row is the first mismatch (or the last row).
// Each logit is the correctly rounded bf16 of the exact dot product (bf16 x
// bf16 products are exact in fp64, and so are the sums met in practice), in
// one of three forms:
//  - 1 token, d <= 4096: one wave per vocab row, 1 KB per load instruction,
//    the lane's hidden-state columns in fp64 registers, the row's partial
//    sums added across the wave (lm_head_row_kernel);
//  - 2..4 tokens: v_mfma_f64_4x4x4_4b_f64 over 4-row tiles, the bf16 hidden
//    states in LDS (lm_head_mfma_kernel);
//  - 1 token with d > 4096, or 5..8 tokens: one lane per vocab row summing in fp64 FMAs, the
//    hidden states widened to fp64 on their way into LDS when they fit
//    (n_tok * d * 8 <= kLdsHBytes), else widened into the workspace by
//    widen_h_kernel and read from there (lm_head_kernel); the inner loop reads
//    them with broadcast LDS loads instead of scalar loads that stall on the
//    scalar cache; per weight 2 conversions + n_tok fp64 FMAs.
// The vocab-wide argmax is a 64-bit atomic max on (orderable logit, ~index);
// the last workgroup to finish evaluates the acceptance rule and clears the
// counters for the next call.
#include "hsmoe_common.h"
#include "hsmoe_internal.h"

namespace hsmoe {
namespace {

constexpr int kMaxTok = 8;
constexpr int kWaves = 8;
constexpr int kRowsPerBlock = 64 * kWaves;
constexpr size_t kLdsHBytes = 128 * 1024;  // hidden states in LDS up to this size (one workgroup per CU)
constexpr int kMfmaMinTok = 2;  // the fp64 MFMA form serves 2..4 tokens (one token: the row-per-lane form)

struct Workspace {
  unsigned long long key[kMaxTok];
  unsigned int done;
  unsigned int pad;
  // followed (256-byte aligned) by double h64[n_tok][d]
};

inline size_t h64_offset() { return 256; }

__global__ void widen_h_kernel(const uint16_t* __restrict__ h, int64_t n, double* __restrict__ h64) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    h64[i] = (double)bf16_bits_to_f32(h[i]);
}

// Orderable key of a bf16 logit: larger value -> larger key; NaN above all.
__device__ __forceinline__ unsigned long long logit_key(uint32_t bits, int64_t v) {
  uint32_t o = (bits & 0x8000u) ? (~bits & 0xffffu) : (bits | 0x8000u);
  if ((bits & 0x7fffu) > 0x7f80u) o = 0x1ffffu;  // NaN: torch.argmax returns the first NaN
  return ((unsigned long long)o << 32) | (unsigned long long)(0xffffffffu - (uint32_t)v);
}

// The acceptance rule, in the last workgroup to arrive (thread 0): pred[t]
// from the vocab-wide keys (cleared for the next call), the longest prefix of
// ids[1..] equal to pred[0..], the counter re-armed.
template <int kTok>
__device__ void accept_tail(const int64_t* __restrict__ ids, int64_t* __restrict__ pred_out,
                            int64_t* __restrict__ result_out, Workspace* __restrict__ ws) {
  int64_t pred[kTok];
#pragma unroll
  for (int t = 0; t < kTok; ++t) {
    const unsigned long long k = __hip_atomic_exchange(&ws->key[t], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    pred[t] = (int64_t)(0xffffffffu - (uint32_t)(k & 0xffffffffu));
    pred_out[t] = pred[t];
  }
  int64_t n_acc = 0;
  for (int t = 0; t + 1 < kTok; ++t) {
    if (pred[t] != ids[t + 1]) break;
    ++n_acc;
  }
  result_out[0] = n_acc;
  result_out[1] = n_acc;
  __hip_atomic_store(&ws->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------- one token, row per wave
// One token, d = 512 kC <= 4096: a wave takes whole vocab rows, each load
// instruction reading 1 KB of one row (lane l: the 16-byte chunks l, l + 64,
// ...), the form HBM streams fastest (measured on a pure-load copy of the
// 129,280 x 4096 head: 166 us, against 175 for 4 rows x 256 B and 202-216
// for a row per lane).  The lane's columns of the hidden state are widened
// to fp64 once, in registers; each row's partial sums (exact fp64 products,
// summed in chunk then element order) are added across the wave by a
// butterfly, so a logit is the row's exact sum rounded once to bf16 whenever
// that sum is exact in fp64, as for the other forms.  Rows are dealt to
// waves grid-stride; the next row's loads are issued before this row's
// sums.
constexpr int kRowWaves = 4;

__device__ __forceinline__ double bf16_elem(const uint4& q, int e) {
  const uint32_t word = e < 2 ? q.x : e < 4 ? q.y : e < 6 ? q.z : q.w;
  return (double)__uint_as_float((e & 1) ? (word & 0xffff0000u) : (word << 16));
}

template <int kC>
__global__ void __launch_bounds__(64 * kRowWaves)
    lm_head_row_kernel(const uint16_t* __restrict__ w, const uint16_t* __restrict__ hb, int64_t vocab,
                       const int64_t* __restrict__ ids, uint16_t* __restrict__ logits, int64_t* __restrict__ pred_out,
                       int64_t* __restrict__ result_out, Workspace* __restrict__ ws) {
  __shared__ unsigned long long s_key[kRowWaves];
  __shared__ int s_last;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int kRowQ = 64 * kC;  // 16-byte chunks per row
  double hv[kC][8];
#pragma unroll
  for (int j = 0; j < kC; ++j) {
    const uint4 q = reinterpret_cast<const uint4*>(hb)[lane + 64 * j];
#pragma unroll
    for (int e = 0; e < 8; ++e) hv[j][e] = bf16_elem(q, e);
  }
  const uint4* __restrict__ wq = reinterpret_cast<const uint4*>(w) + lane;
  const int64_t nwv = (int64_t)gridDim.x * kRowWaves;
  unsigned long long key = 0;
  auto load = [&](uint4 (&q)[kC], int64_t v) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kC; ++j) q[j] = wq[v * kRowQ + 64 * j];
  };
  auto sum_row = [&](const uint4 (&q)[kC], int64_t v) __attribute__((always_inline)) {
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < kC; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = __fma_rn(hv[j][e], bf16_elem(q[j], e), acc);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
    const uint32_t bits = f64_to_bf16_bits(acc);
    if (lane == 0 && logits) logits[v] = (uint16_t)bits;
    const unsigned long long k1 = logit_key(bits, v);
    key = k1 > key ? k1 : key;
  };
  int64_t v = (int64_t)blockIdx.x * kRowWaves + wave;
  uint4 qa[kC], qb[kC];
  if (v < vocab) load(qa, v);
  // two rows per turn: the row after next is loaded while this one is summed
  while (v < vocab) {
    const int64_t v1 = v + nwv;
    if (v1 < vocab) load(qb, v1);
    sum_row(qa, v);
    if (v1 >= vocab) break;
    const int64_t v2 = v1 + nwv;
    if (v2 < vocab) load(qa, v2);
    sum_row(qb, v1);
    v = v2;
  }
  if (lane == 0) s_key[wave] = key;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long k = 0;
#pragma unroll
    for (int q2 = 0; q2 < kRowWaves; ++q2) k = s_key[q2] > k ? s_key[q2] : k;
    __hip_atomic_fetch_max(&ws->key[0], k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(&ws->done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
  __syncthreads();
  if (s_last && threadIdx.x == 0) accept_tail<1>(ids, pred_out, result_out, ws);
}

template <int kC>
int launch_row(const uint16_t* w, const uint16_t* h, int64_t vocab, const int64_t* ids, uint16_t* logits,
               int64_t* pred, int64_t* result, Workspace* ws, hipStream_t st) {
  // one workgroup of 4 waves per CU: 168-174 us over the 129,280 x 4096 head
  // against 179-180 with two per CU (320 or 384 workgroups, uneven over the
  // CUs: 185-205)
  const int64_t blocks = device_cus();
  const int64_t need = (vocab + kRowWaves - 1) / kRowWaves;
  const unsigned nb = (unsigned)(need < blocks ? need : blocks);
  hipLaunchKernelGGL((lm_head_row_kernel<kC>), dim3(nb), dim3(64 * kRowWaves), 0, st, w, h, vocab, ids, logits, pred,
                     result, ws);
  return check_launch("hsmoe_lm_head_accept");
}

// ------------------------------------------------------------- fp64 MFMA form
// For up to 4 tokens the dot products run on v_mfma_f64_4x4x4_4b_f64: four
// blocks of D (4x4) += A (4x4) B (4x4) in fp64 per instruction, operands
// (fitted on the device) A_b[i][k] in lane 16k + 4b + i, B_b[k][j] in lane
// 16k + 4b + j, D_b[i][j] in lane 16i + 4b + j.  A wave works through tiles
// of 4 vocab rows (A row i = tile row i, lane bits 0..1) against the 4 token
// columns j (tokens past n_tok are zero); the 16 (block, k) pairs of a row
// (lane bits 2..5, "slot") take 16 consecutive 16-byte pieces of it, so one
// load instruction reads 256 contiguous bytes of each of the 4 rows and a
// group of W = kMfmaW loads 256 W bytes per row.  Each block sums its own
// quarter of the columns; at the end of a row the 4 blocks' partials are
// added across lanes.  HBM streams long contiguous runs per row best: 64
// bytes per row and group over 16 rows ran at 4.15 TB/s, 128 bytes at 4.5,
// 1 KB over 4 rows at 4.8.  Tiles are dealt to waves grid-stride (wave w
// takes tiles w, w + waves, ...), so that the grid reads one contiguous
// window of the head at a time (a contiguous run of tiles per wave was ~4%
// slower), with the load pipeline running on across a wave's tiles: the
// next group's loads go out while a group is multiplied (one group ahead:
// 202 us at T = 3 over the 129,280 x 4096 head against 207 with four; the
// same loads with no arithmetic run at 182-187).
// The hidden states sit in LDS as bf16 [4][d]; a B lane reads the same
// columns as its A lane in 16-byte LDS loads.  Products of bf16 values are
// exact in fp64 and every partial sum is a subset sum of a row's products,
// so a logit is the row's exact sum rounded once to bf16 whenever that sum is
// exact in fp64, as for the row-per-lane form.
constexpr int kMfmaWaves = 4;
constexpr int kMfmaW = 4;                  // 16-byte loads per lane and group (8 k each)
constexpr int kMfmaAhead = 1;             // groups in flight per wave (64 bytes per lane)
constexpr int kMfmaGroupCols = 128 * kMfmaW;  // columns of a row per group
constexpr int kMfmaResidentWaves = 4096;   // 256 CUs x 4 SIMDs x 4 waves

__device__ __forceinline__ double bf16_lane(const uint4& q, int n) {
  const uint32_t word = n < 2 ? q.x : n < 4 ? q.y : n < 6 ? q.z : q.w;
  return (double)__uint_as_float((n & 1) ? (word & 0xffff0000u) : (word << 16));
}

template <int kTok>
__global__ void __launch_bounds__(64 * kMfmaWaves)
    lm_head_mfma_kernel(const uint16_t* __restrict__ w, const uint16_t* __restrict__ h, int64_t d, int64_t vocab,
                        const int64_t* __restrict__ ids, uint16_t* __restrict__ logits,
                        int64_t* __restrict__ pred_out, int64_t* __restrict__ result_out,
                        Workspace* __restrict__ ws) {
  extern __shared__ uint16_t s_hb[];  // [4][d] bf16, rows >= kTok zero
  __shared__ unsigned long long s_key[kMfmaWaves][4];
  __shared__ int s_last;
  const int chunks = (int)(d / 8);
  for (int c = threadIdx.x; c < 4 * chunks; c += 64 * kMfmaWaves) {
    const int t = c / chunks;
    reinterpret_cast<uint4*>(s_hb)[c] = t < kTok ? reinterpret_cast<const uint4*>(h)[c] : make_uint4(0, 0, 0, 0);
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lo = lane & 3, slot = lane >> 2;  // A row i / B token j; (block, k) pair
  const int64_t ntile = (vocab + 3) / 4;
  // tiles t0, t0 + nwv, t0 + 2 nwv, ...: at any moment the grid streams one contiguous window of the head
  const int64_t t0 = (int64_t)blockIdx.x * kMfmaWaves + wave, nwv = (int64_t)gridDim.x * kMfmaWaves;
  const int64_t ntw = t0 < ntile ? (ntile - 1 - t0) / nwv + 1 : 0;
  const int ng = (int)(d / kMfmaGroupCols);
  const int64_t nf = ntw * ng;  // (tile, group) steps of this wave
  const uint4* hq = reinterpret_cast<const uint4*>(s_hb + (int64_t)lo * d + 8 * slot);
  auto row_ptr = [&](int64_t t) {  // rows past the end read the last row; their sums are dropped
    const int64_t r = 4 * t + lo < vocab ? 4 * t + lo : vocab - 1;
    return reinterpret_cast<const uint4*>(w + r * d + 8 * slot);
  };
  unsigned long long key = 0;
  uint4 q[kMfmaAhead][kMfmaW];
  int64_t lt = t0;  // tile and group of the next load
  int lg = 0;
  const uint4* lp = row_ptr(lt);
#pragma unroll
  for (int p = 0; p < kMfmaAhead; ++p) {
#pragma unroll
    for (int h2 = 0; h2 < kMfmaW; ++h2) q[p][h2] = p < nf ? lp[16 * (kMfmaW * lg + h2)] : make_uint4(0, 0, 0, 0);
    if (p < nf && ++lg == ng) {
      lg = 0;
      lp = row_ptr(lt += nwv);
    }
  }
  double acc0 = 0.0, acc1 = 0.0;
  int cg = 0;  // group of the step being summed
  int64_t ct = t0;
  for (int64_t f0 = 0; f0 < nf; f0 += kMfmaAhead) {
#pragma unroll
    for (int p = 0; p < kMfmaAhead; ++p) {
      if (f0 + p < nf) {
        const bool more = f0 + p + kMfmaAhead < nf;
#pragma unroll
        for (int h2 = 0; h2 < kMfmaW; ++h2) {
          const uint4 cur = q[p][h2];
          if (more) q[p][h2] = lp[16 * (kMfmaW * lg + h2)];
          const uint4 hv = hq[16 * (kMfmaW * cg + h2)];
#pragma unroll
          for (int n = 0; n < 8; n += 2) {
            acc0 = __builtin_amdgcn_mfma_f64_4x4x4f64(bf16_lane(cur, n), bf16_lane(hv, n), acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f64_4x4x4f64(bf16_lane(cur, n + 1), bf16_lane(hv, n + 1), acc1, 0, 0, 0);
          }
        }
        if (more && ++lg == ng) {
          lg = 0;
          lp = row_ptr(lt += nwv);
        }
        if (++cg == ng) {
          // lane (i, b, j): block b's partial of row 4 ct + i, token j; add the 4 blocks
          double s = acc0 + acc1;
          s = s + __shfl_xor(s, 4, 64);
          s = s + __shfl_xor(s, 8, 64);
          const int64_t v = 4 * ct + (lane >> 4);
          if ((lane & 12) == 0 && lo < kTok && v < vocab) {
            const uint32_t bits = f64_to_bf16_bits(s);
            if (logits) logits[lo * vocab + v] = (uint16_t)bits;
            const unsigned long long k1 = logit_key(bits, v);
            key = k1 > key ? k1 : key;
          }
          acc0 = 0.0;
          acc1 = 0.0;
          cg = 0;
          ct += nwv;
        }
      }
    }
  }
  // the wave's best key of token j: lanes with equal lane & 3
#pragma unroll
  for (int off = 4; off < 64; off <<= 1) {
    const unsigned long long o = __shfl_xor(key, off, 64);
    key = o > key ? o : key;
  }
  if (lane < 4) s_key[wave][lane] = key;
  __syncthreads();
  if (threadIdx.x < kTok) {
    unsigned long long k = 0;
#pragma unroll
    for (int q2 = 0; q2 < kMfmaWaves; ++q2) k = s_key[q2][threadIdx.x] > k ? s_key[q2][threadIdx.x] : k;
    __hip_atomic_fetch_max(&ws->key[threadIdx.x], k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(&ws->done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
  __syncthreads();
  if (s_last && threadIdx.x == 0) accept_tail<kTok>(ids, pred_out, result_out, ws);
}

template <int kTok>
int launch_mfma(const uint16_t* w, const uint16_t* h, int64_t d, int64_t vocab, const int64_t* ids, uint16_t* logits,
                int64_t* pred, int64_t* result, Workspace* ws, hipStream_t st) {
  // every wave resident at once (no more waves than tiles)
  const int64_t ntile = (vocab + 3) / 4;
  const int64_t nw = ntile < kMfmaResidentWaves ? ntile : kMfmaResidentWaves;
  const unsigned nb = (unsigned)((nw + kMfmaWaves - 1) / kMfmaWaves);
  const size_t lds = (size_t)4 * (size_t)d * 2;
  constexpr size_t kMaxLds = (size_t)4 * 8192 * 2;  // d <= 8192: 64 KiB of hidden states, beyond the default
  static bool raised = false;                       // allow it once per instantiation
  if (!raised) {
    if (hipFuncSetAttribute((const void*)lm_head_mfma_kernel<kTok>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)kMaxLds) != hipSuccess)
      return fail(HSMOE_ERR_LAUNCH, "hsmoe_lm_head_accept: could not allow %zu bytes of LDS", kMaxLds);
    raised = true;
  }
  hipLaunchKernelGGL((lm_head_mfma_kernel<kTok>), dim3(nb), dim3(64 * kMfmaWaves), lds, st, w, h, d, vocab, ids,
                     logits, pred, result, ws);
  return check_launch("hsmoe_lm_head_accept");
}

extern __shared__ double s_h[];  // [kTok][d] when kLds

template <int kTok, bool kLds>
__global__ void __launch_bounds__(64 * kWaves)
    lm_head_kernel(const uint16_t* __restrict__ w, const uint16_t* __restrict__ hb, const double* __restrict__ h64g,
                   int64_t d, int64_t vocab, const int64_t* __restrict__ ids, uint16_t* __restrict__ logits,
                   int64_t* __restrict__ pred_out, int64_t* __restrict__ result_out, Workspace* __restrict__ ws) {
  __shared__ unsigned long long s_key[kWaves][kTok];
  __shared__ int s_last;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if constexpr (kLds) {  // the bf16 hidden states widened to fp64 on their way into LDS
    for (int64_t c = threadIdx.x; c < kTok * d; c += 64 * kWaves) s_h[c] = (double)bf16_bits_to_f32(hb[c]);
    __syncthreads();
  }
  const double* __restrict__ h64 = kLds ? s_h : h64g;
  const int64_t v = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x;
  const bool on = v < vocab;
  const uint16_t* wr = w + (on ? v : 0) * d;
  double acc[kTok];
#pragma unroll
  for (int t = 0; t < kTok; ++t) acc[t] = 0.0;
  // 8 x 16 B of the row (64 weights) per lane, summed in k order
  auto consume = [&](const uint4 (&q)[8], int64_t k0) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint32_t qq[4] = {q[b].x, q[b].y, q[b].z, q[b].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t bits = (e & 1) ? (qq[e >> 1] & 0xffff0000u) : (qq[e >> 1] << 16);
        const double wv = (double)__uint_as_float(bits);
#pragma unroll
        for (int t = 0; t < kTok; ++t) acc[t] = __fma_rn(h64[t * d + k0 + 8 * b + e], wv, acc[t]);
      }
    }
  };
  auto load = [&](uint4 (&q)[8], int64_t k0) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < 8; ++b) q[b] = *reinterpret_cast<const uint4*>(wr + k0 + 8 * b);
  };
  uint4 qa[8], qb[8];
  if constexpr (kTok == 1) {
    // one token: little arithmetic per byte, so the next 64 weights are
    // loaded while the current ones are summed (measured: 189 -> 181 us for
    // a 129,280 x 4096 head)
    load(qa, 0);
    for (int64_t k0 = 0; k0 < d; k0 += 128) {  // d is a multiple of 512
      load(qb, k0 + 64);
      consume(qa, k0);
      if (k0 + 128 < d) load(qa, k0 + 128);
      consume(qb, k0 + 64);
    }
  } else {
    // several tokens: the FMAs dominate; 128 weights loaded per step, then
    // summed (measured at 3 tokens: 269 -> 260 us; the pipelined form above
    // runs out of registers there)
    for (int64_t k0 = 0; k0 < d; k0 += 128) {
      load(qa, k0);
      load(qb, k0 + 64);
      consume(qa, k0);
      consume(qb, k0 + 64);
    }
  }
#pragma unroll
  for (int t = 0; t < kTok; ++t) {
    const uint32_t bits = f64_to_bf16_bits(acc[t]);
    if (on && logits) logits[t * vocab + v] = (uint16_t)bits;
    unsigned long long k = on ? logit_key(bits, v) : 0ull;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      unsigned long long o = __shfl_xor(k, off, 64);
      k = o > k ? o : k;
    }
    if (lane == 0) s_key[wave][t] = k;
  }
  __syncthreads();
  // Argmax keys and the arrival counter are agent-scope atomics (coherent across
  // XCDs); each block waits for its atomics to complete before it arrives.
  if (threadIdx.x < kTok) {
    unsigned long long k = 0;
#pragma unroll
    for (int q = 0; q < kWaves; ++q) k = s_key[q][threadIdx.x] > k ? s_key[q][threadIdx.x] : k;
    __hip_atomic_fetch_max(&ws->key[threadIdx.x], k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(&ws->done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
  __syncthreads();
  if (!s_last || threadIdx.x != 0) return;
  accept_tail<kTok>(ids, pred_out, result_out, ws);
}

// h: bf16 [kTok][d]; h64: workspace for their fp64 copy, used (and filled by
// widen_h_kernel) only when they do not fit in LDS.
template <int kTok>
int launch(const uint16_t* w, const uint16_t* h, double* h64, int64_t d, int64_t vocab, const int64_t* ids,
           uint16_t* logits, int64_t* pred, int64_t* result, Workspace* ws, hipStream_t st) {
  const unsigned nb = (unsigned)((vocab + kRowsPerBlock - 1) / kRowsPerBlock);
  const size_t lds = (size_t)kTok * (size_t)d * 8;
  if (lds <= kLdsHBytes) {
    static bool raised = false;  // allow more than the default dynamic LDS (once per process)
    if (!raised) {
      if (hipFuncSetAttribute((const void*)lm_head_kernel<kTok, true>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)kLdsHBytes) != hipSuccess)
        return fail(HSMOE_ERR_LAUNCH, "hsmoe_lm_head_accept: could not allow %zu bytes of LDS", kLdsHBytes);
      raised = true;
    }
    hipLaunchKernelGGL((lm_head_kernel<kTok, true>), dim3(nb), dim3(64 * kWaves), lds, st, w, h, h64, d, vocab, ids,
                       logits, pred, result, ws);
  } else {
    hipLaunchKernelGGL(widen_h_kernel, dim3((unsigned)((kTok * d + 255) / 256)), dim3(256), 0, st, h, kTok * d, h64);
    const int rc = check_launch("hsmoe_lm_head_accept(widen)");
    if (rc) return rc;
    hipLaunchKernelGGL((lm_head_kernel<kTok, false>), dim3(nb), dim3(64 * kWaves), 0, st, w, h, h64, d, vocab, ids,
                       logits, pred, result, ws);
  }
  return check_launch("hsmoe_lm_head_accept");
}

}  // namespace
}  // namespace hsmoe

using namespace hsmoe;

extern "C" size_t hsmoe_lm_head_workspace_size(int64_t n_tok, int64_t vocab) {
  (void)vocab;
  if (n_tok < 1 || n_tok > kMaxTok) return 0;
  return h64_offset() + (size_t)n_tok * 8 * 8192;  // room for d <= 8192
}

extern "C" int hsmoe_lm_head_accept(const void* h, const void* lm_head, int64_t n_tok, int64_t d, int64_t vocab,
                                    const int64_t* ids, void* logits_out, int64_t* pred_out, int64_t* result_out,
                                    void* workspace, size_t workspace_bytes, hsmoe_stream_t stream) {
  if (!h || !lm_head || !pred_out || !result_out || vocab < 1 || d < 1)
    return fail(HSMOE_ERR_ARG, "hsmoe_lm_head_accept: null pointer or bad size");
  if (n_tok < 1 || n_tok > kMaxTok) return fail(HSMOE_ERR_SHAPE, "hsmoe_lm_head_accept: n_tok must be in [1, 8]");
  if (n_tok > 1 && !ids) return fail(HSMOE_ERR_ARG, "hsmoe_lm_head_accept: ids required when n_tok > 1");
  if (d % 512 != 0 || d > 8192 || !aligned(lm_head, 16))
    return fail(HSMOE_ERR_SHAPE, "hsmoe_lm_head_accept: d must be a multiple of 512 (<= 8192), lm_head 16-byte aligned");
  if (vocab >= 0xffffffffll) return fail(HSMOE_ERR_SHAPE, "hsmoe_lm_head_accept: vocab too large");
  if (!workspace || workspace_bytes < hsmoe_lm_head_workspace_size(n_tok, vocab) || !aligned(workspace, 256))
    return fail(HSMOE_ERR_WORKSPACE, "hsmoe_lm_head_accept: zero-filled 256-byte aligned workspace of %zu bytes needed",
                hsmoe_lm_head_workspace_size(n_tok, vocab));
  hipStream_t st = (hipStream_t)stream;
  Workspace* ws = (Workspace*)workspace;
  const uint16_t* w = (const uint16_t*)lm_head;
  uint16_t* lg = (uint16_t*)logits_out;
  if (n_tok >= kMfmaMinTok && n_tok <= 4 && aligned(h, 16)) {
    const uint16_t* hb = (const uint16_t*)h;
    switch (n_tok) {
      case 1: return launch_mfma<1>(w, hb, d, vocab, ids, lg, pred_out, result_out, ws, st);
      case 2: return launch_mfma<2>(w, hb, d, vocab, ids, lg, pred_out, result_out, ws, st);
      case 3: return launch_mfma<3>(w, hb, d, vocab, ids, lg, pred_out, result_out, ws, st);
      default: return launch_mfma<4>(w, hb, d, vocab, ids, lg, pred_out, result_out, ws, st);
    }
  }
  if (n_tok == 1 && d <= 4096 && aligned(h, 16)) {  // one token: row per wave (d > 4096: row per lane)
    const uint16_t* hb = (const uint16_t*)h;
    switch (d / 512) {
      case 1: return launch_row<1>(w, hb, vocab, ids, lg, pred_out, result_out, ws, st);
      case 2: return launch_row<2>(w, hb, vocab, ids, lg, pred_out, result_out, ws, st);
      case 3: return launch_row<3>(w, hb, vocab, ids, lg, pred_out, result_out, ws, st);
      case 4: return launch_row<4>(w, hb, vocab, ids, lg, pred_out, result_out, ws, st);
      case 5: return launch_row<5>(w, hb, vocab, ids, lg, pred_out, result_out, ws, st);
      case 6: return launch_row<6>(w, hb, vocab, ids, lg, pred_out, result_out, ws, st);
      case 7: return launch_row<7>(w, hb, vocab, ids, lg, pred_out, result_out, ws, st);
      default: return launch_row<8>(w, hb, vocab, ids, lg, pred_out, result_out, ws, st);
    }
  }
  double* h64 = (double*)((char*)workspace + h64_offset());
  const uint16_t* hb = (const uint16_t*)h;
  switch (n_tok) {
    case 1: return launch<1>(w, hb, h64, d, vocab, ids, lg, pred_out, result_out, ws, st);
    case 2: return launch<2>(w, hb, h64, d, vocab, ids, lg, pred_out, result_out, ws, st);
    case 3: return launch<3>(w, hb, h64, d, vocab, ids, lg, pred_out, result_out, ws, st);
    case 4: return launch<4>(w, hb, h64, d, vocab, ids, lg, pred_out, result_out, ws, st);
    case 5: return launch<5>(w, hb, h64, d, vocab, ids, lg, pred_out, result_out, ws, st);
    case 6: return launch<6>(w, hb, h64, d, vocab, ids, lg, pred_out, result_out, ws, st);
    case 7: return launch<7>(w, hb, h64, d, vocab, ids, lg, pred_out, result_out, ws, st);
    default: return launch<8>(w, hb, h64, d, vocab, ids, lg, pred_out, result_out, ws, st);
  }
}

namespace hsmoe {
namespace {

constexpr int kMaxDraftsRecorded = 15;

// One decode step's emission at temperature 0 (engine.py:2862-2922), from the
// verify's decisions: tokens = [a, d_0 .. d_{n-1}] (the verify's input ids),
// pred = the verify's argmax per row, result = (n_accept, bonus_row):
//   row   = [a, d_0 .. d_{n-1}, pred[bonus_row]]
//   count = 1 + (n_accept > 0) * (n_accept + 1)   tokens emitted
//   next  = pred[bonus_row] if n_accept > 0 else a
// Without drafts (n = 0; pred, result unused): row = [a], count 1, next a.
// Thread 0 writes the single-step outputs that are given and, with `rows`,
// row k of rows [capacity][width] (width n + 2, or 1), counts[k] and
// n_accepts[k], then *cur = next and *k = k + 1; a k outside [0, capacity)
// writes no row.
__global__ void __launch_bounds__(64)
    step_record_kernel(const int64_t* tokens, int n, const int64_t* pred, const int64_t* result, int64_t* row_out,
                       int64_t* count_out, int64_t* next_out, int64_t* nacc_out, int64_t* rows, int64_t* counts,
                       int64_t* naccs, int64_t* k, int64_t capacity, int64_t* cur) {
  if (threadIdx.x != 0) return;
  const int64_t a = tokens[0];
  int64_t nacc = 0, bonus = a;
  if (n > 0) {
    nacc = result[0];
    const int64_t br = result[1] < 0 ? 0 : (result[1] > n ? n : result[1]);
    bonus = pred[br];
  }
  const int width = n > 0 ? n + 2 : 1;
  const int64_t count = nacc > 0 ? nacc + 2 : 1;
  const int64_t next = nacc > 0 ? bonus : a;
  const int64_t kk = rows ? *k : -1;
  const bool keep = rows && kk >= 0 && kk < capacity;
  for (int j = 0; j < width; ++j) {
    const int64_t v = j == 0 ? a : (j <= n ? tokens[j] : bonus);
    if (row_out) row_out[j] = v;
    if (keep) rows[kk * width + j] = v;
  }
  if (count_out) *count_out = count;
  if (next_out) *next_out = next;
  if (nacc_out) *nacc_out = nacc;
  if (keep) {
    counts[kk] = count;
    naccs[kk] = nacc;
  }
  if (rows) *k = kk + 1;
  if (cur) *cur = next;
}

}  // namespace
}  // namespace hsmoe

extern "C" int hsmoe_decode_step_record(const int64_t* tokens, int64_t n_draft, const int64_t* pred,
                                        const int64_t* result, int64_t* row_out, int64_t* count_out,
                                        int64_t* next_out, int64_t* n_accept_out, int64_t* rows, int64_t* counts,
                                        int64_t* n_accepts, int64_t* k, int64_t capacity, int64_t* cur,
                                        hsmoe_stream_t stream) {
  using namespace hsmoe;
  if (!tokens || n_draft < 0 || n_draft > kMaxDraftsRecorded || (n_draft > 0 && (!pred || !result)))
    return fail(HSMOE_ERR_ARG, "hsmoe_decode_step_record: tokens, 0 <= n_draft <= %d, and pred + result with drafts",
                kMaxDraftsRecorded);
  if (rows && (!counts || !n_accepts || !k || capacity < 1))
    return fail(HSMOE_ERR_ARG, "hsmoe_decode_step_record: rows need counts, n_accepts, k and capacity >= 1");
  hipLaunchKernelGGL(step_record_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, tokens, (int)n_draft, pred,
                     result, row_out, count_out, next_out, n_accept_out, rows, counts, n_accepts, k, capacity, cur);
  return check_launch("hsmoe_decode_step_record");
}
