// Routed-expert SwiGLU FFN for many tokens (prefill): a grouped GEMM over the
// experts the tokens select, each expert's weights streamed from HBM once per
// chunk of its tokens (gate/up: up to 32, or 64 for an expert with more than
// 32; down: up to 32).
//
// Restates FusedMoEFFN._forward_legacy at B > 8 and the FP4 grouped route of
// fused_expert_ffn_triton (fused_moe.py:269-380, 458-551) plus the shared
// expert add of _forward_ffn (engine.py:1530-1536), with the arithmetic of
// the decode kernels:
//   gate = x W1^T, up = x W3^T (fp32 accumulation of exact bf16 products);
//   a = w * min(g,L) sigmoid(min(g,L)) clamp(u,-L,L);  y = a W2^T
//   out[t] = sum_j y[t, j] (slot order) + shared(t)
// W = bf16(dequant(FP4)) decoded in registers; the activation enters the down
// GEMM as a bf16 hi + lo pair.  Unlike the reference's dense union GEMM
// (every token through every selected expert), only the (token, expert) pairs
// that routing selects are computed.
//
// Launches (no host synchronisation):
//   group    workgroup e buckets the pairs (t, j) routed to expert e, in (t, j)
//            order (stable, deterministic); one more workgroup places the
//            shared expert's M pairs.  Each bucket is cut into gate/up chunks
//            (<= 32 pairs, or <= 64 for a bucket of more than 32, those first)
//            and into down chunks of <= 32 pairs.
//   gate_up  grid (chunk, 64-row block of I), one launch for the routed
//            experts and one for the shared expert: wave w takes rows
//            +16w..+16 of W1 and W3 over all of D in K-chunks of 256 columns.
//            While chunk kc is multiplied, the token tile of kc+1 is in flight
//            to registers (then LDS) and the weights of kc+2 to a third
//            register buffer (a 64-pair chunk: no weights ahead, for the
//            registers of its four token tiles).  Writes the weighted
//            activation (hi, lo).
//   down     grid (chunk, 128-row block of D), same pipeline over W2 (32 rows
//            per wave) with the activation tile (hi and lo planes); writes one
//            fp32 partial row per pair (no atomics).
//   combine  out[t] = partials of t's pairs in slot order, then the shared one.
// The grids are sized for the most chunks the routing can produce; workgroups
// past the actual count (read from the workspace) exit at once.
#include <math.h>

#include "hsmoe_common.h"
#include "hsmoe_internal.h"
#include "hsmoe_tiles.h"

namespace hsmoe {
namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 32;        // tokens per chunk (two 16-token MFMA tiles)
constexpr int kBigChunk = 64;     // tokens per chunk of an expert with more than kChunk pairs
constexpr int kGuRT = 1;          // 16-row tiles per wave, gate/up (W1 and W3)
constexpr int kDnRT = 2;          // 16-row tiles per wave, down (W2)
constexpr int kGuRows = 64 * kGuRT;  // weight rows per workgroup
constexpr int kDnRows = 64 * kDnRT;
constexpr int kCols = 256;        // columns per K-chunk (2 steps of 128)
constexpr int kPad = 8;           // bf16 elements of padding per LDS row
constexpr int kMaxPairs = 12288;  // m * top_k per call (LDS of the group kernel)
constexpr int kMaxExperts = 1024;

struct Header {
  int n_routed_chunks;  // gate/up chunks of routed experts (big experts' first); the shared expert's follow
  int n_pairs;
  int n_dn_chunks;      // down chunks of routed experts (kChunk pairs each); the shared expert's follow
};

struct PrefillParams {
  const uint16_t* x;       // bf16 [m, d]
  const int64_t* idx;      // [m, top_k]
  const float* wts;        // [m, top_k]
  const uint64_t* table;   // [n_experts][6]
  const uint64_t* shared;  // [6] or null
  Header* hdr;
  int* pair_tok;           // [max_pairs] token of pair p
  float* pair_w;           // [max_pairs] routing weight of pair p
  int* pidx;               // [m][top_k + 1] pair of (t, j); j = top_k: shared; -1 = none
  int* chunk_e;            // [max_chunks] expert (n_experts = shared)
  int* chunk_p0;           // [max_chunks] first pair
  int* chunk_n;            // [max_chunks] pairs in the chunk
  int* dn_e;               // [max_chunks] down chunks: every expert's pairs in chunks of kChunk
  int* dn_p0;
  int* dn_n;
  uint16_t* act_hi;        // bf16 [max_pairs][i]
  uint16_t* act_lo;        // bf16 [max_pairs][i]
  float* part;             // fp32 [max_pairs][d]
  float* out_f32;          // [m, d] or null
  uint16_t* out_bf16;      // [m, d] or null
  int n_experts;
  int m, d, i, top_k;
  int scale_fmt;  // kFp4E8M0 or kFp4F32 for routed FP4 experts
  float limit;
};

// ---------------------------------------------------------------- group
// Pairs per gate/up chunk of an expert with cnt pairs: an expert with more
// than kChunk pairs is cut into chunks of kBigChunk, so that its W1 and W3
// are streamed half as often; big experts' chunks come first, so that the
// longer workgroups start first.  The down pass keeps chunks of kChunk (its
// token tile's size), in expert order: a second list.
__device__ __forceinline__ int chunk_size(int cnt) { return cnt > kChunk ? kBigChunk : kChunk; }

// Sum over the block of v (every thread passes its own value).
__device__ __forceinline__ int block_sum(int v, int* s_red) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
  __syncthreads();
  int t = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) t += s_red[w];
  return t;
}

// Workgroup e < n_experts places the pairs of expert e; workgroup n_experts
// writes the header, the shared expert's pairs and the slots of invalid ids.
// Every workgroup histograms the whole pair list in LDS, so the offsets of
// expert e (pairs and chunks of the experts before it) need no second pass.
// Within an expert, pairs keep (t, j) order: blocks of 256 pairs in order,
// ranked by wave ballots.
__global__ void __launch_bounds__(kThreads) prefill_group_kernel(PrefillParams p) {
  __shared__ int s_e[kMaxPairs];
  __shared__ int s_cnt[kMaxExperts];
  __shared__ bool s_ok[kMaxExperts];  // expert e has a table entry
  __shared__ int s_red[kThreads / 64];
  __shared__ int s_wc[kThreads / 64];
  const int E = p.n_experts, K = p.top_k, P = p.m * K, me = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // which experts have a table entry: one load per expert, not one per pair
  for (int e = threadIdx.x; e < E; e += kThreads) {
    s_cnt[e] = 0;
    s_ok[e] = p.table[(int64_t)e * 6] != 0;
  }
  __syncthreads();
  // the pair ids, kIdBatch loads of a thread in flight at once
  constexpr int kIdBatch = 8;
  for (int q0 = threadIdx.x; q0 < P; q0 += kIdBatch * kThreads) {
    int64_t ev[kIdBatch];
#pragma unroll
    for (int j = 0; j < kIdBatch; ++j) ev[j] = q0 + j * kThreads < P ? p.idx[q0 + j * kThreads] : -1;
#pragma unroll
    for (int j = 0; j < kIdBatch; ++j) {
      const int q = q0 + j * kThreads;
      if (q >= P) break;
      const int64_t e = ev[j];
      const bool ok = e >= 0 && e < E && s_ok[e];
      s_e[q] = ok ? (int)e : -1;
      if (ok) atomicAdd(&s_cnt[e], 1);
    }
  }
  __syncthreads();
  if (me == E) {
    int pairs = 0, chunks = 0, dchunks = 0;
    for (int e = threadIdx.x; e < E; e += kThreads) {
      pairs += s_cnt[e];
      chunks += (s_cnt[e] + chunk_size(s_cnt[e]) - 1) / chunk_size(s_cnt[e]);
      dchunks += (s_cnt[e] + kChunk - 1) / kChunk;
    }
    pairs = block_sum(pairs, s_red);
    chunks = block_sum(chunks, s_red);
    dchunks = block_sum(dchunks, s_red);
    if (threadIdx.x == 0) {
      p.hdr->n_pairs = pairs + (p.shared ? p.m : 0);
      p.hdr->n_routed_chunks = chunks;
      p.hdr->n_dn_chunks = dchunks;
    }
    for (int q = threadIdx.x; q < P; q += kThreads)
      if (s_e[q] < 0) p.pidx[(q / K) * (K + 1) + q % K] = -1;
    for (int t = threadIdx.x; t < p.m; t += kThreads) {
      const int pos = pairs + t;
      p.pidx[t * (K + 1) + K] = p.shared ? pos : -1;
      if (!p.shared) continue;
      p.pair_tok[pos] = t;
      p.pair_w[pos] = 1.0f;
      if (t % kChunk == 0) {
        const int ch = chunks + t / kChunk, dch = dchunks + t / kChunk;
        p.chunk_e[ch] = p.dn_e[dch] = E;
        p.chunk_p0[ch] = p.dn_p0[dch] = pos;
        p.chunk_n[ch] = p.dn_n[dch] = min(kChunk, p.m - t);
      }
    }
    return;
  }
  const int cnt = s_cnt[me];
  if (cnt == 0) return;  // uniform across the workgroup
  // chunks: the big experts' (expert order), then one per small expert (expert order)
  const bool big = cnt > kChunk;
  int off = 0, choff = 0, dnoff = 0;
  for (int e = threadIdx.x; e < E; e += kThreads) {
    const int c = s_cnt[e];
    if (e < me) off += c;
    if (e < me) dnoff += (c + kChunk - 1) / kChunk;
    if (c > kChunk && (!big || e < me)) choff += (c + kBigChunk - 1) / kBigChunk;  // every big expert's chunks first
    else if (!big && e < me && c > 0) ++choff;
  }
  off = block_sum(off, s_red);
  choff = block_sum(choff, s_red);
  dnoff = block_sum(dnoff, s_red);
  const int cs = chunk_size(cnt);
  int base = off;
  for (int q0 = 0; q0 < P; q0 += kThreads) {
    const int q = q0 + threadIdx.x;
    const bool hit = q < P && s_e[q] == me;
    const unsigned long long bal = __ballot(hit);
    if (lane == 0) s_wc[wave] = __popcll(bal);
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {
      before += w < wave ? s_wc[w] : 0;
      total += s_wc[w];
    }
    if (hit) {
      const int pos = base + before + __popcll(bal & ((1ull << lane) - 1ull));
      p.pair_tok[pos] = q / K;
      p.pair_w[pos] = p.wts[q];
      p.pidx[(q / K) * (K + 1) + q % K] = pos;
    }
    base += total;
    __syncthreads();
  }
  for (int c = threadIdx.x; c * cs < cnt; c += kThreads) {
    p.chunk_e[choff + c] = me;
    p.chunk_p0[choff + c] = off + c * cs;
    p.chunk_n[choff + c] = min(cs, cnt - c * cs);
  }
  for (int c = threadIdx.x; c * kChunk < cnt; c += kThreads) {
    p.dn_e[dnoff + c] = me;
    p.dn_p0[dnoff + c] = off + c * kChunk;
    p.dn_n[dnoff + c] = min(kChunk, cnt - c * kChunk);
  }
}

// B operand (16 token columns x 32 k) from an LDS tile [kChunk][cols + kPad]:
// lane (c, g) takes token tile*16 + c, columns 128*st + 32g + 8j .. +8.
__device__ __forceinline__ bf16x8 tile_frag(const uint16_t* t, int cols, int tile, int c, int g, int st, int j) {
  return *reinterpret_cast<const bf16x8*>(t + (tile * 16 + c) * (cols + kPad) + st * 128 + g * 32 + 8 * j);
}

struct Chunk {
  int e, p0, n;
  const uint64_t* ent;
};

// Chunk q of the routed experts (kShared = false) or of the shared expert,
// from the gate/up list or (kDown) the down list.
template <bool kShared, bool kDown>
__device__ __forceinline__ bool load_chunk(const PrefillParams& p, int q, Chunk& ch) {
  const int nr = kDown ? p.hdr->n_dn_chunks : p.hdr->n_routed_chunks;
  if (kShared) {
    if (q * kChunk >= p.m) return false;
    q += nr;
  } else if (q >= nr) {
    return false;
  }
  ch.e = kDown ? p.dn_e[q] : p.chunk_e[q];
  ch.p0 = kDown ? p.dn_p0[q] : p.chunk_p0[q];
  ch.n = kDown ? p.dn_n[q] : p.chunk_n[q];
  ch.ent = kShared ? p.shared : p.table + (int64_t)ch.e * 6;
  return true;
}

// This thread's share of a token tile [kC][kCols] of kPlanes planes,
// held in registers between its global loads and its LDS store.  Rows past
// the chunk's n tokens are zero and never loaded.
template <int kPlanes, int kC>
struct XStage {
  static constexpr int kPer = kC * kCols / 8 / kThreads;  // uint4 per thread and plane
  uint4 v[kPlanes][kPer];
  template <typename Src>
  __device__ __forceinline__ void load(Src& src, int kc, int n) {
#pragma unroll
    for (int pl = 0; pl < kPlanes; ++pl)
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int q = threadIdx.x + u * kThreads, tt = q / (kCols / 8), cc = q % (kCols / 8);
        v[pl][u] = tt < n ? ldg<uint4>(src(pl, tt) + kc * kCols + cc * 8) : make_uint4(0, 0, 0, 0);
      }
  }
  __device__ __forceinline__ void store(uint16_t* lds) const {
#pragma unroll
    for (int pl = 0; pl < kPlanes; ++pl)
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int q = threadIdx.x + u * kThreads, tt = q / (kCols / 8), cc = q % (kCols / 8);
        *reinterpret_cast<uint4*>(lds + pl * kC * (kCols + kPad) + tt * (kCols + kPad) + cc * 8) = v[pl][u];
      }
  }
};

// The weights of one K-chunk for a wave: kMats matrices x kRT row tiles.
template <int F, int kMats, int kRT>
struct WBuf {
  static constexpr int kSteps = kCols / 128;
  Batch<F, kSteps> b[kMats][kRT];
  __device__ __forceinline__ void load(const Mat (&mats)[kMats], int row, int k, int kc, int g) {
#pragma unroll
    for (int q = 0; q < kMats; ++q)
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) b[q][rt].load(mats[q], row + 16 * rt, k, kc * kSteps, g);
  }
};

// Software pipeline over K-chunks of the kMats matrices ([n_rows][k]) at
// ent[w_slot], ent[w_slot + 2], ...  While chunk kc is multiplied, the token
// tile of kc + 1 is in flight to registers and the weights of kc + 2 to the
// third weight buffer; the tile loads are issued before the weight loads.
// Buffers rotate statically (three steps per loop turn).
// kC: token tile rows; kBufs: weight buffers (3: the weights of kc + 2 in
// flight, 2: those of kc + 1, 1: none ahead, for the larger token tile's
// register budget).
template <int F, int kMats, int kRT, int kPlanes, int kC, int kBufs, typename Src, typename Mul>
__device__ __forceinline__ void pipeline(const uint64_t* ent, int w_slot, int n_rows, int row, int k, int g, int n,
                                         uint16_t* lds, Src&& src, Mul&& mul) {
  using W = WBuf<F, kMats, kRT>;
  const int nkc = k / kCols;
  Mat mats[kMats];
#pragma unroll
  for (int q = 0; q < kMats; ++q) mats[q] = make_mat<F>(ent[w_slot + 2 * q], ent[w_slot + 2 * q + 1], n_rows, k);
  XStage<kPlanes, kC> xr;
  if constexpr (F == kBf16 || kBufs == 1) {
    // bf16 weights (a compatibility format, 4x the bytes), or one buffer
    // asked for: no weight prefetch, so that this path never raises the
    // kernel's registers
    W w;
    for (int kc = 0; kc < nkc; ++kc) {
      xr.load(src, kc, n);
      w.load(mats, row, k, kc, g);
      __syncthreads();
      xr.store(lds);
      __syncthreads();
      mul(w);
    }
    return;
  }
  if constexpr (kBufs == 2) {
    W w0, w1;
    xr.load(src, 0, n);
    w0.load(mats, row, k, 0, g);
    auto step2 = [&](const W& wc, W& wl, int kc) {
      __syncthreads();
      xr.store(lds);
      __syncthreads();
      if (kc + 1 < nkc) {
        xr.load(src, kc + 1, n);
        wl.load(mats, row, k, kc + 1, g);
      }
      mul(wc);
    };
    for (int kc = 0; kc < nkc; kc += 2) {
      step2(w0, w1, kc);
      if (kc + 1 < nkc) step2(w1, w0, kc + 1);
    }
    return;
  }
  W w0, w1, w2;
  xr.load(src, 0, n);
  w0.load(mats, row, k, 0, g);
  if (nkc > 1) w1.load(mats, row, k, 1, g);
  auto step = [&](const W& wc, W& wl, int kc) {
    __syncthreads();
    xr.store(lds);
    __syncthreads();
    if (kc + 1 < nkc) xr.load(src, kc + 1, n);
    if (kc + 2 < nkc) wl.load(mats, row, k, kc + 2, g);
    mul(wc);
  };
  for (int kc = 0; kc < nkc; kc += 3) {
    step(w0, w2, kc);
    if (kc + 1 < nkc) step(w1, w0, kc + 1);
    if (kc + 2 < nkc) step(w2, w1, kc + 2);
  }
}

// ---------------------------------------------------------------- gate / up
// The E8M0 scale bytes lane (r, g) needs for steps [s0, s0 + kSteps) of
// weight row `row` (k columns): byte j of c[q] is the group-g scale of step
// s0 + 4q + j.  A K-chunk uses two steps' bytes; reading them per K-chunk
// touched each row's 128-byte scale line sixteen times, far enough apart in
// time that the weight stream had evicted it from L2 in between (measured:
// ~0.6 GB of the gate/up fetch of the M=512 prefill against 0.13 GB of
// scales).  fill() reads the row's kSteps steps of scales once (lane g: steps
// s0 + 4g .. +3, 16 bytes) and deals each step's word to the row's four lanes
// (ds_bpermute from lanes r + 16q); consume() advances past a K-chunk.
struct ScaleCache {
  static constexpr int kSteps = 16;  // 8 K-chunks
  uint32_t c[4];
  __device__ __forceinline__ void fill(const BufRsrc& s, int row, int k, int s0, int g) {
    const int r = (threadIdx.x & 63) & 15;
    const uint4 u = bload128(s, (uint32_t)row * (uint32_t)(k / 32) + (uint32_t)(s0 + 4 * g) * 4);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) c[q] = 0u;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t v = (uint32_t)__builtin_amdgcn_ds_bpermute((r + 16 * q) * 4, (int)w[j]);
        c[q] |= ((v >> (8 * g)) & 0xffu) << (8 * j);
      }
  }
  // scale byte of step b of K-chunk kc (two steps per K-chunk)
  __device__ __forceinline__ uint32_t byte(int kc, int b) const { return (c[0] >> (8 * (2 * (kc & 1) + b))) & 0xffu; }
  __device__ __forceinline__ void consume(int kc) {
    if (kc & 1) {
#pragma unroll
      for (int q = 0; q < 3; ++q) c[q] = c[q + 1];
      c[3] = 0u;
    }
  }
};

// Wave rows r0 .. r0+16*kGuRT-1 of W1 and W3 against the chunk's tokens; lane
// (r, g) ends holding rows r0 + 16 rt + 4g + q of token tile*16 + r.
// F = kFp4E8M0Split: E8M0 scales through a ScaleCache per matrix (the same
// decoded weights as kFp4E8M0).
template <int F, int kC, int kBufs>
__device__ void gate_up_chunk(const PrefillParams& p, const Chunk& ch, int r0, uint16_t* xs, const int* s_tok) {
  using W = WBuf<F, 2, kGuRT>;
  constexpr int kTiles = kC / 16;
  constexpr bool kSplit = F == kFp4E8M0Split;
  static_assert(!kSplit || (kGuRT == 1 && W::kSteps == 2), "scale cache: one row tile, two steps per K-chunk");
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int ntile = (ch.n + 15) / 16;
  f32x4 ag[kGuRT][kTiles], au[kGuRT][kTiles];
#pragma unroll
  for (int rt = 0; rt < kGuRT; ++rt)
#pragma unroll
    for (int t = 0; t < kTiles; ++t) ag[rt][t] = au[rt][t] = f32x4{0, 0, 0, 0};
  ScaleCache s1, s3;
  const BufRsrc sr1 = make_mat<F>(ch.ent[0], ch.ent[1], p.i, p.d).s, sr3 = make_mat<F>(ch.ent[2], ch.ent[3], p.i, p.d).s;
  if constexpr (kSplit) {
    s1.fill(sr1, r0 + r, p.d, 0, g);
    s3.fill(sr3, r0 + r, p.d, 0, g);
  }
  int kc = 0;
  auto src = [&](int, int tt) { return p.x + (int64_t)s_tok[tt] * p.d; };
  pipeline<F, 2, kGuRT, 1, kC, kBufs>(ch.ent, 0, p.i, r0 + r, p.d, g, ch.n, xs, src, [&](const W& w) {
    if constexpr (kSplit) {
      if (kc > 0 && (kc & (ScaleCache::kSteps / 2 - 1)) == 0) {  // the next kSteps steps' scales
        s1.fill(sr1, r0 + r, p.d, 2 * kc, g);
        s3.fill(sr3, r0 + r, p.d, 2 * kc, g);
      }
    }
#pragma unroll
    for (int b = 0; b < W::kSteps; ++b) {
      uint32_t e1 = 0, e3 = 0;
      if constexpr (kSplit) {
        e1 = s1.byte(kc, b);
        e3 = s3.byte(kc, b);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int rt = 0; rt < kGuRT; ++rt) {
          bf16x8 f1, f3;
          if constexpr (kSplit) {
            f1 = w.b[0][rt].frag_e(b, j, e1);
            f3 = w.b[1][rt].frag_e(b, j, e3);
          } else {
            f1 = w.b[0][rt].frag(b, j, g);
            f3 = w.b[1][rt].frag(b, j, g);
          }
#pragma unroll
          for (int tile = 0; tile < kTiles; ++tile) {
            if (tile >= ntile) break;
            const bf16x8 xf = tile_frag(xs, kCols, tile, r, g, b, j);
            ag[rt][tile] = mfma16x16x32(f1, xf, ag[rt][tile]);
            au[rt][tile] = mfma16x16x32(f3, xf, au[rt][tile]);
          }
        }
      }
    }
    if constexpr (kSplit) {
      s1.consume(kc);
      s3.consume(kc);
    }
    ++kc;
  });
#pragma unroll
  for (int tile = 0; tile < kTiles; ++tile) {
    const int tt = tile * 16 + r;
    if (tile >= ntile || tt >= ch.n) continue;
    const int64_t pr = ch.p0 + tt;
    const float wt = p.pair_w[pr];
#pragma unroll
    for (int rt = 0; rt < kGuRT; ++rt) {
      uint32_t hi[4], lo[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float a = __fmul_rn(wt, swiglu(ag[rt][tile][q], au[rt][tile][q], p.limit));
        hi[q] = f32_to_bf16_bits(a);
        lo[q] = f32_to_bf16_bits(__fadd_rn(a, -bf16_bits_to_f32(hi[q])));
      }
      const int64_t o = pr * p.i + r0 + 16 * rt + 4 * g;
      *reinterpret_cast<uint2*>(p.act_hi + o) = make_uint2(hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16));
      *reinterpret_cast<uint2*>(p.act_lo + o) = make_uint2(lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16));
    }
  }
}

// F: format of the chunks' weights (routed FP4 of the call's scale kind, or
// the shared expert's FP8); table entries without scales take the bf16 path.
template <int F, bool kShared>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(F == kFp8Block ? 2 : 4)))
prefill_gate_up_kernel(PrefillParams p) {
  __shared__ __align__(16) uint16_t xs[kBigChunk * (kCols + kPad)];
  __shared__ int s_tok[kBigChunk];
  const int nrb = p.i / kGuRows;
  Chunk ch;
  if (!load_chunk<kShared, false>(p, blockIdx.x / nrb, ch)) return;
  if (threadIdx.x < kBigChunk) s_tok[threadIdx.x] = threadIdx.x < ch.n ? p.pair_tok[ch.p0 + threadIdx.x] : 0;
  __syncthreads();
  const int r0 = (blockIdx.x % nrb) * kGuRows + 16 * kGuRT * (threadIdx.x >> 6);
  // routed E8M0 chunks read their scales through a per-lane cache (same weights)
  constexpr int FG = F == kFp4E8M0 ? kFp4E8M0Split : F;
  if (!kShared && ch.n > kChunk && ch.ent[1]) {  // a big expert's chunk (the shared expert's hold at most kChunk)
    gate_up_chunk<FG, kBigChunk, 1>(p, ch, r0, xs, s_tok);
  } else if (ch.n > kChunk) {  // bf16 weights: the chunk as two kChunk halves (registers)
    for (int h0 = 0; h0 < ch.n; h0 += kChunk) {
      Chunk sub = ch;
      sub.p0 = ch.p0 + h0;
      sub.n = min(kChunk, ch.n - h0);
      gate_up_chunk<kBf16, kChunk, 3>(p, sub, r0, xs, s_tok + h0);
    }
  } else if (ch.ent[1]) {
    gate_up_chunk<FG, kChunk, 3>(p, ch, r0, xs, s_tok);
  } else {
    gate_up_chunk<kBf16, kChunk, 3>(p, ch, r0, xs, s_tok);
  }
}

// ---------------------------------------------------------------- down
// F = kFp4E8M0Split: W2's E8M0 scales through a ScaleCache per row tile.
template <int F>
__device__ void down_chunk(const PrefillParams& p, const Chunk& ch, int r0, uint16_t* as) {
  using W = WBuf<F, 1, kDnRT>;
  constexpr bool kSplit = F == kFp4E8M0Split;
  static_assert(!kSplit || W::kSteps == 2, "scale cache: two steps per K-chunk");
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int ntile = (ch.n + 15) / 16;
  const uint16_t* ls = as + kChunk * (kCols + kPad);
  f32x4 acc[kDnRT][2];
#pragma unroll
  for (int rt = 0; rt < kDnRT; ++rt) acc[rt][0] = acc[rt][1] = f32x4{0, 0, 0, 0};
  ScaleCache sc[kDnRT];
  const BufRsrc sr = make_mat<F>(ch.ent[4], ch.ent[5], p.d, p.i).s;
  if constexpr (kSplit) {
#pragma unroll
    for (int rt = 0; rt < kDnRT; ++rt) sc[rt].fill(sr, r0 + r + 16 * rt, p.i, 0, g);
  }
  int kc = 0;
  auto src = [&](int pl, int tt) { return (pl ? p.act_lo : p.act_hi) + (int64_t)(ch.p0 + tt) * p.i; };
  pipeline<F, 1, kDnRT, 2, kChunk, 3>(ch.ent, 4, p.d, r0 + r, p.i, g, ch.n, as, src, [&](const W& w) {
    if constexpr (kSplit) {
      if (kc > 0 && (kc & (ScaleCache::kSteps / 2 - 1)) == 0) {  // the next kSteps steps' scales
#pragma unroll
        for (int rt = 0; rt < kDnRT; ++rt) sc[rt].fill(sr, r0 + r + 16 * rt, p.i, 2 * kc, g);
      }
    }
#pragma unroll
    for (int b = 0; b < W::kSteps; ++b) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int tile = 0; tile < 2; ++tile) {
          if (tile >= ntile) break;
          const bf16x8 hf = tile_frag(as, kCols, tile, r, g, b, j), lf = tile_frag(ls, kCols, tile, r, g, b, j);
#pragma unroll
          for (int rt = 0; rt < kDnRT; ++rt) {
            bf16x8 wf;
            if constexpr (kSplit) wf = w.b[0][rt].frag_e(b, j, sc[rt].byte(kc, b));
            else wf = w.b[0][rt].frag(b, j, g);
            acc[rt][tile] = mfma16x16x32(wf, hf, acc[rt][tile]);
            acc[rt][tile] = mfma16x16x32(wf, lf, acc[rt][tile]);
          }
        }
      }
    }
    if constexpr (kSplit) {
#pragma unroll
      for (int rt = 0; rt < kDnRT; ++rt) sc[rt].consume(kc);
    }
    ++kc;
  });
#pragma unroll
  for (int tile = 0; tile < 2; ++tile) {
    const int tt = tile * 16 + r;
    if (tile >= ntile || tt >= ch.n) continue;
#pragma unroll
    for (int rt = 0; rt < kDnRT; ++rt) {
      float* o = p.part + (int64_t)(ch.p0 + tt) * p.d + r0 + 16 * rt + 4 * g;
      *reinterpret_cast<float4*>(o) = make_float4(acc[rt][tile][0], acc[rt][tile][1], acc[rt][tile][2], acc[rt][tile][3]);
    }
  }
}

template <int F, bool kShared>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(F == kFp8Block ? 2 : 3)))
prefill_down_kernel(PrefillParams p) {
  __shared__ __align__(16) uint16_t as[2 * kChunk * (kCols + kPad)];  // hi plane, lo plane
  const int nrb = p.d / kDnRows;
  Chunk ch;
  if (!load_chunk<kShared, true>(p, blockIdx.x / nrb, ch)) return;
  const int r0 = (blockIdx.x % nrb) * kDnRows + 16 * kDnRT * (threadIdx.x >> 6);
  if (ch.ent[1]) down_chunk<F == kFp4E8M0 ? kFp4E8M0Split : F>(p, ch, r0, as);  // routed E8M0: cached scales
  else down_chunk<kBf16>(p, ch, r0, as);
}

// ---------------------------------------------------------------- combine
// grid (m, d / 1024): thread -> 4 consecutive columns of one token.
__global__ void __launch_bounds__(kThreads) prefill_combine_kernel(PrefillParams p) {
  const int t = blockIdx.x;
  const int col = (blockIdx.y * kThreads + threadIdx.x) * 4;
  if (col >= p.d) return;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  const int* pi = p.pidx + (int64_t)t * (p.top_k + 1);
  for (int j = 0; j <= p.top_k; ++j) {
    const int pr = pi[j];
    if (pr < 0) continue;
    const float4 v = *reinterpret_cast<const float4*>(p.part + (int64_t)pr * p.d + col);
    acc.x = __fadd_rn(acc.x, v.x);
    acc.y = __fadd_rn(acc.y, v.y);
    acc.z = __fadd_rn(acc.z, v.z);
    acc.w = __fadd_rn(acc.w, v.w);
  }
  const int64_t o = (int64_t)t * p.d + col;
  if (p.out_f32) *reinterpret_cast<float4*>(p.out_f32 + o) = acc;
  if (p.out_bf16)
    *reinterpret_cast<uint2*>(p.out_bf16 + o) =
        make_uint2(f32_to_bf16_bits(acc.x) | (f32_to_bf16_bits(acc.y) << 16),
                   f32_to_bf16_bits(acc.z) | (f32_to_bf16_bits(acc.w) << 16));
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

struct Layout {
  size_t hdr, pair_tok, pair_w, pidx, chunk_e, chunk_p0, chunk_n, dn_e, dn_p0, dn_n, act_hi, act_lo, part, total;
};

int64_t max_pairs(int64_t m, int top_k) { return m * top_k + m; }
// Chunks of the routed experts in either list: at most sum over experts of
// ceil(n_e / kChunk) <= (experts with a pair) + (pairs) / kChunk (a gate/up
// chunk of kBigChunk covers two down chunks).
int64_t max_routed_chunks(int64_t m, int64_t n_experts, int top_k) {
  const int64_t pk = m * top_k;
  return (n_experts < pk ? n_experts : pk) + (pk + kChunk - 1) / kChunk;
}
int64_t max_chunks(int64_t m, int64_t n_experts, int top_k) {
  return max_routed_chunks(m, n_experts, top_k) + (m + kChunk - 1) / kChunk;
}

Layout layout(int64_t m, int64_t d, int64_t i, int64_t n_experts, int top_k) {
  const int64_t P = max_pairs(m, top_k), C = max_chunks(m, n_experts, top_k);
  Layout L;
  size_t o = 0;
  L.hdr = o;
  o += 256;
  L.pair_tok = o;
  o += align256((size_t)P * 4);
  L.pair_w = o;
  o += align256((size_t)P * 4);
  L.pidx = o;
  o += align256((size_t)m * (top_k + 1) * 4);
  L.chunk_e = o;
  o += align256((size_t)C * 4);
  L.chunk_p0 = o;
  o += align256((size_t)C * 4);
  L.chunk_n = o;
  o += align256((size_t)C * 4);
  L.dn_e = o;
  o += align256((size_t)C * 4);
  L.dn_p0 = o;
  o += align256((size_t)C * 4);
  L.dn_n = o;
  o += align256((size_t)C * 4);
  L.act_hi = o;
  o += align256((size_t)P * i * 2);
  L.act_lo = o;
  o += align256((size_t)P * i * 2);
  L.part = o;
  o += align256((size_t)P * d * 4);
  L.total = o;
  return L;
}

}  // namespace
}  // namespace hsmoe

using namespace hsmoe;

extern "C" size_t hsmoe_moe_prefill_workspace_size(int64_t m, int64_t d, int64_t i, int64_t n_experts, int top_k) {
  if (m < 1 || d < 1 || i < 1 || n_experts < 1 || top_k < 1) return 0;
  return layout(m, d, i, n_experts, top_k).total;
}

extern "C" int hsmoe_moe_prefill(const void* x, int64_t m, int64_t d, int64_t i, const int64_t* topk_idx,
                                 const float* topk_w, int top_k, const uint64_t* expert_table, int64_t n_experts,
                                 int scale_kind, const uint64_t* shared, float swiglu_limit, float* out_f32,
                                 void* out_bf16, void* workspace, size_t workspace_bytes, hsmoe_stream_t stream) {
  const char* name = "hsmoe_moe_prefill";
  if (!x || !topk_idx || !topk_w || !expert_table || (!out_f32 && !out_bf16))
    return fail(HSMOE_ERR_ARG, "%s: null pointer or no output", name);
  if (scale_kind != HSMOE_SCALE_E8M0 && scale_kind != HSMOE_SCALE_F32)
    return fail(HSMOE_ERR_ARG, "%s: unknown scale_kind %d", name, scale_kind);
  if (n_experts < 1 || n_experts > kMaxExperts || top_k < 1 || top_k > 16 || m < 1 || m * top_k > kMaxPairs)
    return fail(HSMOE_ERR_SHAPE, "%s: need 1 <= n_experts <= %d, 1 <= top_k <= 16, 1 <= m*top_k <= %d", name,
                kMaxExperts, kMaxPairs);
  if (d % 1024 != 0 || i % 512 != 0 || d > 65536 || i > 65536)
    return fail(HSMOE_ERR_SHAPE, "%s: d must be a multiple of 1024 and i of 512 (d=%lld i=%lld)", name, (long long)d,
                (long long)i);
  if (!expert_fits(d, i))
    return fail(HSMOE_ERR_SHAPE, "%s: d*i too large (an expert matrix must stay below 4 GiB)", name);
  if (!aligned(x, 16) || (out_f32 && !aligned(out_f32, 16)) || (out_bf16 && !aligned(out_bf16, 8)))
    return fail(HSMOE_ERR_SHAPE, "%s: x and out_f32 must be 16-byte aligned, out_bf16 8-byte aligned", name);
  const Layout L = layout(m, d, i, n_experts, top_k);
  if (!workspace || workspace_bytes < L.total || !aligned(workspace, 256))
    return fail(HSMOE_ERR_WORKSPACE, "%s: workspace of %zu bytes (256-byte aligned) needed", name, L.total);
  char* ws = (char*)workspace;
  PrefillParams p;
  p.x = (const uint16_t*)x;
  p.idx = topk_idx;
  p.wts = topk_w;
  p.table = expert_table;
  p.shared = shared;
  p.hdr = (Header*)(ws + L.hdr);
  p.pair_tok = (int*)(ws + L.pair_tok);
  p.pair_w = (float*)(ws + L.pair_w);
  p.pidx = (int*)(ws + L.pidx);
  p.chunk_e = (int*)(ws + L.chunk_e);
  p.chunk_p0 = (int*)(ws + L.chunk_p0);
  p.chunk_n = (int*)(ws + L.chunk_n);
  p.dn_e = (int*)(ws + L.dn_e);
  p.dn_p0 = (int*)(ws + L.dn_p0);
  p.dn_n = (int*)(ws + L.dn_n);
  p.act_hi = (uint16_t*)(ws + L.act_hi);
  p.act_lo = (uint16_t*)(ws + L.act_lo);
  p.part = (float*)(ws + L.part);
  p.out_f32 = out_f32;
  p.out_bf16 = (uint16_t*)out_bf16;
  p.n_experts = (int)n_experts;
  p.m = (int)m;
  p.d = (int)d;
  p.i = (int)i;
  p.top_k = top_k;
  p.scale_fmt = scale_kind == HSMOE_SCALE_E8M0 ? kFp4E8M0 : kFp4F32;
  p.limit = swiglu_limit;
  hipStream_t st = (hipStream_t)stream;
  const int64_t C = max_routed_chunks(m, n_experts, top_k), CS = shared ? (m + kChunk - 1) / kChunk : 0;
  hipLaunchKernelGGL(prefill_group_kernel, dim3((unsigned)n_experts + 1), dim3(kThreads), 0, st, p);
  int rc = check_launch(name);
  if (rc) return rc;
  const dim3 blk(kThreads), gu((unsigned)(C * (i / kGuRows))), dn((unsigned)(C * (d / kDnRows)));
  if (scale_kind == HSMOE_SCALE_E8M0) hipLaunchKernelGGL((prefill_gate_up_kernel<kFp4E8M0, false>), gu, blk, 0, st, p);
  else hipLaunchKernelGGL((prefill_gate_up_kernel<kFp4F32, false>), gu, blk, 0, st, p);
  if ((rc = check_launch(name))) return rc;
  if (CS) {
    hipLaunchKernelGGL((prefill_gate_up_kernel<kFp8Block, true>), dim3((unsigned)(CS * (i / kGuRows))), blk, 0, st, p);
    if ((rc = check_launch(name))) return rc;
  }
  if (scale_kind == HSMOE_SCALE_E8M0) hipLaunchKernelGGL((prefill_down_kernel<kFp4E8M0, false>), dn, blk, 0, st, p);
  else hipLaunchKernelGGL((prefill_down_kernel<kFp4F32, false>), dn, blk, 0, st, p);
  if ((rc = check_launch(name))) return rc;
  if (CS) {
    hipLaunchKernelGGL((prefill_down_kernel<kFp8Block, true>), dim3((unsigned)(CS * (d / kDnRows))), blk, 0, st, p);
    if ((rc = check_launch(name))) return rc;
  }
  hipLaunchKernelGGL(prefill_combine_kernel, dim3((unsigned)m, (unsigned)(d / (4 * kThreads))), dim3(kThreads), 0,
                     st, p);
  return check_launch(name);
}
