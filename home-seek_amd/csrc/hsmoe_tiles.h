// Weight-streaming tiles shared by the decode kernels (stage kernels of
// hsmoe_moe_decode and the fused layer kernel of hsmoe_moe_layer_decode).
//
// A "step" is 128 consecutive columns of one weight row.  Lane (r, g) of a
// wave owns columns 128*st + 32g .. +32 of row r: the 4 lanes of a row read the
// step's bytes contiguously, and MFMA j of the step uses the lane's columns
// +8j .. +8j+7 (so its k-slot 8g+jj is column 128*st + 32g + 8j + jj).
// Batch<F, kB> holds the raw loads of kB consecutive steps; nothing is decoded
// until every load of the batch has been issued.
//
// Weight formats of a slot: routed experts are FP4 (e2m1) with E8M0 or fp32
// per-32 scales, or bf16 when the table entry has no scale pointer; the shared
// expert is e4m3 with fp32 128x128 block scales, or bf16 likewise.
#pragma once
#include "hsmoe_common.h"

namespace hsmoe {

enum Fmt : int { kFp4E8M0 = 0, kFp4F32 = 1, kFp8Block = 2, kBf16 = 3, kFp4E8M0Split = 4 };
// kFp4E8M0Split: FP4 with E8M0 scales whose bytes the caller reads itself
// (batches hold the weights only; the matrix is that of kFp4E8M0).

// One weight matrix of format F ([rows][cols], row-major) and its scales, as
// buffer resources of their exact sizes: every load of a batch is an
// immediate offset from one per-lane offset, and nothing past either array is
// read.  Sizes must stay below 4 GiB (the entry points check their shapes).
struct Mat {
  BufRsrc w, s;
};
template <int F>
__device__ __forceinline__ Mat make_mat(uint64_t w, uint64_t sc, int rows, int cols) {
  const uint32_t n = (uint32_t)rows * (uint32_t)cols;
  Mat m;
  if constexpr (F == kFp4E8M0 || F == kFp4E8M0Split) {
    m.w = make_buf(w, n / 2);
    m.s = make_buf(sc, n / 32);
  } else if constexpr (F == kFp4F32) {
    m.w = make_buf(w, n / 2);
    m.s = make_buf(sc, n / 32 * 4);
  } else if constexpr (F == kFp8Block) {
    m.w = make_buf(w, n);
    m.s = make_buf(sc, (uint32_t)((rows + 127) / 128) * (uint32_t)((cols + 127) / 128) * 4);
  } else {
    m.w = make_buf(w, 2 * n);
    m.s = make_buf(w, 0);
  }
  return m;
}

template <int F, int kB>
struct Batch;

template <int kB>
struct Batch<kFp4E8M0, kB> {
  uint4 a[kB];
  uint4 sq[kB >= 4 ? kB / 4 : 1];  // kB >= 4: 16 scale bytes per 4 steps (bytes 4b..4b+3 = step b)
  uint32_t sw[kB];                 // kB < 4: the 4 scale bytes of each step (byte g = group g)
  __device__ __forceinline__ void load(const Mat& m, int row, int k, int st, int g) {
    const uint32_t wo = (uint32_t)row * (uint32_t)(k / 2) + st * 64 + g * 16;
#pragma unroll
    for (int b = 0; b < kB; ++b) a[b] = bload128(m.w, wo + b * 64);
    const uint32_t so = (uint32_t)row * (uint32_t)(k / 32) + st * 4;
    if constexpr (kB >= 4) {
#pragma unroll
      for (int q = 0; q < kB / 4; ++q) sq[q] = bload128(m.s, so + 16 * q);
    } else if constexpr (kB == 2) {  // both steps' scale words in one load
      const uint2 w2 = bload64(m.s, so);
      sw[0] = w2.x;
      sw[1] = w2.y;
    } else {
      sw[0] = bload32(m.s, so);
    }
  }
  __device__ __forceinline__ bf16x8 frag(int b, int j, int g) const {
    const uint4& q = a[b];
    const uint32_t dw = j == 0 ? q.x : j == 1 ? q.y : j == 2 ? q.z : q.w;
    uint32_t e;
    if constexpr (kB >= 4) {
      const uint4& s4 = sq[b / 4];
      const int d = b & 3;
      const uint32_t word = d == 0 ? s4.x : d == 1 ? s4.y : d == 2 ? s4.z : s4.w;
      e = (word >> (8 * g)) & 0xffu;
    } else {
      e = (sw[b] >> (8 * g)) & 0xffu;
    }
    return fp4x8_to_bf16_e8m0(dw, e8m0_as_f32(e));
  }
};

template <int kB>
struct Batch<kFp4E8M0Split, kB> {
  uint4 a[kB];
  __device__ __forceinline__ void load(const Mat& m, int row, int k, int st, int g) {
    const uint32_t wo = (uint32_t)row * (uint32_t)(k / 2) + st * 64 + g * 16;
#pragma unroll
    for (int b = 0; b < kB; ++b) a[b] = bload128(m.w, wo + b * 64);
  }
  // the weights of MFMA j of step b, decoded with scale exponent byte e
  __device__ __forceinline__ bf16x8 frag_e(int b, int j, uint32_t e) const {
    const uint4& q = a[b];
    const uint32_t dw = j == 0 ? q.x : j == 1 ? q.y : j == 2 ? q.z : q.w;
    return fp4x8_to_bf16_e8m0(dw, e8m0_as_f32(e));
  }
};

template <int kB>
struct Batch<kFp4F32, kB> {
  uint4 a[kB];
  float s[kB];
  __device__ __forceinline__ void load(const Mat& m, int row, int k, int st, int g) {
    const uint32_t wo = (uint32_t)row * (uint32_t)(k / 2) + st * 64 + g * 16;
    const uint32_t so = 4 * ((uint32_t)row * (uint32_t)(k / 32) + st * 4 + g);
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      a[b] = bload128(m.w, wo + b * 64);
      s[b] = bloadf(m.s, so + 16 * b);
    }
  }
  __device__ __forceinline__ bf16x8 frag(int b, int j, int) const {
    const uint4& q = a[b];
    const uint32_t dw = j == 0 ? q.x : j == 1 ? q.y : j == 2 ? q.z : q.w;
    return fp4x8_to_bf16_f32(dw, s[b]);
  }
};

template <int kB>
struct Batch<kFp8Block, kB> {
  uint4 a[kB], c[kB];
  float s[kB];
  __device__ __forceinline__ void load(const Mat& m, int row, int k, int st, int g) {
    const uint32_t wo = (uint32_t)row * (uint32_t)k + st * 128 + g * 32;
    const uint32_t so = 4 * ((uint32_t)(row / 128) * (uint32_t)(k / 128) + st);
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      a[b] = bload128(m.w, wo + b * 128);
      c[b] = bload128(m.w, wo + b * 128 + 16);
      s[b] = bloadf(m.s, so + 4 * b);
    }
  }
  __device__ __forceinline__ bf16x8 frag(int b, int j, int) const {
    const uint4& q = j < 2 ? a[b] : c[b];
    const uint32_t d0 = (j & 1) ? q.z : q.x, d1 = (j & 1) ? q.w : q.y;
    bf16x8 f;
    fp8x4_to_bf16(d0, s[b], f, 0);
    fp8x4_to_bf16(d1, s[b], f, 1);
    return f;
  }
};

template <int kB>
struct Batch<kBf16, kB> {
  uint4 a[kB][4];
  __device__ __forceinline__ void load(const Mat& m, int row, int k, int st, int g) {
    const uint32_t wo = 2 * ((uint32_t)row * (uint32_t)k + st * 128 + g * 32);
#pragma unroll
    for (int b = 0; b < kB; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j) a[b][j] = bload128(m.w, wo + b * 256 + j * 16);
  }
  __device__ __forceinline__ bf16x8 frag(int b, int j, int) const { return __builtin_bit_cast(bf16x8, a[b][j]); }
};

// Steps per batch of the gate/up streams (register budget: ~64 VGPRs of raw
// weights per matrix) and of the down stream (one matrix: FP4 twice the
// steps; FP8 and bf16 twice the steps only with kDeep, for kernels whose
// register budget holds 64 VGPRs of raw weights -- the split decode kernel's
// 128-VGPR budget does not).  The batch size never changes the arithmetic.
template <int F>
constexpr int gate_up_batch() {
  return (F == kFp4E8M0 || F == kFp4F32) ? 8 : (F == kFp8Block ? 4 : 2);
}
template <int F, bool kDeep = false>
constexpr int down_batch() {
  return (F == kFp4E8M0 || F == kFp4F32 || kDeep) ? 2 * gate_up_batch<F>() : gate_up_batch<F>();
}

// Format of the slot whose table entry is `ent`.
__device__ __forceinline__ int slot_format(int routed_scale_fmt, const uint64_t* ent, bool is_shared) {
  if (is_shared) return ent[1] ? kFp8Block : kBf16;
  return ent[1] ? routed_scale_fmt : kBf16;
}

// B operand from an LDS tile laid out [16 columns][kcols] bf16: lane (c, g)
// takes columns 128*st + 32g + 8j .. +8 of tile column c (zero when c >= ncol).
__device__ __forceinline__ bf16x8 lds_frag(const uint16_t* tile, int kcols, int c, int g, int st, int j, int ncol) {
  bf16x8 z = {};
  if (c >= ncol) return z;
  return *reinterpret_cast<const bf16x8*>(tile + c * kcols + st * 128 + g * 32 + 8 * j);
}

// The four B fragments (j = 0..3) of step st, as lds_frag.  The MFMA loops
// read step st + 1's fragments before multiplying step st, so the LDS latency
// of one step hides behind the previous step's MFMAs instead of stalling
// every MFMA on its own read.
struct Frags {
  bf16x8 f[4];
  __device__ __forceinline__ void read(const uint16_t* tile, int kcols, int c, int g, int st, int ncol) {
#pragma unroll
    for (int j = 0; j < 4; ++j) f[j] = lds_frag(tile, kcols, c, g, st, j, ncol);
  }
};

// ------------------------------------------------------------ gate / up
// One wave: rows r0..r0+15 of W1 and W3 ([i][d]) of the slot `ent` over steps
// [st0, st1) against the m token rows of x ([m][d] bf16 in LDS).  The MFMA
// accumulators hold D[4*(lane/16) + q][lane%16] = row r0 + 4*(lane/16) + q,
// token lane%16.
template <int F, int kB>
__device__ __forceinline__ void gate_up_rows(const uint64_t* ent, const uint16_t* xs, int m, int d, int i, int r0,
                                             int st0, int st1, f32x4& ag, f32x4& au) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int row = r0 + r;
  const Mat w1 = make_mat<F>(ent[0], ent[1], i, d), w3 = make_mat<F>(ent[2], ent[3], i, d);
  for (int st = st0; st < st1; st += kB) {
    Batch<F, kB> b1, b3;
    b1.load(w1, row, d, st, g);
    b3.load(w3, row, d, st, g);
#pragma unroll
    for (int b = 0; b < kB; ++b) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bf16x8 xf = lds_frag(xs, d, r, g, st + b, j, m);
        ag = mfma16x16x32(b1.frag(b, j, g), xf, ag);
        au = mfma16x16x32(b3.frag(b, j, g), xf, au);
      }
    }
  }
}

template <int F>
__device__ __forceinline__ void gate_up_any(const uint64_t* ent, const uint16_t* xs, int m, int d, int i, int r0,
                                            int st0, int st1, f32x4& ag, f32x4& au) {
  constexpr int kMax = gate_up_batch<F>();
  if ((st1 - st0) % kMax == 0) gate_up_rows<F, kMax>(ent, xs, m, d, i, r0, st0, st1, ag, au);
  else gate_up_rows<F, 1>(ent, xs, m, d, i, r0, st0, st1, ag, au);
}

__device__ __forceinline__ void gate_up_slot(int fmt, const uint64_t* ent, const uint16_t* xs, int m, int d, int i,
                                             int r0, int st0, int st1, f32x4& ag, f32x4& au) {
  switch (fmt) {
    case kFp4E8M0: gate_up_any<kFp4E8M0>(ent, xs, m, d, i, r0, st0, st1, ag, au); break;
    case kFp4F32: gate_up_any<kFp4F32>(ent, xs, m, d, i, r0, st0, st1, ag, au); break;
    case kFp8Block: gate_up_any<kFp8Block>(ent, xs, m, d, i, r0, st0, st1, ag, au); break;
    default: gate_up_any<kBf16>(ent, xs, m, d, i, r0, st0, st1, ag, au); break;
  }
}

// One wave: rows r0..r0+15 of ONE of W1 / W3 (weights w, scales sc, [i][d])
// over steps [st0, st1) against the m token rows of x: the same MFMA sequence
// as that matrix's accumulator in gate_up_rows, so the sums are identical.
template <int F, int kB>
__device__ __forceinline__ void gate_or_up_rows(uint64_t w, uint64_t sc, const uint16_t* xs, int m, int d, int i,
                                                int r0, int st0, int st1, f32x4& acc) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int row = r0 + r;
  const Mat wm = make_mat<F>(w, sc, i, d);
  for (int st = st0; st < st1; st += kB) {
    Batch<F, kB> bw;
    bw.load(wm, row, d, st, g);
#pragma unroll
    for (int b = 0; b < kB; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc = mfma16x16x32(bw.frag(b, j, g), lds_frag(xs, d, r, g, st + b, j, m), acc);
  }
}

// gate_or_up_rows in batches of twice the gate/up batch (one matrix instead
// of two) when that divides the steps, else one step at a time (the *_any
// helpers instantiate only these two sizes: every further size is code that
// the decode shapes never run, fetched into the instruction cache nonetheless).
template <int F>
__device__ __forceinline__ void gate_or_up_any(uint64_t w, uint64_t sc, const uint16_t* xs, int m, int d, int i,
                                               int r0, int st0, int st1, f32x4& acc) {
  constexpr int kMax = 2 * gate_up_batch<F>();
  if ((st1 - st0) % kMax == 0) gate_or_up_rows<F, kMax>(w, sc, xs, m, d, i, r0, st0, st1, acc);
  else gate_or_up_rows<F, 1>(w, sc, xs, m, d, i, r0, st0, st1, acc);
}

// SwiGLU of the reference's M<=8 route (fused_moe.py:390-395) in fp32:
// min(g, L) * sigmoid(min(g, L)) * clamp(u, -L, L); NaN passes both clamps.
__device__ __forceinline__ float swiglu(float gsum, float usum, float L) {
  const float gc = gsum > L ? L : gsum;
  const float uc = usum < -L ? -L : (usum > L ? L : usum);
  const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-gc)));  // torch sigmoid
  return __fmul_rn(__fmul_rn(gc, sig), uc);
}

// ------------------------------------------------------------ down
// One wave: rows r0..r0+15 of W2 ([d][i]) of the slot `ent` over steps
// [st0, st1) of the i/128 against the activation tile as ([2m][i] bf16 in
// LDS: hi rows then lo rows).  `ready()` runs (block-wide) after the first
// batch's loads are issued and before the tile is read, so the weight loads
// overlap whatever it waits for.
template <int F, int kB, typename Ready>
__device__ __forceinline__ void down_rows(const uint64_t* ent, const uint16_t* as, int m, int i, int d, int r0,
                                          int st0, int st1, f32x4& acc, Ready&& ready) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int row = r0 + r;
  const Mat w2 = make_mat<F>(ent[4], ent[5], d, i);
  Batch<F, kB> bw;
  if (st0 < st1) bw.load(w2, row, i, st0, g);
  ready();
  if (st0 >= st1) return;  // (an empty range: the sum stays zero)
  Frags ac;
  ac.read(as, i, r, g, st0, 2 * m);
  for (int st = st0; st < st1; st += kB) {
    if (st != st0) bw.load(w2, row, i, st, g);
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      Frags an;
      an.read(as, i, r, g, min(st + b + 1, st1 - 1), 2 * m);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc = mfma16x16x32(bw.frag(b, j, g), ac.f[j], acc);
      ac = an;
    }
  }
}

// Batches of min(down_batch, kCap) steps when that divides the steps, else one
// step at a time.
template <int F, bool kDeep, int kCap = 64, typename Ready>
__device__ __forceinline__ void down_any(const uint64_t* ent, const uint16_t* as, int m, int i, int d, int r0,
                                         int st0, int st1, f32x4& acc, Ready&& ready) {
  constexpr int kMax = down_batch<F, kDeep>() < kCap ? down_batch<F, kDeep>() : kCap;
  if ((st1 - st0) % kMax == 0) down_rows<F, kMax>(ent, as, m, i, d, r0, st0, st1, acc, ready);
  else down_rows<F, 1>(ent, as, m, i, d, r0, st0, st1, acc, ready);
}

template <int F, bool kDeep, typename Ready>
__device__ __forceinline__ void down_any(const uint64_t* ent, const uint16_t* as, int m, int i, int d, int r0,
                                         f32x4& acc, Ready&& ready) {
  down_any<F, kDeep>(ent, as, m, i, d, r0, 0, i / 128, acc, ready);
}

// The shared expert's split of the i/128 down steps: [0, half) and
// [half, i/128), each accumulated from zero, the two sums added (first +
// second) -- one split for every path, so that they agree bit for bit.
__device__ __forceinline__ int shared_down_half(int i) { return (i / 128) / 2; }

template <bool kDeep = false, typename Ready>
__device__ __forceinline__ void down_slot(int fmt, const uint64_t* ent, const uint16_t* as, int m, int i, int d,
                                          int r0, f32x4& acc, Ready&& ready) {
  switch (fmt) {
    case kFp4E8M0: down_any<kFp4E8M0, kDeep>(ent, as, m, i, d, r0, acc, ready); break;
    case kFp4F32: down_any<kFp4F32, kDeep>(ent, as, m, i, d, r0, acc, ready); break;
    case kFp8Block: down_any<kFp8Block, kDeep>(ent, as, m, i, d, r0, acc, ready); break;
    default: down_any<kBf16, kDeep>(ent, as, m, i, d, r0, acc, ready); break;
  }
}

// down_slot over steps [st0, st1) only.
template <bool kDeep = false, typename Ready>
__device__ __forceinline__ void down_slot(int fmt, const uint64_t* ent, const uint16_t* as, int m, int i, int d,
                                          int r0, int st0, int st1, f32x4& acc, Ready&& ready) {
  switch (fmt) {
    case kFp4E8M0: down_any<kFp4E8M0, kDeep>(ent, as, m, i, d, r0, st0, st1, acc, ready); break;
    case kFp4F32: down_any<kFp4F32, kDeep>(ent, as, m, i, d, r0, st0, st1, acc, ready); break;
    case kFp8Block: down_any<kFp8Block, kDeep>(ent, as, m, i, d, r0, st0, st1, acc, ready); break;
    default: down_any<kBf16, kDeep>(ent, as, m, i, d, r0, st0, st1, acc, ready); break;
  }
}

// Agent-scope (cross-XCD coherent, L2-bypassing) loads and stores used for
// every value one workgroup hands to another inside a launch.
__device__ __forceinline__ void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int load_agent(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned load_agent(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_agent(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned add_agent(unsigned* p, unsigned v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Fixed-order sum over n slots of agent-scope values base[s * stride]
// (s = 0 .. n-1, then `extra` when non-null): the loads go out 8 at a time so
// a chain of them costs one memory round trip per 8 slots, and the additions
// keep slot order.
__device__ __forceinline__ float sum_slots_agent(const float* base, int64_t stride, int n, const float* extra) {
  float v = 0.0f;
  for (int s0 = 0; s0 < n; s0 += 8) {
    float pv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) pv[j] = (s0 + j < n) ? load_agent(base + (int64_t)(s0 + j) * stride) : 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (s0 + j < n) v = __fadd_rn(v, pv[j]);
  }
  if (extra) v = __fadd_rn(v, load_agent(extra));
  return v;
}

}  // namespace hsmoe
