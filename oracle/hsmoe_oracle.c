/*
 * CPU oracle for the routed-expert MoE hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker or the timed CPU baseline.  The product
 * (libhsmoe.so and the home_seek_amd package) never links or calls it.
 *
 * Every routine restates one step of the reference's PyTorch algorithm; the
 * reference file:line it follows is given above each one.  Build with
 * -ffp-contract=off so that every float operation rounds exactly once, the way
 * the matching device code (which uses __fmul_rn/__fadd_rn) does.
 *
 * Parity pins (see tests/test_oracle_*.py):
 *   e2m1 decode       -- the reference's _FP4_LUT table, all 16 codes
 *   e8m0 / e4m3       -- torch's own float8 casts, all 256 bytes
 *   bf16 rounding     -- torch's own float32->bfloat16 cast on edge patterns
 *   dequant           -- interleave / per-group-scale KATs of the reference tests
 *   splitmix64        -- the published splitmix64 output sequence for seed 0
 *   exact dot         -- integer brute force on small inputs (exactly representable)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define HSO_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------ */
/* number formats                                                      */
/* ------------------------------------------------------------------ */

static inline float u32_as_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_as_u32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* bf16 -> fp32 is a 16-bit shift (exact). */
HSO_API float hso_bf16_to_f32(uint16_t h) { return u32_as_f32((uint32_t)h << 16); }

/* fp32 -> bf16, round to nearest even; NaN -> 0x7FC0.  This is what
 * torch's Tensor.to(torch.bfloat16) does on the CPU, which every ".to(bf16)"
 * in the reference path relies on (e.g. fused_moe.py:26, fused_moe.py:394). */
HSO_API uint16_t hso_f32_to_bf16(float f) {
  uint32_t u = f32_as_u32(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* fp64 -> bf16 with ONE rounding (round to nearest even).  Used for logits
 * whose exact value is accumulated in fp64 (router.py:27-29 rounds the fp32
 * matmul result to bf16; the oracle rounds the exact sum instead). */
HSO_API uint16_t hso_f64_to_bf16(double d) {
  if (isnan(d)) return 0x7fc0;
  uint64_t u; memcpy(&u, &d, 8);
  uint16_t sign = (uint16_t)((u >> 48) & 0x8000u);
  double a = fabs(d);
  if (a == 0.0) return sign;
  /* largest finite bf16 is (2 - 2^-7) * 2^127; values at or beyond the
   * midpoint to the next binade (2 - 2^-8) * 2^127 overflow to inf. */
  if (a >= ldexp(2.0 - ldexp(1.0, -8), 127)) return (uint16_t)(sign | 0x7f80u);
  int e;
  frexp(a, &e);               /* a = m * 2^e, m in [0.5, 1) */
  int ulp_exp = e - 8;        /* bf16 keeps 8 significant bits */
  if (ulp_exp < -133) ulp_exp = -133; /* subnormal spacing 2^-133 */
  double q = ldexp(a, -ulp_exp);      /* exact: scaling by a power of two */
  double r = nearbyint(q);            /* default rounding mode: ties to even */
  double v = ldexp(r, ulp_exp);       /* exact bf16 value as a double */
  /* re-encode v (exactly representable in fp32 and bf16) */
  float vf = (float)v;
  return (uint16_t)(sign | (uint16_t)(f32_as_u32(vf) >> 16));
}

/* e2m1 decode, fused_moe.py:604-608 (_FP4_LUT) and _fp4.py:79-90:
 * s = bit3, e = bits2-1, m = bit0; e == 0 -> m * 0.5, else (1 + m/2) * 2^(e-1).
 * Code 8 is -0.0. */
HSO_API float hso_e2m1(int code) {
  int s = (code >> 3) & 1, e = (code >> 1) & 3, m = code & 1;
  float mag = (e == 0) ? 0.5f * (float)m : ldexpf(1.0f + 0.5f * (float)m, e - 1);
  return s ? -mag : mag;
}

/* E8M0 -> fp32 as torch's float8_e8m0fnu.to(float32) does on the engine's GPU
 * tier (engine.py:1260-1271): 2^(e-127) for every e < 255 (e == 0 gives the
 * fp32 subnormal 2^-127), NaN for e == 255. */
HSO_API float hso_e8m0_cast(uint8_t e) {
  if (e == 255) return NAN;
  if (e == 0) return ldexpf(1.0f, -127);
  return u32_as_f32((uint32_t)e << 23);
}

/* E8M0 -> fp32 by the bit trick of weight_loader.py:14-19 (_ue8m0_to_f32) and
 * _fp4.py:59-69 (transform_sf): bits = e << 23.  e == 0 gives +0.0, e == 255
 * gives +inf. */
HSO_API float hso_e8m0_shift(uint8_t e) { return u32_as_f32((uint32_t)e << 23); }

/* OCP e4m3fn decode (torch.float8_e4m3fn -> float32), used by
 * load_fp8_weight / cast_back (weight_loader.py:22-32, _fp4.py:98-110):
 * bias 7, no infinities, S.1111.111 is NaN, exponent 0 is subnormal m/8*2^-6. */
HSO_API float hso_e4m3(uint8_t b) {
  int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
  float mag;
  if (e == 15 && m == 7) return NAN;
  if (e == 0) mag = ldexpf((float)m / 8.0f, -6);
  else mag = ldexpf(1.0f + (float)m / 8.0f, e - 7);
  return s ? -mag : mag;
}

/* ------------------------------------------------------------------ */
/* dequantisation                                                      */
/* ------------------------------------------------------------------ */

/* FP4 -> bf16 with per-32-column scales, _dequantize_fp4_to_bf16
 * (fused_moe.py:22-26), load_fp4_weight (weight_loader.py:35-45) and the CPU
 * branch of triton_dequantize_fp4_to_bf16 (fused_moe.py:687-691):
 *   out[n, 2j]   = bf16(e2m1(p & 0xF) * s[n, 2j / 32])
 *   out[n, 2j+1] = bf16(e2m1(p >> 4)  * s[n, (2j+1) / 32])
 * fp32 product, one bf16 rounding.  Scales are fp32 values here; the caller
 * decides how E8M0 bytes become fp32 (hso_e8m0_cast or hso_e8m0_shift). */
HSO_API void hso_dequant_fp4(const uint8_t* packed, const float* scale, int64_t n_rows, int64_t k,
                             uint16_t* out) {
  float lut[16];
  for (int c = 0; c < 16; ++c) lut[c] = hso_e2m1(c); /* the same decode, tabulated once */
  int64_t kh = k / 2, ks = k / 32;
  for (int64_t n = 0; n < n_rows; ++n) {
    for (int64_t j = 0; j < kh; ++j) {
      uint8_t p = packed[n * kh + j];
      float s = scale[n * ks + (2 * j) / 32];
      out[n * k + 2 * j] = hso_f32_to_bf16(lut[p & 15] * s);
      out[n * k + 2 * j + 1] = hso_f32_to_bf16(lut[p >> 4] * s);
    }
  }
}

/* FP8 e4m3 -> bf16 with [ceil(N/128), ceil(K/128)] block scales
 * (cast_back(..., 'bf16', (128, 128)), _fp4.py:98-110, via load_fp8_weight,
 * weight_loader.py:22-32): bf16(fp32(e4m3) * s[n/128, k/128]). */
HSO_API void hso_dequant_fp8_block(const uint8_t* data, const float* scale, int64_t n_rows, int64_t k,
                                   uint16_t* out) {
  float lut[256];
  for (int b = 0; b < 256; ++b) lut[b] = hso_e4m3((uint8_t)b);
  int64_t kb = (k + 127) / 128;
  for (int64_t n = 0; n < n_rows; ++n)
    for (int64_t c = 0; c < k; ++c)
      out[n * k + c] = hso_f32_to_bf16(lut[data[n * k + c]] * scale[(n / 128) * kb + c / 128]);
}

/* ------------------------------------------------------------------ */
/* exact dot products (router logits, lm_head logits)                  */
/* ------------------------------------------------------------------ */

/* logits[m, r] = bf16(sum_k x[m, k] * W[r, k]) for bf16 x and W, summed in
 * fp64 (each bf16 x bf16 product is exact in fp64) and rounded ONCE to bf16.
 * Restates torch.matmul(x.bf16, W.t()) -> bf16 of router.py:27 and of the
 * lm_head matmul (engine.py:2483, 2846), whose fp32 accumulation order is left
 * to the BLAS; the oracle defines the value as the correctly rounded sum.
 * If bias != NULL, follows router.py:28-29: bf16(bf16(logit) + bf16(bias)). */
HSO_API void hso_logits_bf16(const uint16_t* x, const uint16_t* w, const float* bias, int64_t m_rows,
                             int64_t n_rows, int64_t k, uint16_t* out) {
  /* one token's hidden row widened to fp64, for any k */
  double* xs = (double*)malloc((size_t)(k > 0 ? k : 1) * sizeof(double));
  if (!xs) abort();
  for (int64_t m = 0; m < m_rows; ++m) {
    for (int64_t c = 0; c < k; ++c) xs[c] = (double)hso_bf16_to_f32(x[m * k + c]);
    for (int64_t r = 0; r < n_rows; ++r) {
      const uint16_t* wr = w + r * k;
      double acc = 0.0;
      for (int64_t c = 0; c < k; ++c) acc += xs[c] * (double)hso_bf16_to_f32(wr[c]);
      uint16_t l = hso_f64_to_bf16(acc);
      if (bias) {
        float b = hso_bf16_to_f32(hso_f32_to_bf16(bias[r]));
        l = hso_f32_to_bf16(hso_bf16_to_f32(l) + b);
      }
      out[m * n_rows + r] = l;
    }
  }
  free(xs);
}

/* ------------------------------------------------------------------ */
/* counter-based RNG for the synthetic workloads                       */
/* ------------------------------------------------------------------ */

/* splitmix64 finaliser (Steele, Lea, Flood 2014; Vigna's splitmix64.c).
 * rand(key, i) is the (i+1)-th output of splitmix64 seeded with `key`, so
 * rand(0, 0) = 0xE220A8397B1DCDAF as published. */
static inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
HSO_API uint64_t hso_rand(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull); }
HSO_API uint64_t hso_key(uint64_t seed, uint64_t tag) { return hso_rand(seed, tag); }

/* bytes[b] = byte (b % 8) of rand(key, b / 8), little-endian: packed e2m1
 * codes uniform over all 16 values. */
HSO_API void hso_gen_bytes(uint64_t key, int64_t n, uint8_t* out) {
  for (int64_t w = 0; w * 8 < n; ++w) {
    uint64_t r = hso_rand(key, (uint64_t)w);
    for (int q = 0; q < 8 && w * 8 + q < n; ++q) out[w * 8 + q] = (uint8_t)(r >> (8 * q));
  }
}

/* e4m3 codes: random bytes with the two NaN codes (0x7F, 0xFF) mapped to
 * 0x7E / 0xFE (+-448). */
HSO_API void hso_gen_e4m3(uint64_t key, int64_t n, uint8_t* out) {
  hso_gen_bytes(key, n, out);
  for (int64_t i = 0; i < n; ++i)
    if ((out[i] & 0x7f) == 0x7f) out[i] ^= 1;
}

/* E8M0 exponent bytes uniform over [lo, lo + span): lo + floor(hi32 * span / 2^32). */
HSO_API void hso_gen_e8m0(uint64_t key, int64_t n, int lo, int span, uint8_t* out) {
  for (int64_t i = 0; i < n; ++i) {
    uint64_t r = hso_rand(key, (uint64_t)i);
    out[i] = (uint8_t)(lo + (int)(((r >> 32) * (uint64_t)span) >> 32));
  }
}

/* Approximately normal N(mean, std): z = (u0+u1+u2+u3 - 2*65535) * sqrt(3)/65536
 * (Irwin-Hall sum of the four 16-bit lanes of rand(key, i), unit variance up to
 * a 2^-16 relative bias, tails bounded at 3.46 sigma); v = mean + std * z with
 * every product and sum rounded once in fp32. */
static inline float normal_f32(uint64_t key, uint64_t i, float mean, float std) {
  uint64_t r = hso_rand(key, i);
  int32_t s = (int32_t)(r & 0xffff) + (int32_t)((r >> 16) & 0xffff) + (int32_t)((r >> 32) & 0xffff) +
              (int32_t)((r >> 48) & 0xffff);
  float z = (float)(s - 131070) * 2.642899103e-05f;
  float t = std * z;
  return mean + t;
}
HSO_API void hso_gen_normal_f32(uint64_t key, int64_t n, float mean, float std, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = normal_f32(key, (uint64_t)i, mean, std);
}
HSO_API void hso_gen_normal_bf16(uint64_t key, int64_t n, float mean, float std, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = hso_f32_to_bf16(normal_f32(key, (uint64_t)i, mean, std));
}

/* Uniform U(lo, hi) in fp32 times `mul`: f = (r >> 40) * 2^-24 (exact),
 * v = (lo + (hi - lo) * f) * mul, each operation rounded once. */
HSO_API void hso_gen_uniform_f32(uint64_t key, int64_t n, float lo, float hi, float mul, float* out) {
  for (int64_t i = 0; i < n; ++i) {
    uint64_t r = hso_rand(key, (uint64_t)i);
    float f = (float)(r >> 40) * 5.9604644775390625e-08f;
    float t = (hi - lo) * f;
    float v = lo + t;
    out[i] = v * mul;
  }
}

/* Uniform integers in [0, n_values): floor(hi32 * n_values / 2^32). */
HSO_API void hso_gen_index(uint64_t key, int64_t n, int64_t n_values, int64_t* out) {
  for (int64_t i = 0; i < n; ++i) {
    uint64_t r = hso_rand(key, (uint64_t)i);
    out[i] = (int64_t)(((r >> 32) * (uint64_t)n_values) >> 32);
  }
}
