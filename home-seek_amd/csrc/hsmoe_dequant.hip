// Standalone FP4 -> bf16 and FP8(block-scaled) -> bf16 dequantisation.
//
// Not on the fast path (the FFN kernels decode in registers); this is the
// drop-in for triton_dequantize_fp4_to_bf16 (fused_moe.py:672-710) used by the
// T>1 BF16 loaders, and the bit-exactness anchor of the decode the FFN kernels
// share.  HBM-bound: reads 17 B, writes 64 B per 32 weights.
#include "hsmoe_common.h"
#include "hsmoe_internal.h"

namespace hsmoe {
namespace {

constexpr int kThreads = 256;

// One thread = one 32-column scale group of one row: 16 packed bytes in,
// 64 bytes of bf16 out.
template <int kScale>
__global__ void __launch_bounds__(kThreads) fp4_dequant_kernel(const uint8_t* __restrict__ packed,
                                                                const void* __restrict__ scale, int64_t n_rows,
                                                                int64_t groups_per_row, int64_t packed_stride,
                                                                int64_t scale_stride, uint16_t* __restrict__ out,
                                                                int64_t out_stride) {
  int64_t total = n_rows * groups_per_row;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    int64_t n = t / groups_per_row, g = t - n * groups_per_row;
    uint4 p = *reinterpret_cast<const uint4*>(packed + n * packed_stride + g * 16);
    bf16x8 f0, f1, f2, f3;
    if (kScale == kScaleE8M0) {
      float s = e8m0_as_f32(reinterpret_cast<const uint8_t*>(scale)[n * scale_stride + g]);
      f0 = fp4x8_to_bf16_e8m0(p.x, s);
      f1 = fp4x8_to_bf16_e8m0(p.y, s);
      f2 = fp4x8_to_bf16_e8m0(p.z, s);
      f3 = fp4x8_to_bf16_e8m0(p.w, s);
    } else {
      float s = reinterpret_cast<const float*>(scale)[n * scale_stride + g];
      f0 = fp4x8_to_bf16_f32(p.x, s);
      f1 = fp4x8_to_bf16_f32(p.y, s);
      f2 = fp4x8_to_bf16_f32(p.z, s);
      f3 = fp4x8_to_bf16_f32(p.w, s);
    }
    bf16x8* o = reinterpret_cast<bf16x8*>(out + n * out_stride + g * 32);
    o[0] = f0;
    o[1] = f1;
    o[2] = f2;
    o[3] = f3;
  }
}

// One thread = 8 consecutive e4m3 bytes of a row.
__global__ void __launch_bounds__(kThreads) fp8_dequant_kernel(const uint8_t* __restrict__ data,
                                                                const float* __restrict__ scale, int64_t n_rows,
                                                                int64_t k, uint16_t* __restrict__ out) {
  int64_t per_row = k / 8, kb = (k + 127) / 128;
  int64_t total = n_rows * per_row;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    int64_t n = t / per_row, c = (t - n * per_row) * 8;
    uint2 w = *reinterpret_cast<const uint2*>(data + n * k + c);
    float s = scale[(n / 128) * kb + c / 128];
    bf16x8 r;
    fp8x4_to_bf16(w.x, s, r, 0);
    fp8x4_to_bf16(w.y, s, r, 1);
    *reinterpret_cast<bf16x8*>(out + n * k + c) = r;
  }
}

// Block-scaled dequant of any shape: one thread = one data byte (two FP4
// columns, or one e4m3 column) of one row; the code's exact fp32 value times
// the fp32 scale of its (row block, column block), one fp32 rounding, then
// stored as fp32 or rounded to bf16 (RNE).  FP4 rows hold ceil(k / 2) bytes.
template <bool kFp4, bool kOutF32>
__global__ void __launch_bounds__(kThreads) dequant_blocked_kernel(const uint8_t* __restrict__ data,
                                                                    const float* __restrict__ scale, int64_t n_rows,
                                                                    int64_t k, int64_t br, int64_t bc,
                                                                    int64_t scale_cols, void* __restrict__ out) {
  const int64_t bytes_per_row = kFp4 ? (k + 1) / 2 : k;
  const int64_t total = n_rows * bytes_per_row;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = t / bytes_per_row, j = t - n * bytes_per_row;
    const uint32_t b = data[t];
    const float* srow = scale + (n / br) * scale_cols;
    float v[2];
    int cnt = 1;
    int64_t c0 = j;
    if (kFp4) {
      const f32x2 f = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(b, 1.0f, 0);  // low nibble = column 2j
      v[0] = f[0];
      v[1] = f[1];
      c0 = 2 * j;
      cnt = c0 + 1 < k ? 2 : 1;
    } else {
      v[0] = __builtin_amdgcn_cvt_pk_f32_fp8(b, false)[0];
    }
    for (int u = 0; u < cnt; ++u) {
      const int64_t c = c0 + u;
      const float x = __fmul_rn(v[u], srow[c / bc]);
      if (kOutF32) reinterpret_cast<float*>(out)[n * k + c] = x;
      else reinterpret_cast<uint16_t*>(out)[n * k + c] = (uint16_t)f32_to_bf16_bits(x);
    }
  }
}

inline int blocks_for(int64_t n_items) {
  int64_t b = (n_items + kThreads - 1) / kThreads;
  if (b > 1048576) b = 1048576;
  return (int)(b < 1 ? 1 : b);
}

}  // namespace
}  // namespace hsmoe

using namespace hsmoe;

extern "C" int hsmoe_fp4_dequant_bf16(const void* packed, const void* scale, int scale_kind, int64_t n_rows,
                                      int64_t k, int64_t packed_row_stride, int64_t scale_row_stride, void* out,
                                      int64_t out_row_stride, hsmoe_stream_t stream) {
  if (!packed || !scale || !out || n_rows < 0 || k < 0)
    return fail(HSMOE_ERR_ARG, "hsmoe_fp4_dequant_bf16: null pointer or negative size");
  if (scale_kind != HSMOE_SCALE_E8M0 && scale_kind != HSMOE_SCALE_F32)
    return fail(HSMOE_ERR_ARG, "hsmoe_fp4_dequant_bf16: unknown scale_kind %d", scale_kind);
  if (k % 32 != 0) return fail(HSMOE_ERR_SHAPE, "hsmoe_fp4_dequant_bf16: k=%lld is not a multiple of 32", (long long)k);
  if (packed_row_stride < k / 2 || scale_row_stride < k / 32 || out_row_stride < k)
    return fail(HSMOE_ERR_SHAPE, "hsmoe_fp4_dequant_bf16: row stride smaller than the row");
  if (!aligned(packed, 16) || packed_row_stride % 16 != 0 || !aligned(out, 16) || out_row_stride % 8 != 0)
    return fail(HSMOE_ERR_SHAPE, "hsmoe_fp4_dequant_bf16: packed rows and out rows must be 16-byte aligned");
  if (scale_kind == HSMOE_SCALE_F32 && !aligned(scale, 4))
    return fail(HSMOE_ERR_SHAPE, "hsmoe_fp4_dequant_bf16: fp32 scales must be 4-byte aligned");
  if (n_rows == 0 || k == 0) return HSMOE_OK;
  int64_t groups = k / 32;
  int nb = blocks_for(n_rows * groups);
  if (scale_kind == HSMOE_SCALE_E8M0)
    hipLaunchKernelGGL(fp4_dequant_kernel<kScaleE8M0>, dim3(nb), dim3(kThreads), 0, (hipStream_t)stream,
                       (const uint8_t*)packed, scale, n_rows, groups, packed_row_stride, scale_row_stride,
                       (uint16_t*)out, out_row_stride);
  else
    hipLaunchKernelGGL(fp4_dequant_kernel<kScaleF32>, dim3(nb), dim3(kThreads), 0, (hipStream_t)stream,
                       (const uint8_t*)packed, scale, n_rows, groups, packed_row_stride, scale_row_stride,
                       (uint16_t*)out, out_row_stride);
  return check_launch("hsmoe_fp4_dequant_bf16");
}

extern "C" int hsmoe_fp8_dequant_bf16(const void* data, const float* scale, int64_t n_rows, int64_t k, void* out,
                                      hsmoe_stream_t stream) {
  if (!data || !scale || !out || n_rows < 0 || k < 0)
    return fail(HSMOE_ERR_ARG, "hsmoe_fp8_dequant_bf16: null pointer or negative size");
  if (k % 8 != 0) return fail(HSMOE_ERR_SHAPE, "hsmoe_fp8_dequant_bf16: k=%lld is not a multiple of 8", (long long)k);
  if (!aligned(data, 8) || !aligned(out, 16) || !aligned(scale, 4))
    return fail(HSMOE_ERR_SHAPE, "hsmoe_fp8_dequant_bf16: misaligned data/out/scale");
  if (n_rows == 0 || k == 0) return HSMOE_OK;
  hipLaunchKernelGGL(fp8_dequant_kernel, dim3(blocks_for(n_rows * (k / 8))), dim3(kThreads), 0, (hipStream_t)stream,
                     (const uint8_t*)data, scale, n_rows, k, (uint16_t*)out);
  return check_launch("hsmoe_fp8_dequant_bf16");
}

extern "C" int hsmoe_dequant_blocked(const void* data, int data_kind, const float* scale, int64_t n_rows, int64_t k,
                                     int64_t block_rows, int64_t block_cols, int64_t scale_cols, void* out,
                                     int out_kind, hsmoe_stream_t stream) {
  const char* name = "hsmoe_dequant_blocked";
  if (!data || !scale || !out || n_rows < 0 || k < 0) return fail(HSMOE_ERR_ARG, "%s: null pointer or negative size", name);
  if (data_kind != HSMOE_DATA_FP4 && data_kind != HSMOE_DATA_E4M3)
    return fail(HSMOE_ERR_ARG, "%s: unknown data_kind %d", name, data_kind);
  if (out_kind != HSMOE_OUT_F32 && out_kind != HSMOE_OUT_BF16)
    return fail(HSMOE_ERR_ARG, "%s: unknown out_kind %d", name, out_kind);
  if (block_rows < 1 || block_cols < 1 || scale_cols < (k + block_cols - 1) / block_cols)
    return fail(HSMOE_ERR_SHAPE, "%s: blocks must be >= 1 and a scale row must cover k columns", name);
  if (data_kind == HSMOE_DATA_FP4 && k % 2 != 0)
    return fail(HSMOE_ERR_SHAPE, "%s: FP4 rows hold two columns per byte (k=%lld is odd)", name, (long long)k);
  if (!aligned(scale, 4) || !aligned(out, out_kind == HSMOE_OUT_F32 ? 4 : 2))
    return fail(HSMOE_ERR_SHAPE, "%s: misaligned scale or out", name);
  if (n_rows == 0 || k == 0) return HSMOE_OK;
  const bool fp4 = data_kind == HSMOE_DATA_FP4, f32 = out_kind == HSMOE_OUT_F32;
  const int nb = blocks_for(n_rows * (fp4 ? k / 2 : k));
  const dim3 grid(nb), block(kThreads);
  hipStream_t st = (hipStream_t)stream;
  const uint8_t* d = (const uint8_t*)data;
  if (fp4 && f32) hipLaunchKernelGGL((dequant_blocked_kernel<true, true>), grid, block, 0, st, d, scale, n_rows, k, block_rows, block_cols, scale_cols, out);
  else if (fp4) hipLaunchKernelGGL((dequant_blocked_kernel<true, false>), grid, block, 0, st, d, scale, n_rows, k, block_rows, block_cols, scale_cols, out);
  else if (f32) hipLaunchKernelGGL((dequant_blocked_kernel<false, true>), grid, block, 0, st, d, scale, n_rows, k, block_rows, block_cols, scale_cols, out);
  else hipLaunchKernelGGL((dequant_blocked_kernel<false, false>), grid, block, 0, st, d, scale, n_rows, k, block_rows, block_cols, scale_cols, out);
  return check_launch(name);
}
