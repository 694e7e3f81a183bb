// Counter-based synthetic data generators.  Value i of a stream depends only on
// (key, i), so the host oracle regenerates any slice bit for bit.  Every float
// operation is an explicitly rounded single op (__fmul_rn/__fadd_rn), so no
// contraction into FMA can change a result.
#include "hsmoe_common.h"
#include "hsmoe_internal.h"

namespace hsmoe {
namespace {

constexpr int kThreads = 256;

inline int blocks_for(int64_t n_items) {
  int64_t b = (n_items + kThreads - 1) / kThreads;
  if (b > 65536) b = 65536;  // grid-stride loops cover the rest
  return (int)(b < 1 ? 1 : b);
}

// bytes[b] = byte (b % 8) of rand(key, b / 8); e4m3 mode maps 0x7F/0xFF to 0x7E/0xFE.
template <bool kE4M3>
__global__ void gen_bytes_kernel(uint64_t key, int64_t n, uint8_t* __restrict__ out) {
  int64_t n_words = (n + 7) / 8;
  for (int64_t w = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; w < n_words; w += (int64_t)gridDim.x * blockDim.x) {
    uint64_t r = rand64(key, (uint64_t)w);
    if (kE4M3) {
      // per byte: if (b & 0x7F) == 0x7F then b ^= 1
      uint64_t low7 = r & 0x7f7f7f7f7f7f7f7full;
      uint64_t is_nan = ((low7 + 0x0101010101010101ull) & 0x8080808080808080ull) >> 7;  // 1 where low7 == 0x7F
      r ^= is_nan;
    }
    if (w * 8 + 8 <= n) {
      *reinterpret_cast<uint64_t*>(out + w * 8) = r;
    } else {
      for (int q = 0; w * 8 + q < n; ++q) out[w * 8 + q] = (uint8_t)(r >> (8 * q));
    }
  }
}

__global__ void gen_e8m0_kernel(uint64_t key, int64_t n, int lo, int span, uint8_t* __restrict__ out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    uint64_t r = rand64(key, (uint64_t)i);
    out[i] = (uint8_t)(lo + (int)(((r >> 32) * (uint64_t)span) >> 32));
  }
}

__device__ __forceinline__ float normal_f32(uint64_t key, uint64_t i, float mean, float stdv) {
  uint64_t r = rand64(key, i);
  int32_t s = (int32_t)(r & 0xffff) + (int32_t)((r >> 16) & 0xffff) + (int32_t)((r >> 32) & 0xffff) +
              (int32_t)((r >> 48) & 0xffff);
  float z = __fmul_rn((float)(s - 131070), 2.642899103e-05f);
  return __fadd_rn(mean, __fmul_rn(stdv, z));
}

template <bool kBf16>
__global__ void gen_normal_kernel(uint64_t key, int64_t n, float mean, float stdv, void* __restrict__ out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float v = normal_f32(key, (uint64_t)i, mean, stdv);
    if (kBf16)
      reinterpret_cast<uint16_t*>(out)[i] = (uint16_t)f32_to_bf16_bits(v);
    else
      reinterpret_cast<float*>(out)[i] = v;
  }
}

__global__ void gen_uniform_kernel(uint64_t key, int64_t n, float lo, float hi, float mul, float* __restrict__ out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    uint64_t r = rand64(key, (uint64_t)i);
    float f = __fmul_rn((float)(r >> 40), 5.9604644775390625e-08f);
    float v = __fadd_rn(lo, __fmul_rn(__fadd_rn(hi, -lo), f));
    out[i] = __fmul_rn(v, mul);
  }
}

// Index uniform over [0, n_values): ((r >> 32) * n_values) >> 32.
__global__ void gen_index_kernel(uint64_t key, int64_t n, uint32_t n_values, int64_t* __restrict__ out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const uint64_t r = rand64(key, (uint64_t)i);
    out[i] = (int64_t)(((r >> 32) * (uint64_t)n_values) >> 32);
  }
}

}  // namespace
}  // namespace hsmoe

using namespace hsmoe;

extern "C" int hsmoe_gen_bytes(uint64_t key, int64_t n, void* out, hsmoe_stream_t stream) {
  if (n < 0 || (n > 0 && !out)) return fail(HSMOE_ERR_ARG, "hsmoe_gen_bytes: bad arguments");
  if (!aligned(out, 8)) return fail(HSMOE_ERR_SHAPE, "hsmoe_gen_bytes: output must be 8-byte aligned");
  if (n == 0) return HSMOE_OK;
  hipLaunchKernelGGL(gen_bytes_kernel<false>, dim3(blocks_for((n + 7) / 8)), dim3(kThreads), 0, (hipStream_t)stream,
                     key, n, (uint8_t*)out);
  return check_launch("hsmoe_gen_bytes");
}

extern "C" int hsmoe_gen_e4m3(uint64_t key, int64_t n, void* out, hsmoe_stream_t stream) {
  if (n < 0 || (n > 0 && !out)) return fail(HSMOE_ERR_ARG, "hsmoe_gen_e4m3: bad arguments");
  if (!aligned(out, 8)) return fail(HSMOE_ERR_SHAPE, "hsmoe_gen_e4m3: output must be 8-byte aligned");
  if (n == 0) return HSMOE_OK;
  hipLaunchKernelGGL(gen_bytes_kernel<true>, dim3(blocks_for((n + 7) / 8)), dim3(kThreads), 0, (hipStream_t)stream,
                     key, n, (uint8_t*)out);
  return check_launch("hsmoe_gen_e4m3");
}

extern "C" int hsmoe_gen_e8m0(uint64_t key, int64_t n, int lo, int span, void* out, hsmoe_stream_t stream) {
  if (n < 0 || (n > 0 && !out) || span < 1 || lo < 0 || lo + span > 256)
    return fail(HSMOE_ERR_ARG, "hsmoe_gen_e8m0: bad arguments");
  if (n == 0) return HSMOE_OK;
  hipLaunchKernelGGL(gen_e8m0_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, (hipStream_t)stream, key, n, lo, span,
                     (uint8_t*)out);
  return check_launch("hsmoe_gen_e8m0");
}

extern "C" int hsmoe_gen_normal(uint64_t key, int64_t n, float mean, float stdv, int as_bf16, void* out,
                                hsmoe_stream_t stream) {
  if (n < 0 || (n > 0 && !out)) return fail(HSMOE_ERR_ARG, "hsmoe_gen_normal: bad arguments");
  if (n == 0) return HSMOE_OK;
  if (as_bf16)
    hipLaunchKernelGGL(gen_normal_kernel<true>, dim3(blocks_for(n)), dim3(kThreads), 0, (hipStream_t)stream, key, n,
                       mean, stdv, out);
  else
    hipLaunchKernelGGL(gen_normal_kernel<false>, dim3(blocks_for(n)), dim3(kThreads), 0, (hipStream_t)stream, key, n,
                       mean, stdv, out);
  return check_launch("hsmoe_gen_normal");
}

extern "C" int hsmoe_gen_uniform(uint64_t key, int64_t n, float lo, float hi, float mul, float* out,
                                 hsmoe_stream_t stream) {
  if (n < 0 || (n > 0 && !out)) return fail(HSMOE_ERR_ARG, "hsmoe_gen_uniform: bad arguments");
  if (n == 0) return HSMOE_OK;
  hipLaunchKernelGGL(gen_uniform_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, (hipStream_t)stream, key, n, lo, hi,
                     mul, out);
  return check_launch("hsmoe_gen_uniform");
}

extern "C" int hsmoe_gen_index(uint64_t key, int64_t n, int64_t n_values, int64_t* out, hsmoe_stream_t stream) {
  if (n < 0 || (n > 0 && !out) || n_values < 1 || n_values > 0xffffffffll)
    return fail(HSMOE_ERR_ARG, "hsmoe_gen_index: bad arguments");
  if (n == 0) return HSMOE_OK;
  hipLaunchKernelGGL(gen_index_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, (hipStream_t)stream, key, n,
                     (uint32_t)n_values, out);
  return check_launch("hsmoe_gen_index");
}
