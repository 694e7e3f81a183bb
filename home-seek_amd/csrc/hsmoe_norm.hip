// RMSNorm between MoE layers, restating rms_norm (utils.py:6-9):
//   var = mean(float(x)^2); y = float(w) * (float(x) * rsqrt(var + eps)); out = bf16(y)
// One workgroup per row; fixed-order tree sum, so results are deterministic.
#include "hsmoe_common.h"
#include "hsmoe_internal.h"

namespace hsmoe {
namespace {

__global__ void __launch_bounds__(256) rms_norm_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                       int64_t d, float eps, uint16_t* __restrict__ out) {
  __shared__ float part[256];
  const uint16_t* xr = x + (int64_t)blockIdx.x * d;
  float s = 0.0f;
  for (int64_t c = threadIdx.x; c < d; c += 256) {
    const float v = bf16_bits_to_f32(xr[c]);
    s = __fmaf_rn(v, v, s);
  }
  part[threadIdx.x] = s;
  __syncthreads();
  for (int off = 128; off >= 1; off >>= 1) {
    if (threadIdx.x < off) part[threadIdx.x] = __fadd_rn(part[threadIdx.x], part[threadIdx.x + off]);
    __syncthreads();
  }
  const float var = __fdiv_rn(part[0], (float)d);
  const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(var, eps)));
  uint16_t* orow = out + (int64_t)blockIdx.x * d;
  for (int64_t c = threadIdx.x; c < d; c += 256) {
    const float xn = __fmul_rn(bf16_bits_to_f32(xr[c]), inv);
    orow[c] = (uint16_t)f32_to_bf16_bits(__fmul_rn(bf16_bits_to_f32(w[c]), xn));
  }
}

}  // namespace
}  // namespace hsmoe

using namespace hsmoe;

extern "C" int hsmoe_rms_norm(const void* x, const void* w, int64_t rows, int64_t d, float eps, void* out,
                              hsmoe_stream_t stream) {
  if (!x || !w || !out || rows < 0 || d < 1) return fail(HSMOE_ERR_ARG, "hsmoe_rms_norm: bad arguments");
  if (rows == 0) return HSMOE_OK;
  hipLaunchKernelGGL(rms_norm_kernel, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream, (const uint16_t*)x,
                     (const uint16_t*)w, d, eps, (uint16_t*)out);
  return check_launch("hsmoe_rms_norm");
}
