// XOR checksum of a device buffer: a read-only stream at the HBM read rate.
//
// The expert store is written once (generated on the device or loaded from a
// checkpoint) and then only read; its checksum is the XOR of all its 16-byte
// words, a value the host can recompute from the same bytes and that is
// linear over concatenation (the checksum of a buffer is the XOR of the
// checksums of its pieces), so a store of any size can be checked piecewise.
// The same kernel is the library's measure of the read bandwidth a
// single-pass stream reaches on the device (it moves nothing but loads).
//
// Pass 1: workgroup b XORs the 32 KiB chunks b, b + G, b + 2G, ...: every
// lane has 8 loads of 16 bytes in flight per chunk (the chunk's next 4 KiB
// per load instruction of the workgroup, 1 KiB contiguous per wave), and
// the lane's words of the next chunk are loaded before the current chunk is
// folded.  G is one workgroup per CU: about 32-64 KiB in flight per CU is
// where the stream reads fastest on MI355X (6.45-6.49 TB/s over 1 GiB);
// 4 workgroups of 64 KiB chunks per CU (256 KiB in flight) read at
// 5.87-5.92 TB/s, the queues behind each channel only adding latency.
// The workgroup's XOR goes to partial[b].  Pass 2: one workgroup folds the
// G partials.
#include "hsmoe_internal.h"
#include "hsmoe_common.h"

namespace hsmoe {
namespace {

constexpr int kThreads = 256;
constexpr int kLoads = 8;                                 // 16-byte loads per lane per chunk
constexpr int64_t kChunk = (int64_t)kThreads * kLoads;  // 16-byte words per chunk (32 KiB)
constexpr int kMaxGrid = 4096;

__device__ __forceinline__ uint4 xor4(uint4 a, uint4 b) {
  return make_uint4(a.x ^ b.x, a.y ^ b.y, a.z ^ b.z, a.w ^ b.w);
}

__device__ __forceinline__ uint4 wave_xor(uint4 v) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) {
    v.x ^= __shfl_xor(v.x, s);
    v.y ^= __shfl_xor(v.y, s);
    v.z ^= __shfl_xor(v.z, s);
    v.w ^= __shfl_xor(v.w, s);
  }
  return v;
}

// XOR of the block's values into out (thread 0 stores it).
__device__ __forceinline__ void block_xor_store(uint4 acc, uint4* out) {
  __shared__ uint4 part[kThreads / 64];
  acc = wave_xor(acc);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint4 r = part[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) r = xor4(r, part[w]);
    *out = r;
  }
}

__global__ void __launch_bounds__(kThreads) xor_stream_kernel(const uint4* __restrict__ src, int64_t n16,
                                                              uint4* __restrict__ partial) {
  const int64_t n_chunks = (n16 + kChunk - 1) / kChunk;
  uint4 acc = make_uint4(0u, 0u, 0u, 0u);
  int64_t c = blockIdx.x;
  uint4 v[kLoads];
  auto issue = [&](int64_t chunk) {
    const int64_t base = chunk * kChunk + threadIdx.x;
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const int64_t k = base + (int64_t)j * kThreads;
      v[j] = k < n16 ? ldg<uint4>(src + k) : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  if (c < n_chunks) issue(c);
  while (c < n_chunks) {
    uint4 cur[kLoads];
#pragma unroll
    for (int j = 0; j < kLoads; ++j) cur[j] = v[j];
    c += gridDim.x;
    if (c < n_chunks) issue(c);  // the next chunk's loads go out before this one is folded
#pragma unroll
    for (int j = 0; j < kLoads; ++j) acc = xor4(acc, cur[j]);
  }
  block_xor_store(acc, partial + blockIdx.x);
}

__global__ void __launch_bounds__(kThreads) xor_fold_kernel(const uint4* __restrict__ partial, int n,
                                                            uint4* __restrict__ out) {
  uint4 acc = make_uint4(0u, 0u, 0u, 0u);
  for (int k = threadIdx.x; k < n; k += kThreads) acc = xor4(acc, partial[k]);
  block_xor_store(acc, out);
}

int grid_for(int64_t n16) {
  const int64_t n_chunks = (n16 + kChunk - 1) / kChunk;
  int64_t g = device_cus();  // one workgroup (4 waves) per CU
  if (g > kMaxGrid) g = kMaxGrid;
  if (g > n_chunks) g = n_chunks;
  return g < 1 ? 1 : (int)g;
}

}  // namespace
}  // namespace hsmoe

using namespace hsmoe;

extern "C" size_t hsmoe_xor_checksum_workspace_size(void) { return (size_t)kMaxGrid * 16; }

extern "C" int hsmoe_xor_checksum(const void* data, int64_t nbytes, void* out, void* workspace,
                                  size_t workspace_bytes, hsmoe_stream_t stream) {
  const char* name = "hsmoe_xor_checksum";
  if (!out || (!data && nbytes > 0)) return fail(HSMOE_ERR_ARG, "%s: null pointer", name);
  if (nbytes < 0 || nbytes % 16 != 0)
    return fail(HSMOE_ERR_SHAPE, "%s: nbytes must be a non-negative multiple of 16 (got %lld)", name,
                (long long)nbytes);
  if ((data && !aligned(data, 16)) || !aligned(out, 16))
    return fail(HSMOE_ERR_SHAPE, "%s: data and out must be 16-byte aligned", name);
  if (!workspace || workspace_bytes < hsmoe_xor_checksum_workspace_size() || !aligned(workspace, 16))
    return fail(HSMOE_ERR_WORKSPACE, "%s: workspace of %zu bytes (16-byte aligned) needed", name,
                hsmoe_xor_checksum_workspace_size());
  const int64_t n16 = nbytes / 16;
  const int grid = grid_for(n16);
  uint4* partial = (uint4*)workspace;
  hipLaunchKernelGGL(xor_stream_kernel, dim3((unsigned)grid), dim3(kThreads), 0, (hipStream_t)stream,
                     (const uint4*)data, n16, partial);
  int rc = check_launch(name);
  if (rc) return rc;
  hipLaunchKernelGGL(xor_fold_kernel, dim3(1), dim3(kThreads), 0, (hipStream_t)stream, (const uint4*)partial, grid,
                     (uint4*)out);
  return check_launch(name);
}
