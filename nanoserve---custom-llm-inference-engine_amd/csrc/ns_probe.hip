// Bandwidth reference for the benchmark (not part of the sampler's ABI): the decode batch's
// rows read in exactly the layout and cache policy of the one-workgroup-per-row top-k kernel
// (1024 threads per row, 16-byte chunk q * 1024 + t to thread t, 16 chunks per thread, all
// held in registers, non-temporal buffer loads), with no sampling work: each wave reduces its
// bits with cross-lane operations and one lane stores the wave's result.  Its time per call is
// the floor a one-pass kernel over these rows reaches.  (A reduction through one LDS word, all
// threads atomically, serialises 1024 LDS atomics per row and costs about 3 us on its own.)
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {
constexpr int kThreads = 1024;
constexpr int kChunks = 16;
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void read_rows_kernel(const unsigned char* src, int64_t row_stride_bytes,
                                                             uint32_t row_bytes, uint32_t* out) {
  const unsigned char* rp = src + (int64_t)blockIdx.x * row_stride_bytes;
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(rp), (short)0, (int)row_bytes, 0x00020000);
  v4u v[kChunks];
#pragma unroll
  for (int q = 0; q < kChunks; ++q) {
    v[q] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(
                                       r, (int)((uint32_t)(q * kThreads + threadIdx.x) * 16u), 0, 2));
    __builtin_amdgcn_sched_barrier(0);
  }
  uint32_t m = 0u;
#pragma unroll
  for (int q = 0; q < kChunks; ++q) m = max(m, max(max(v[q].x, v[q].y), max(v[q].z, v[q].w)));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o));
  if ((threadIdx.x & 63) == 0) out[blockIdx.x * (kThreads / 64) + threadIdx.x / 64] = m;
}
}  // namespace

// Read rows [0, rows) of `src` (row_stride_bytes apart, row_bytes each, both multiples of 16,
// row_bytes <= 16 * 1024 * 16): out[r * 16 + w] receives a reduction of wave w's share of row
// r (out holds rows * 16 words).  0 on success.
extern "C" int ns_probe_read_rows(const void* src, int64_t row_stride_bytes, int64_t row_bytes, int32_t rows,
                                  uint32_t* out, hipStream_t stream) {
  if (src == nullptr || out == nullptr || rows <= 0 || row_bytes <= 0 || row_bytes % 16 != 0 ||
      row_stride_bytes < row_bytes || row_bytes > (int64_t)kThreads * kChunks * 16)
    return 1;
  hipLaunchKernelGGL(read_rows_kernel, dim3((unsigned)rows), dim3(kThreads), 0, stream,
                     static_cast<const unsigned char*>(src), row_stride_bytes, (uint32_t)row_bytes, out);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
