// Streaming-read floor: what a kernel that only reads K/V-sized buffers achieves, the bound the
// decode kernels are measured against (no counterpart in the reference: a measurement aid).
//
// Every workgroup reads one contiguous slice of the buffer with 16-byte loads, eight in flight a
// lane (nontemporal, as the decode tiles are read, or plain), and folds them by XOR into one word
// so the loads stay; the workgroup's word goes to sink[block]. The XOR of all words equals the
// XOR of the buffer's 32-bit words exactly when every 16 bytes were read once.
#include "bg_kernels.h"

namespace bg {

typedef unsigned u32x4d __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ u32x4d rd16(const u32x4d* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}

template <bool NT>
__global__ __launch_bounds__(512) void stream_read_kernel(const u32x4d* __restrict__ p, size_t n16, unsigned* sink) {
  const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const size_t b0 = (size_t)blockIdx.x * per;
  const size_t b1 = b0 + per < n16 ? b0 + per : n16;
  const size_t bd = blockDim.x;
  unsigned acc = 0;
  size_t i = b0 + threadIdx.x;
  for (; i + 7 * bd < b1; i += 8 * bd) {
    u32x4d v[8];
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = rd16<NT>(p + i + j * bd);
#pragma unroll
    for (int j = 0; j < 8; j++) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  }
  for (; i < b1; i += bd) {
    const u32x4d v = rd16<NT>(p + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  // workgroup fold: lanes by shuffles, waves through LDS
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o);
  __shared__ unsigned wacc[16];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) wacc[wave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned a = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) a ^= wacc[w];
    sink[blockIdx.x] = a;
  }
}

hipError_t launch_stream_read(const void* buf, size_t bytes, int workgroups, bool nontemporal, unsigned* sink,
                              hipStream_t st) {
  const size_t n16 = bytes / 16;
  if (nontemporal)
    hipLaunchKernelGGL(stream_read_kernel<true>, dim3(workgroups), dim3(512), 0, st, (const u32x4d*)buf, n16, sink);
  else
    hipLaunchKernelGGL(stream_read_kernel<false>, dim3(workgroups), dim3(512), 0, st, (const u32x4d*)buf, n16, sink);
  return hipGetLastError();
}

}  // namespace bg
