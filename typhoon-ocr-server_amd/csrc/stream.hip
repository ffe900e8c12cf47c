// stream.hip -- a plain streaming read of a device buffer: the floor a
// kernel launch that reads the same bytes once can reach on this device
// (launch, first-byte latency, ramp and drain included).  A measurement aid
// for the HBM-bound GEMVs: their time over this kernel's time for the same
// byte count is how close they stand to what the hardware gives a single
// launch, which the 8 TB/s peak does not show for a few MB.
//
// Grid-stride loop of U non-temporal 16-byte loads per lane in flight (the
// loads of the GEMV weight stream), folded by xor; the fold is written only
// if it equals a value no buffer of this library produces, which keeps the
// loads live without a store per work-group.
#include "tl_common.h"
#include "tl_kernels.h"

namespace tl {

template <int U>
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ p, size_t n16,
                                                          uint32_t* sink) {
  typedef unsigned int v4u_t __attribute__((ext_vector_type(4)));
  const v4u_t* q = reinterpret_cast<const v4u_t*>(p);
  uint32_t acc = 0;
  const size_t stride = (size_t)gridDim.x * 256 * U;
  size_t i = (size_t)blockIdx.x * 256 * U + threadIdx.x;
  for (; i + 256 * (U - 1) < n16; i += stride) {
    v4u_t v[U];
#pragma unroll
    for (int u = 0; u < U; u++) v[u] = __builtin_nontemporal_load(q + i + 256 * u);
#pragma unroll
    for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  // the last partial pass: one load at a time
  for (; i < n16; i += 256) {
    const v4u_t v = __builtin_nontemporal_load(q + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

hipError_t launch_stream_read(const void* p, size_t bytes, int grid, int u, uint32_t* sink, hipStream_t st) {
  if (!p || !sink || bytes == 0 || bytes % 16 != 0 || (((uintptr_t)p) & 15) != 0) return hipErrorInvalidValue;
  if (grid < 1 || grid > 65536 || (u != 4 && u != 8)) return hipErrorInvalidValue;
  const size_t n16 = bytes / 16;
  if (u == 4) hipLaunchKernelGGL(stream_read_kernel<4>, dim3(grid), dim3(256), 0, st, (const uint4*)p, n16, sink);
  else hipLaunchKernelGGL(stream_read_kernel<8>, dim3(grid), dim3(256), 0, st, (const uint4*)p, n16, sink);
  return hipGetLastError();
}

}  // namespace tl

extern "C" hipError_t tlk_launch_stream_read(const void* p, size_t bytes, int grid, int u, uint32_t* sink,
                                             hipStream_t st) {
  return tl::launch_stream_read(p, bytes, grid, u, sink, st);
}
