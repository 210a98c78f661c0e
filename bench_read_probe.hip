// bench_read_probe.hip -- bandwidth reference for bench.py, not part of the
// library: the time of a plain read of N bytes, which bounds what any kernel
// reading those N bytes once can reach on this device.  Two access shapes,
// each with U independent 16-byte loads in flight per lane:
//   mode 0: grid stride over the whole buffer;
//   mode 1: each workgroup reads one contiguous span (as the decode's
//           workgroups read their token chunks), every lane issuing its U
//           loads before it uses any.
// The loaded words are xor-folded into a value that is stored only if it
// equals a constant, so no load is optimised away.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kBlock = 256;

template <int U>
__global__ __launch_bounds__(kBlock) void read_stride_kernel(const uint4 *__restrict__ p, size_t n16,
                                                             uint32_t *sink) {
  const size_t stride = (size_t)gridDim.x * kBlock;
  size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (U - 1) * stride < n16; i += U * stride) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) v[u] = p[i + u * stride];
#pragma unroll
    for (int u = 0; u < U; u++) acc ^= v[u].x + v[u].y + v[u].z + v[u].w;
  }
  for (; i < n16; i += stride) {
    const uint4 v = p[i];
    acc ^= v.x + v.y + v.z + v.w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;  // practically never; keeps the loads
}

template <int U>
__global__ __launch_bounds__(kBlock) void read_span_kernel(const uint4 *__restrict__ p, size_t n16, uint32_t *sink) {
  const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const size_t b0 = (size_t)blockIdx.x * per;
  const size_t b1 = b0 + per < n16 ? b0 + per : n16;
  uint32_t acc = 0;
  size_t i = b0 + threadIdx.x;
  for (; i + (U - 1) * kBlock < b1; i += U * kBlock) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) v[u] = p[i + u * kBlock];
#pragma unroll
    for (int u = 0; u < U; u++) acc ^= v[u].x + v[u].y + v[u].z + v[u].w;
  }
  for (; i < b1; i += kBlock) {
    const uint4 v = p[i];
    acc ^= v.x + v.y + v.z + v.w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

template <int U>
void launch(int mode, const uint4 *p, size_t n16, int grid, uint32_t *sink, hipStream_t s) {
  if (mode == 0) hipLaunchKernelGGL(read_stride_kernel<U>, dim3((unsigned)grid), dim3(kBlock), 0, s, p, n16, sink);
  else hipLaunchKernelGGL(read_span_kernel<U>, dim3((unsigned)grid), dim3(kBlock), 0, s, p, n16, sink);
}

}  // namespace

// Reads `bytes` (a multiple of 16, 16-byte aligned) with `grid` workgroups of
// 256 lanes, `unroll` in {1, 4, 8} loads in flight per lane, access `mode` 0
// or 1.  Returns 0, or 1 for invalid arguments, 2 for a launch error.
extern "C" int tq_probe_read(const void *buf, size_t bytes, int grid, int unroll, int mode, void *sink,
                             hipStream_t stream) {
  if (!buf || !sink || grid <= 0 || (bytes & 15u) || ((uintptr_t)buf & 15u) || (mode != 0 && mode != 1)) return 1;
  const uint4 *p = static_cast<const uint4 *>(buf);
  uint32_t *sk = static_cast<uint32_t *>(sink);
  if (unroll == 1) launch<1>(mode, p, bytes / 16, grid, sk, stream);
  else if (unroll == 4) launch<4>(mode, p, bytes / 16, grid, sk, stream);
  else if (unroll == 8) launch<8>(mode, p, bytes / 16, grid, sk, stream);
  else return 1;
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
