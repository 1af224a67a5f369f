// Measurement helper for bench.py (not part of the W8A16 C ABI): a plain
// streaming read of a device buffer, the same non-temporal 128-bit loads the
// decode GEMV issues for its weights, with no arithmetic, no activations and
// no epilogue.  Timed over the same sequence of byte counts as a decode step,
// it gives the rate that launch structure allows on the device (launch gaps,
// ramp-up and drain included): the envelope the GEMV is compared against.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__global__ __launch_bounds__(512) void stream_read_kernel(const uint4* __restrict__ p, size_t n16,
                                                          uint32_t* sink) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  uint32_t acc = 0;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
#pragma unroll 8
  for (; i < n16; i += stride) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p) + i);
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  // Data-dependent store that (almost) never happens keeps the loads alive.
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

}  // namespace

// Reads `bytes` (a multiple of 16) at `p` on `stream`; `sink` is a 4-byte
// device word the kernel may write.  Grid measured on MI355X: 1024 x 512 up
// to 40 MB, 2048 x 512 above.  Returns the hipError_t of the launch.
extern "C" int rf_bench_stream_read(const void* p, size_t bytes, void* sink, void* stream) {
  if (!p || !sink || bytes == 0 || bytes % 16 != 0) return (int)hipErrorInvalidValue;
  const int blocks = bytes <= (40u << 20) ? 1024 : 2048;
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(512), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(p), bytes / 16, static_cast<uint32_t*>(sink));
  return (int)hipGetLastError();
}
