// C-ABI layer: validation, kernel choice, workspace sizing, weight packing.
//
// Validation mirrors the reference launchers' TORCH_CHECKs
// (src/ops/rpu_linear.cpp:1119-1134 -- int8 [N,K] weight, fp16 [N] scale,
// byte extents; src/ops/rpu_linear_gemv.cpp:105-123 -- scale.numel()==N,
// alignment) but returns status codes; the torch op turns them into errors.
// Unlike the RPU the kernels accept every M, N >= 1 and K % 8 == 0: there is
// no core partition to satisfy (runtime/weights.py:97-135), only the
// 16-byte activation-row alignment of a 128-bit load.
#include <limits.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "../../include/w8a16.h"
#include "w8a16_common.h"
#include "w8a16_internal.h"

namespace rf {

// ---------------------------------------------------------------------------
// Device properties, cached per device (read-only after the first query).
// ---------------------------------------------------------------------------
int device_info(DeviceInfo* out) {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> state[kMaxDevices];  // 0 = unknown, 1 = cached
  static DeviceInfo cache[kMaxDevices];
  static std::mutex mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return RF_W8A16_EHIP;
  if (dev < 0 || dev >= kMaxDevices) return RF_W8A16_EDEVICE;
  if (state[dev].load(std::memory_order_acquire) == 0) {
    std::lock_guard<std::mutex> g(mu);
    if (state[dev].load(std::memory_order_relaxed) == 0) {
      hipDeviceProp_t prop;
      if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return RF_W8A16_EHIP;
      DeviceInfo d;
      d.cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
      d.gfx950 = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
      cache[dev] = d;
      state[dev].store(1, std::memory_order_release);
    }
  }
  *out = cache[dev];
  return RF_W8A16_OK;
}

// ---------------------------------------------------------------------------
// Device repack kernel: one thread per 16-byte lane chunk of a tile.
// ---------------------------------------------------------------------------
namespace {
__global__ void pack_kernel(const int8_t* __restrict__ q, int64_t N, int64_t K, int64_t ldq,
                            uint8_t* __restrict__ dst, int64_t kblocks, int64_t chunks) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= chunks) return;
  const int64_t tile = idx >> 6;
  const int lane = (int)(idx & 63);
  const int64_t nb = tile / kblocks, kb = tile % kblocks;
  const int64_t n = nb * 16 + (lane & 15);
  const int64_t k0 = kb * 64 + 16 * (lane >> 4);
  uint32_t words[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t v = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int64_t k = k0 + w * 4 + b;
      const uint8_t qb = (n < N && k < K) ? (uint8_t)q[n * ldq + k] : 0u;
      v |= (uint32_t)(uint8_t)(qb ^ 0x80u) << (8 * b);
    }
    words[w] = v;
  }
  *reinterpret_cast<uint4*>(dst + idx * 16) = make_uint4(words[0], words[1], words[2], words[3]);
}
}  // namespace

// Int4 (TILE16X128_I4): nibble of position i (0..7) inside a dword.
__host__ __device__ inline int i4_nibble(int i) { return (i & 1) ? 4 + (i >> 1) : (i >> 1); }

namespace {
__global__ void pack4_kernel(const int8_t* __restrict__ q, int64_t N, int64_t K, int64_t ldq,
                             uint8_t* __restrict__ dst, int64_t ktiles, int64_t chunks) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= chunks) return;
  const int64_t tile = idx >> 6;
  const int lane = (int)(idx & 63);
  const int64_t nb = tile / ktiles, kt = tile % ktiles;
  const int64_t n = nb * 16 + (lane & 15);
  const int64_t k0 = kt * 128 + 32 * (lane >> 4);
  uint32_t words[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t k = k0 + 8 * w + i;
      const int qv = (n < N && k < K) ? (int)q[n * ldq + k] : 0;
      v |= (uint32_t)((qv + 8) & 0xF) << (4 * i4_nibble(i));
    }
    words[w] = v;
  }
  *reinterpret_cast<uint4*>(dst + idx * 16) = make_uint4(words[0], words[1], words[2], words[3]);
}
}  // namespace

hipError_t launch_pack4(const int8_t* q, int64_t N, int64_t K, int64_t ldq, uint8_t* dst,
                        hipStream_t stream) {
  const int64_t ktiles = ceil_div(K, 128);
  const int64_t chunks = ceil_div(N, 16) * ktiles * 64;
  const int64_t blocks = ceil_div(chunks, 256);
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(pack4_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, q, N, K, ldq, dst,
                     ktiles, chunks);
  return hipGetLastError();
}

hipError_t launch_pack(const int8_t* q, int64_t N, int64_t K, int64_t ldq, uint8_t* dst,
                       hipStream_t stream) {
  const int64_t kblocks = ceil_div(K, 64);
  const int64_t chunks = ceil_div(N, 16) * kblocks * 64;
  const int64_t blocks = ceil_div(chunks, 256);
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, q, N, K, ldq, dst,
                     kblocks, chunks);
  return hipGetLastError();
}

}  // namespace rf

using rf::ceil_div;
using rf::round_up;

namespace {

constexpr int64_t kMaxDim = (int64_t)1 << 30;

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int check_nk(int64_t N, int64_t K) {
  if (N < 1 || K < 1 || N > kMaxDim || K > kMaxDim) return RF_W8A16_EINVAL;
  return RF_W8A16_OK;
}

// Kernel the AUTO policy picks (N summed over a launch's projections).
// Measured on MI355X over the projections of Qwen3 0.6B..32B, Qwen3-VL-32B,
// Qwen2.5-VL 3B / 7B and the Pi0.5 Gemma decoder and expert (each alone and
// q/k/v, gate/up fused): the GEMV wins up to M = 16; from M = 17 the
// small-tile split-K GEMM wins on every shape but small weights, where the
// GEMV keeps its lead: N*K < 2^25 up to M = 24 (Qwen3-8B q/k/v 6144 x 4096
// at M 24: 10.4 against 12.2 us), N*K <= 2^24 up to M = 28, and up to M = 32
// N*K <= 2^23, or N*K <= 2^24 on N <= 2048 (Qwen3-1.7B down 2048 x 6144 at
// M 32: 9.0 against 12.5 us).  The GEMV runs up to M = 64 when forced.
int auto_kernel(int64_t M, int64_t N, int64_t K) {
  if (M <= 16) return RF_W8A16_KERNEL_GEMV;
  const int64_t nk = N * K;
  if ((M <= 24 && nk < ((int64_t)1 << 25)) || (M <= 28 && nk <= ((int64_t)1 << 24)) ||
      (M <= 32 && (nk <= ((int64_t)1 << 23) || (N <= 2048 && nk <= ((int64_t)1 << 24)))))
    return RF_W8A16_KERNEL_GEMV;
  return RF_W8A16_KERNEL_GEMM;
}

// W4A16 keeps the GEMV up to its M = 64 limit (its GEMM has no small tiles).
int auto_kernel_int4(int64_t M) { return M <= 64 ? RF_W8A16_KERNEL_GEMV : RF_W8A16_KERNEL_GEMM; }

}  // namespace

// ---------------------------------------------------------------------------
// Scratch of rf_w8a16_linear_multi_noalloc: a fixed device array per GPU
// (split-K counters, then fp32 partials), so that entry point allocates
// nothing.  In host code `scratch` is only a stand-in for the symbol: its
// device address, which differs per GPU, comes from hipGetSymbolAddress on
// each device and is the only form passed to kernels.
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint8_t scratch[RF_W8A16_NOALLOC_SCRATCH_BYTES];

namespace {

__global__ void zero_u4_kernel(uint4* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = make_uint4(0, 0, 0, 0);
}

// Device address of the current device's scratch array, looked up once per
// device (with that device current).  A __device__ array without an
// initializer is zero when the code object loads, so the counters start at
// zero, and every call leaves them so.  The first lookup on an uncaptured
// stream clears the counter region once more with a fill kernel (no memset
// node); under graph capture it does not, since the fill would be recorded
// into the graph and re-zero the shared counters on every replay.
int noalloc_scratch(hipStream_t stream, void** out) {
  constexpr int kMaxDevices = 64;
  static std::atomic<void*> ptrs[kMaxDevices];
  static std::mutex mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return RF_W8A16_EHIP;
  if (dev < 0 || dev >= kMaxDevices) return RF_W8A16_EDEVICE;
  void* p = ptrs[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> g(mu);
    p = ptrs[dev].load(std::memory_order_relaxed);
    if (!p) {
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return RF_W8A16_EHIP;
      if (!aligned(p, 256)) return RF_W8A16_EHIP;
      hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing(stream, &cap) != hipSuccess) return RF_W8A16_EHIP;
      if (cap == hipStreamCaptureStatusNone) {
        constexpr int n = (int)(RF_W8A16_WS_COUNTER_BYTES / 16);
        hipLaunchKernelGGL(zero_u4_kernel, dim3((n + 255) / 256), dim3(256), 0, stream,
                           static_cast<uint4*>(p), n);
        if (hipGetLastError() != hipSuccess) return RF_W8A16_EHIP;
      }
      ptrs[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return RF_W8A16_OK;
}

}  // namespace

extern "C" {

const char* rf_w8a16_status_str(int status) {
  switch (status) {
    case RF_W8A16_OK: return "ok";
    case RF_W8A16_EINVAL: return "invalid argument (shape, size or null pointer)";
    case RF_W8A16_EALIGN:
      return "misaligned operand (x must be 16-byte aligned with ldx % 8 == 0 and K % 8 == 0)";
    case RF_W8A16_ELAYOUT:
      return "weight layout not accepted: pack the row-major int8 weight with "
             "rf_w8a16_pack_weight (layout TILE16X64) first";
    case RF_W8A16_EWORKSPACE: return "workspace missing or smaller than rf_w8a16_workspace_bytes()";
    case RF_W8A16_EHIP: return "HIP runtime error";
    case RF_W8A16_EDEVICE: return "current HIP device is not gfx950 (MI355X)";
    case RF_W8A16_EKERNEL:
      return "requested kernel cannot run this shape (GEMV: M > 64, or a row stride ldx whose "
             "32-bit offsets over 16 rows overflow)";
    case RF_W8A16_ESCRATCH:
      return "shape needs more split-K scratch than rf_w8a16_linear_multi_noalloc holds "
             "(RF_W8A16_NOALLOC_SCRATCH_BYTES); call rf_w8a16_linear_multi with a workspace";
    default: return "unknown rf_w8a16 status";
  }
}

int rf_w8a16_abi_version(void) { return RF_W8A16_ABI_VERSION; }

size_t rf_w8a16_packed_bytes(int64_t N, int64_t K) {
  if (check_nk(N, K) != RF_W8A16_OK) return 0;
  return (size_t)round_up(N, 16) * (size_t)round_up(K, 64);
}

int rf_w8a16_pack_weight(const int8_t* q, int64_t N, int64_t K, int64_t ldq, void* dst,
                         size_t dst_bytes) {
  if (check_nk(N, K) != RF_W8A16_OK || !q || !dst || ldq < K) return RF_W8A16_EINVAL;
  if (dst_bytes < rf_w8a16_packed_bytes(N, K)) return RF_W8A16_EINVAL;
  const int64_t kblocks = ceil_div(K, 64), nstrips = ceil_div(N, 16);
  uint8_t* out = static_cast<uint8_t*>(dst);
  for (int64_t nb = 0; nb < nstrips; ++nb) {
    for (int64_t kb = 0; kb < kblocks; ++kb) {
      uint8_t* tile = out + (nb * kblocks + kb) * 1024;
      for (int l = 0; l < 64; ++l) {
        const int64_t n = nb * 16 + (l & 15);
        const int64_t k0 = kb * 64 + 16 * (l >> 4);
        for (int j = 0; j < 16; ++j) {
          const int64_t k = k0 + j;
          const uint8_t qb = (n < N && k < K) ? (uint8_t)q[n * ldq + k] : 0u;
          tile[l * 16 + j] = (uint8_t)(qb ^ 0x80u);
        }
      }
    }
  }
  return RF_W8A16_OK;
}

int rf_w8a16_unpack_weight(const void* packed, int64_t N, int64_t K, int8_t* q, int64_t ldq) {
  if (check_nk(N, K) != RF_W8A16_OK || !packed || !q || ldq < K) return RF_W8A16_EINVAL;
  const int64_t kblocks = ceil_div(K, 64);
  const uint8_t* in = static_cast<const uint8_t*>(packed);
  for (int64_t n = 0; n < N; ++n) {
    const int64_t nb = n >> 4;
    const int nl = (int)(n & 15);
    for (int64_t k = 0; k < K; ++k) {
      const int64_t kb = k >> 6;
      const int kk = (int)(k & 63);
      const int l = nl + 16 * (kk >> 4);
      q[n * ldq + k] = (int8_t)(in[(nb * kblocks + kb) * 1024 + l * 16 + (kk & 15)] ^ 0x80u);
    }
  }
  return RF_W8A16_OK;
}

int rf_w8a16_pack_weight_device(const int8_t* q_dev, int64_t N, int64_t K, int64_t ldq,
                                void* dst_dev, size_t dst_bytes, void* stream) {
  if (check_nk(N, K) != RF_W8A16_OK || !q_dev || !dst_dev || ldq < K) return RF_W8A16_EINVAL;
  if (dst_bytes < rf_w8a16_packed_bytes(N, K)) return RF_W8A16_EINVAL;
  if (!aligned(dst_dev, 16)) return RF_W8A16_EALIGN;
  hipError_t e = rf::launch_pack(q_dev, N, K, ldq, static_cast<uint8_t*>(dst_dev),
                                 static_cast<hipStream_t>(stream));
  return e == hipSuccess ? RF_W8A16_OK : RF_W8A16_EHIP;
}

int rf_w8a16_select_kernel(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || M > kMaxDim || check_nk(N, K) != RF_W8A16_OK) return -RF_W8A16_EINVAL;
  return auto_kernel(M, N, K);
}

int rf_w8a16_plan(int64_t M, const int64_t* Ns, int32_t count, int64_t K, int32_t kernel,
                  int32_t format, int32_t cus, rf_w8a16_plan_info* out) {
  if (!out || !Ns || count < 1 || count > RF_W8A16_MAX_PROJ || M < 1 || M > kMaxDim)
    return RF_W8A16_EINVAL;
  if (format != RF_W8A16_FORMAT_INT8 && format != RF_W8A16_FORMAT_INT4 &&
      format != RF_W8A16_FORMAT_INT4_GROUP)
    return RF_W8A16_EINVAL;
  const bool int4 = format != RF_W8A16_FORMAT_INT8;
  int n32[RF_W8A16_MAX_PROJ];
  int64_t ntotal = 0;
  for (int i = 0; i < count; ++i) {
    if (check_nk(Ns[i], K) != RF_W8A16_OK) return RF_W8A16_EINVAL;
    if (int4 && Ns[i] % 16 != 0) return RF_W8A16_EINVAL;  // as rf_w4a16_linear
    n32[i] = (int)Ns[i];
    ntotal += Ns[i];
  }
  // The compute entry points' other refusals for this shape (x contiguous:
  // ldx = K).
  if (int4 && K % 64 != 0) return RF_W8A16_EINVAL;
  if (!int4 && K % 8 != 0) return RF_W8A16_EALIGN;
  rf::DeviceInfo dev;
  if (cus > 0) {
    dev.cus = cus;
    dev.gfx950 = true;
  } else {
    const int st = rf::device_info(&dev);
    if (st != RF_W8A16_OK) return st;
  }
  if (kernel == RF_W8A16_KERNEL_AUTO) {
    kernel = int4 ? auto_kernel_int4(M) : auto_kernel(M, ntotal, K);
    if (kernel == RF_W8A16_KERNEL_GEMV && !rf::gemv_offsets_fit(M, K))
      kernel = RF_W8A16_KERNEL_GEMM;  // the fallback the compute entry points take
  }
  if (kernel != RF_W8A16_KERNEL_GEMV && kernel != RF_W8A16_KERNEL_GEMM) return RF_W8A16_EINVAL;
  if (kernel == RF_W8A16_KERNEL_GEMV && (M > 64 || !rf::gemv_offsets_fit(M, K)))
    return RF_W8A16_EKERNEL;
  memset(out, 0, sizeof(*out));
  out->kernel = kernel;
  if (kernel == RF_W8A16_KERNEL_GEMV) {
    const rf::GemvPlan p = int4 ? rf::plan_gemv_int4((int)M, n32, count, (int)K,
                                                     format == RF_W8A16_FORMAT_INT4_GROUP, dev)
                                : rf::plan_gemv((int)M, n32, count, (int)K, dev);
    int waves = 0;
    bool xl = false;
    rf::gemv_cfg_info(p, (int)M, int4, &waves, &xl);
    out->tile_m = 16 * p.mt;
    out->tile_n = 16 * p.ns;
    out->splits = p.splits;
    out->waves = waves;
    out->workgroups = p.groups * p.splits;
    out->workspace_bytes = rf::gemv_workspace_bytes(p, (int)M, n32, count);
    snprintf(out->name, sizeof(out->name), "gemv %dx%d strips, %d waves%s", p.mt, p.ns, waves,
             xl ? ", x in LDS" : "");
  } else {
    const rf::GemmPlan p = rf::gemm_plan_for_stride(rf::plan_gemm((int)M, n32, count, (int)K, dev, int4),
                                                    (int)M, n32, count, K, (int)K, int4);
    // The int4 GEMM has no 64-bit-address kernel (rf_w4a16_linear refuses).
    if (int4 && !rf::gemm_offsets_fit(p, K, (int)K, true)) {
      memset(out, 0, sizeof(*out));
      return RF_W8A16_EKERNEL;
    }
    out->tile_m = p.bm;
    out->tile_n = p.bn;
    out->splits = p.splits;
    out->waves = rf::gemm_cfg_waves(p.cfg);
    out->workgroups = p.tiles_m * p.tiles_n * p.splits;
    out->workspace_bytes = rf::gemm_workspace_bytes(p);
    snprintf(out->name, sizeof(out->name), "gemm %s", rf::gemm_cfg_name(p.cfg, format, (int)M));
  }
  return RF_W8A16_OK;
}

size_t rf_w8a16_workspace_bytes_multi(int64_t M, const int64_t* Ns, int32_t count, int64_t K) {
  if (!Ns || count < 1 || count > RF_W8A16_MAX_PROJ || M < 1 || M > kMaxDim) return 0;
  int n32[RF_W8A16_MAX_PROJ];
  for (int i = 0; i < count; ++i) {
    if (check_nk(Ns[i], K) != RF_W8A16_OK) return 0;
    n32[i] = (int)Ns[i];
  }
  rf::DeviceInfo dev;
  if (rf::device_info(&dev) != RF_W8A16_OK) {
    dev.cus = 256;
    dev.gfx950 = false;
  }
  // Enough for either kernel family (the caller may force the GEMM at M <= 64).
  size_t extra = rf::gemm_workspace_bytes(rf::plan_gemm((int)M, n32, count, (int)K, dev));
  if (M <= 64) {
    const rf::GemvPlan p = rf::plan_gemv((int)M, n32, count, (int)K, dev);
    const size_t g = rf::gemv_workspace_bytes(p, (int)M, n32, count);
    extra = g > extra ? g : extra;
  }
  return RF_W8A16_WS_COUNTER_BYTES + extra;
}

size_t rf_w8a16_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  return rf_w8a16_workspace_bytes_multi(M, &N, 1, K);
}

// rf_w8a16_linear_multi and its no-allocation variant (noalloc: the
// workspace arguments are ignored and the library's scratch array is used).
static int linear_multi_impl(const void* x, int64_t ldx, int32_t layout,
                             const rf_w8a16_proj* projs, int32_t count, int64_t M, int64_t K,
                             int32_t kernel, void* workspace, size_t workspace_bytes, void* stream,
                             bool noalloc) {
  if (!x || !projs || count < 1 || count > RF_W8A16_MAX_PROJ) return RF_W8A16_EINVAL;
  if (M < 1 || M > kMaxDim || K < 1 || K > kMaxDim || ldx < K) return RF_W8A16_EINVAL;
  for (int i = 0; i < count; ++i) {
    const rf_w8a16_proj& q = projs[i];
    if (!q.w_packed || !q.scale || !q.y) return RF_W8A16_EINVAL;
    if (check_nk(q.N, K) != RF_W8A16_OK || q.ldy < q.N) return RF_W8A16_EINVAL;
  }
  if (layout != RF_W8A16_LAYOUT_TILE16X64) return RF_W8A16_ELAYOUT;
  if (K % 8 != 0 || ldx % 8 != 0 || !aligned(x, 16)) return RF_W8A16_EALIGN;
  for (int i = 0; i < count; ++i) {
    const rf_w8a16_proj& q = projs[i];
    if (!aligned(q.w_packed, 16) || !aligned(q.scale, 2) || !aligned(q.y, 2) ||
        (q.bias && !aligned(q.bias, 2)))
      return RF_W8A16_EALIGN;
  }

  rf::DeviceInfo dev;
  int st = rf::device_info(&dev);
  if (st != RF_W8A16_OK) return st;
  if (!dev.gfx950) return RF_W8A16_EDEVICE;

  if (kernel == RF_W8A16_KERNEL_AUTO) {
    int64_t ntotal = 0;
    for (int i = 0; i < count; ++i) ntotal += projs[i].N;
    kernel = auto_kernel(M, ntotal, K);
    // A row stride too large for the GEMV's 32-bit offsets: the GEMM (with
    // its 64-bit-address kernel) runs instead.
    if (kernel == RF_W8A16_KERNEL_GEMV && !rf::gemv_offsets_fit(M, ldx))
      kernel = RF_W8A16_KERNEL_GEMM;
  }
  if (kernel != RF_W8A16_KERNEL_GEMV && kernel != RF_W8A16_KERNEL_GEMM) return RF_W8A16_EINVAL;
  if (kernel == RF_W8A16_KERNEL_GEMV && (M > 64 || !rf::gemv_offsets_fit(M, ldx)))
    return RF_W8A16_EKERNEL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (noalloc) {
    st = noalloc_scratch(s, &workspace);
    if (st != RF_W8A16_OK) return st;
    workspace_bytes = RF_W8A16_NOALLOC_SCRATCH_BYTES;
  }
  // A plan needing more workspace than is at hand: the caller's buffer is too
  // small (EWORKSPACE), or the library's fixed scratch is (ESCRATCH).
  const int too_small = noalloc ? RF_W8A16_ESCRATCH : RF_W8A16_EWORKSPACE;

  rf::LinearProblem pr;
  pr.x = static_cast<const _Float16*>(x);
  pr.ldx = ldx;
  pr.M = (int)M;
  pr.K = (int)K;
  pr.nproj = count;
  int n32[RF_W8A16_MAX_PROJ];
  for (int i = 0; i < count; ++i) {
    rf::Projection& d = pr.proj[i];
    d.w = static_cast<const uint8_t*>(projs[i].w_packed);
    d.scale = static_cast<const _Float16*>(projs[i].scale);
    d.bias = static_cast<const _Float16*>(projs[i].bias);
    d.y = static_cast<_Float16*>(projs[i].y);
    d.ldy = projs[i].ldy;
    d.N = (int)projs[i].N;
    n32[i] = d.N;
  }
  auto workspace_ok = [&](size_t extra) {
    return workspace && workspace_bytes >= RF_W8A16_WS_COUNTER_BYTES + extra &&
           aligned(workspace, 256);
  };
  hipError_t e;
  if (kernel == RF_W8A16_KERNEL_GEMV) {
    const rf::GemvPlan p = rf::plan_gemv(pr.M, n32, count, pr.K, dev);
    if (p.splits > 1 && !workspace_ok(rf::gemv_workspace_bytes(p, pr.M, n32, count)))
      return too_small;
    e = rf::launch_gemv(pr, p, p.splits > 1 ? workspace : nullptr, s);
  } else {
    const rf::GemmPlan p = rf::plan_gemm(pr.M, n32, count, pr.K, dev);
    if (p.splits > 1 && !workspace_ok(rf::gemm_workspace_bytes(p))) return too_small;
    e = rf::launch_gemm(pr, p, p.splits > 1 ? workspace : nullptr, s);
  }
  return e == hipSuccess ? RF_W8A16_OK : RF_W8A16_EHIP;
}

int rf_w8a16_linear_multi(const void* x, int64_t ldx, int32_t layout, const rf_w8a16_proj* projs,
                          int32_t count, int64_t M, int64_t K, int32_t kernel, void* workspace,
                          size_t workspace_bytes, void* stream) {
  return linear_multi_impl(x, ldx, layout, projs, count, M, K, kernel, workspace, workspace_bytes,
                           stream, false);
}

int rf_w8a16_linear_multi_noalloc(const void* x, int64_t ldx, int32_t layout,
                                  const rf_w8a16_proj* projs, int32_t count, int64_t M, int64_t K,
                                  int32_t kernel, void* stream) {
  return linear_multi_impl(x, ldx, layout, projs, count, M, K, kernel, nullptr, 0, stream, true);
}

int rf_w8a16_linear(const void* x, int64_t ldx, const void* w_packed, int32_t layout,
                    const void* scale, const void* bias, void* y, int64_t ldy, int64_t M,
                    int64_t N, int64_t K, int32_t kernel, void* workspace,
                    size_t workspace_bytes, void* stream) {
  rf_w8a16_proj q;
  q.w_packed = w_packed;
  q.scale = scale;
  q.bias = bias;
  q.y = y;
  q.ldy = ldy;
  q.N = N;
  return rf_w8a16_linear_multi(x, ldx, layout, &q, 1, M, K, kernel, workspace, workspace_bytes,
                               stream);
}

// ---------------------------------------------------------------------------
// W4A16
// ---------------------------------------------------------------------------
size_t rf_w4a16_packed_bytes(int64_t N, int64_t K) {
  if (check_nk(N, K) != RF_W8A16_OK) return 0;
  return (size_t)round_up(N, 16) * (size_t)round_up(K, 128) / 2;
}

int rf_w4a16_pack_weight(const int8_t* q, int64_t N, int64_t K, int64_t ldq, void* dst,
                         size_t dst_bytes) {
  if (check_nk(N, K) != RF_W8A16_OK || !q || !dst || ldq < K) return RF_W8A16_EINVAL;
  if (dst_bytes < rf_w4a16_packed_bytes(N, K)) return RF_W8A16_EINVAL;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k)
      if (q[n * ldq + k] < -8 || q[n * ldq + k] > 7) return RF_W8A16_EINVAL;
  const int64_t ktiles = ceil_div(K, 128), nstrips = ceil_div(N, 16);
  uint8_t* out = static_cast<uint8_t*>(dst);
  for (int64_t nb = 0; nb < nstrips; ++nb)
    for (int64_t kt = 0; kt < ktiles; ++kt) {
      uint8_t* tile = out + (nb * ktiles + kt) * 1024;
      for (int l = 0; l < 64; ++l) {
        const int64_t n = nb * 16 + (l & 15);
        for (int w = 0; w < 4; ++w) {
          uint32_t v = 0;
          for (int i = 0; i < 8; ++i) {
            const int64_t k = kt * 128 + 32 * (l >> 4) + 8 * w + i;
            const int qv = (n < N && k < K) ? (int)q[n * ldq + k] : 0;
            v |= (uint32_t)(qv + 8) << (4 * rf::i4_nibble(i));
          }
          memcpy(tile + l * 16 + 4 * w, &v, 4);  // little-endian dword
        }
      }
    }
  return RF_W8A16_OK;
}

int rf_w4a16_unpack_weight(const void* packed, int64_t N, int64_t K, int8_t* q, int64_t ldq) {
  if (check_nk(N, K) != RF_W8A16_OK || !packed || !q || ldq < K) return RF_W8A16_EINVAL;
  const int64_t ktiles = ceil_div(K, 128);
  const uint8_t* in = static_cast<const uint8_t*>(packed);
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) {
      const int64_t kt = k >> 7;
      const int kk = (int)(k & 127);
      const int l = (int)(n & 15) + 16 * (kk >> 5), w = (kk >> 3) & 3, i = kk & 7;
      uint32_t v;
      memcpy(&v, in + ((n >> 4) * ktiles + kt) * 1024 + l * 16 + 4 * w, 4);
      q[n * ldq + k] = (int8_t)((int)((v >> (4 * rf::i4_nibble(i))) & 0xF) - 8);
    }
  return RF_W8A16_OK;
}

int rf_w4a16_pack_weight_device(const int8_t* q_dev, int64_t N, int64_t K, int64_t ldq,
                                void* dst_dev, size_t dst_bytes, void* stream) {
  if (check_nk(N, K) != RF_W8A16_OK || !q_dev || !dst_dev || ldq < K) return RF_W8A16_EINVAL;
  if (dst_bytes < rf_w4a16_packed_bytes(N, K)) return RF_W8A16_EINVAL;
  if (!aligned(dst_dev, 16)) return RF_W8A16_EALIGN;
  hipError_t e = rf::launch_pack4(q_dev, N, K, ldq, static_cast<uint8_t*>(dst_dev),
                                  static_cast<hipStream_t>(stream));
  return e == hipSuccess ? RF_W8A16_OK : RF_W8A16_EHIP;
}

size_t rf_w4a16_workspace_bytes_multi(int64_t M, const int64_t* Ns, int32_t count, int64_t K) {
  if (!Ns || count < 1 || count > RF_W8A16_MAX_PROJ || M < 1 || M > kMaxDim) return 0;
  int n32[RF_W8A16_MAX_PROJ];
  for (int i = 0; i < count; ++i) {
    if (check_nk(Ns[i], K) != RF_W8A16_OK) return 0;
    n32[i] = (int)Ns[i];
  }
  rf::DeviceInfo dev;
  if (rf::device_info(&dev) != RF_W8A16_OK) {
    dev.cus = 256;
    dev.gfx950 = false;
  }
  size_t extra = rf::gemm_workspace_bytes(rf::plan_gemm((int)M, n32, count, (int)K, dev, true));
  if (M <= 64) {
    // Either scale format: the plans may differ.
    for (const bool grouped : {false, true}) {
      const rf::GemvPlan p = rf::plan_gemv_int4((int)M, n32, count, (int)K, grouped, dev);
      const size_t g = rf::gemv_workspace_bytes(p, (int)M, n32, count);
      extra = g > extra ? g : extra;
    }
  }
  return RF_W8A16_WS_COUNTER_BYTES + extra;
}

size_t rf_w4a16_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  return rf_w4a16_workspace_bytes_multi(M, &N, 1, K);
}

int rf_w4a16_linear_multi(const void* x, int64_t ldx, const rf_w8a16_proj* projs, int32_t count,
                          int32_t group_size, int64_t M, int64_t K, int32_t kernel,
                          void* workspace, size_t workspace_bytes, void* stream) {
  if (!x || !projs || count < 1 || count > RF_W8A16_MAX_PROJ) return RF_W8A16_EINVAL;
  if (M < 1 || M > kMaxDim || K < 1 || K > kMaxDim || ldx < K) return RF_W8A16_EINVAL;
  if (group_size != 0 && group_size != 32 && group_size != 64 && group_size != 128)
    return RF_W8A16_EINVAL;
  if (K % 64 != 0 || (group_size && K % group_size != 0)) return RF_W8A16_EINVAL;
  for (int i = 0; i < count; ++i) {
    const rf_w8a16_proj& q = projs[i];
    if (!q.w_packed || !q.scale || !q.y) return RF_W8A16_EINVAL;
    if (check_nk(q.N, K) != RF_W8A16_OK || q.ldy < q.N || q.N % 16 != 0) return RF_W8A16_EINVAL;
  }
  if (ldx % 8 != 0 || !aligned(x, 16)) return RF_W8A16_EALIGN;
  for (int i = 0; i < count; ++i) {
    const rf_w8a16_proj& q = projs[i];
    // group-wise scale rows are copied with 16-byte DMAs
    if (!aligned(q.w_packed, 16) || !aligned(q.scale, group_size ? 16 : 2) || !aligned(q.y, 2) ||
        (q.bias && !aligned(q.bias, 2)))
      return RF_W8A16_EALIGN;
  }

  rf::DeviceInfo dev;
  int st = rf::device_info(&dev);
  if (st != RF_W8A16_OK) return st;
  if (!dev.gfx950) return RF_W8A16_EDEVICE;

  if (kernel == RF_W8A16_KERNEL_AUTO) {
    kernel = auto_kernel_int4(M);
    if (kernel == RF_W8A16_KERNEL_GEMV && !rf::gemv_offsets_fit(M, ldx))
      kernel = RF_W8A16_KERNEL_GEMM;
  }
  if (kernel != RF_W8A16_KERNEL_GEMV && kernel != RF_W8A16_KERNEL_GEMM) return RF_W8A16_EINVAL;
  if (kernel == RF_W8A16_KERNEL_GEMV && (M > 64 || !rf::gemv_offsets_fit(M, ldx)))
    return RF_W8A16_EKERNEL;
  hipStream_t s = static_cast<hipStream_t>(stream);

  rf::LinearProblem pr;
  pr.x = static_cast<const _Float16*>(x);
  pr.ldx = ldx;
  pr.M = (int)M;
  pr.K = (int)K;
  pr.nproj = count;
  pr.wf = group_size ? rf::kWfInt4Grp : rf::kWfInt4;
  pr.gshift = group_size == 128 ? 2 : group_size == 64 ? 1 : 0;
  int n32[RF_W8A16_MAX_PROJ];
  for (int i = 0; i < count; ++i) {
    rf::Projection& d = pr.proj[i];
    d.w = static_cast<const uint8_t*>(projs[i].w_packed);
    d.scale = static_cast<const _Float16*>(projs[i].scale);
    d.bias = static_cast<const _Float16*>(projs[i].bias);
    d.y = static_cast<_Float16*>(projs[i].y);
    d.ldy = projs[i].ldy;
    d.N = (int)projs[i].N;
    n32[i] = d.N;
  }
  auto workspace_ok = [&](size_t extra) {
    return workspace && workspace_bytes >= RF_W8A16_WS_COUNTER_BYTES + extra &&
           aligned(workspace, 256);
  };
  hipError_t e;
  if (kernel == RF_W8A16_KERNEL_GEMV) {
    const rf::GemvPlan p = rf::plan_gemv_int4(pr.M, n32, count, pr.K, group_size != 0, dev);
    if (p.splits > 1 && !workspace_ok(rf::gemv_workspace_bytes(p, pr.M, n32, count)))
      return RF_W8A16_EWORKSPACE;
    e = rf::launch_gemv(pr, p, p.splits > 1 ? workspace : nullptr, s);
  } else {
    const rf::GemmPlan p = rf::plan_gemm(pr.M, n32, count, pr.K, dev, true);
    // The int4 GEMM has no 64-bit-address kernel.
    if (!rf::gemm_offsets_fit(p, ldx, pr.K, true)) return RF_W8A16_EKERNEL;
    if (p.splits > 1 && !workspace_ok(rf::gemm_workspace_bytes(p))) return RF_W8A16_EWORKSPACE;
    e = rf::launch_gemm(pr, p, p.splits > 1 ? workspace : nullptr, s);
  }
  return e == hipSuccess ? RF_W8A16_OK : RF_W8A16_EHIP;
}

int rf_w4a16_linear(const void* x, int64_t ldx, const void* w_packed, const void* scale,
                    int32_t group_size, const void* bias, void* y, int64_t ldy, int64_t M,
                    int64_t N, int64_t K, int32_t kernel, void* workspace, size_t workspace_bytes,
                    void* stream) {
  rf_w8a16_proj q;
  q.w_packed = w_packed;
  q.scale = scale;
  q.bias = bias;
  q.y = y;
  q.ldy = ldy;
  q.N = N;
  return rf_w4a16_linear_multi(x, ldx, &q, 1, group_size, M, K, kernel, workspace,
                               workspace_bytes, stream);
}

size_t rf_w8a16_workspace_bytes_argmax(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || M > 64 || check_nk(N, K) != RF_W8A16_OK || N > INT32_MAX - 1) return 0;
  rf::DeviceInfo dev;
  if (rf::device_info(&dev) != RF_W8A16_OK) {
    dev.cus = 256;
    dev.gfx950 = false;
  }
  const int n32 = (int)N;
  const rf::GemvPlan p = rf::plan_gemv((int)M, &n32, 1, (int)K, dev);
  return RF_W8A16_WS_COUNTER_BYTES +
         (size_t)rf::round_up((int64_t)rf::gemv_workspace_bytes(p, (int)M, &n32, 1), 256) +
         rf::argmax_slot_bytes(p, (int)M);
}

int rf_w8a16_linear_argmax(const void* x, int64_t ldx, const void* w_packed, int32_t layout,
                           const void* scale, const void* bias, void* y, int64_t ldy,
                           int32_t* index, int64_t M, int64_t N, int64_t K, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (!x || !w_packed || !scale || !index) return RF_W8A16_EINVAL;
  if (M < 1 || M > kMaxDim || check_nk(N, K) != RF_W8A16_OK || ldx < K) return RF_W8A16_EINVAL;
  if (N > INT32_MAX - 1 || (y && ldy < N)) return RF_W8A16_EINVAL;
  if (layout != RF_W8A16_LAYOUT_TILE16X64) return RF_W8A16_ELAYOUT;
  if (K % 8 != 0 || ldx % 8 != 0 || !aligned(x, 16) || !aligned(w_packed, 16) ||
      !aligned(scale, 2) || (bias && !aligned(bias, 2)) || (y && !aligned(y, 2)) ||
      !aligned(index, 4))
    return RF_W8A16_EALIGN;
  if (M > 64 || !rf::gemv_offsets_fit(M, ldx)) return RF_W8A16_EKERNEL;
  rf::DeviceInfo dev;
  int st = rf::device_info(&dev);
  if (st != RF_W8A16_OK) return st;
  if (!dev.gfx950) return RF_W8A16_EDEVICE;

  rf::LinearProblem pr;
  pr.x = static_cast<const _Float16*>(x);
  pr.ldx = ldx;
  pr.M = (int)M;
  pr.K = (int)K;
  pr.nproj = 1;
  pr.proj[0].w = static_cast<const uint8_t*>(w_packed);
  pr.proj[0].scale = static_cast<const _Float16*>(scale);
  pr.proj[0].bias = static_cast<const _Float16*>(bias);
  pr.proj[0].y = static_cast<_Float16*>(y);
  pr.proj[0].ldy = y ? ldy : 0;
  pr.proj[0].N = (int)N;
  const int n32 = (int)N;
  const rf::GemvPlan p = rf::plan_gemv(pr.M, &n32, 1, pr.K, dev);
  const size_t slots_off = RF_W8A16_WS_COUNTER_BYTES +
      (size_t)rf::round_up((int64_t)rf::gemv_workspace_bytes(p, pr.M, &n32, 1), 256);
  const size_t need = slots_off + rf::argmax_slot_bytes(p, pr.M);
  if (!workspace || workspace_bytes < need || !aligned(workspace, 256)) return RF_W8A16_EWORKSPACE;
  rf::ArgmaxTarget am;  // per-workgroup keys in the scratch part of the workspace
  am.slots = reinterpret_cast<uint64_t*>(static_cast<uint8_t*>(workspace) + slots_off);
  am.index = index;
  const hipError_t e = rf::launch_gemv(pr, p, workspace, static_cast<hipStream_t>(stream), &am);
  return e == hipSuccess ? RF_W8A16_OK : RF_W8A16_EHIP;
}

}  // extern "C"
