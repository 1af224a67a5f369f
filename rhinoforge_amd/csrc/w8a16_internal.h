// Host-side internals shared by the C-ABI layer and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/w8a16.h"

namespace rf {

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

// Arguments of one W8A16 linear call, already validated.
struct LinearArgs {
  const _Float16* x;
  int64_t ldx;
  const uint8_t* w;      // TILE16X64 packed
  const _Float16* scale; // [N]
  const _Float16* bias;  // [N] or nullptr
  _Float16* y;
  int64_t ldy;
  int M, N, K;
  int kblocks;  // Kp / 64
  int nstrips;  // Np / 16
};

// One projection of a GEMV launch (weights, per-channel scale, optional bias,
// output) and a launch of up to RF_W8A16_MAX_PROJ projections sharing x.
struct GemvProjection {
  const uint8_t* w;      // TILE16X64 packed
  const _Float16* scale; // [N]
  const _Float16* bias;  // [N] or nullptr
  _Float16* y;
  int64_t ldy;
  int N;
};

struct GemvProblem {
  const _Float16* x;
  int64_t ldx;
  int M, K;
  int nproj;
  GemvProjection proj[RF_W8A16_MAX_PROJ];
};

// Decode GEMV / skinny-GEMM launch plan (M <= 64).
struct GemvPlan {
  int cfg;       // kernel configuration id (w8a16_gemv.hip)
  int mt;        // 16-row m tiles per wavefront (1, 2 or 4)
  int ns;        // 16-channel strips per workgroup
  int splits;    // K splits across workgroups (1 = no workspace use)
  int kb_per_split;
  int groups;    // ceil(nstrips / ns)
};

// Prefill GEMM launch plan.
struct GemmPlan {
  int cfg;       // tile configuration id (w8a16_gemm.hip)
  int bm, bn;    // workgroup tile
  int tiles_m, tiles_n;
  int group_m;   // output-tile rows per scheduling group
};

struct DeviceInfo {
  int cus;           // compute units
  bool gfx950;
};

// Cached per-device properties (read-only after first query).
int device_info(DeviceInfo* out);

GemvPlan plan_gemv(int M, const int* Ns, int nproj, int K, const DeviceInfo& dev);
GemmPlan plan_gemm(int M, int N, int K, const DeviceInfo& dev);
size_t gemv_workspace_bytes(const GemvPlan& p, int M, const int* Ns, int nproj);

// Launchers: return hipSuccess or the launch error.
hipError_t launch_gemv(const GemvProblem& pr, const GemvPlan& p, void* workspace,
                       hipStream_t stream);
hipError_t launch_gemm(const LinearArgs& a, const GemmPlan& p, hipStream_t stream);
hipError_t launch_pack(const int8_t* q, int64_t N, int64_t K, int64_t ldq,
                       uint8_t* dst, hipStream_t stream);

}  // namespace rf
