// Host-side internals shared by the C-ABI layer and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/w8a16.h"

namespace rf {

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

// One projection of a launch (weights, per-channel scale, optional bias,
// output) and a launch of up to RF_W8A16_MAX_PROJ projections sharing x,
// already validated.
struct Projection {
  const uint8_t* w;      // TILE16X64 (int8) or TILE16X128_I4 (int4) packed
  const _Float16* scale; // [N], or [K/group][N] for group-wise int4
  const _Float16* bias;  // [N] or nullptr
  _Float16* y;
  int64_t ldy;
  int N;
};

struct LinearProblem {
  const _Float16* x;
  int64_t ldx;
  int M, K;
  int nproj;
  Projection proj[RF_W8A16_MAX_PROJ];
  int wf = 0;      // weight format (w8a16_common.h WeightFormat): 0 int8, 1 int4, 2 int4 group-wise
  int gshift = 0;  // group-wise int4: log2(group_size / 32)
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
  int tiles_m, tiles_n;  // tiles_n summed over the launch's projections
  int group_m;   // output-tile rows per scheduling group
  int splits;    // K splits across workgroups (1 = no workspace use)
  int kb_per_split;
};

struct DeviceInfo {
  int cus;           // compute units
  bool gfx950;
};

// Cached per-device properties (read-only after first query).
int device_info(DeviceInfo* out);

GemvPlan plan_gemv(int M, const int* Ns, int nproj, int K, const DeviceInfo& dev);

// The GEMV addresses activations as a 64-bit base per 16-row m-tile plus a
// per-lane 32-bit byte offset spanning at most 15 rows (and 256 bytes of
// lane-group and chunk offsets): true when that offset cannot overflow.
inline bool gemv_offsets_fit(int64_t M, int64_t ldx) {
  const uint64_t rows = (uint64_t)((M < 16 ? M : 16) - 1);
  return rows * (uint64_t)ldx * 2u + 256u < (1ull << 32);
}
// True when the 32-bit tile offsets of the GEMM kernels fit for this plan
// and row stride (otherwise int8 launches take the 64-bit-address kernel;
// int4 launches have none).
bool gemm_offsets_fit(const GemmPlan& p, int64_t ldx, int K, bool int4);
// The plan launch_gemm runs at row stride ldx: int8 plans whose offsets do
// not fit become the 64-bit-address kernel (unsplit); int4 plans unchanged.
GemmPlan gemm_plan_for_stride(const GemmPlan& p, int M, const int* Ns, int nproj, int64_t ldx,
                              int K, bool int4);
// int4: packed-int4 weights (TILE16X128_I4) take the large-tile rules only.
GemmPlan plan_gemm(int M, const int* Ns, int nproj, int K, const DeviceInfo& dev,
                   bool int4 = false);
// GEMV plan of packed-int4 weights (nproj projections sharing x); grouped:
// group-wise scales (their per-tile scale loads change which configuration
// wins).
GemvPlan plan_gemv_int4(int M, const int* Ns, int nproj, int K, bool grouped,
                        const DeviceInfo& dev);
// Workspace bytes past the RF_W8A16_WS_COUNTER_BYTES counter region.
size_t gemv_workspace_bytes(const GemvPlan& p, int M, const int* Ns, int nproj);
size_t gemm_workspace_bytes(const GemmPlan& p);
// Plan descriptions for rf_w8a16_plan: wavefronts per workgroup and x staging
// of a GEMV configuration; the name of a GEMM configuration as it runs for
// weight format wf at M rows.
void gemv_cfg_info(const GemvPlan& p, int M, bool int4, int* waves, bool* x_in_lds);
const char* gemm_cfg_name(int cfg, int wf, int M);
// Wavefronts per workgroup of a GEMM configuration.
int gemm_cfg_waves(int cfg);

// Fused argmax of a single-projection GEMV launch (M <= 64): the GEMV
// stores every workgroup's best 64-bit key per row to `slots` (scratch,
// argmax_slot_bytes), a second launch reduces them into the int32 result.
struct ArgmaxTarget {
  uint64_t* slots;  // [M][groups]
  int32_t* index;   // [M]
};
size_t argmax_slot_bytes(const GemvPlan& p, int M);

// Split-K arrival counters (4 B per workgroup group or tile) fill the
// zero-between-calls counter region at the start of every workspace.
constexpr int kMaxSplitCounters = (int)(RF_W8A16_WS_COUNTER_BYTES / 4);

// Launchers: return hipSuccess or the launch error.
hipError_t launch_gemv(const LinearProblem& pr, const GemvPlan& p, void* workspace,
                       hipStream_t stream, const ArgmaxTarget* am = nullptr);
hipError_t launch_gemm(const LinearProblem& pr, const GemmPlan& p, void* workspace,
                       hipStream_t stream);
hipError_t launch_pack4(const int8_t* q, int64_t N, int64_t K, int64_t ldq, uint8_t* dst,
                        hipStream_t stream);
hipError_t launch_pack(const int8_t* q, int64_t N, int64_t K, int64_t ldq,
                       uint8_t* dst, hipStream_t stream);

}  // namespace rf
