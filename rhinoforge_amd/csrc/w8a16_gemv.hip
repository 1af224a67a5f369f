// Decode GEMV / skinny GEMM for W8A16, M <= 64 (gfx950).
//
// HBM-bound: every call streams N*K weight bytes once.  Design:
//   * one workgroup = 4 wavefronts = `NS` strips of 16 output channels over
//     one K split; the wavefronts interleave the split's 1 KB weight tiles
//     (wave w takes tiles w, w+4, ...), so each wavefront-wide load is one
//     fully coalesced 1 KB tile and a workgroup step reads 4 KB contiguous;
//   * weights are dequantized in registers (v_perm + v_pk_add, exact) and
//     fed to v_mfma_f32_16x16x32_f16 with the activation rows as the A
//     operand, so the K reduction inside a tile happens in the matrix core;
//   * loads are software-pipelined: the next stage of U tiles per wavefront
//     is in flight while the current one is converted and multiplied;
//   * the four wavefronts' fp32 partials are summed through LDS; with K
//     split across workgroups, partials go to the workspace and the last
//     workgroup to arrive (device-scope counter) adds them in split order
//     (deterministic), applies scale and bias, stores fp16, and re-zeroes
//     the counter.
// The per-channel scale is applied once in the epilogue: s[n] factors out
// of the K sum, y[m,n] = s[n] * sum_k x[m,k] q[n,k] (+ b[n]).
#include "w8a16_common.h"
#include "w8a16_internal.h"
#include "../../include/w8a16.h"

namespace rf {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;

struct GemvKernelArgs {
  const _Float16* x;
  int64_t ldx;
  const uint8_t* w;
  const _Float16* scale;
  const _Float16* bias;
  _Float16* y;
  int64_t ldy;
  int M, N, K;
  int kblocks;
  int nstrips;
  int splits;
  int kb_per_split;
  int np;              // padded N (nstrips * 16), row stride of partials
  float* partial;      // [splits][M][np]
  uint32_t* counters;  // [groups]
};

// Activation fragment of one tile for m-tile `mt`: x[m][k .. k+15] with
// m = 16*mt + lane%16 and k = 64*kb + 16*(lane/16); zero outside [M) x [K).
template <int MT>
__device__ __forceinline__ void load_x(const GemvKernelArgs& a, int kb, int lane,
                                       half8 (&xa)[MT][2]) {
  const int k = kb * kTileK + 16 * (lane >> 4);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + (lane & 15);
    uint4 v0 = make_uint4(0, 0, 0, 0), v1 = make_uint4(0, 0, 0, 0);
    if (m < a.M) {
      const _Float16* p = a.x + (int64_t)m * a.ldx + k;
      if (k < a.K) v0 = load_u4(p);
      if (k + 8 < a.K) v1 = load_u4(p + 8);
    }
    xa[mt][0] = as_half8(v0);
    xa[mt][1] = as_half8(v1);
  }
}

template <int MT, int NS, int U>
__global__ __launch_bounds__(kThreads) void w8a16_gemv_kernel(GemvKernelArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int group = blockIdx.x;
  const int split = blockIdx.y;
  const int strip0 = group * NS;
  const int kb0 = split * a.kb_per_split;
  const int kb1 = min(kb0 + a.kb_per_split, a.kblocks);

  floatx4 acc[MT][NS];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < NS; ++s) acc[mt][s] = floatx4{0.f, 0.f, 0.f, 0.f};

  // Strip s of this group exists iff strip0 + s < nstrips (uniform per WG).
  bool strip_ok[NS];
  const uint8_t* wbase[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    strip_ok[s] = (strip0 + s) < a.nstrips;
    wbase[s] = a.w + ((int64_t)(strip0 + s) * a.kblocks) * kTileBytes + lane * 16;
  }

  // Stage buffers: U tiles per wavefront per stage.
  uint4 wcur[U][NS], wnxt[U][NS];
  half8 xcur[U][MT][2], xnxt[U][MT][2];

  auto load_stage = [&](int it, uint4 (&wv)[U][NS], half8 (&xv)[U][MT][2]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kb = kb0 + wave + kWaves * (it * U + u);
      const bool ok = kb < kb1;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        wv[u][s] = (ok && strip_ok[s]) ? load_u4_stream(wbase[s] + (int64_t)kb * kTileBytes)
                                       : make_uint4(0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u);
      }
      if (ok) {
        load_x<MT>(a, kb, lane, xv[u]);
      } else {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) xv[u][mt][0] = xv[u][mt][1] = half8{};
      }
    }
  };

  const int my_tiles = (kb1 - kb0 - wave + kWaves - 1) / kWaves;  // tiles for this wave
  const int stages = (my_tiles + U - 1) / U;

  if (stages > 0) load_stage(0, wcur, xcur);
  for (int it = 0; it < stages; ++it) {
    if (it + 1 < stages) load_stage(it + 1, wnxt, xnxt);
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const half8 b0 = dequant8(wcur[u][s].x, wcur[u][s].y);
        const half8 b1 = dequant8(wcur[u][s].z, wcur[u][s].w);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc[mt][s] = mfma16x16x32(xcur[u][mt][0], b0, acc[mt][s]);
          acc[mt][s] = mfma16x16x32(xcur[u][mt][1], b1, acc[mt][s]);
        }
      }
    }
    if (it + 1 < stages) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int s = 0; s < NS; ++s) wcur[u][s] = wnxt[u][s];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          xcur[u][mt][0] = xnxt[u][mt][0];
          xcur[u][mt][1] = xnxt[u][mt][1];
        }
      }
    }
  }

  // ---- cross-wavefront reduction through LDS --------------------------
  __shared__ floatx4 red[kWaves][MT * NS][kWave];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < NS; ++s) red[wave][mt * NS + s][lane] = acc[mt][s];
  __syncthreads();

  // Tile t = mt*NS + s is finished by wavefront t % 4.
  const int n_in_strip = lane & 15;
  const int m_sub = 4 * (lane >> 4);
  for (int t = wave; t < MT * NS; t += kWaves) {
    const int mt = t / NS, s = t % NS;
    floatx4 sum = red[0][t][lane];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) sum += red[w][t][lane];
    const int n = (strip0 + s) * 16 + n_in_strip;
    if (a.splits == 1) {
      if (n < a.N) {
        const float sc = (float)a.scale[n];
        const float bi = a.bias ? (float)a.bias[n] : 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = mt * 16 + m_sub + r;
          if (m < a.M) a.y[(int64_t)m * a.ldy + n] = (_Float16)__builtin_fmaf(sum[r], sc, bi);
        }
      }
    } else if (strip0 + s < a.nstrips) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = mt * 16 + m_sub + r;
        if (m < a.M) a.partial[((int64_t)split * a.M + m) * a.np + n] = sum[r];
      }
    }
  }
  if (a.splits == 1) return;

  // ---- split-K: last workgroup to arrive reduces in split order ---------
  __shared__ uint32_t is_last;
  __threadfence();  // release this workgroup's partials (device scope)
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = atomicAdd(&a.counters[group], 1u);
    is_last = (prev == (uint32_t)(a.splits - 1)) ? 1u : 0u;
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();  // acquire the other workgroups' partials

  // Each thread finishes (m, n) outputs of this group, coalesced along n.
  const int nrows = min(NS, a.nstrips - strip0) * 16;
  const int total = a.M * nrows;
  for (int i = threadIdx.x; i < total; i += kThreads) {
    const int m = i / nrows;
    const int n = strip0 * 16 + (i % nrows);
    float sum = 0.f;
    for (int sp = 0; sp < a.splits; ++sp)
      sum += __builtin_nontemporal_load(&a.partial[((int64_t)sp * a.M + m) * a.np + n]);
    if (n < a.N) {
      const float sc = (float)a.scale[n];
      const float bi = a.bias ? (float)a.bias[n] : 0.f;
      a.y[(int64_t)m * a.ldy + n] = (_Float16)__builtin_fmaf(sum, sc, bi);
    }
  }
  if (threadIdx.x == 0) atomicExch(&a.counters[group], 0u);  // leave the counter zeroed
}

template <int MT, int NS, int U>
hipError_t launch_t(const GemvKernelArgs& ka, const GemvPlan& p, hipStream_t stream) {
  dim3 grid(p.groups, p.splits, 1);
  hipLaunchKernelGGL((w8a16_gemv_kernel<MT, NS, U>), grid, dim3(kThreads), 0, stream, ka);
  return hipGetLastError();
}

}  // namespace

size_t gemv_workspace_bytes(const GemvPlan& p, int M, int N) {
  if (p.splits <= 1) return 0;
  const int64_t np = round_up(N, 16);
  return (size_t)p.splits * (size_t)M * (size_t)np * sizeof(float);
}

hipError_t launch_gemv(const LinearArgs& a, const GemvPlan& p, void* workspace,
                       hipStream_t stream) {
  GemvKernelArgs ka;
  ka.x = a.x;
  ka.ldx = a.ldx;
  ka.w = a.w;
  ka.scale = a.scale;
  ka.bias = a.bias;
  ka.y = a.y;
  ka.ldy = a.ldy;
  ka.M = a.M;
  ka.N = a.N;
  ka.K = a.K;
  ka.kblocks = a.kblocks;
  ka.nstrips = a.nstrips;
  ka.splits = p.splits;
  ka.kb_per_split = p.kb_per_split;
  ka.np = a.nstrips * 16;
  // Workspace: [counters | partials]; counter region size fixed by the ABI.
  ka.counters = reinterpret_cast<uint32_t*>(workspace);
  ka.partial = workspace ? reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + RF_W8A16_WS_COUNTER_BYTES)
                         : nullptr;

  switch (p.mt * 100 + p.ns) {
    case 101: return launch_t<1, 1, 4>(ka, p, stream);
    case 102: return launch_t<1, 2, 4>(ka, p, stream);
    case 104: return launch_t<1, 4, 2>(ka, p, stream);
    case 201: return launch_t<2, 1, 2>(ka, p, stream);
    case 202: return launch_t<2, 2, 2>(ka, p, stream);
    case 401: return launch_t<4, 1, 2>(ka, p, stream);
    case 402: return launch_t<4, 2, 1>(ka, p, stream);
    default: return hipErrorInvalidValue;
  }
}

GemvPlan plan_gemv(int M, int N, int K, const DeviceInfo& dev) {
  GemvPlan p;
  const int nstrips = (int)ceil_div(N, 16);
  const int kblocks = (int)ceil_div(K, 64);
  p.mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  p.ns = 1;
  p.groups = (int)ceil_div(nstrips, p.ns);
  // Enough workgroups to cover every CU twice; each wavefront keeps >= 2
  // tiles per split so the pipeline has something to overlap.
  const int target = 2 * dev.cus;
  int splits = (int)ceil_div(target, p.groups);
  const int max_splits = kblocks / (2 * kWaves);
  if (splits > max_splits) splits = max_splits;
  if (splits > 16) splits = 16;
  if (splits < 1) splits = 1;
  if (p.groups > 16384) splits = 1;  // counter region holds 16384 counters
  p.kb_per_split = (int)ceil_div(kblocks, splits);
  p.splits = (int)ceil_div(kblocks, p.kb_per_split);  // drop empty splits
  return p;
}

}  // namespace rf
