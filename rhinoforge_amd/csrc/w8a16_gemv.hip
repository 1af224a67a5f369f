// Decode GEMV / skinny GEMM for W8A16, M <= 64 (gfx950).
//
// HBM-bound: every call streams N*K weight bytes once.  Design:
//   * a workgroup of W wavefronts owns NS strips of 16 output channels over
//     one K split; the wavefronts interleave the split's 1 KB weight tiles
//     (wave w takes tiles w, w+W, ...), so each wavefront-wide load is one
//     fully coalesced 1 KB tile and a workgroup step reads W KB contiguous
//     per strip;
//   * weights are dequantized in registers (v_perm + v_pk_add, exact) and
//     fed to v_mfma_f32_16x16x32_f16 with the activation rows as the A
//     operand, so the K reduction inside a tile happens in the matrix core;
//     the activation fragment of a tile is reused for all NS strips;
//   * weight loads are software-pipelined two stages deep: the next U tiles
//     per wavefront are in flight while the current U are converted and
//     multiplied;
//   * activations come either straight from global memory (L2-resident,
//     prefetched with the weights) or, when XL is set, from a copy of the
//     split's x[0:M, Krange] that the workgroup stages in LDS once;
//   * the wavefronts' fp32 partials are summed through LDS in a fixed order;
//     with K split across workgroups the partials go to the workspace and
//     the last workgroup to arrive sums them in split order (deterministic),
//     applies scale and bias, stores fp16 and re-zeroes its counter.
//
// Split-K hand-off without L2 flushes: on gfx950 each XCD has its own L2,
// and a device-scope fence (__threadfence) writes back and invalidates the
// whole L2 of the issuing XCD.  Instead the partials are written and read
// with relaxed device-scope atomic stores/loads (global_store/load ... sc1,
// coherent at device scope by themselves), and each workgroup waits for its
// stores to complete (s_waitcnt vmcnt(0)) before it bumps the counter.
//
// The per-channel scale is applied once in the epilogue: s[n] factors out
// of the K sum, y[m,n] = s[n] * sum_k x[m,k] q[n,k] (+ b[n]).
#include <algorithm>

#include "w8a16_common.h"
#include "w8a16_internal.h"
#include "../../include/w8a16.h"

namespace rf {
namespace {

constexpr int kMaxSplits = 16;
constexpr int kMaxProj = RF_W8A16_MAX_PROJ;
constexpr int kMaxGroupsSplit = kMaxSplitCounters;

// One weight matrix of a launch.  Several projections that share the
// activation x (q/k/v, or gate/up) run in one launch: workgroups are
// numbered projection-major, projection p owning groups [group0, next group0).
struct GemvProj {
  const uint8_t* w;
  const _Float16* scale;
  const _Float16* bias;
  _Float16* y;
  int64_t ldy;
  int N;
  int nstrips;
  int group0;  // first workgroup (blockIdx.x) of this projection
  int col0;    // first column of this projection in the partial buffer
};

struct GemvKernelArgs {
  const _Float16* x;
  int64_t ldx;
  int M, K;
  int kblocks;
  int nproj;
  GemvProj proj[kMaxProj];
  int splits;
  int kb_per_split;
  int np;              // padded columns of all projections: row stride of partials
  float* partial;      // [splits][M][np]
  uint32_t* counters;  // [groups]
  // Fused argmax (nullptr: none): every workgroup's best key per row,
  // [M][gridDim.x], reduced by argmax_finish_kernel after this launch.
  unsigned long long* amax_slots;
  // Group-wise int4: log2(group_size / 32); scale row of tile position k is
  // k / group_size.
  int gshift;
  // Nonzero: groups per XCD run (xcd_group), the launch's groups / 8.
  int xcd_run;
};

// Argmax key of output value v at column n: the fp16 value mapped to an
// unsigned order (NaN above everything, -0 equal to +0, as torch.argmax
// compares), +1 so that every key beats the reset value 0, in the high half;
// ~n in the low half, so among equal values the lowest column wins.
__device__ __forceinline__ unsigned long long argmax_key(_Float16 v, int n) {
  uint32_t h = __builtin_bit_cast(uint16_t, v);
  if (h == 0x8000u) h = 0;
  uint32_t ord;
  if ((h & 0x7fffu) > 0x7c00u) ord = 0xffffu;
  else ord = (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u);
  return ((unsigned long long)(ord + 1) << 32) | (uint32_t)(0xffffffffu - (uint32_t)n);
}

__device__ __forceinline__ int32_t argmax_index_of(unsigned long long key) {
  return (int32_t)(0xffffffffu - (uint32_t)key);
}

__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Activation fragment of one tile for every m-tile read from global memory:
// x[m][k .. k+15] with m = 16*mt + lane%16, k = 64*kb + 16*(lane/16).
// Addresses are a wave-uniform 64-bit base per m-tile (xrow[mt] = first row
// of the m-tile, plus 64*kb: scalar) and a per-lane 32-bit offset fixed for
// the whole call (xoff[mt]: row within the m-tile, lane group), so a load
// costs no vector address math.  The 32-bit part spans at most 15 rows; the
// host checks that it cannot overflow (gemv_offsets_fit).  Rows m >= M read
// row M-1 instead (their MFMA output rows are never stored).  KT (K % 64 != 0, a launch-time
// choice) clamps every chunk into the row and zeroes the chunks past K with
// selects; without it the load path has no branch or select at all, which
// keeps the compiler's load-wait bookkeeping exact (a branch around a load
// makes it fall back to waiting for every load in flight).
// K % 8 == 0, so a chunk that starts below K ends below K.
template <int MT, bool KT>
__device__ __forceinline__ void load_x_global(const GemvKernelArgs& a, int kb,
                                              const uint8_t* const (&xrow)[MT],
                                              const uint32_t (&xoff)[MT], int lane,
                                              half8 (&xa)[MT][2]) {
  if (!KT) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint8_t* xb = xrow[mt] + (int64_t)kb * (kTileK * 2);
      xa[mt][0] = as_half8(load_u4(xb + xoff[mt]));
      xa[mt][1] = as_half8(load_u4(xb + xoff[mt] + 16));
    }
  } else {
    const int k = kb * kTileK + 16 * (lane >> 4);
    // byte offsets (<= 0) that pull each chunk back inside the row
    const int d0 = (min(k, a.K - 8) - k) * 2, d1 = (min(k + 8, a.K - 8) - (k + 8)) * 2;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint8_t* xb = xrow[mt] + (int64_t)kb * (kTileK * 2);
      const half8 v0 = as_half8(load_u4(xb + xoff[mt] + d0));
      const half8 v1 = as_half8(load_u4(xb + xoff[mt] + 16 + d1));
      xa[mt][0] = k < a.K ? v0 : half8{};
      xa[mt][1] = k + 8 < a.K ? v1 : half8{};
    }
  }
}

// Activation fragment of one int4 tile (128 input positions): lane l reads
// x[m][128*kb + 32*(l/16) .. +31] as four half8, m = 16*mt + l%16, with the
// same wave-uniform base plus fixed per-lane offset as above.  K % 64 == 0
// for int4, so with KT (K % 128 == 64) a lane's 32 positions are either all
// below K or all past it; the latter read a clamped chunk and are zeroed.
template <int MT, bool KT>
__device__ __forceinline__ void load_x_global4(const GemvKernelArgs& a, int kb,
                                               const uint8_t* const (&xrow)[MT],
                                               const uint32_t (&xoff)[MT], int lane,
                                               half8 (&xa)[MT][4]) {
  const int k = kb * kTileK4 + 32 * (lane >> 4);
  const int d = KT ? (min(k, a.K - 32) - k) * 2 : 0;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const uint8_t* xb = xrow[mt] + (int64_t)kb * (kTileK4 * 2);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const half8 v = as_half8(load_u4(xb + xoff[mt] + d + 16 * c));
      xa[mt][c] = (!KT || k < a.K) ? v : half8{};
    }
  }
}

// The same fragment read from the LDS copy of x (row pitch `pitch` bytes,
// column 0 = first K position of the split; the copy is zero past K).  Rows
// m >= M read row M-1; tiles past the split read tile kl_max and are zeroed.
template <int MT>
__device__ __forceinline__ void load_x_lds(const uint8_t* xs, int pitch, int M, int kl, int kl_max,
                                           int lane, half8 (&xa)[MT][2]) {
  const bool valid = kl <= kl_max;
  const int k = min(kl, kl_max) * kTileK + 16 * (lane >> 4);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = min(mt * 16 + (lane & 15), M - 1);
    const uint8_t* p = xs + m * pitch + k * 2;
    const half8 v0 = as_half8(*reinterpret_cast<const uint4*>(p));
    const half8 v1 = as_half8(*reinterpret_cast<const uint4*>(p + 16));
    xa[mt][0] = valid ? v0 : half8{};
    xa[mt][1] = valid ? v1 : half8{};
  }
}

// The int4 fragment (four half8, positions 32*(l/16) .. +31 of the tile)
// from the LDS copy of x; same conventions as load_x_lds.
template <int MT>
__device__ __forceinline__ void load_x_lds4(const uint8_t* xs, int pitch, int M, int kl, int kl_max,
                                            int lane, half8 (&xa)[MT][4]) {
  const bool valid = kl <= kl_max;
  const int k = min(kl, kl_max) * kTileK4 + 32 * (lane >> 4);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = min(mt * 16 + (lane & 15), M - 1);
    const uint8_t* p = xs + m * pitch + k * 2;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const half8 v = as_half8(*reinterpret_cast<const uint4*>(p + 16 * c));
      xa[mt][c] = valid ? v : half8{};
    }
  }
}

// Dynamic LDS bytes the kernel needs: max(x copy, cross-wave reduction);
// tk = input positions per weight tile (64 int8, 128 int4).
inline size_t gemv_lds_bytes(int MT, int NS, int W, bool XL, int M, int kb_per_split,
                             int tk = kTileK) {
  const size_t red = (size_t)W * MT * NS * kWave * sizeof(floatx4);
  // x copy, rounded up to whole 1 KB DMA chunks
  const size_t xb = XL ? ((size_t)M * (size_t)(kb_per_split * tk * 2 + 16) + 1023) / 1024 * 1024 : 0;
  return red > xb ? red : xb;
}

// Split-K: each workgroup has stored its partials; the last one to arrive
// at the group's counter sums every split in split order (deterministic),
// applies scale and bias, stores fp16 (and feeds the fused argmax), and
// re-zeroes the counter.  Returns whether this workgroup was the last.
template <int NS, bool SC>
__device__ __forceinline__ bool split_k_reduce(const GemvKernelArgs& a, int group, int strip0,
                                               int P_nstrips, int P_N, int P_col0,
                                               const _Float16* P_scale, const _Float16* P_bias,
                                               _Float16* P_y, int64_t P_ldy, bool amax,
                                               unsigned long long* row_key, int tid, int nthreads) {
  __shared__ uint32_t is_last;
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // partial stores complete
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(&a.counters[group], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = (prev == (uint32_t)(a.splits - 1)) ? 1u : 0u;
  }
  __syncthreads();
  if (!is_last) return false;

  const int nrows = min(NS, P_nstrips - strip0) * 16;
  const int total = a.M * nrows;
  for (int i = tid; i < total; i += nthreads) {
    const int m = i / nrows;
    const int n = strip0 * 16 + (i - m * nrows);
    // Issue every split's load before summing (one memory round trip), then
    // add in split order.
    float part[kMaxSplits];
#pragma unroll
    for (int sp = 0; sp < kMaxSplits; ++sp)
      part[sp] = sp < a.splits
                     ? load_coherent(&a.partial[((int64_t)sp * a.M + m) * a.np + P_col0 + n])
                     : 0.f;
    float sum = part[0];
#pragma unroll
    for (int sp = 1; sp < kMaxSplits; ++sp)
      if (sp < a.splits) sum += part[sp];
    if (n < P_N) {
      const float sc = SC ? (float)P_scale[n] : 1.f;
      const float bi = P_bias ? (float)P_bias[n] : 0.f;
      const _Float16 v = (_Float16)__builtin_fmaf(sum, sc, bi);
      if (P_y) P_y[(int64_t)m * P_ldy + n] = v;
      if (amax)
        __hip_atomic_fetch_max(&row_key[m], argmax_key(v, n), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
  if (tid == 0)
    __hip_atomic_store(&a.counters[group], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// Fused argmax: this workgroup's per-row best keys (row_key, LDS) go to its
// group's own slots with plain stores -- no atomics on shared addresses,
// which with thousands of workgroups on one row would serialise -- and the
// next launch on the stream (argmax_finish_kernel) reduces the slots.
__device__ __forceinline__ void argmax_store(const GemvKernelArgs& a, const unsigned long long* row_key,
                                             int group, int tid, int nthreads) {
  __syncthreads();  // row_key complete
  for (int m = tid; m < a.M; m += nthreads)
    a.amax_slots[(int64_t)m * gridDim.x + group] = row_key[m];
}

// Group (strip range) of workgroup bx out of G = gridDim.x.  The hardware
// deals workgroups to the 8 XCDs round-robin by dispatch id, x fastest, so
// with group = bx adjacent strips run on different XCDs.  A 128-byte line of
// a group-wise scale row holds the scales of four adjacent strips (32 bytes
// each), and every XCD's L2 would fetch it: up to four times the scale
// traffic.  Here the groups an XCD runs form one contiguous range of
// `run` = G / 8 groups (the first 8 * run workgroups of each split; any rest
// keep their id), a bijection of [0, G) either way; run = 0 keeps every id.
// The K split stays blockIdx.y, so the splits of one group keep sharing an
// XCD when G % 8 == 0 (a split-major order, one K slice of x per XCD, measured
// slower on every int8 and int4 K-split launch tried).
__device__ __forceinline__ int xcd_group(int bx, int run) {
  return bx < 8 * run ? (bx & 7) * run + (bx >> 3) : bx;
}

// WF (WeightFormat): int8 tiles (64 input positions, two MFMAs per tile and
// strip) or int4 tiles (128 positions, four MFMAs); group-wise int4 loads one
// scale per lane, tile and strip alongside the weights and applies it at
// dequantization, the other formats scale in the epilogue.
template <int MT, int NS, int W, int U, bool XL, bool NT, bool KT, int WF = kWfInt8>
__global__ __launch_bounds__(W * 64) void w8a16_gemv_kernel(GemvKernelArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int kThreads = W * kWave;
  constexpr int T = MT * NS;  // 16x16 output tiles per workgroup
  constexpr int XN = WF ? 4 : 2;  // half8 activation chunks per tile and m-tile
  constexpr int TK = WF ? kTileK4 : kTileK;  // input positions per weight tile
  constexpr bool GS = WF == kWfInt4Grp;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
  // (only group-wise launches renumber: the others need not wait for xcd_run)
  const int group = GS ? xcd_group(blockIdx.x, a.xcd_run) : (int)blockIdx.x;
  const int split = blockIdx.y;
  // Projection of this workgroup (uniform across it).  Its fields are loaded
  // once pi is known, a second scalar-memory trip.  Reading one field of each
  // 64-byte argument line with the first loads (the loop below reads the
  // group0 of projections 1..3) brings every line into the scalar cache, so
  // that trip hits it.
  int pi = 0;
  __asm__ volatile("" ::"s"(a.M), "s"(a.proj[0].group0), "s"(a.kb_per_split));
#pragma unroll
  for (int i = 1; i < kMaxProj; ++i)
    if (i < a.nproj && group >= a.proj[i].group0) pi = i;
  const uint8_t* const P_w = a.proj[pi].w;
  const _Float16* const P_scale = a.proj[pi].scale;
  const _Float16* const P_bias = a.proj[pi].bias;
  _Float16* const P_y = a.proj[pi].y;
  const int64_t P_ldy = a.proj[pi].ldy;
  const int P_N = a.proj[pi].N;
  const int P_nstrips = a.proj[pi].nstrips;
  const int P_col0 = a.proj[pi].col0;
  const int strip0 = (group - a.proj[pi].group0) * NS;
  const int kb0 = split * a.kb_per_split;
  const int kb1 = min(kb0 + a.kb_per_split, a.kblocks);
  const int ntiles = kb1 - kb0;

  // LDS row pitch of the x copy: 128 B per tile (+16 B in the register-
  // staged K-tail path, so rows start on different banks).
  const int pitch = XL ? ntiles * TK * 2 + (KT ? 16 : 0) : 0;

  // CH independent accumulator chains (the two K halves of a tile, and
  // alternate tiles when registers allow): a single chain would make every
  // MFMA wait for the previous one, and the wavefront could not issue its
  // next loads meanwhile.  The chains are summed in a fixed order at the end.
  constexpr int CH = (MT * NS <= 2) ? 4 : 2;
  floatx4 accs[CH][MT][NS];
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int s = 0; s < NS; ++s) accs[c][mt][s] = floatx4{0.f, 0.f, 0.f, 0.f};

  // Strip s of this group exists iff strip0 + s < nstrips (uniform per WG);
  // a missing strip loads the projection's last strip instead and its
  // outputs are never stored.  Tile bases are wave-uniform (scalar); lane l
  // reads bytes [16*l, 16*l + 16) of a tile.
  const uint8_t* wstrip[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int strip = min(strip0 + s, P_nstrips - 1);
    wstrip[s] = P_w + ((int64_t)strip * a.kblocks + kb0) * kTileBytes;
  }
  const uint32_t woff = lane * 16;
  // Activation rows: a wave-uniform base per m-tile (its first row, clamped
  // to M-1) and a per-lane offset of at most 15 rows (load_x_global).
  const uint8_t* xrow[MT];
  uint32_t xoff[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r0 = min(mt * 16, a.M - 1);
    xrow[mt] = reinterpret_cast<const uint8_t*>(a.x + (int64_t)r0 * a.ldx);
    xoff[mt] = (uint32_t)((int64_t)(min(mt * 16 + (lane & 15), a.M - 1) - r0) * a.ldx * 2) +
               (WF ? 64 : 32) * (lane >> 4);
  }
  // Group-wise int4 scale of lane l, strip s, tile kl: scale row
  // (4*(kb0 + kl) + l/16) >> gshift (4 lane groups of 32 positions per
  // tile), column 16*strip + l%16.  Wave-uniform row part per tile, fixed
  // per-lane part.
  const _Float16* sstrip[GS ? NS : 1];
  uint32_t slane = 0;
  if (GS) {
#pragma unroll
    for (int s = 0; s < NS; ++s) sstrip[s] = P_scale + 16 * min(strip0 + s, P_nstrips - 1);
    slane = (uint32_t)(((lane >> 4) >> a.gshift) * P_N + (lane & 15));
  }

  // Tiles of this wavefront: local index kl = wave + W*i, i in [0, my).
  // Every load below is unconditional: a tile past the split (the last
  // stage may be partial) loads tile ntiles-1 and is skipped in compute (a
  // wave-uniform branch with no loads in it, so in-flight loads are not
  // waited for; overwriting their registers would be).
  const int my = ntiles > wave ? (ntiles - wave + W - 1) / W : 0;
  const int stages = (my + U - 1) / U;

  uint4 wA[U][NS], wB[U][NS];
  half8 xA[XL ? 1 : U][MT][XN], xB[XL ? 1 : U][MT][XN];
  _Float16 sA[GS ? U : 1][NS], sB[GS ? U : 1][NS];

  // nvalid < U (a wave-uniform count, U at every pipelined call): only the
  // stage's first nvalid tiles are loaded; see the one-stage path below.
  auto load_stage = [&](int st, uint4 (&wv)[U][NS], half8 (&xv)[XL ? 1 : U][MT][XN],
                        _Float16 (&sv)[GS ? U : 1][NS], int nvalid) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (u >= nvalid) break;  // wave-uniform
      const int kl = wave + W * (st * U + u);
      const int klc = min(kl, ntiles - 1);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const uint8_t* p = wstrip[s] + (int64_t)klc * kTileBytes + woff;
        wv[u][s] = NT ? load_u4_stream(p) : load_u4(p);
      }
      if (GS) {
        if (KT) {
          // K % 128 == 64: the last tile's lanes 32..63 lie past K (their
          // activations are zero); clamp their scale row into the matrix.
          const int srow = min((4 * (kb0 + klc) + (lane >> 4)) >> a.gshift,
                               (a.K >> (5 + a.gshift)) - 1);
#pragma unroll
          for (int s = 0; s < NS; ++s)
            sv[GS ? u : 0][s] = sstrip[GS ? s : 0][(int64_t)srow * P_N + (lane & 15)];
        } else {
          const int srow = (4 * (kb0 + klc)) >> a.gshift;  // wave-uniform
#pragma unroll
          for (int s = 0; s < NS; ++s)
            sv[GS ? u : 0][s] = sstrip[GS ? s : 0][(int64_t)srow * P_N + slane];
        }
      }
      if constexpr (WF != kWfInt8) {
        if (!XL) load_x_global4<MT, KT>(a, kb0 + klc, xrow, xoff, lane, xv[XL ? 0 : u]);
      } else if (!XL) {
        load_x_global<MT, KT>(a, kb0 + klc, xrow, xoff, lane, xv[XL ? 0 : u]);
      }
    }
  };

  auto compute_stage = [&](int st, const uint4 (&wv)[U][NS], half8 (&xv)[XL ? 1 : U][MT][XN],
                           const _Float16 (&sv)[GS ? U : 1][NS]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kl = wave + W * (st * U + u);
      if (kl >= ntiles) break;  // wave-uniform
      if constexpr (WF != kWfInt8) {
        // Four MFMAs per tile and strip: dword j holds positions 8j..8j+7 of
        // the lane's 32, matching activation chunk j.
        half8 xl4[MT][4];
        if (XL) load_x_lds4<MT>(smem, pitch, a.M, kl, ntiles - 1, lane, xl4);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const uint32_t wd[4] = {wv[u][s].x, wv[u][s].y, wv[u][s].z, wv[u][s].w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const half8 b = GS ? dequant8_i4_scaled(wd[j], sv[GS ? u : 0][s]) : dequant8_i4(wd[j]);
            const int c = (4 * u + j) % CH;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              accs[c][mt][s] = mfma16x16x32(XL ? xl4[mt][j] : xv[XL ? 0 : u][mt][j], b, accs[c][mt][s]);
          }
        }
      } else {
        half8 xl[MT][2];
        if (XL) load_x_lds<MT>(smem, pitch, a.M, kl, ntiles - 1, lane, xl);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const half8 b0 = dequant8(wv[u][s].x, wv[u][s].y);
          const half8 b1 = dequant8(wv[u][s].z, wv[u][s].w);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const half8 x0 = XL ? xl[mt][0] : xv[XL ? 0 : u][mt][0];
            const half8 x1 = XL ? xl[mt][1] : xv[XL ? 0 : u][mt][1];
            const int c = (2 * u) % CH;  // chains c (first K half), c+1 (second)
            accs[c][mt][s] = mfma16x16x32(x0, b0, accs[c][mt][s]);
            accs[c + 1][mt][s] = mfma16x16x32(x1, b1, accs[c + 1][mt][s]);
          }
        }
      }
    }
  };

  // x[0:M, split's K range] -> LDS by DMA (K % 64 == 0: no zero fill):
  // 1 KB chunk j of the row-major copy (pitch = 128 B per tile) is written by
  // wavefront j % W; lanes past the end read the last chunk again and land
  // in the rounded-up tail of the allocation.  Issued first: the weight
  // loads below may then stay in flight while it is waited for.
  if (XL && !KT) {
    const int total = a.M * pitch;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_u8*)smem;
    for (int j = wave; j * 1024 < total; j += W) {
      const int pb = min(j * 1024 + lane * 16, total - 16);
      int m = 0;  // pb / pitch, by M - 1 compares (x is staged for small M only)
      for (int r = 1; r < a.M; ++r) m += pb >= r * pitch ? 1 : 0;
      const int c = pb - m * pitch;
      const uint8_t* src = reinterpret_cast<const uint8_t*>(a.x + (int64_t)m * a.ldx + kb0 * TK) + c;
      dma16(src, lds0 + j * 1024);
    }
  }
  // ---- stage x[0:M, split's K range] in LDS (zero past K) ----------------
  // Called once the first weight stages are out; `issued` (0..2) full
  // stages of them may stay in flight past the x copy's wait (0: that wait
  // covers every load issued so far).
  auto stage_x = [&](int issued) {
    if (XL && KT) {
      // Columns past K need zeros: staged through registers (after the first
      // weight tiles went out, so the two round trips overlap).
      const int row_chunks = ntiles * (TK / 8);
      const int total = a.M * row_chunks;
      for (int c = tid; c < total; c += kThreads) {
        const int m = c / row_chunks, cc = c - m * row_chunks;
        const int k = kb0 * TK + cc * 8;
        const uint4 v = load_u4(a.x + (int64_t)m * a.ldx + min(k, a.K - 8));
        *reinterpret_cast<uint4*>(smem + m * pitch + cc * 16) = k < a.K ? v : make_uint4(0, 0, 0, 0);
      }
      __syncthreads();
    } else if (XL) {
      // The DMAs were issued before the weight loads (xdma above): wait for
      // this wave's share (every load issued after them may stay in flight),
      // then for everyone's.
      // (loads per stage: U*NS weight tiles, and as many group scales)
      constexpr int LPS = U * NS * (GS ? 2 : 1);
      if (issued > 1) __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * LPS) : "memory");
      else if (issued > 0) __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(LPS) : "memory");
      else __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
      barrier_lds();
    }
  };

  // Two-stage pipeline, unrolled by two so the buffers never move: a
  // stage's buffer is refilled (two stages ahead) as soon as it is consumed.
  // The compiler waits for a stage's loads by counting the loads issued
  // after them, and where paths that issued different numbers of loads
  // meet it must assume the fewest, i.e. wait for the next stage's loads
  // too.  So with one m-tile (M <= 16) a wavefront with two or more stages
  // takes a path on which every load is unconditional up to a tail of two
  // or three stages: the prologue's two stages and both refills of the
  // steady-state loop (which runs zero times for two or three stages); a
  // stage is then computed as soon as its own loads are in, with the next
  // one still in flight.  The instances with two or four m-tiles keep the
  // plain loop: on that path the compiler holds more values live at once,
  // and their register budget (up to four m-tiles of activations per
  // stage) has no room for them.
  if (MT == 1 && stages >= 2) {
    load_stage(0, wA, xA, sA, U);
    load_stage(1, wB, xB, sB, U);
    // (the prologue's loads all go out before any MFMA: the scheduler would
    // otherwise sink each tile's loads to just before its use)
    __builtin_amdgcn_sched_barrier(0);
    stage_x(2);
    int st = 0;
    // (the scheduling barriers keep each refill ahead of the next stage's
    // MFMAs, which the scheduler would otherwise interleave with it)
    for (; st + 3 < stages; st += 2) {
      compute_stage(st, wA, xA, sA);
      load_stage(st + 2, wA, xA, sA, U);
      __builtin_amdgcn_sched_barrier(0);
      compute_stage(st + 1, wB, xB, sB);
      load_stage(st + 3, wB, xB, sB, U);
      __builtin_amdgcn_sched_barrier(0);
    }
    // two or three stages left, the last possibly partial
    compute_stage(st, wA, xA, sA);
    if (st + 2 < stages) {
      load_stage(st + 2, wA, xA, sA, U);
      __builtin_amdgcn_sched_barrier(0);
      compute_stage(st + 1, wB, xB, sB);
      compute_stage(st + 2, wA, xA, sA);
    } else {
      compute_stage(st + 1, wB, xB, sB);
    }
  } else if (stages <= 1) {
    // At most one stage: its loads all go out before any MFMA (the
    // scheduling barrier: the scheduler would otherwise sink each tile's
    // loads to just before its use, one memory round trip per tile).  A
    // partial stage loads only its tiles (nothing is pipelined behind it);
    // the x copy's exact wait counts a full stage, so it then waits for
    // every load.
    const bool full = my >= U;
    if (stages > 0) load_stage(0, wA, xA, sA, full ? U : my);
    __builtin_amdgcn_sched_barrier(0);
    stage_x(full ? stages : 0);
    if (stages > 0) compute_stage(0, wA, xA, sA);
  } else {
    // The first two stages of weight tiles go out before anything waits.
    load_stage(0, wA, xA, sA, U);
    load_stage(1, wB, xB, sB, U);
    __builtin_amdgcn_sched_barrier(0);
    stage_x(stages);
    for (int st = 0; st < stages; st += 2) {
      compute_stage(st, wA, xA, sA);
      if (st + 2 < stages) load_stage(st + 2, wA, xA, sA, U);
      if (st + 1 >= stages) break;
      compute_stage(st + 1, wB, xB, sB);
      if (st + 3 < stages) load_stage(st + 3, wB, xB, sB, U);
    }
  }

  floatx4 acc[MT][NS];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      acc[mt][s] = accs[0][mt][s] + accs[1][mt][s];
#pragma unroll
      for (int c = 2; c < CH; c += 2) acc[mt][s] += accs[c][mt][s] + accs[c + 1][mt][s];
    }

  // ---- cross-wavefront reduction through LDS (fixed order) --------------
  const bool amax = a.amax_slots != nullptr;  // fused argmax (M <= 64 rows)
  __shared__ unsigned long long row_key[64];
  if (amax)
    for (int i = tid; i < 64; i += kThreads) row_key[i] = 0;
  if (XL) __syncthreads();  // everyone is done with the x copy
  float* red = reinterpret_cast<float*>(smem);  // [W][T][64 lanes][4]
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < NS; ++s)
      *reinterpret_cast<floatx4*>(&red[((wave * T + mt * NS + s) * kWave + lane) * 4]) = acc[mt][s];
  __syncthreads();

  // Element e = (tile t, lane ln, row r) of the workgroup's T tiles; lane ln
  // of an MFMA result holds D[4*(ln/16) + r][ln%16].
  for (int e = tid; e < T * 256; e += kThreads) {
    const int t = e >> 8, j = e & 255, ln = j >> 2, r = j & 3;
    float sum = red[t * 256 + j];
#pragma unroll
    for (int w = 1; w < W; ++w) sum += red[(w * T + t) * 256 + j];
    const int mt = t / NS, s = t % NS;
    const int n = (strip0 + s) * 16 + (ln & 15);
    const int m = mt * 16 + 4 * (ln >> 4) + r;
    if (m >= a.M || strip0 + s >= P_nstrips) continue;
    if (a.splits == 1) {
      if (n < P_N) {
        const float sc = GS ? 1.f : (float)P_scale[n];
        const float bi = P_bias ? (float)P_bias[n] : 0.f;
        const _Float16 v = (_Float16)__builtin_fmaf(sum, sc, bi);
        if (P_y) P_y[(int64_t)m * P_ldy + n] = v;
        if (amax)
          __hip_atomic_fetch_max(&row_key[m], argmax_key(v, n), __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    } else {
      store_coherent(&a.partial[((int64_t)split * a.M + m) * a.np + P_col0 + n], sum);
    }
  }
  if (a.splits > 1 && !split_k_reduce<NS, !GS>(a, group, strip0, P_nstrips, P_N, P_col0, P_scale,
                                          P_bias, P_y, P_ldy, amax, row_key, tid, kThreads))
    return;
  if (amax) argmax_store(a, row_key, group, tid, kThreads);
}

// One workgroup per row: the largest key over the GEMV's slots[m][0..G),
// decoded to its column (lowest column among equal values, see argmax_key).
// Each thread keeps four independent maxima over 16-byte loads, so its loads
// are all in flight together; then a tree over the workgroup.
constexpr int kFinishThreads = 1024;
__global__ __launch_bounds__(kFinishThreads) void argmax_finish_kernel(
    const unsigned long long* slots, int G, int32_t* index) {
  __shared__ unsigned long long best[kFinishThreads];
  const int m = blockIdx.x, tid = threadIdx.x;
  const unsigned long long* row = slots + (int64_t)m * G;
  unsigned long long k[4] = {0, 0, 0, 0};
  // G * 8 bytes per row: the row starts 16-byte aligned when m * G is even.
  const int lead = ((m * G) & 1) ? 1 : 0;
  if (lead && tid == 0) k[0] = row[0];
  const int pairs = (G - lead) / 2;
  const ulonglong2* row2 = reinterpret_cast<const ulonglong2*>(row + lead);
  int i = tid;
#pragma unroll 1
  for (; i + 3 * kFinishThreads < pairs; i += 4 * kFinishThreads) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const ulonglong2 v = row2[i + u * kFinishThreads];
      const unsigned long long w = v.x > v.y ? v.x : v.y;
      k[u] = w > k[u] ? w : k[u];
    }
  }
  for (; i < pairs; i += kFinishThreads) {
    const ulonglong2 v = row2[i];
    const unsigned long long w = v.x > v.y ? v.x : v.y;
    k[0] = w > k[0] ? w : k[0];
  }
  if (tid == 0 && lead + 2 * pairs < G) k[1] = row[G - 1] > k[1] ? row[G - 1] : k[1];
  k[0] = k[0] > k[1] ? k[0] : k[1];
  k[2] = k[2] > k[3] ? k[2] : k[3];
  best[tid] = k[0] > k[2] ? k[0] : k[2];
  __syncthreads();
  for (int w = kFinishThreads / 2; w > 0; w >>= 1) {
    if (tid < w && best[tid + w] > best[tid]) best[tid] = best[tid + w];
    __syncthreads();
  }
  if (tid == 0) index[m] = argmax_index_of(best[0]);
}

template <int MT, int NS, int W, int U, bool XL, bool NT, int WF = kWfInt8>
hipError_t launch_t(const GemvKernelArgs& ka, const GemvPlan& p, hipStream_t stream) {
  const size_t lds = gemv_lds_bytes(MT, NS, W, XL, ka.M, ka.kb_per_split, WF ? kTileK4 : kTileK);
  if (lds > 65536) return hipErrorInvalidValue;
  dim3 grid(p.groups, p.splits, 1);
  if ((ka.K % (WF ? kTileK4 : kTileK)) != 0)  // K-tail variant: chunks past K are zeroed
    hipLaunchKernelGGL((w8a16_gemv_kernel<MT, NS, W, U, XL, NT, true, WF>), grid, dim3(W * kWave),
                       lds, stream, ka);
  else
    hipLaunchKernelGGL((w8a16_gemv_kernel<MT, NS, W, U, XL, NT, false, WF>), grid, dim3(W * kWave),
                       lds, stream, ka);
  return hipGetLastError();
}

GemvKernelArgs make_args(const LinearProblem& pr, const GemvPlan& p, void* workspace) {
  GemvKernelArgs ka;
  ka.x = pr.x;
  ka.ldx = pr.ldx;
  ka.M = pr.M;
  ka.K = pr.K;
  // Weight tiles along K: 64 input positions per int8 tile, 128 per int4 tile.
  ka.kblocks = (int)ceil_div(pr.K, pr.wf ? kTileK4 : kTileK);
  ka.gshift = pr.gshift;
  ka.nproj = pr.nproj;
  int group = 0, col = 0;
  for (int i = 0; i < kMaxProj; ++i) {
    GemvProj& q = ka.proj[i];
    if (i < pr.nproj) {
      q.w = pr.proj[i].w;
      q.scale = pr.proj[i].scale;
      q.bias = pr.proj[i].bias;
      q.y = pr.proj[i].y;
      q.ldy = pr.proj[i].ldy;
      q.N = pr.proj[i].N;
      q.nstrips = (int)ceil_div(pr.proj[i].N, 16);
      q.group0 = group;
      q.col0 = col;
      group += (int)ceil_div(q.nstrips, p.ns);
      col += q.nstrips * 16;
    } else {
      q = ka.proj[0];
      q.group0 = 0x7fffffff;  // never selected
    }
  }
  ka.splits = p.splits;
  ka.kb_per_split = p.kb_per_split;
  ka.np = col;
  // Workspace: [counters | partials]; counter region size fixed by the ABI.
  ka.counters = reinterpret_cast<uint32_t*>(workspace);
  ka.partial = workspace ? reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) +
                                                    RF_W8A16_WS_COUNTER_BYTES)
                         : nullptr;
  ka.amax_slots = nullptr;
  // Contiguous strip ranges per XCD on every group-wise launch: without them
  // each XCD's L2 fetches the scale lines of its strips' neighbours too
  // (FETCH_SIZE at M = 1, gs = 32: 1.34x the algorithmic bytes on 4096 x 4096
  // and on the fused 24576 x 4096 gate/up, 1.12x on the fused q/k/v, against
  // 1.003..1.016x with the ranges).  Graph-timed on MI355X: launches of 16 MB
  // or more 5..12% faster at M = 1 and 2..3% at M = 16, smaller ones within
  // +-2%; int8 launches (no scale lines) keep the hardware's order, which
  // measured 7..9% faster on q / o at M = 1..4.
  ka.xcd_run = pr.wf == kWfInt4Grp ? p.groups / 8 : 0;
  return ka;
}

// Kernel configurations the planner chooses from (all stream weights with
// non-temporal loads).  Measured on MI355X over the BASELINE decode shapes.
enum GemvCfgId {
  kG1x1W16U2,    // MT=1 NS=1 W=16 U=2  (U=4 without LDS staging spills at 128 VGPRs)
  kG1x1W16U4XL,  // MT=1 NS=1 W=16 U=4, x staged in LDS (M = 1, short K)
  kG1x1W8U4,     // MT=1 NS=1 W=8  U=4   (long K)
  kG1x1W8U4XL,   // MT=1 NS=1 W=8  U=4, x staged in LDS (many strips / long K)
  kG1x1W4U4,     // MT=1 NS=1 W=4  U=4
  kG1x2W16U2,    // MT=1 NS=2 W=16 U=2
  kG1x4W8U2,     // MT=1 NS=4 W=8  U=2   (M 5..16: x fragment reused 4x)
  kG1x4W4U2,     // MT=1 NS=4 W=4  U=2
  kG1x2W8U2,     // MT=1 NS=2 W=8  U=2
  kG2x4W4U2,     // MT=2 NS=4 W=4  U=2
  kG2x2W8U1,     // MT=2 NS=2 W=8  U=1
  kG2x1W8U4,     // MT=2 NS=1 W=8  U=4
  kG4x2W8U1,     // MT=4 NS=2 W=8  U=1
  kG4x2W4U1,     // MT=4 NS=2 W=4  U=1
  // Launches of many strips at M 5..16: as many strips per workgroup as give
  // about one workgroup per CU (or two, NS=3), so the activation fragment
  // each wavefront loads serves 3..7 weight tiles (int4 at half the unroll).
  kG1x3W8U2,     // MT=1 NS=3 W=8  U=2
  kG1x5W8U1,     // MT=1 NS=5 W=8  U=1
  kG1x6W8U1,     // MT=1 NS=6 W=8  U=1
  kG1x7W8U1,     // MT=1 NS=7 W=8  U=1
  kG2x2W16U1,    // MT=2 NS=2 W=16 U=1  (int8, M 17..32 on <= 128 strips, 4-way K split)
  kGemvCfgCount
};

struct GemvCfgDesc {
  int mt, ns, w;
  bool xl;
};

constexpr GemvCfgDesc kGemvCfgs[kGemvCfgCount] = {
    {1, 1, 16, false}, {1, 1, 16, true}, {1, 1, 8, false}, {1, 1, 8, true}, {1, 1, 4, false},
    {1, 2, 16, false}, {1, 4, 8, false}, {1, 4, 4, false}, {1, 2, 8, false},
    {2, 4, 4, false},  {2, 2, 8, false}, {2, 1, 8, false}, {4, 2, 8, false}, {4, 2, 4, false},
    {1, 3, 8, false},  {1, 5, 8, false}, {1, 6, 8, false}, {1, 7, 8, false},
    {2, 2, 16, false},
};

bool lds_fits(int cfg, int M, int kb_per_split) {
  const GemvCfgDesc& d = kGemvCfgs[cfg];
  return gemv_lds_bytes(d.mt, d.ns, d.w, d.xl, M, kb_per_split) <= 65536;
}

hipError_t launch_gemv_cfg(const GemvKernelArgs& ka, const GemvPlan& p, hipStream_t stream) {
  switch (p.cfg) {
    case kG1x1W16U2: return launch_t<1, 1, 16, 2, false, true>(ka, p, stream);
    case kG1x1W16U4XL: return launch_t<1, 1, 16, 4, true, true>(ka, p, stream);
    case kG1x1W8U4: return launch_t<1, 1, 8, 4, false, true>(ka, p, stream);
    case kG1x1W8U4XL: return launch_t<1, 1, 8, 4, true, true>(ka, p, stream);
    case kG1x1W4U4: return launch_t<1, 1, 4, 4, false, true>(ka, p, stream);
    case kG1x2W16U2: return launch_t<1, 2, 16, 2, false, true>(ka, p, stream);
    case kG1x4W8U2: return launch_t<1, 4, 8, 2, false, true>(ka, p, stream);
    case kG1x4W4U2: return launch_t<1, 4, 4, 2, false, true>(ka, p, stream);
    case kG1x2W8U2: return launch_t<1, 2, 8, 2, false, true>(ka, p, stream);
    case kG2x4W4U2: return launch_t<2, 4, 4, 2, false, true>(ka, p, stream);
    case kG2x2W8U1: return launch_t<2, 2, 8, 1, false, true>(ka, p, stream);
    case kG2x1W8U4: return launch_t<2, 1, 8, 4, false, true>(ka, p, stream);
    case kG4x2W8U1: return launch_t<4, 2, 8, 1, false, true>(ka, p, stream);
    case kG4x2W4U1: return launch_t<4, 2, 4, 1, false, true>(ka, p, stream);
    case kG1x3W8U2: return launch_t<1, 3, 8, 2, false, true>(ka, p, stream);
    case kG1x5W8U1: return launch_t<1, 5, 8, 1, false, true>(ka, p, stream);
    case kG1x7W8U1: return launch_t<1, 7, 8, 1, false, true>(ka, p, stream);
    case kG2x2W16U1: return launch_t<2, 2, 16, 1, false, true>(ka, p, stream);
    default: return hipErrorInvalidValue;  // (kG1x6W8U1: planned for int4 only)
  }
}

// Int4 launches take the same rules with K counted in 128-wide tiles (one
// 1 KB tile per 128 positions, as an int8 tile holds 64): a configuration
// runs with half its unroll (its int4 tiles carry twice the activation
// registers), except one per-channel XL instance below.
template <int WF>
hipError_t launch_gemv4_cfg(const GemvKernelArgs& ka, const GemvPlan& p, hipStream_t stream) {
  // x staged in LDS where the planner asks for it and int4's 256 bytes of x
  // per row and tile still fit.
  auto xl_fits = [&](int ns, int w) {
    return gemv_lds_bytes(1, ns, w, true, ka.M, ka.kb_per_split, kTileK4) <= 65536;
  };
  switch (p.cfg) {
    // With x in LDS no activation registers ride the pipeline, so the
    // 16-wavefront per-channel instance keeps the int8 unroll (down 4096 x
    // 12288 at M 1: 7.36..7.70 instead of 7.78..8.33 us).  At the int8
    // unroll the group-wise instances lose 10..13% to their scale loads and
    // the 8-wavefront one 1..2%, so they keep half.
    case kG1x1W16U4XL:
      if (xl_fits(1, 16)) {
        if (WF == kWfInt4) return launch_t<1, 1, 16, 2, true, true, WF>(ka, p, stream);
        return launch_t<1, 1, 16, 1, true, true, WF>(ka, p, stream);
      }
      return launch_t<1, 1, 16, 1, false, true, WF>(ka, p, stream);
    case kG1x1W8U4XL:
      if (xl_fits(1, 8)) return launch_t<1, 1, 8, 2, true, true, WF>(ka, p, stream);
      return launch_t<1, 1, 8, 2, false, true, WF>(ka, p, stream);
    case kG1x1W16U2: return launch_t<1, 1, 16, 1, false, true, WF>(ka, p, stream);
    case kG1x1W8U4: return launch_t<1, 1, 8, 2, false, true, WF>(ka, p, stream);
    case kG1x1W4U4: return launch_t<1, 1, 4, 2, false, true, WF>(ka, p, stream);
    case kG1x2W16U2: return launch_t<1, 2, 16, 1, false, true, WF>(ka, p, stream);
    case kG1x4W8U2: return launch_t<1, 4, 8, 1, false, true, WF>(ka, p, stream);
    case kG1x4W4U2: return launch_t<1, 4, 4, 1, false, true, WF>(ka, p, stream);
    case kG1x2W8U2: return launch_t<1, 2, 8, 1, false, true, WF>(ka, p, stream);
    case kG2x4W4U2: return launch_t<2, 4, 4, 1, false, true, WF>(ka, p, stream);
    case kG2x2W8U1: return launch_t<2, 2, 8, 1, false, true, WF>(ka, p, stream);
    case kG2x1W8U4: return launch_t<2, 1, 8, 2, false, true, WF>(ka, p, stream);
    case kG4x2W8U1: return launch_t<4, 2, 8, 1, false, true, WF>(ka, p, stream);
    case kG4x2W4U1: return launch_t<4, 2, 4, 1, false, true, WF>(ka, p, stream);
    case kG1x3W8U2: return launch_t<1, 3, 8, 1, false, true, WF>(ka, p, stream);
    case kG1x6W8U1: return launch_t<1, 6, 8, 1, false, true, WF>(ka, p, stream);
    case kG1x7W8U1: return launch_t<1, 7, 8, 1, false, true, WF>(ka, p, stream);
    default: return hipErrorInvalidValue;  // (kG1x5W8U1: not planned for int4)
  }
}

}  // namespace

void gemv_cfg_info(const GemvPlan& p, int M, bool int4, int* waves, bool* x_in_lds) {
  const bool ok = p.cfg >= 0 && p.cfg < kGemvCfgCount;
  *waves = ok ? kGemvCfgs[p.cfg].w : 0;
  // int4 stages x in LDS only where its 256 bytes per row and tile fit
  // (launch_gemv4_cfg)
  *x_in_lds = ok && kGemvCfgs[p.cfg].xl &&
              (!int4 || gemv_lds_bytes(1, 1, *waves, true, M, p.kb_per_split, kTileK4) <= 65536);
}

size_t gemv_workspace_bytes(const GemvPlan& p, int M, const int* Ns, int nproj) {
  if (p.splits <= 1) return 0;
  int64_t np = 0;
  for (int i = 0; i < nproj; ++i) np += round_up(Ns[i], 16);
  return (size_t)p.splits * (size_t)M * (size_t)np * sizeof(float);
}

hipError_t launch_gemv(const LinearProblem& pr, const GemvPlan& p, void* workspace,
                       hipStream_t stream, const ArgmaxTarget* am) {
  if (pr.nproj < 1 || pr.nproj > kMaxProj) return hipErrorInvalidValue;
  GemvKernelArgs ka = make_args(pr, p, workspace);
  if (pr.wf != kWfInt8) {
    if (am) return hipErrorInvalidValue;
    return pr.wf == kWfInt4 ? launch_gemv4_cfg<kWfInt4>(ka, p, stream)
                            : launch_gemv4_cfg<kWfInt4Grp>(ka, p, stream);
  }
  if (am) {
    if (pr.nproj != 1 || pr.M > 64 || !am->slots || !am->index) return hipErrorInvalidValue;
    ka.amax_slots = reinterpret_cast<unsigned long long*>(am->slots);
    const hipError_t e = launch_gemv_cfg(ka, p, stream);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(pr.M), dim3(kFinishThreads), 0, stream,
                       static_cast<const unsigned long long*>(ka.amax_slots), p.groups, am->index);
    return hipGetLastError();
  }
  return launch_gemv_cfg(ka, p, stream);
}

size_t argmax_slot_bytes(const GemvPlan& p, int M) { return (size_t)M * (size_t)p.groups * 8; }

GemvPlan plan_gemv_rules(int M, const int* Ns, int nproj, int K, const DeviceInfo& dev,
                         bool int8_rules);

// Int4 launches: the int8 rules over K counted in 128-wide tiles (one 1 KB
// tile per 128 positions), with these changes, measured on MI355X (cfg1 and
// Qwen3-VL-32B shapes, N 1024..25600, K 1024..25600, per-channel and
// group-wise scales, graph-timed):
//   * M <= 4 on fewer than 257 strips (N <= 4096), where the int8 rules give
//     one strip per workgroup: an int4 tile reads two activation chunks per
//     wavefront load for every 128 positions, so staging x in LDS pays off
//     from a shorter K than for int8 (K >= 2176 per-channel; from K 8192 at
//     M <= 3 group-wise, whose scale loads share the load queue), and the
//     16-wavefront staging instance beats the 8-wavefront one from K 8192
//     (M = 1, 4096 x 12288: 7.10 against 7.64 us; M = 2: 7.38 against
//     8.83 us); K <= 1024 keeps the 4-wavefront instance per-channel only
//     (group-wise it loses 5..20%), and 1024 < K <= 2048 keeps 16 wavefronts
//     of one tile each;
//   * M <= 4 on 257..639 strips with K >= 8192: x in LDS at M = 1 (and at
//     M = 2 per-channel) where it fits, else two strips per 16-wavefront
//     workgroup (int4's x copy is twice int8's per weight byte and stops
//     fitting in LDS at M = 2 from K 16384; VL-32B down 5120 x 25600 at
//     M = 2: 22.1 against 28.4 us);
//   * M 3..4 with many strips: x staged in LDS (an int4 tile reads four
//     activation chunks per weight load, so the LDS copy pays off beyond
//     M = 2);
//   * M 8..16 on >= 1536 strips: four strips per 4-wavefront workgroup
//     (int8 takes two below 2048 strips; 25600 x 5120 at M = 16: 20.5
//     against 26.8 us; at 1024..1280 strips, or at M = 5, it loses up to
//     20%);
//   * M 5..16 on 257..511 strips: from K 16384 four strips per workgroup
//     with a 2-way K split (5120 x 25600 at M = 16: 25.9 against 34.4 us),
//     and at M >= 8 from K 8192 two strips per 8-wavefront workgroup;
//   * M 5..16, a long K with fewer strips: two strips per workgroup and a
//     2-way K split;
//   * M 5..8 on <= 64 strips: no K split (1024 x 4096 at M = 8: 5.1
//     against 5.8 us);
//   * M 5..16, about three, six or seven strips per CU (513..768,
//     1281..1536, 1537..1792 strips, no K split): that many strips per
//     8-wave workgroup, one workgroup per CU (three strips, two per CU, at
//     six per CU below M 12), so each activation fragment -- four chunks
//     per wavefront and tile -- serves 3..7 weight tiles (per-channel and
//     group-wise alike: 12288 x 4096 at M 5..16 7.3..9.1 against
//     8.8..9.7 us; 24576 x 4096 at M 16 13.7 against 16.4 us, at M 8 12.3
//     against 14.1 us; 25600 x 5120 at M 16 19.1 against 20.8 us).
// Ahead of those, rules measured over the decode projections of the
// reference's model families (Qwen3 0.6B..32B, Qwen3-VL-32B, Qwen2.5-VL
// 3B / 7B, the Pi0.5 Gemma decoder and expert) at M 1 / 2 / 4 / 8 / 16,
// per-channel and group-wise (128), against every configuration and K
// split; checked against the rules above on the 80 launches they change:
// 0.884 of the time (geometric mean), worst +1.7%:
//   * M 2..4 on >= 1024 strips from 24 tiles (M 3..4 from 16), and M 1 at
//     24..39 tiles: two strips per 8-wave workgroup instead of x in LDS
//     (Qwen3-8B gate/up 24576 x 4096 at M 4: 12.5 against 13.7 us
//     per-channel, 12.8 against 16.2 us group-wise);
//   * M <= 4 on 257..511 strips from 128 tiles: x in LDS split 2-way (4-way
//     from 192 tiles) at M <= 2, two strips split 4-way at M 3..4
//     (Qwen3-VL-32B down 5120 x 25600 at M 2: 16.2 against 17.9 us); M 3..4
//     on <= 128 strips from 64 tiles: two strips split 4-way (Qwen2.5-VL-3B
//     down 2048 x 11008 at M 4: 7.2 against 8.0 us);
//   * M 8..16 at five strips per CU (1025..1280 strips): three strips per
//     workgroup, six from M 12 (Qwen3-4B gate/up 19456 x 2560 at M 16: 9.4
//     against 11.7 us);
//   * M 2..4 from 128 tiles below 257 strips: two strips per workgroup,
//     split to about one workgroup per CU (Pi0.5 Gemma down 2048 x 16384 at
//     M 4: 8.0 against 10.6 us);
//   * per-channel M <= 2 at 64..127 tiles below 257 strips: x in LDS with 8
//     wavefronts instead of 16 (Qwen3-8B down 4096 x 12288 at M 1: 6.7
//     against 7.4 us);
//   * M 8..16 on >= 2048 strips: four strips per 8-wave workgroup, or three
//     or seven where they keep the rounds of 256 workgroups more than 5%
//     fuller, where one of them fills 85% (Qwen3-14B gate/up 34816 x 5120 at
//     M 8: three, 19.6 against 22.3 us);
//   * M 8..16 on <= 128 strips from 64 tiles (48 from M 12): two strips,
//     4-way split (Pi0.5 Gemma down at M 16: 9.6 against 11.1 us);
//     M 12..16 on 129..256 strips from 64 tiles: four strips, 4-way split;
//   * M 8..16 on 257..511 strips from 128 tiles: three strips and a 2-way
//     split at M 8, six strips and a 4-way split above (Qwen3-VL-32B down
//     5120 x 25600 at M 16: 19.8 against 24.2 us);
//   * M 9..16 on <= 64 strips below 32 tiles: one strip per 16-wave
//     workgroup, no split (Pi0.5 expert o 1024 x 2048 at M 16: 4.2 against
//     5.4 us);
//   * M 17..32 (int4 stays on the GEMV to M 64) below 1024 strips: two
//     strips per 4-wave workgroup from 640 strips (Qwen3-VL-32B q/k/v 10240
//     x 5120 at M 32: 17.8 against 27.8 us); on 65..256 strips one strip
//     per 8-wave workgroup of four tiles a stage below 24 tiles, else two
//     strips split 2-way (129..256, below 128 tiles) or 4-way (Qwen2.5-VL-3B
//     down 2048 x 11008 at M 32: 11.9 against 26.3 us); on <= 64 strips no
//     split up to M 24 below 24 tiles;
//   * M 33..64: from 512 strips four strips per 4-wave workgroup (two per
//     8-wave workgroup at <= 8 tiles), split 2-way on 512..767 strips from
//     32 tiles; on 257..511 strips two strips per 8-wave workgroup without
//     a split, or per 4-wave workgroup split 4-way from 128 tiles (Qwen3-14B
//     q/k/v at M 48: 20.0 against 25.2 us; Qwen3-VL-32B down: 67.2 against
//     85.2 us); below 257 strips a 4-way split up to 128 strips and none at
//     <= 8 tiles (Qwen3-0.6B q/k/v 4096 x 1024 at M 48: 6.3 against 7.9 us).
GemvPlan plan_gemv_int4(int M, const int* Ns, int nproj, int K, bool grouped,
                        const DeviceInfo& dev) {
  const int keff = (int)(round_up(K, kTileK4) / 2);
  GemvPlan p = plan_gemv_rules(M, Ns, nproj, keff, dev, false);
  const int ktiles = (int)ceil_div(K, kTileK4);
  // The rules see the launch's strips of all projections together.
  int nstrips = 0;
  for (int i = 0; i < nproj; ++i) nstrips += (int)ceil_div(Ns[i], 16);
  const int cu = dev.cus > 0 ? dev.cus : 256;
  auto strips_ge = [&](int n256) { return (int64_t)nstrips * 256 >= (int64_t)n256 * cu; };
  auto fits_xl = [&](int w) { return gemv_lds_bytes(1, 1, w, true, M, ktiles, kTileK4) <= 65536; };
  int cfg = p.cfg, splits = p.splits;
  const int64_t spc = ((int64_t)nstrips + cu - 1) / cu;  // strips per CU, rounded up
  auto groups = [&](int ns) { return (nstrips + ns - 1) / ns; };
  // M 8..16 on >= 2048 strips: four strips per 8-wave workgroup unless three
  // or seven keep the rounds of `cu` workgroups more than 5% fuller; -1
  // (the rules below) where none fills them to 85%.
  int many_strips_cfg = -1;
  if (M >= 8 && M <= 16 && strips_ge(2048)) {
    auto fill = [&](int ns) {
      const int g = groups(ns);
      return (double)g / (double)(((g + cu - 1) / cu) * cu);
    };
    int c = kG1x4W8U2;
    double best = fill(4) * 1.05;
    if (fill(3) > best) { c = kG1x3W8U2; best = fill(3); }
    if (fill(7) > best) c = kG1x7W8U1;
    if (std::max(fill(4), std::max(fill(3), fill(7))) >= 0.85) many_strips_cfg = c;
  }
  if (M >= 17 && M <= 32 && !strips_ge(1024)) {
    // (two m-tiles per wavefront)
    if (strips_ge(640)) {
      cfg = kG2x4W4U2;
      splits = 1;
    } else if (strips_ge(257)) {
      cfg = ktiles >= 128 ? kG2x4W4U2 : kG2x2W8U1;
      splits = ktiles >= 128 ? 4 : 1;
    } else if (strips_ge(129) && ktiles >= 128) {
      cfg = kG2x4W4U2;
      splits = 4;
    } else if (strips_ge(65)) {
      cfg = ktiles < 24 ? kG2x1W8U4 : kG2x2W8U1;
      splits = ktiles < 24 ? 1 : strips_ge(129) ? 2 : 4;
    } else {
      cfg = kG2x1W8U4;
      splits = M <= 24 && ktiles < 24 ? 1 : 4;
    }
  } else if (M >= 33 && M <= 64) {
    // (four m-tiles per wavefront)
    if (strips_ge(512)) {
      cfg = ktiles <= 8 ? kG4x2W8U1 : kG4x2W4U1;
      splits = !strips_ge(768) && ktiles >= 32 ? 2 : 1;
    } else if (strips_ge(257)) {
      cfg = ktiles >= 128 ? kG4x2W4U1 : kG4x2W8U1;
      splits = ktiles >= 128 ? 4 : 1;
    } else {
      cfg = kG4x2W8U1;
      splits = !strips_ge(129) ? 4 : ktiles <= 8 ? 1 : 2;
    }
  } else if (M <= 4 && strips_ge(1024) &&
             (ktiles >= 24 ? (M >= 2 || ktiles < 40) : (M >= 3 && ktiles >= 16))) {
    cfg = kG1x2W8U2;
    splits = 1;
  } else if (M <= 4 && ktiles >= 128 && strips_ge(257) && !strips_ge(512)) {
    // x in LDS split 2- or 4-way at M <= 2, two strips split 4-way at M 3..4
    cfg = M <= 2 ? kG1x1W8U4XL : kG1x2W8U2;
    splits = M <= 2 && ktiles < 192 ? 2 : 4;
    if (cfg == kG1x1W8U4XL &&
        gemv_lds_bytes(1, 1, 8, true, M, (int)ceil_div(ktiles, splits), kTileK4) > 65536)
      cfg = kG1x2W8U2;
  } else if (M >= 3 && M <= 4 && ktiles >= 64 && !strips_ge(129)) {
    cfg = kG1x2W8U2;
    splits = 4;
  } else if (M >= 2 && M <= 4 && ktiles >= 128 && !strips_ge(257)) {
    cfg = kG1x2W8U2;
    splits = std::max(1, std::min(8, (cu + groups(2) / 2) / groups(2)));
  } else if (!grouped && M <= 2 && !strips_ge(257) && ktiles >= 64 && ktiles < 128 && fits_xl(8)) {
    cfg = kG1x1W8U4XL;
  } else if (many_strips_cfg >= 0) {
    cfg = many_strips_cfg;
    splits = 1;
  } else if (M >= 8 && M <= 16 && (ktiles >= 64 || (M >= 12 && ktiles >= 48)) && !strips_ge(129)) {
    cfg = kG1x2W8U2;
    splits = 4;
  } else if (M >= 12 && M <= 16 && ktiles >= 64 && strips_ge(129) && !strips_ge(257)) {
    cfg = kG1x4W8U2;
    splits = 4;
  } else if (M >= 8 && M <= 16 && ktiles >= 128 && strips_ge(257) && !strips_ge(512)) {
    cfg = M <= 8 ? kG1x3W8U2 : kG1x6W8U1;
    splits = M <= 8 ? 2 : 4;
  } else if (M >= 9 && M <= 16 && !strips_ge(65) && ktiles < 32) {
    cfg = kG1x1W16U2;
    splits = 1;
  } else if (M >= 5 && M <= 16 && p.splits == 1 && strips_ge(513) &&
             (spc == 3 || spc == 6 || spc == 7 || (spc == 5 && M >= 8))) {
    cfg = spc == 3 ? kG1x3W8U2 : spc == 7 ? kG1x7W8U1 : M >= 12 ? kG1x6W8U1 : kG1x3W8U2;
  } else if (M <= 4 && p.splits == 1 && !strips_ge(257) && ktiles < 128) {
    // Below 64 tiles the x copy (at most 4 rows of 63 * 256 bytes) fits.
    if (ktiles <= 8) {
      cfg = grouped ? kG1x1W16U2 : kG1x1W4U4;
    } else if (ktiles <= 16) {
      cfg = !grouped && M == 1 ? kG1x1W8U4XL : kG1x1W16U2;
    } else if (ktiles < 64) {
      if (!grouped) cfg = kG1x1W8U4XL;
      else cfg = M == 1 || (M == 2 && ktiles >= 40) ? kG1x1W16U4XL : kG1x1W16U2;
    } else if (M <= 3) {
      cfg = fits_xl(16) ? kG1x1W16U4XL : kG1x1W16U2;
    }
  } else if (M <= 4 && p.splits == 1 && strips_ge(257) && !strips_ge(640) && ktiles >= 64) {
    cfg = (M == 1 || (M == 2 && !grouped)) && fits_xl(8) ? kG1x1W8U4XL : kG1x2W16U2;
  } else if (M >= 3 && M <= 4 && cfg == kG1x2W8U2 && fits_xl(8)) {
    cfg = kG1x1W8U4XL;
  } else if (M >= 8 && M <= 16 && strips_ge(1536)) {
    cfg = kG1x4W4U2;
  } else if (M >= 5 && M <= 16 && cfg == kG1x2W16U2 && p.splits == 1 &&
             (ktiles >= 128 || (M >= 8 && ktiles >= 64))) {
    // (257..511 strips)
    if (ktiles >= 128) {
      cfg = kG1x4W8U2;
      splits = 2;
    } else {
      cfg = kG1x2W8U2;
    }
  } else if (M >= 5 && M <= 16 && cfg == kG1x1W16U2 && ktiles >= 64 &&
             (int64_t)nstrips * 256 <= 511LL * cu) {
    cfg = kG1x2W8U2;
    splits = 2;
  } else if (M >= 5 && M <= 8 && cfg == kG1x2W16U2 && p.splits > 1 && !strips_ge(65)) {
    cfg = kG1x1W16U2;
    splits = 1;
  }
  if (cfg == p.cfg && splits == p.splits) return p;
  GemvPlan q;
  q.cfg = cfg;
  q.mt = kGemvCfgs[cfg].mt;
  q.ns = kGemvCfgs[cfg].ns;
  q.groups = 0;
  for (int i = 0; i < nproj; ++i) q.groups += (int)ceil_div(ceil_div(Ns[i], 16), q.ns);
  if (q.groups > kMaxGroupsSplit) splits = 1;
  if (splits > ktiles) splits = ktiles;
  q.kb_per_split = (int)ceil_div(ktiles, splits);
  q.splits = (int)ceil_div(ktiles, q.kb_per_split);
  return q;
}


// Int8 rules at M <= 16 measured over the decode projections of the
// reference's model families -- Qwen3 0.6B / 1.7B / 4B / 8B / 14B / 32B and
// Qwen3-VL-32B, Qwen2.5-VL 3B / 7B, the Pi0.5 Gemma decoder (2048 wide, MLP
// 16384) and action expert (1024 wide, MLP 4096), each projection alone and
// q/k/v and gate/up fused, at M 1..16 -- against every configuration and K
// split (MI355X, graph-timed, 600 MB of rotated weights, three interleaved
// rounds).  Sets cfg / splits and returns true where they replace the
// general rules below; returns false elsewhere.
//   * M <= 4 on 257..639 strips from K 1088: two strips per 8-wave
//     workgroup, no K split (Qwen3-14B q 5120 x 5120 at M 1 / 2: 7.0 against
//     7.7 / 7.9 us with x in LDS; Qwen3-14B down 5120 x 17408: 17.5 against
//     19.6 us with an 8-way split; Qwen3-4B q/k/v 6144 x 2560: 5.25 against
//     5.53 us with 16 wavefronts), except at M <= 2 for K 8192..16383, where
//     x in LDS and two strips tie to within the spread between boxes
//     (Qwen3-VL-32B o 5120 x 8192: -2.6..+4.5%);
//   * M <= 4 below 257 strips from K 1088: x staged in LDS at M 1 and 2, at
//     M 3 below 256 strips and at M 4 up to 128, with a 2-way K split where
//     only that fits (Qwen3-0.6B down 1024 x 3072 at M 2: 3.68 against 4.32
//     us; Qwen2.5-VL-7B down 3584 x 18944 at M 1: 12.9 against 16.7 us;
//     Qwen2.5-VL-3B down 2048 x 11008 at M 3: 8.2 against 9.6 us); else 16
//     wavefronts, or from K 16384 two strips per workgroup split to about
//     one workgroup per CU (Qwen3-8B down at M 4: 10.7 against 11.1 us with
//     8 wavefronts; Qwen2.5-VL-7B down at M 2..4: 14.3..14.6 against
//     17.0..17.7 us);
//   * M 5..16 on >= 2048 strips: from M 9 and K 3072 five strips per
//     8-wave workgroup (Qwen3-14B gate/up 34816 x 5120 at M 16: 31.9
//     against 37.7 us with four strips per 4-wave workgroup; Qwen2.5-VL-7B
//     gate/up 37888 x 3584: 23.5 against 27.4 us; Qwen3-14B lm_head 151936
//     x 5120 ties; at K 2048, Pi0.5 gate/up 32768 x 2048, four per 4-wave
//     workgroup stay 7% faster), and at M 5..8 from K 1088 three or five strips,
//     whichever keeps the rounds of 256 workgroups fuller (Qwen2.5-VL-7B
//     gate/up at M 8: five, 22.6 against 26.7 us with three; the Qwen3-14B
//     lm_head stays at three, 116.7 us at M 8);
//   * M 5..16 from K 16384: five strips per workgroup and a 4-way K split on
//     257..511 strips (Qwen3-14B down at M 16: 19.6 against 25.1 us with two
//     strips and 8 splits), four strips on 129..256 (Qwen2.5-VL-7B down at
//     M 16: 16.6 against 21.5 us), two on fewer;
//   * M 5..16, K 8192..16383, up to 128 strips: two strips, 4-way K split
//     (Qwen2.5-VL-3B down at M 16: 10.2 against 11.3 us with four strips),
//     one strip per 8-wave workgroup split 2-way up to M 6 (M 8 below
//     K 10240); on 257..511 strips from M 8 three strips split 2-way, or
//     five split 4-way from K 10240 and M 12 where that fits one round of
//     workgroups (from M 12 also at K 8192);
//   * M 13..16 on 65..128 strips at K 5120..8191: two strips per 16-wave
//     workgroup split 4-way;
//     on 129..256 strips at M 5..6: one strip per 16-wave workgroup, no
//     split (Qwen3-8B down at M 5: 10.8 against 11.7 us with two strips and
//     two splits), and from M 8 three strips split 4-way where 4 x the
//     workgroups of three strips fit one round of 256;
//   * M 5..16 on <= 64 strips: one strip per 16-wave workgroup and no K
//     split, or at M >= 8 from K 5120 one per 8-wave workgroup and a 4-way
//     split (Pi0.5 expert o 1024 x 2048 at M 8: 3.8 against 5.9 us with
//     two strips and four splits; Qwen3-14B k 1024 x 5120 at M 16: 6.6
//     against 7.2 us).
static bool plan_int8_rules(int M, int nstrips, int kblocks, int cu, int* cfg, int* splits) {
  auto strips_ge = [&](int n256) { return (int64_t)nstrips * 256 >= (int64_t)n256 * cu; };
  auto groups = [&](int ns) { return (nstrips + ns - 1) / ns; };
  *splits = 1;
  if (M > 16 || (M <= 4 && kblocks <= 16)) return false;
  if (M <= 4) {
    if (strips_ge(640) || (strips_ge(512) && kblocks >= 256)) return false;
    if (strips_ge(257)) {
      if (M <= 2 && kblocks >= 128 && kblocks < 256) return false;
      *cfg = kG1x2W8U2;
      return true;
    }
    // (M 1, K 4096..5119, <= 64 strips: sixteen wavefronts of one stage
    // each stay 2% faster, Qwen3-8B k 1024 x 4096)
    if (M == 1 && kblocks >= 64 && kblocks < 80 && !strips_ge(65)) return false;
    const bool few = !strips_ge(129);
    const bool xl_rows = M <= 2 || (M == 3 && !strips_ge(256)) || (M == 4 && few);
    if (xl_rows && lds_fits(kG1x1W8U4XL, M, kblocks)) {
      *cfg = kG1x1W8U4XL;
    } else if (xl_rows && few && lds_fits(kG1x1W8U4XL, M, (kblocks + 1) / 2)) {
      *cfg = kG1x1W8U4XL;
      *splits = 2;
    } else if (kblocks >= 256) {
      *cfg = kG1x2W8U2;
      *splits = std::max(1, std::min(8, (cu + groups(2) / 2) / groups(2)));
    } else {
      *cfg = kG1x1W16U2;
    }
    return true;
  }
  if (strips_ge(2048)) {
    if (kblocks <= 16) return false;
    if (M >= 9) {
      if (kblocks < 48) return false;
      *cfg = kG1x5W8U1;
    } else {
      // Busy share of the rounds of `cu` workgroups the launch needs.
      auto fill = [&](int ns) {
        const int g = groups(ns);
        return (double)g / (double)(((g + cu - 1) / cu) * cu);
      };
      *cfg = fill(5) > fill(3) ? kG1x5W8U1 : kG1x3W8U2;
    }
    return true;
  }
  if (strips_ge(512)) return false;
  if (kblocks >= 256) {
    *cfg = strips_ge(257) ? kG1x5W8U1 : strips_ge(129) ? kG1x4W8U2 : kG1x2W8U2;
    *splits = 4;
    return true;
  }
  if (strips_ge(257)) {
    // K 8192..16383 from M 8: three strips split 2-way, or from K 10240 and
    // M 12 five strips split 4-way (Qwen3-VL-32B o 5120 x 8192 at M 16: 12.5
    // against 13.3 us; 5120 x 10240 at M 16: 14.3 against 16.6 us)
    if (kblocks >= 128 && M >= 8 && (kblocks >= 160 || M >= 12)) {
      const bool five = kblocks >= 160 && M >= 12 && (int64_t)groups(5) * 4 <= cu;
      *cfg = five ? kG1x5W8U1 : kG1x3W8U2;
      *splits = five ? 4 : 2;
      return true;
    }
    return false;
  }
  if (kblocks >= 128) {
    if (!strips_ge(129)) {
      // (up to M 6, and M 8 below K 10240, one strip per 8-wave workgroup
      // split 2-way: 2048 x 8192 at M 8 7.7 against 8.6 us)
      const bool one = M <= 6 || (M <= 8 && kblocks < 160);
      *cfg = one ? kG1x1W8U4 : kG1x2W8U2;
      *splits = one ? 2 : 4;
      return true;
    }
    if (M <= 6) {
      *cfg = kG1x1W16U2;
      return true;
    }
    if (M >= 8 && (int64_t)groups(3) * 4 <= cu) {
      // three strips split 4-way where that stays within one round
      // (Qwen3-4B down 2560 x 9728 at M 8 / 16: 9.4 / 10.8 against 10.1 /
      // 11.6 us with two strips split 2-way)
      *cfg = kG1x3W8U2;
      *splits = 4;
      return true;
    }
    return false;
  }
  if (M >= 13 && kblocks >= 80 && strips_ge(65) && !strips_ge(129)) {
    // two strips per 16-wave workgroup split 4-way (Qwen3-1.7B down 2048 x
    // 6144 at M 16: 8.3 against 8.8 us)
    *cfg = kG1x2W16U2;
    *splits = 4;
    return true;
  }
  if (!strips_ge(65)) {
    const bool split = M >= 8 && kblocks >= 80;
    *cfg = split ? kG1x1W8U4 : kG1x1W16U2;
    *splits = split ? 4 : 1;
    return true;
  }
  return false;
}

// Kernel choice per shape: the analogue of the reference's W8A16 tile
// tables (src/ops/rpu_linear_tiling.h:69-127, selectors :544-595), but as
// rules over (M, strips of 16 channels, 64-wide K blocks), tuned on MI355X:
//   * M <= 4: the activation fragment is nearly free, so one strip per
//     workgroup and as many wavefronts as keep ~16 per CU busy;
//   * M 5..16: the fragment costs twice the weight bytes per tile, so four
//     strips share it when there are enough strips to fill the chip;
//   * M 17..64: two / four 16-row m-tiles per wavefront;
//   * K splits only where the strips alone cannot fill 256 CUs.
// int8_rules: the rules measured on int8 launches alone -- at M 5..16 the
// ones that give a workgroup three to seven strips (kG1x3W8U2 .. kG1x7W8U1,
// sized to about one or two workgroups per CU), eight wavefronts on 257..511
// strips at long K and the 2-way K split at K >= 8192, and the 16-wavefront
// rule at M 17..32 (kG2x2W16U1); the int4 planner starts from the rules
// without them.
GemvPlan plan_gemv_rules(int M, const int* Ns, int nproj, int K, const DeviceInfo& dev,
                         bool int8_rules) {
  // Rules see the launch's strips of all projections together.
  int nstrips = 0;
  for (int i = 0; i < nproj; ++i) nstrips += (int)ceil_div(Ns[i], 16);
  const int kblocks = (int)ceil_div(K, 64);
  // Thresholds are in strips for a 256-CU part; scale for smaller parts.
  const int cu = dev.cus > 0 ? dev.cus : 256;
  auto strips_ge = [&](int n256) { return (int64_t)nstrips * 256 >= (int64_t)n256 * cu; };
  int cfg, splits = 1;
  if (int8_rules && plan_int8_rules(M, nstrips, kblocks, cu, &cfg, &splits)) {
    // (measured int8 rules above)
  } else if (M <= 16 && !strips_ge(640) && kblocks >= 256) {
    // Very long K (>= 16384) on few strips (Qwen3-VL-32B down_proj): two
    // strips per 8-wavefront workgroup and an 8-way K split.
    cfg = kG1x2W8U2;
    splits = 8;
  } else if (M <= 4 && strips_ge(257) && !strips_ge(640) && kblocks >= 80) {
    // Long K (>= 5120) on 257..639 strips (Qwen3-VL-32B q_proj, o_proj):
    // x in LDS at M <= 2, two strips per workgroup at M 3..4.
    cfg = (M <= 2 && lds_fits(kG1x1W8U4XL, M, kblocks)) ? kG1x1W8U4XL : kG1x2W8U2;
  } else if (M <= 4) {
    // x staged in LDS (one DMA copy per workgroup instead of every
    // wavefront re-reading the same L2 lines) pays off at M <= 2.
    if (strips_ge(640)) {
      // Many strips: two strips per workgroup share the x fragment at M 3..4.
      cfg = M >= 3 ? kG1x2W8U2 : kG1x1W8U4XL;
      if (!lds_fits(cfg, M, kblocks)) cfg = kG1x1W4U4;
    } else if (strips_ge(257)) {
      cfg = kG1x2W16U2;
    } else if (kblocks >= 128 || (M == 1 && kblocks >= 80)) {
      // (at M = 1 from K = 5120: ten tiles per wavefront instead of five,
      // Qwen3-VL-32B k/v 1024 x 5120 4.84 instead of 5.15 us).  x is staged
      // in LDS at M = 1.
      cfg = (M == 1 && lds_fits(kG1x1W8U4XL, M, kblocks)) ? kG1x1W8U4XL : kG1x1W8U4;
    } else if (kblocks <= 16) {
      // K <= 1024: four wavefronts of four tiles, one pipeline stage each,
      // and a 4-way cross-wavefront sum instead of 16 (Qwen3-0.6B q/k/v
      // 3072 x 1024 at M 1 / 4: 3.12 / 3.24 us instead of 3.61 / 3.77 us).
      cfg = kG1x1W4U4;
    } else {
      // (short K: one tile per wavefront does not amortize the staging wait)
      cfg = (M == 1 && kblocks >= 48 && lds_fits(kG1x1W16U4XL, M, kblocks)) ? kG1x1W16U4XL
                                                                             : kG1x1W16U2;
    }
  } else if (M <= 16) {
    // Strips per CU, rounded up (one-round rules below).
    const int64_t spc = ((int64_t)nstrips + cu - 1) / cu;
    if (strips_ge(2048)) {
      // M 5..8 (rows 8..15 of the activation fragment repeat row M-1, so
      // it costs less): three strips per workgroup (32768 x 4096: 23.3
      // instead of 25.1 us); int8 from K 1088 in plan_int8_rules.
      cfg = (int8_rules && M <= 8) ? kG1x3W8U2 : kG1x4W4U2;
    } else if (int8_rules && strips_ge(1025) && spc <= 7) {
      // 5..7 strips per CU: that many strips per 8-wave workgroup, one
      // workgroup per CU, so each activation fragment serves 5..7 weight
      // tiles; at 6 per CU three strips, two workgroups per CU (MI355X, four
      // rotated weight copies: Qwen3-8B fused gate/up 24576 x 4096 at M 16:
      // 18.8 instead of 21.6 us, at M 5..12 17.7..18.0 instead of 18.9..20.6
      // us; 20480 x 4096 at M 16: 16.1 instead of 20.2 us; 28672 x 4096:
      // 21.7 instead of 25.9 us).  Since each wavefront waits only for its
      // own stage (the one-m-tile pipeline), three strips also beat six at
      // M 13..16: 24576 x 4096 at M 16 18.1 against 18.6 us (graph-timed,
      // 600 MB of rotated weights, three interleaved rounds).
      cfg = spc == 5 ? kG1x5W8U1 : spc == 7 ? kG1x7W8U1 : kG1x3W8U2;
    } else if (strips_ge(1024)) {
      cfg = kG1x2W8U2;
    } else if (int8_rules && strips_ge(513) && spc == 3) {
      // 3 strips per CU: three strips per 8-wave workgroup, one workgroup
      // per CU (12288 x 4096 at M 5 / 8 / 16: 10.4 / 10.9 / 11.2 instead of
      // 12.6 / 12.8 / 13.1 us with four strips per workgroup).
      cfg = kG1x3W8U2;
    } else if (strips_ge(640)) {
      cfg = kG1x4W8U2;
    } else if (strips_ge(512)) {
      cfg = kG1x2W8U2;  // 512 strips: four per workgroup leaves half the CUs idle
    } else if (strips_ge(257)) {
      // From K 5120 eight wavefronts of twice the tiles each stream longer
      // than sixteen (5120 x 5120 at M 5 / 8 / 12 / 16: 7.4 / 8.1 / 9.0 /
      // 10.0 against 8.0 / 8.7 / 9.8 / 10.8 us; at K 4096 the two tie).
      cfg = (int8_rules && kblocks >= 80) ? kG1x2W8U2 : kG1x2W16U2;
    } else if (kblocks >= 128) {
      if (int8_rules && strips_ge(129)) {
        // 129..256 strips: two strips per workgroup and a 2-way K split
        // (Qwen3-8B down 4096 x 12288 at M 8 / 12 / 16: 11.4 / 12.1 / 13.0
        // against 12.2 / 12.9 / 13.1 us with four strips and four splits).
        cfg = kG1x2W8U2;
        splits = 2;
      } else {
        cfg = kG1x4W8U2;
        splits = 4;
      }
    } else if (!strips_ge(65)) {
      cfg = kG1x2W16U2;
      splits = 4;
    } else {
      cfg = kG1x1W16U2;
    }
  } else if (M <= 32) {
    // int8 below 640 strips, measured over the projections of the model
    // families that stay on the GEMV at M 17..32 (graph-timed, 600 MB of
    // rotated weights): from K 8192 on <= 256 strips, two strips per
    // 16-wavefront workgroup split 4-way (<= 128 strips) or 2-way
    // (Qwen2.5-VL-3B down 2048 x 11008 at M 24: 10.7 against 16.7 us;
    // Qwen3-4B down 2560 x 9728: 13.7 against 15.9 us); at K 3072..8191 on
    // 129..256 strips the same 2-way (Qwen3-8B o at M 24: 8.7 against
    // 9.7 us); below K 3072 one strip per 8-wavefront workgroup of four
    // tiles a stage on 65..256 strips (Pi0.5 Gemma 2B q/k/v 2560 x 2048 at
    // M 24: 5.8 against 6.4 us), two strips per 16-wavefront workgroup on
    // 257..639 (Qwen3-0.6B gate/up 6144 x 1024: 4.8 against 5.0 us), and no
    // K split on <= 64 strips up to M 24 and K 2048 (Qwen3-0.6B o 1024 x
    // 2048: 5.7 against 6.1 us).
    const bool k_short = kblocks < 48;
    if (strips_ge(1024)) {
      cfg = kG2x4W4U2;
    } else if (int8_rules && kblocks >= 128 && !strips_ge(257)) {
      cfg = kG2x2W16U1;
      splits = strips_ge(129) ? 2 : 4;
    } else if (kblocks >= 128) {
      cfg = kG2x4W4U2;
      splits = 4;
    } else if (int8_rules && strips_ge(129) && !strips_ge(257) && !k_short) {
      cfg = kG2x2W16U1;
      splits = 2;
    } else if (int8_rules && strips_ge(65) && !strips_ge(257) && k_short) {
      cfg = kG2x1W8U4;
    } else if (int8_rules && strips_ge(257) && !strips_ge(640) && k_short) {
      cfg = kG2x2W16U1;
    } else if (int8_rules && !strips_ge(65) && kblocks <= 32 && M <= 24) {
      cfg = kG2x1W8U4;
    } else if (int8_rules && !strips_ge(129) && kblocks >= 64) {
      // <= 128 strips, K 4096..8191 (int8): two strips per 16-wavefront
      // workgroup and a 4-way K split (MI355X, 600 MB of rotated weights:
      // Qwen3-8B k and v together, 2048 x 4096, at M 24 / 32 7.6 / 8.0
      // instead of 9.7 / 11.1 us; k alone, 1024 x 4096, 6.9 / 7.4 instead
      // of 7.7 / 8.3 us; 1024 x 5120 -4%).
      cfg = kG2x2W16U1;
      splits = 4;
    } else if (!strips_ge(65)) {
      cfg = kG2x1W8U4;
      splits = 4;
    } else {
      cfg = kG2x2W8U1;
    }
  } else {
    if (strips_ge(512)) {
      cfg = kG4x2W4U1;
    } else {
      cfg = kG4x2W8U1;
      splits = 2;
    }
  }
  GemvPlan p;
  p.cfg = cfg;
  p.mt = kGemvCfgs[cfg].mt;
  p.ns = kGemvCfgs[cfg].ns;
  p.groups = 0;
  for (int i = 0; i < nproj; ++i) p.groups += (int)ceil_div(ceil_div(Ns[i], 16), p.ns);
  if (p.groups > kMaxGroupsSplit) splits = 1;  // counter region holds kMaxGroupsSplit counters
  if (splits > kblocks) splits = kblocks;
  p.kb_per_split = (int)ceil_div(kblocks, splits);
  p.splits = (int)ceil_div(kblocks, p.kb_per_split);  // drop empty splits
  return p;
}

GemvPlan plan_gemv(int M, const int* Ns, int nproj, int K, const DeviceInfo& dev) {
  return plan_gemv_rules(M, Ns, nproj, K, dev, true);
}

}  // namespace rf
