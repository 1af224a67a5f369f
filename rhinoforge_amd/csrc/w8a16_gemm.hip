// Prefill GEMM for W8A16 (gfx950): LDS-staged INT8 weight tiles dequantized
// into fp16 MFMA operands, fp32 accumulation.
//
// Workgroup tile BM x BN, WAVES_M x WAVES_N wavefronts, each owning a
// (BM/WAVES_M) x (BN/WAVES_N) block of 16x16 v_mfma_f32_16x16x32_f16
// accumulators.
//   * operands move global -> LDS with global_load_lds_dwordx4 (no VGPR
//     staging) into a ring of STAGES 64-wide K blocks, so up to STAGES-1 K
//     blocks are in flight while one is multiplied;
//   * A (activations, fp16) rows are 128 bytes per K block, chunk-swizzled
//     (a_swizzle) so fragment reads are free of LDS bank conflicts;
//   * B (weights) stays INT8 in LDS (half the LDS bytes and half the
//     global->LDS traffic of an fp16 tile): TILE16X64 tiles are copied
//     verbatim and each lane's 16 bytes are exactly its two MFMA B operands,
//     dequantized in registers right before the MFMAs (exact, v_perm +
//     v_pk_add);
//   * in a 1 x N wavefront grid no two wavefronts read the same B strip, so
//     the 128x256 and 128x128 (3 per CU) tiles skip LDS for B: each wavefront
//     loads its strips one K block ahead straight into VGPRs (BR), which
//     halves the LDS writes of a 128x256 tile and cuts its LDS reads by 20%;
//   * tiles are ordered so that the workgroups one XCD runs at the same time
//     (the hardware deals workgroup ids round-robin over the 8 XCDs) cover a
//     compact block of output tiles and share A and B rows in their L2;
//   * one launch can cover up to RF_W8A16_MAX_PROJ weight matrices that
//     share the activation (q/k/v, gate/up): their tile columns are laid
//     side by side and each workgroup resolves its matrix from its column;
//   * when the output has fewer tiles than the chip has workgroup slots, K
//     is split across workgroups: each split writes its fp32 partial tile to
//     the workspace and the last split to arrive sums all partials in split
//     order (deterministic) before the epilogue;
//   * the per-channel scale and bias are applied in the fp32 epilogue.
#include <type_traits>

#include "w8a16_common.h"
#include "w8a16_internal.h"

namespace rf {
namespace {

constexpr int kXcds = 8;
constexpr int kMaxProj = RF_W8A16_MAX_PROJ;
static_assert(kMaxProj == 4, "target_of selects among exactly four projections");

// One weight matrix of a launch; its tile columns are [tn0, next tn0).
struct GemmProj {
  const uint8_t* w;       // TILE16X64 packed
  const _Float16* scale;  // [N]
  const _Float16* bias;   // [N] or nullptr
  _Float16* y;
  int64_t ldy;
  int N;
  int nstrips;
  int tn0;
};

struct GemmKernelArgs {
  const _Float16* x;
  int64_t ldx;
  int M, K;
  int kblocks;
  int tiles_m, tiles_n;  // tiles_n summed over the projections
  int group_m;           // output-tile rows per scheduling group
  int nproj;
  GemmProj proj[kMaxProj];
  int splits;            // K splits (blockIdx.y); 1 = no workspace
  int kb_per_split;
  float* partial;        // [splits][tiles][BM*BN], fp32
  uint32_t* counters;    // [tiles], zero between calls
  int wtiles;            // 1 KB weight tiles per strip along K (64 positions int8, 128 int4)
  int gshift;            // group-wise int4: log2(group_size / 32)
};

// The weight matrix (and its tile column) behind global tile column tile_n.
struct TileTarget {
  const uint8_t* w;
  const _Float16* scale;
  const _Float16* bias;
  _Float16* y;
  int64_t ldy;
  int N;
  int nstrips;
  int tn;
};

__device__ __forceinline__ TileTarget target_of(const GemmKernelArgs& a, int tile_n) {
  int p = 0;
#pragma unroll
  for (int i = 1; i < kMaxProj; ++i) p = (i < a.nproj && tile_n >= a.proj[i].tn0) ? i : p;
  // Selects, not an indexed load: the argument block stays in SGPRs.
#define RF_PICK(f) (p == 0 ? a.proj[0].f : p == 1 ? a.proj[1].f : p == 2 ? a.proj[2].f : a.proj[3].f)
  TileTarget t;
  t.w = RF_PICK(w);
  t.scale = RF_PICK(scale);
  t.bias = RF_PICK(bias);
  t.y = RF_PICK(y);
  t.ldy = RF_PICK(ldy);
  t.N = RF_PICK(N);
  t.nstrips = RF_PICK(nstrips);
  t.tn = tile_n - RF_PICK(tn0);
#undef RF_PICK
  return t;
}

// Workgroup id -> (tile_m, tile_n).  Ids are first regrouped so that the
// ids one XCD receives (id % 8 == x) form one contiguous run of tile
// indices, then the run is walked in groups of `group_m` tile rows,
// column-major inside a group, so concurrently running workgroups share
// both A rows (same tile_m) and B strips (same tile_n).
__device__ __forceinline__ void tile_of(int bid, const GemmKernelArgs& a, int& tm, int& tn) {
  const int total = a.tiles_m * a.tiles_n;
  int t = bid;
  if (total % kXcds == 0) t = (bid % kXcds) * (total / kXcds) + bid / kXcds;
  const int per_group = a.group_m * a.tiles_n;
  const int g = t / per_group;
  const int first_m = g * a.group_m;
  const int gm = min(a.group_m, a.tiles_m - first_m);
  const int r = t - g * per_group;
  tm = first_m + r % gm;
  tn = r / gm;
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// dma16 (w8a16_common.h) with a wave-uniform SGPR base and a per-lane
// 32-bit byte offset (global_load_lds_dwordx4 voff, s[base]).
__device__ __forceinline__ void dma16s(uint32_t voff, const void* sbase, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Chunk swizzle of the LDS A tile: 16-byte chunk c of row r is stored in
// slot c ^ a_swizzle(r).  An MFMA A-fragment read has 16 lanes on rows
// r0..r0+15 (r0 % 16 == 0) at one chunk, and the next 16 lanes on the same
// rows at chunk ^ 2; with this swizzle the accesses of every 8-, 16- and
// 32-lane group cover distinct LDS banks (64 or 128 banks of 4 bytes).
__device__ __forceinline__ int a_swizzle(int r) { return (r & 7) ^ (((r >> 3) & 1) * 5); }

// Buffer resource over the split-K partials; accesses use sc1 (device-scope
// coherent: written through / re-fetched past the issuing XCD's L2, the
// same instructions as relaxed agent-scope atomic stores and loads).
// 0x00020000: raw 32-bit data format word of CDNA buffer descriptors.
constexpr int kCoherent = 16;  // cache-policy bit sc1
__device__ __forceinline__ __amdgpu_buffer_rsrc_t partial_rsrc(float* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, (short)0, (int)bytes, 0x00020000);
}

// fp32 epilogue: y = acc * scale[n] + bias[n].  Lane l holds
// D[4*(l/16) + r][l%16] of each 16x16 tile; a full tile stores without
// per-element checks.
template <int TM, int TN, bool SC = true>
__device__ __forceinline__ void store_tile(const TileTarget& t, const floatx4 (&acc)[TM][TN],
                                           int m0w, int n0w, int lane, int M, bool full) {
  const int nl = n0w + (lane & 15);
  const int ml = m0w + 4 * (lane >> 4);
  _Float16* yl = t.y + (int64_t)ml * t.ldy + nl;
  float sc[TN], bi[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = nl + j * 16;
    sc[j] = n < t.N ? (SC ? (float)t.scale[n] : 1.f) : 0.f;
    bi[j] = (t.bias && n < t.N) ? (float)t.bias[n] : 0.f;
  }
  if (full) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        _Float16* yr = yl + (int64_t)(i * 16 + r) * t.ldy;
#pragma unroll
        for (int j = 0; j < TN; ++j) yr[j * 16] = (_Float16)__builtin_fmaf(acc[i][j][r], sc[j], bi[j]);
      }
  } else {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (ml + i * 16 + r >= M) continue;
        _Float16* yr = yl + (int64_t)(i * 16 + r) * t.ldy;
#pragma unroll
        for (int j = 0; j < TN; ++j)
          if (nl + j * 16 < t.N) yr[j * 16] = (_Float16)__builtin_fmaf(acc[i][j][r], sc[j], bi[j]);
      }
  }
}

// ---------------------------------------------------------------------------
// Main kernel.  Each DMA is global_load_lds_dwordx4 voff, s[base]: the
// per-lane byte offset from the tile's first row / strip is fixed for the
// whole K loop, and one scalar add per K block moves the bases, so the loop
// issues no vector address math.  OCC workgroups per CU are requested from
// the register allocator.  Offsets are 32-bit: the host checks that
// BM*ldx*2 + 2K and the strip span of BN/16 strips fit (v3_offsets_fit).
//
// LDS A rows are unpadded (128 B) and chunk-swizzled: slot p of row r holds
// global chunk p ^ a_swizzle(r).  Rows past M and strips past N load clamped
// (valid) addresses; their results are never stored.  Columns past K (the
// last K block when K % 64 != 0) are zeroed in LDS after their load lands.
// ---------------------------------------------------------------------------
//
// WF (WeightFormat) int4: a 1 KB TILE16X128_I4 tile covers two K blocks; the
// half for K block kb (lanes 32*(kb%2) .. +31 of the tile, 512 contiguous
// bytes) is copied per strip, and lane (g = l/16, c = l%16) reads the eight
// bytes holding positions 16g .. 16g+15 of the block for channel c: bytes
// 8*(g%2) .. +7 of half-tile lane c + 16*(g/2), i.e. the two MFMA operands
// of the int8 path (so the A operand path is shared unchanged).  Group-wise
// int4 also copies the block's scale rows ([K/gs][N], BN columns; one row,
// or two for gs = 32) into LDS, by wavefront 0, and scales at dequantization.
//
// IL (int8 only): both K steps' A fragments of a block are read up front, the
// second step's reads are interleaved one per MFMA with the first step's
// MFMAs (sched_group_barrier), and the wavefront runs its MFMA section at
// raised issue priority (s_setprio 1).  Same arithmetic in the same order;
// chosen where two wavefronts per SIMD are resident (see plan_gemm).
//
// KG: K groups per workgroup (1 or 2).  With two, the workgroup runs two
// WAVES_M x WAVES_N grids of wavefronts; group g multiplies K blocks g,
// g + 2, ... of the split (each stage holds one block per group), so a
// launch of one tile per CU still keeps two wavefronts on every SIMD, each
// with the instruction mix of the one-group tile.  At the end group 1 hands
// its accumulators to group 0 through LDS, which adds them (fixed order).
template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int OCC, int WF = kWfInt8,
          bool IL = false, bool BR = false, int KG = 1>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64 * KG) __attribute__((amdgpu_waves_per_eu(OCC * WAVES_M * WAVES_N * KG / 4, 8)))
void w8a16_gemm_v3_kernel(GemmKernelArgs a) {
  constexpr int NT = WAVES_M * WAVES_N * 64;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int A_BYTES = BM * 128;
  constexpr int B_TILES = BN / 16;
  constexpr int B_STRIP = WF ? kTileBytes / 2 : kTileBytes;  // per strip and K block
  constexpr int B_BYTES = B_TILES * B_STRIP;
  constexpr bool GS = WF == kWfInt4Grp;
  constexpr int S_BYTES = GS ? 1024 : 0;  // one wavefront DMA of scale rows
  static_assert(!GS || 2 * BN * 2 <= S_BYTES, "two scale rows of BN fp16 fit one DMA");
  // BR: each wavefront loads its own B strips straight into registers (in a
  // 1 x N grid no two wavefronts share a strip, so staging B in LDS only adds
  // a DMA write and a read per byte); LDS then holds A (and scales) only.
  constexpr int S_OFF = A_BYTES + (BR ? 0 : B_BYTES);
  constexpr int SUB = S_OFF + S_BYTES;  // one K block's LDS
  constexpr int STAGE = KG * SUB;       // one block per K group
  static_assert(KG == 1 || (KG == 2 && !IL && WF == kWfInt8),
                "two K groups: int8, plain schedule");
  constexpr int A_LOADS = A_BYTES / (NT * 16);
  constexpr int B_LOADS = BR ? 0 : B_BYTES / (NT * 16);
  constexpr int LOADS = A_LOADS + B_LOADS;
  static_assert(A_LOADS >= 1 && (BR || B_LOADS >= 1) && A_LOADS * NT * 16 == A_BYTES &&
                    (BR || B_LOADS * NT * 16 == B_BYTES),
                "tile does not split into whole 1 KB wavefront loads");
  static_assert(STAGES >= 2 && STAGES <= 4, "2..4 stages");
  static_assert(!BR || (STAGES == 2 && WAVES_M == 1 && !IL), "register B: 2 stages, 1 x N grid");

  // Two K groups: group 1's accumulators are handed to group 0 through LDS
  // at the end, which for the 128x256 register-B tile needs more than the
  // stages hold.
  constexpr int HANDOFF = KG == 2 ? WAVES_M * WAVES_N * TM * TN * 64 * 16 : 0;
  constexpr int SMEM_BYTES = STAGES * STAGE > HANDOFF ? STAGES * STAGE : HANDOFF;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave: index within the wavefront's K group (kg_u, wave-uniform).
  constexpr int NW = WAVES_M * WAVES_N;
  const int wave = KG == 1 ? (tid >> 6) : (tid >> 6) % NW;
  const int kg_u = KG == 1 ? 0 : __builtin_amdgcn_readfirstlane((tid >> 6) / NW);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int tile = blockIdx.x;
  const int split = blockIdx.y;
  int tile_m, tile_n;
  tile_of(tile, a, tile_m, tile_n);
  const TileTarget tt = target_of(a, tile_n);
  const int m0 = tile_m * BM;
  const int strip0 = tt.tn * B_TILES;
  const int kb0 = split * a.kb_per_split;
  const int nk = min(a.kblocks - kb0, a.kb_per_split);  // K blocks of this split (>= 1)

  // Wave-uniform bases and per-lane 32-bit offsets.
  const uint8_t* abase = reinterpret_cast<const uint8_t*>(a.x + (int64_t)m0 * a.ldx);
  const uint8_t* bbase = tt.w + (int64_t)strip0 * a.wtiles * kTileBytes;
  uint32_t aoff[A_LOADS], arow_off[A_LOADS];
  int acol[A_LOADS];
#pragma unroll
  for (int i = 0; i < A_LOADS; ++i) {
    const int p = (wave * A_LOADS + i) * 64 + lane;
    const int row = p >> 3;
    const int chunk = (p & 7) ^ a_swizzle(row);
    acol[i] = chunk * 8;
    const int r = min(m0 + row, a.M - 1) - m0;
    arow_off[i] = (uint32_t)((int64_t)r * a.ldx * 2);
    aoff[i] = arow_off[i] + acol[i] * 2;
  }
  uint32_t boff[B_LOADS > 0 ? B_LOADS : 1];
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i) {
    if (WF) {
      // 16-byte chunk p of the stage's B: strip p/32, chunk p%32 of its half tile
      const int p = (wave * B_LOADS + i) * 64 + lane;
      const int t = min(strip0 + (p >> 5), tt.nstrips - 1) - strip0;
      boff[i] = (uint32_t)t * (uint32_t)a.wtiles * kTileBytes + (p & 31) * 16;
    } else {
      const int t = min(strip0 + wave * B_LOADS + i, tt.nstrips - 1) - strip0;
      boff[i] = (uint32_t)t * (uint32_t)a.wtiles * kTileBytes + lane * 16;
    }
  }
  // Group-wise int4 scale rows: chunk q = lane of row q / (BN/8) (lanes past
  // the rows repeat the last chunk into the unused tail of the region);
  // columns past N are clamped into the row (their outputs are not stored).
  const _Float16* sbase = nullptr;
  uint32_t soff = 0;
  if (GS) {
    const int gpb = a.gshift == 0 ? 2 : 1;  // scale rows per 64-wide K block
    const int q = min(lane, gpb * (BN / 8) - 1);
    const int r = q / (BN / 8), cc = q % (BN / 8);
    const int n0 = strip0 * 16;
    sbase = tt.scale + n0;
    soff = (uint32_t)(r * tt.N * 2 + min(n0 * 2 + cc * 16, tt.N * 2 - 16) - n0 * 2);
  }
  const bool k_tail = (a.K & 63) != 0;

  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_u8*)smem;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  // Local K block i of this split = global K block kb0 + i, LDS stage i % STAGES.
  // may_tail = false (a constant at every call site) drops the K-tail check.
  // Two K groups: stage i holds group g's block 2i + g at offset g * SUB; a
  // block past the split's end is replaced by its last block (tail-safe
  // addresses, never computed), so every stage issues the same loads.
  auto issue = [&](int i, bool may_tail) {
    int blk = i;
    uint32_t st = lds0 + (i % STAGES) * STAGE;
    if constexpr (KG == 2) {
      blk = KG * i + kg_u;
      st += kg_u * SUB;
      if (blk >= nk) {
        blk = nk - 1;
        may_tail = true;
      }
    }
    const int kb = kb0 + blk;
    if (may_tail && k_tail && kb == a.kblocks - 1) {
      // Last block with columns past K: those chunks load column 0 instead
      // and are zeroed after they land (fix_tail).
#pragma unroll
      for (int l = 0; l < A_LOADS; ++l) {
        const uint32_t o = kb * 64 + acol[l] < a.K ? aoff[l] + kb * 128 : arow_off[l];
        dma16s(o, abase, st + (wave_u * A_LOADS + l) * 1024);
      }
    } else {
      const uint8_t* ab = abase + kb * 128;
#pragma unroll
      for (int l = 0; l < A_LOADS; ++l) dma16s(aoff[l], ab, st + (wave_u * A_LOADS + l) * 1024);
    }
    const uint8_t* bb = bbase + (WF ? (int64_t)(kb >> 1) * kTileBytes + (kb & 1) * (kTileBytes / 2)
                                    : (int64_t)kb * kTileBytes);
#pragma unroll
    for (int l = 0; l < B_LOADS; ++l) dma16s(boff[l], bb, st + A_BYTES + (wave_u * B_LOADS + l) * 1024);
    (void)bb;
    if (GS && wave_u == 0)
      dma16s(soff, sbase + (int64_t)((2 * kb) >> a.gshift) * tt.N, st + S_OFF);
  };
  auto fix_tail = [&](int i) {  // local K block i (two K groups: zeroed by its group)
    const int kb = kb0 + i;
    uint8_t* st = smem + (i % STAGES) * STAGE;
    if constexpr (KG == 2) st = smem + ((i / KG) % STAGES) * STAGE + (i % KG) * SUB;
#pragma unroll
    for (int l = 0; l < A_LOADS; ++l)
      if (kb * 64 + acol[l] >= a.K)
        *reinterpret_cast<uint4*>(st + (wave * A_LOADS + l) * 1024 + lane * 16) = make_uint4(0, 0, 0, 0);
  };

  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int arow = wm * WM + (lane & 15);
  const int sw = a_swizzle(arow);  // same for arow + 16*i
  const int aoff0 = arow * 128 + (((2 * (lane >> 4)) ^ sw) * 16);
  const int aoff1 = arow * 128 + (((2 * (lane >> 4) + 1) ^ sw) * 16);
  // int4: half-tile lane and byte offset of this lane's eight bytes
  const int b4off = ((lane & 15) + 16 * (lane >> 5)) * 16 + 8 * ((lane >> 4) & 1);
  // group-wise: this lane's scale row in the block (gs = 32: positions 16g..16g+15
  // lie in group g/2 of the block's two)
  const int s4off = GS ? (((a.gshift == 0) ? (lane >> 5) : 0) * BN + wn * TN * 16 + (lane & 15)) * 2 : 0;
  // Register B: this lane's byte offset in each of the wavefront's strips.
  uint32_t broff[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int t = min(strip0 + wn * TN + j, tt.nstrips - 1) - strip0;
    broff[j] = (uint32_t)t * (uint32_t)a.wtiles * kTileBytes + (WF ? (uint32_t)b4off : (uint32_t)lane * 16);
  }
  using BRaw = typename std::conditional<WF != kWfInt8, uint2, uint4>::type;
  BRaw breg[TN];
  const __amdgpu_buffer_rsrc_t brsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(bbase), (short)0, -1, 0x00020000);
  // Issued right after the A DMA; the memory clobber keeps the compiler from
  // sinking them behind the MFMAs of the current block.
  auto load_b = [&](int i) {  // stage i (two K groups: this group's block, the last past the end)
    const int kb = kb0 + (KG == 2 ? min(KG * i + kg_u, nk - 1) : i);
    const uint32_t boffk = WF ? (uint32_t)(kb >> 1) * kTileBytes + (kb & 1) * (kTileBytes / 2)
                              : (uint32_t)kb * kTileBytes;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (WF == kWfInt8) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(brsrc, broff[j], boffk, 0);
        breg[j] = *reinterpret_cast<const BRaw*>(&v);
      } else {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(brsrc, broff[j], boffk, 0);
        breg[j] = *reinterpret_cast<const BRaw*>(&v);
      }
    }
    __asm__ volatile("" ::: "memory");
  };
  // Dequantize the registers of block i; the empty asm pins the results
  // before the next block's loads are issued, so the compiler's own wait for
  // these loads is a vmcnt(0) that the loop's wait has already satisfied.
  auto dequant_b = [&](int i, half8 (&bq)[2][TN]) {
    const uint8_t* st = smem + (i % STAGES) * STAGE;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (WF == kWfInt8) {
        const uint4 d = *reinterpret_cast<const uint4*>(&breg[j]);
        bq[0][j] = dequant8(d.x, d.y);
        bq[1][j] = dequant8(d.z, d.w);
      } else {
        const uint2 d = *reinterpret_cast<const uint2*>(&breg[j]);
        if constexpr (GS) {
          const _Float16 sc = *reinterpret_cast<const _Float16*>(st + S_OFF + s4off + j * 32);
          bq[0][j] = dequant8_i4_scaled(d.x, sc);
          bq[1][j] = dequant8_i4_scaled(d.y, sc);
        } else {
          bq[0][j] = dequant8_i4(d.x);
          bq[1][j] = dequant8_i4(d.y);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) __asm__ volatile("" ::"v"(bq[0][j]), "v"(bq[1][j]));
  };
  auto compute_br = [&](int i, const half8 (&bq)[2][TN]) {
    const uint8_t* st = smem + (i % STAGES) * STAGE + (KG == 2 ? kg_u * SUB : 0);
#pragma unroll
    for (int step = 0; step < 2; ++step) {
      half8 af[TM];
      const int ao = step == 0 ? aoff0 : aoff1;
#pragma unroll
      for (int r = 0; r < TM; ++r) af[r] = *reinterpret_cast<const half8*>(st + ao + r * 16 * 128);
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < TM; ++r) acc[r][j] = mfma16x16x32(af[r], bq[step][j], acc[r][j]);
    }
  };
  auto compute = [&](int i) {
    const uint8_t* st = smem + (i % STAGES) * STAGE;
    if constexpr (KG == 2) st += kg_u * SUB;  // this wavefront's group's block
    if constexpr (WF != kWfInt8 && IL) {
      // The int8 interleaved schedule below with int4 B (and group-wise
      // scale reads among the first LDS reads).
      __builtin_amdgcn_s_setprio(1);
      uint2 braw[TN];
      _Float16 sc[GS ? TN : 1];
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        braw[j] = *reinterpret_cast<const uint2*>(st + A_BYTES + (wn * TN + j) * B_STRIP + b4off);
        if (GS) sc[GS ? j : 0] = *reinterpret_cast<const _Float16*>(st + S_OFF + s4off + j * 32);
      }
      half8 af0[TM], af1[TM];
#pragma unroll
      for (int r = 0; r < TM; ++r) af0[r] = *reinterpret_cast<const half8*>(st + aoff0 + r * 16 * 128);
#pragma unroll
      for (int r = 0; r < TM; ++r) af1[r] = *reinterpret_cast<const half8*>(st + aoff1 + r * 16 * 128);
#pragma unroll
      for (int step = 0; step < 2; ++step)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const uint32_t d = step == 0 ? braw[j].x : braw[j].y;
          const half8 b = GS ? dequant8_i4_scaled(d, sc[GS ? j : 0]) : dequant8_i4(d);
#pragma unroll
          for (int r = 0; r < TM; ++r) acc[r][j] = mfma16x16x32(step == 0 ? af0[r] : af1[r], b, acc[r][j]);
        }
      __builtin_amdgcn_sched_group_barrier(0x100, (GS ? 2 : 1) * TN + TM, 0);
#pragma unroll
      for (int r = 0; r < TM; ++r) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * TM * TN - TM, 0);
      __builtin_amdgcn_s_setprio(0);
    } else if constexpr (WF != kWfInt8) {
      uint2 braw[TN];
      _Float16 sc[GS ? TN : 1];
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        braw[j] = *reinterpret_cast<const uint2*>(st + A_BYTES + (wn * TN + j) * B_STRIP + b4off);
        if (GS) sc[GS ? j : 0] = *reinterpret_cast<const _Float16*>(st + S_OFF + s4off + j * 32);
      }
#pragma unroll
      for (int step = 0; step < 2; ++step) {
        half8 af[TM];
        const int ao = step == 0 ? aoff0 : aoff1;
#pragma unroll
        for (int r = 0; r < TM; ++r) af[r] = *reinterpret_cast<const half8*>(st + ao + r * 16 * 128);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const uint32_t d = step == 0 ? braw[j].x : braw[j].y;
          const half8 b = GS ? dequant8_i4_scaled(d, sc[GS ? j : 0]) : dequant8_i4(d);
#pragma unroll
          for (int r = 0; r < TM; ++r) acc[r][j] = mfma16x16x32(af[r], b, acc[r][j]);
        }
      }
    } else if constexpr (IL) {
      __builtin_amdgcn_s_setprio(1);
      uint4 braw[TN];
#pragma unroll
      for (int j = 0; j < TN; ++j)
        braw[j] = *reinterpret_cast<const uint4*>(st + A_BYTES + (wn * TN + j) * kTileBytes + lane * 16);
      half8 af0[TM], af1[TM];
#pragma unroll
      for (int r = 0; r < TM; ++r) af0[r] = *reinterpret_cast<const half8*>(st + aoff0 + r * 16 * 128);
#pragma unroll
      for (int r = 0; r < TM; ++r) af1[r] = *reinterpret_cast<const half8*>(st + aoff1 + r * 16 * 128);
#pragma unroll
      for (int step = 0; step < 2; ++step)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const half8 b = step == 0 ? dequant8(braw[j].x, braw[j].y) : dequant8(braw[j].z, braw[j].w);
#pragma unroll
          for (int r = 0; r < TM; ++r) acc[r][j] = mfma16x16x32(step == 0 ? af0[r] : af1[r], b, acc[r][j]);
        }
      // Masks: 0x100 LDS reads, 0x008 MFMA.  The B and first-step A reads
      // go first, then each second-step A read follows one MFMA.
      __builtin_amdgcn_sched_group_barrier(0x100, TN + TM, 0);
#pragma unroll
      for (int r = 0; r < TM; ++r) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * TM * TN - TM, 0);
      __builtin_amdgcn_s_setprio(0);
    } else {
      uint4 braw[TN];
#pragma unroll
      for (int j = 0; j < TN; ++j)
        braw[j] = *reinterpret_cast<const uint4*>(st + A_BYTES + (wn * TN + j) * kTileBytes + lane * 16);
#pragma unroll
      for (int step = 0; step < 2; ++step) {
        half8 af[TM];
        const int ao = step == 0 ? aoff0 : aoff1;
#pragma unroll
        for (int r = 0; r < TM; ++r) af[r] = *reinterpret_cast<const half8*>(st + ao + r * 16 * 128);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const half8 b = step == 0 ? dequant8(braw[j].x, braw[j].y) : dequant8(braw[j].z, braw[j].w);
#pragma unroll
          for (int r = 0; r < TM; ++r) acc[r][j] = mfma16x16x32(af[r], b, acc[r][j]);
        }
      }
    }
  };

  if constexpr (BR) {
    // Two stages: A(i+1) by DMA and B(i+1) into registers are in flight
    // during compute(i); every wait is a full vmcnt(0).  With two K groups
    // a stage holds one block per group (as below), and a block past the
    // split's end is loaded again and not multiplied.
    const int nsb = (nk + KG - 1) / KG;
    issue(0, true);
    load_b(0);
    int i = 0;
    for (; i < nsb - 2; ++i) {  // the blocks issued here are never the split's last
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
      barrier_lds();
      half8 bq[2][TN];
      dequant_b(i, bq);
      issue(i + 1, false);
      load_b(i + 1);
      compute_br(i, bq);
    }
    for (; i < nsb; ++i) {
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
      if constexpr (KG == 1) {
        if (k_tail && kb0 + i == a.kblocks - 1) fix_tail(i);
      } else {
        if (k_tail && kb0 + nk - 1 == a.kblocks - 1 && i == (nk - 1) / KG && kg_u == (nk - 1) % KG)
          fix_tail(nk - 1);
      }
      barrier_lds();
      half8 bq[2][TN];
      dequant_b(i, bq);
      if (i + 1 < nsb) {
        issue(i + 1, true);
        load_b(i + 1);
      }
      if (KG == 1 || KG * i + kg_u < nk) compute_br(i, bq);
    }
  } else {
  const int ns = (nk + KG - 1) / KG;  // stages: one block per K group each
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < ns) issue(s, true);
  // Group-wise int4: wavefront 0 issues one more DMA per K block (scale rows).
  const bool extra = GS && wave_u == 0;
  // Steady state: the block issued (i + STAGES - 1 <= nk - 2) is never the
  // last one, so it holds no K tail, and STAGES - 2 blocks stay in flight
  // after block i; the loop carries no tail checks (their branches cost
  // about 4% on a 12288-deep K).
  int i = 0;
  for (; i < ns - STAGES; ++i) {
    if constexpr (STAGES - 2 >= 2) {
      if (extra) __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * (LOADS + 1)) : "memory");
      else __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * LOADS) : "memory");
    } else if constexpr (STAGES - 2 == 1) {
      if (extra) __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(LOADS + 1) : "memory");
      else __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(LOADS) : "memory");
    } else {
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    barrier_lds();
    issue(i + STAGES - 1, false);
    if (KG == 1 || KG * i + kg_u < nk) compute(i);
  }
  // The last STAGES blocks (or all of a short split): the block issued may be
  // the K tail, and fewer blocks remain in flight.
  for (; i < ns; ++i) {
    const int ahead = min(STAGES - 2, ns - 1 - i);  // stages issued after i
    if (ahead >= 2) {
      if (extra) __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * (LOADS + 1)) : "memory");
      else __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * LOADS) : "memory");
    } else if (ahead == 1) {
      if (extra) __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(LOADS + 1) : "memory");
      else __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(LOADS) : "memory");
    } else {
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    if constexpr (KG == 1) {
      if (k_tail && kb0 + i == a.kblocks - 1) fix_tail(i);
    } else {
      if (k_tail && kb0 + nk - 1 == a.kblocks - 1 && i == (nk - 1) / KG && kg_u == (nk - 1) % KG)
        fix_tail(nk - 1);
    }
    barrier_lds();
    // Everyone is past compute(i-1): its stage can be refilled.
    if (i + STAGES - 1 < ns) issue(i + STAGES - 1, true);
    if (KG == 1 || KG * i + kg_u < nk) compute(i);  // none past the split's end
  }
  }
  if constexpr (KG == 2) {
    // Every wavefront is past its last compute, so the stages are free: group
    // 1 leaves its accumulators there and group 0 adds them to its own.
    static_assert(NW * TM * TN * 64 * 16 <= SMEM_BYTES, "hand-off fits the LDS");
    barrier_lds();
    floatx4* red = reinterpret_cast<floatx4*>(smem);
    if (kg_u == 1) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) red[((wave * TM + i) * TN + j) * 64 + lane] = acc[i][j];
    }
    barrier_lds();
    if (kg_u == 0) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = acc[i][j] + red[((wave * TM + i) * TN + j) * 64 + lane];
    }
  }

  if (a.splits > 1) {
    // Partial tile in lane order: element (wave, i, j, r) of lane l at
    // ((((wave*TM + i)*TN + j)*4 + r)*64 + l) floats, so every store and
    // load below moves 256 contiguous bytes per wavefront.
    constexpr uint32_t TILE_F = BM * BN;
    const int tiles = a.tiles_m * a.tiles_n;
    const __amdgpu_buffer_rsrc_t pr =
        partial_rsrc(a.partial, (uint32_t)((uint64_t)a.splits * tiles * TILE_F * 4));
    const uint32_t own = ((uint32_t)split * tiles + tile) * TILE_F * 4;
    if (kg_u == 0) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t off = ((((wave * TM + i) * TN + j) * 4 + r) * 64 + lane) * 4;
            // Copy the element out first: a bit cast of the vector-element
            // lvalue itself reads element 0 whatever r is.
            const float v = acc[i][j][r];
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), pr, own + off,
                                                  0, kCoherent);
          }
    }
    __shared__ uint32_t is_last;
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's partial stores landed
    barrier_lds();
    if (tid == 0) {
      const uint32_t prev =
          __hip_atomic_fetch_add(&a.counters[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      is_last = prev == (uint32_t)(a.splits - 1) ? 1u : 0u;
    }
    barrier_lds();
    if (!is_last) return;
    // Last to arrive: sum every split's partial (its own included, read
    // back) in split order, so the result does not depend on arrival order.
    for (int sp = 0; sp < a.splits && kg_u == 0; ++sp) {
      const uint32_t base = ((uint32_t)sp * tiles + tile) * TILE_F * 4;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t off = ((((wave * TM + i) * TN + j) * 4 + r) * 64 + lane) * 4;
            const float v = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(pr, base + off, 0, kCoherent));
            acc[i][j][r] = sp == 0 ? v : acc[i][j][r] + v;
          }
    }
    if (tid == 0)
      __hip_atomic_store(&a.counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  if (kg_u != 0) return;  // group 0 holds the tile's sums
  const bool full = m0 + BM <= a.M && (strip0 + B_TILES) * 16 <= tt.N;
  store_tile<TM, TN, !GS>(tt, acc, m0 + wm * WM, (strip0 + wn * TN) * 16, lane, a.M, full);
}

// True when the 32-bit DMA offsets of w8a16_gemm_v3_kernel cannot overflow
// for any projection of the launch.
inline bool v3_offsets_fit(const GemmKernelArgs& ka, int bm, int bn) {
  const uint64_t a_span = (uint64_t)bm * (uint64_t)ka.ldx * 2 + (uint64_t)ka.kblocks * 128;
  const uint64_t b_span = (uint64_t)(bn / 16) * (uint64_t)ka.wtiles * kTileBytes;
  return a_span < (1ull << 32) && b_span < (1ull << 32);
}

// ---------------------------------------------------------------------------
// 64-bit fallback: the same pipeline with full per-lane addresses, for
// shapes whose 32-bit tile offsets could overflow (huge ldx or K).  One K
// range (no split).
// ---------------------------------------------------------------------------
template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64) void w8a16_gemm_dma_kernel(GemmKernelArgs a) {
  constexpr int NT = WAVES_M * WAVES_N * 64;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int A_BYTES = BM * 128;
  constexpr int B_TILES = BN / 16;
  constexpr int B_BYTES = B_TILES * kTileBytes;
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int A_LOADS = A_BYTES / (NT * 16);
  constexpr int B_LOADS = B_BYTES / (NT * 16);
  constexpr int LOADS = A_LOADS + B_LOADS;
  static_assert(A_LOADS >= 1 && B_LOADS >= 1 && A_LOADS * NT * 16 == A_BYTES &&
                    B_LOADS * NT * 16 == B_BYTES,
                "tile does not split into whole 1 KB wavefront loads");
  static_assert(STAGES >= 2 && STAGES <= 3, "2..3 stages");

  __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  int tile_m, tile_n;
  tile_of(blockIdx.x, a, tile_m, tile_n);
  const TileTarget tt = target_of(a, tile_n);
  const int m0 = tile_m * BM;
  const int strip0 = tt.tn * B_TILES;
  const int nk = a.kblocks;

  const _Float16* asrc[A_LOADS];
  int acol[A_LOADS];
#pragma unroll
  for (int i = 0; i < A_LOADS; ++i) {
    const int p = (wave * A_LOADS + i) * 64 + lane;
    const int row = p >> 3;
    const int chunk = (p & 7) ^ a_swizzle(row);
    acol[i] = chunk * 8;
    const int m = min(m0 + row, a.M - 1);
    asrc[i] = a.x + (int64_t)m * a.ldx + acol[i];
  }
  const uint8_t* bsrc[B_LOADS];
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i) {
    const int strip = min(strip0 + wave * B_LOADS + i, tt.nstrips - 1);
    bsrc[i] = tt.w + (int64_t)strip * a.wtiles * kTileBytes + lane * 16;
  }
  const bool k_tail = (a.K & 63) != 0;

  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_u8*)smem;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  auto issue = [&](int kb) {
    const uint32_t st = lds0 + (kb % STAGES) * STAGE;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const _Float16* src = kb * 64 + acol[i] < a.K ? asrc[i] + kb * 64 : asrc[i] - acol[i];
      dma16(src, st + (wave_u * A_LOADS + i) * 1024);
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i)
      dma16(bsrc[i] + (int64_t)kb * kTileBytes, st + A_BYTES + (wave_u * B_LOADS + i) * 1024);
  };
  auto fix_tail = [&](int kb) {
    uint8_t* st = smem + (kb % STAGES) * STAGE;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i)
      if (kb * 64 + acol[i] >= a.K)
        *reinterpret_cast<uint4*>(st + (wave * A_LOADS + i) * 1024 + lane * 16) = make_uint4(0, 0, 0, 0);
  };

  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int arow = wm * WM + (lane & 15);
  const int sw = a_swizzle(arow);
  const int aoff0 = arow * 128 + (((2 * (lane >> 4)) ^ sw) * 16);
  const int aoff1 = arow * 128 + (((2 * (lane >> 4) + 1) ^ sw) * 16);
  auto compute = [&](int kb) {
    const uint8_t* st = smem + (kb % STAGES) * STAGE;
    uint4 braw[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j)
      braw[j] = *reinterpret_cast<const uint4*>(st + A_BYTES + (wn * TN + j) * kTileBytes + lane * 16);
#pragma unroll
    for (int step = 0; step < 2; ++step) {
      half8 af[TM];
      const int ao = step == 0 ? aoff0 : aoff1;
#pragma unroll
      for (int r = 0; r < TM; ++r) af[r] = *reinterpret_cast<const half8*>(st + ao + r * 16 * 128);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const half8 b = step == 0 ? dequant8(braw[j].x, braw[j].y) : dequant8(braw[j].z, braw[j].w);
#pragma unroll
        for (int r = 0; r < TM; ++r) acc[r][j] = mfma16x16x32(af[r], b, acc[r][j]);
      }
    }
  };

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < nk) issue(s);
  for (int kb = 0; kb < nk; ++kb) {
    const int ahead = min(STAGES - 2, nk - 1 - kb);
    if (ahead >= 1) __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(LOADS) : "memory");
    else __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (k_tail && kb == nk - 1) fix_tail(kb);
    barrier_lds();
    if (kb + STAGES - 1 < nk) issue(kb + STAGES - 1);
    compute(kb);
  }

  const bool full = m0 + BM <= a.M && (strip0 + B_TILES) * 16 <= tt.N;
  store_tile<TM, TN>(tt, acc, m0 + wm * WM, (strip0 + wn * TN) * 16, lane, a.M, full);
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int OCC, int WF = kWfInt8,
          bool IL = false, bool BR = false, int KG = 1>
hipError_t launch_v3_t(const GemmKernelArgs& ka, hipStream_t stream) {
  const int64_t tiles = (int64_t)ka.tiles_m * ka.tiles_n;
  if (tiles <= 0 || tiles > 0x7fffffff || ka.splits < 1 || ka.splits > 65535 ||
      !v3_offsets_fit(ka, BM, BN))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL((w8a16_gemm_v3_kernel<BM, BN, WAVES_M, WAVES_N, STAGES, OCC, WF, IL, BR, KG>),
                     dim3((unsigned)tiles, (unsigned)ka.splits), dim3(WAVES_M * WAVES_N * 64 * KG), 0,
                     stream, ka);
  return hipGetLastError();
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES>
hipError_t launch_dma_t(const GemmKernelArgs& ka, hipStream_t stream) {
  const int64_t tiles = (int64_t)ka.tiles_m * ka.tiles_n;
  if (tiles <= 0 || tiles > 0x7fffffff || ka.splits != 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL((w8a16_gemm_dma_kernel<BM, BN, WAVES_M, WAVES_N, STAGES>),
                     dim3((unsigned)tiles), dim3(WAVES_M * WAVES_N * 64), 0, stream, ka);
  return hipGetLastError();
}

}  // namespace

// Tile configurations (measured on MI355X over the BASELINE prefill shapes).
enum GemmCfgId {
  kV3M128N256,    // 4 wavefronts 1x4, 2 stages, 2 workgroups/CU, B in registers: wide launches,
                  // and every launch beyond six 128x128 tiles per CU
  kV3M128N128,    // 4 wavefronts 1x4, 2 stages, 3 workgroups/CU, B in registers: M >= 1024 up to
                  // six 128x128 tiles per CU, and K-split launches above one workgroup per CU
  kV3M128N128S3,  // 4 wavefronts 1x4, 3 stages, 2 workgroups/CU: 128 <= M < 1024, N < 16384
  kV3M64N256,     // 4 wavefronts 1x4, 3 stages, 2 workgroups/CU: M < 128; wide mid-M launches
  kDmaM128N128,   // 64-bit addresses: when the v3 32-bit offsets could overflow
  kV3M32N64,      // 4 wavefronts 1x4, 3 stages, 4 workgroups/CU: M <= 32, with K splits
  kV3M64N64,      // 4 wavefronts 1x4, 4 stages, 4 workgroups/CU: M 33..64, with K splits
  kV3M128N128IL,  // kV3M128N128 with the interleaved MFMA schedule: 1..2 tiles per CU
  kV3M32N128,     // 4 wavefronts 1x4, 4 stages, 3 workgroups/CU: M <= 32, >= 0.75 tiles per CU
  kV3M32N256,     // 4 wavefronts 1x4, 3 stages, 2 workgroups/CU: M <= 32, >= 0.75 tiles per CU
  kV3M128N128KG,  // two K groups of 4 wavefronts, 3 stages, 1 workgroup/CU: int8 M 33..2048,
  kV3M64N128KG,   //   launches of few tiles or one round of tiles (plan_two_k_groups),
  kV3M64N64KG,    //   128x128 / 64x128 / 64x64 tiles (64x64: 4 stages)
  kV3M128N256KG,  // two K groups of the 128x256 register-B tile, 1 workgroup/CU: int8 long K
                  //   in about one round of tiles (plan_long_k_two_groups)
  kGemmCfgCount
};

// {BM, BN, workgroups per CU}
constexpr int kGemmTile[kGemmCfgCount][3] = {{128, 256, 2}, {128, 128, 3}, {128, 128, 2},
                                             {64, 256, 2},  {128, 128, 1}, {32, 64, 4},
                                             {64, 64, 4},   {128, 128, 3}, {32, 128, 3},
                                             {32, 256, 2},  {128, 128, 1}, {64, 128, 1},
                                             {64, 64, 1},   {128, 256, 1}};

// Wavefronts per workgroup of a configuration.
int gemm_cfg_waves(int cfg) {
  return (cfg == kV3M128N128KG || cfg == kV3M64N128KG || cfg == kV3M64N64KG ||
          cfg == kV3M128N256KG)
             ? 8
             : 4;
}

// Short description of a configuration as it runs for weight format wf and
// M rows (group-wise int4 at M >= 1024 runs the interleaved tile's register-B
// form, see launch_gemm4).
const char* gemm_cfg_name(int cfg, int wf, int M) {
  switch (cfg) {
    case kV3M128N256: return "128x256 B-in-registers";
    case kV3M128N128: return "128x128 B-in-registers";
    case kV3M128N128S3: return "128x128 3-stage";
    case kV3M64N256: return "64x256 3-stage";
    case kDmaM128N128: return "128x128 64-bit-address";
    case kV3M32N64: return "32x64 3-stage";
    case kV3M64N64: return "64x64 4-stage";
    case kV3M128N128IL:
      return (wf == kWfInt4Grp && M >= 1024) ? "128x128 B-in-registers" : "128x128 interleaved";
    case kV3M32N128: return "32x128 4-stage";
    case kV3M32N256: return "32x256 3-stage";
    case kV3M128N128KG: return "128x128 two K groups";
    case kV3M64N128KG: return "64x128 two K groups";
    case kV3M64N64KG: return "64x64 two K groups";
    case kV3M128N256KG: return "128x256 two K groups, B-in-registers";
    default: return "?";
  }
}

namespace {

template <int WF>
hipError_t launch_gemm4(int cfg, const GemmKernelArgs& ka, hipStream_t stream) {
  switch (cfg) {
    case kV3M128N256: return launch_v3_t<128, 256, 1, 4, 2, 2, WF, false, true>(ka, stream);
    case kV3M128N128: return launch_v3_t<128, 128, 1, 4, 2, 3, WF, false, true>(ka, stream);
    case kV3M128N128S3: return launch_v3_t<128, 128, 1, 4, 3, 2, WF>(ka, stream);
    case kV3M64N256: return launch_v3_t<64, 256, 1, 4, 3, 2, WF>(ka, stream);
    case kV3M128N128IL:
      // Group-wise at M >= 1024 (where the plan replaced the 128x128 tile
      // with B in registers): that tile is 4% faster than the interleaved
      // schedule (its scale reads sit in the LDS read groups); below M 1024
      // the interleaved schedule replaces the 3-stage tile, +14%.
      if (WF == kWfInt4Grp && ka.M >= 1024)
        return launch_v3_t<128, 128, 1, 4, 2, 3, WF, false, true>(ka, stream);
      return launch_v3_t<128, 128, 1, 4, 2, 3, WF, true>(ka, stream);
    default: return hipErrorInvalidValue;
  }
}

constexpr int kMaxGemmSplits = 8;
constexpr int kMinKbPerSplit = 16;  // 1024 input channels per split at least
constexpr int kMaxSplitTiles = kMaxSplitCounters;

void set_tiles(GemmPlan& p, int M, const int* Ns, int nproj) {
  p.bm = kGemmTile[p.cfg][0];
  p.bn = kGemmTile[p.cfg][1];
  p.tiles_m = (int)ceil_div(M, p.bm);
  p.tiles_n = 0;
  for (int i = 0; i < nproj; ++i) p.tiles_n += (int)ceil_div(Ns[i], p.bn);
  p.group_m = p.tiles_m < 4 ? p.tiles_m : 4;
}

}  // namespace

// Kernel choice per shape: the analogue of the reference's W8A16 tile
// tables (src/ops/rpu_linear_tiling.h:69-127, selectors :544-595), as rules
// over (M, total N) tuned on MI355X, plus a K split when the output has
// fewer tiles than the chip has workgroup slots.
//
// M <= 32 (int8): one tile row of 32.  The widest tile that still gives
// >= 0.75 tiles per CU runs unsplit (32x256, then 32x128): every tile
// streams its weight strips once and re-reads the M x K activation panel,
// so wider tiles cut that re-read.  Otherwise 32x64 tiles with a 4-way K
// split (8-way from 192 K blocks), fewer when a split would hold < 8 K
// blocks or the launch exceed three workgroups per CU.  (MI355X, four
// rotated weight copies, M = 32: Qwen3-VL-32B gate 25600 x 5120 28.3 us on
// 200 32x128 tiles instead of 31.9 on 400 32x64; fused gate/up 51200 x 5120
// 50.4 instead of 53.0 us with 64x256; fused q/k/v 10240 x 5120 13.8 us and
// o 5120 x 8192 13.2 us with 4 splits instead of 14.6 / 14.2 us with the
// previous 4-stage tile or 8 splits; Qwen3-8B o 4096 x 4096 9.3 instead of
// 10.2 us; down 5120 x 25600 34.6 us with 8 splits.)
//
// M 33..64 (int8): 64x64 tiles (four per CU) and a K split that brings the
// launch to about three workgroups per CU -- the largest power of two <= 768
// / tiles, at most 8, each split at least 8 K blocks -- or 64x256 tiles on
// wide launches, or the 64x64 tile with two K groups (below).
// Launches of few tiles at M 33..2048 (int8): the tile with two K groups,
// which keeps two wavefronts on every SIMD at one workgroup per CU, in place
// of a K split through memory.  Taken at <= 128 tiles of 128x128 unless K >=
// 8192 with >= 96 of them (where the K-split plans with B in registers stay
// ahead).  Among 128x128 / 64x128 / 64x64 and 1 / 2 / 4 splits that fit one
// round (tiles x splits <= CUs, >= 16 K blocks per split) it takes the least
// estimated time: the work per workgroup at 3.0 / 2.7 / 2.0 TFLOP/s per CU
// (measured rates of the three tiles) plus 6 us for a split's hand-off.
// Measured on 45 shapes (M 128..512, N 2048..8192, K 4096..12288, MI355X,
// four rotated weight copies) against the plans below: -8.9% on average,
// e.g. 2048 x 4096 at M 128 -35%, 4096 x 4096 at M 256 -16%, 4096 x 4096 at
// M 512 -10.5%; none more than 2% slower.  At M 80..112 (N 1024..4096, K
// 4096..8192) against the 64x256 tiles: -22..-41%.  At M 640..2048 (N 512..
// 2048, K 2048..5120) with >= 0.75 workgroups per CU: -3.5..-33% (e.g. 1024 x
// 4096 at M 2048 27.8 -> 24.9 us); there K 8192, more splits or fewer
// workgroups lost up to 16%, hence the extra conditions.
static bool plan_two_k_groups(int M, const int* Ns, int nproj, int K, int cus, int64_t t128,
                              GemmPlan& out) {
  const int kblocks = (int)ceil_div(K, 64);
  // One round of 129..CUs 128x128 tiles at M 128..512 with K <= 5120: the
  // unsplit tile with two K groups, in place of the unsplit 3-stage tile
  // (256 tiles) or two K splits with B in registers (the candidates below
  // leave only it, since a split or a smaller tile no longer fits one round).
  // Measured on nine shapes (MI355X, four rotated weight copies, same run):
  // Qwen3-VL-32B q at M 512 45.6 -> 44.3 us, Qwen3-8B fused q/k/v at M 512
  // 34.7 -> 33.0, fused gate/up at M 128 42.1 -> 37.6, Qwen3-VL-32B gate at
  // M 128 53.0 -> 46.5, 12288 x 4096 at M 192 / 256 33.8 -> 32.6 / 35.1 ->
  // 32.8, 8192 x 4096 at M 384 / 512 34.5 -> 32.9 / 38.6 -> 37.6, 16384 x
  // 5120 at M 256 50.7 -> 49.3 (-2..-12%).  Longer K (Qwen3-VL-32B o and
  // down at M 512) stays with the K-split plans, which measured faster.
  const bool one_round = M >= 128 && M <= 512 && kblocks <= 80 && t128 <= cus;
  if ((t128 > 128 && !one_round) || (kblocks >= 128 && t128 >= 96)) return false;
  // Beyond M 512 only where the forms measured faster: K <= 5120, at most
  // two K splits and >= 0.75 workgroups per CU.
  const bool beyond = M > 512;
  if (beyond && kblocks > 80) return false;
  // At M 33..64 only the 64x64 form with four K splits over <= 64 tiles
  // (K >= 4096): -8..-14% against the 64x64 4-stage tile with 8 splits at
  // N 1024..4096, K 4096..8192; at N 5120 / 8192 mixed (-7..+4%).
  const bool one_row = M <= 64;
  if (one_row && kblocks < 64) return false;
  struct Cand {
    int cfg;
    double rate;  // TFLOP/s per CU
  };
  const Cand cands[] = {{kV3M128N128KG, 3.0}, {kV3M64N128KG, 2.7}, {kV3M64N64KG, 2.0}};
  double best = 0;
  bool found = false;
  for (const Cand& c : cands) {
    GemmPlan p;
    p.cfg = c.cfg;
    set_tiles(p, M, Ns, nproj);
    const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
    if (one_row && (c.cfg != kV3M64N64KG || 4 * tiles > cus)) continue;
    for (int s = 1; s <= 4; s *= 2) {
      if (tiles * s > cus || kblocks < 16 * s || (s > 1 && tiles > kMaxSplitTiles)) continue;
      if (beyond && (s > 2 || 4 * tiles * s < 3LL * cus)) continue;
      const int kbs = (int)ceil_div(kblocks, s);
      const double us = 2.0 * p.bm * p.bn * 64.0 * kbs / (c.rate * 1e6) + (s > 1 ? 6.0 : 0.0);
      if (!found || us < best) {
        found = true;
        best = us;
        p.kb_per_split = kbs;
        p.splits = (int)ceil_div(kblocks, kbs);
        out = p;
      }
    }
  }
  return found;
}

// Long K (>= 8192) at M 512..2048 in about one round of 128x256 tiles (int8):
// the 128x256 tile with B in registers as two K groups (eight wavefronts, one
// workgroup per CU), with the fewest K splits (1..3) that bring the launch to
// 0.75..1 workgroups per CU while each split keeps >= 96 K blocks.  Measured
// on nine shapes against the plans they replace (MI355X, four rotated weight
// copies, same run): Qwen3-8B down (4096 x 12288) at M 1024 / 1536 / 2048
// 97.4 -> 89.5 / 133.4 -> 129.9 / 157.2 -> 152.9 us, Qwen3-VL-32B down (5120 x
// 25600) at M 512 130.1 -> 122.4 us, 2048 x 12288 at M 2048 91.2 -> 88.0 us,
// 4096 x 8192 at M 2048 106.1 -> 104.5 us (-1.4..-8%).  Not taken where no
// split count fits (VL down at M 1024, 160 tiles: 253 -> 274 us) or the
// splits would be shorter (4096 x 8192 at M 1024, 4096 x 12288 at M 512: even).
static bool plan_long_k_two_groups(int M, const int* Ns, int nproj, int K, int cus,
                                   GemmPlan& out) {
  const int kblocks = (int)ceil_div(K, 64);
  if (M < 512 || kblocks < 128) return false;
  GemmPlan p;
  p.cfg = kV3M128N256KG;
  set_tiles(p, M, Ns, nproj);
  const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
  for (int s = 1; s <= 3; ++s) {
    if (tiles * s > cus || kblocks < 96 * s || (s > 1 && tiles > kMaxSplitTiles)) return false;
    if (4 * tiles * s < 3LL * cus) continue;
    p.kb_per_split = (int)ceil_div(kblocks, s);
    p.splits = (int)ceil_div(kblocks, p.kb_per_split);
    out = p;
    return true;
  }
  return false;
}

GemmPlan plan_gemm(int M, const int* Ns, int nproj, int K, const DeviceInfo& dev, bool int4) {
  const int cus = dev.cus > 0 ? dev.cus : 256;
  if (M <= 32 && !int4) {
    GemmPlan p;
    const int kblocks = (int)ceil_div(K, 64);
    int64_t t256 = 0, t128 = 0;
    for (int i = 0; i < nproj; ++i) {
      t256 += ceil_div(Ns[i], 256);
      t128 += ceil_div(Ns[i], 128);
    }
    if (4 * t256 >= 3LL * cus || 4 * t128 >= 3LL * cus) {
      p.cfg = 4 * t256 >= 3LL * cus ? kV3M32N256 : kV3M32N128;
      set_tiles(p, M, Ns, nproj);
      p.splits = 1;
      p.kb_per_split = kblocks;
      return p;
    }
    p.cfg = kV3M32N64;
    set_tiles(p, M, Ns, nproj);
    const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
    int s = kblocks >= 192 ? 8 : 4;
    while (s > 1 && (s * tiles > 3LL * cus || kblocks < 8 * s)) s /= 2;
    if (tiles > kMaxSplitTiles) s = 1;
    p.kb_per_split = (int)ceil_div(kblocks, s);
    p.splits = (int)ceil_div(kblocks, p.kb_per_split);
    return p;
  }
  if (M <= 64 && !int4) {
    GemmPlan p;
    const int kblocks = (int)ceil_div(K, 64);
    // Wide launches: every workgroup reads its M x K activation panel, so the
    // activation traffic is (tile columns) x M x K x 2 bytes -- as large as
    // the weights themselves with 64-column tiles at N = 51200.  64x256 tiles
    // read it a quarter as often: taken when they alone give >= 0.75
    // workgroups per CU, or with a 2-way K split at >= 0.375
    // (Qwen3-VL-32B gate/up at M 32..64: 52..57 us instead of 63..84 us;
    // Qwen3-8B gate/up at M 48..64: 28.5 instead of 30.5..32 us; MI355X).
    int64_t w256 = 0;
    for (int i = 0; i < nproj; ++i) w256 += ceil_div(Ns[i], 256);
    const bool wide = w256 * 4 >= 3LL * cus;
    if (wide || (w256 * 8 >= 3LL * cus && kblocks >= 2 * kMinKbPerSplit)) {
      p.cfg = kV3M64N256;
      set_tiles(p, M, Ns, nproj);
      p.kb_per_split = wide ? kblocks : (int)ceil_div(kblocks, 2);
      p.splits = (int)ceil_div(kblocks, p.kb_per_split);
      return p;
    }
    GemmPlan kgp;
    if (plan_two_k_groups(M, Ns, nproj, K, cus, /*t128=*/0, kgp)) return kgp;
    p.cfg = kV3M64N64;
    set_tiles(p, M, Ns, nproj);
    const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
    int s = 1;
    while (s < 8 && (int64_t)(2 * s) * tiles <= 3LL * cus && kblocks / (2 * s) >= 8) s *= 2;
    if (tiles > kMaxSplitTiles) s = 1;
    p.kb_per_split = (int)ceil_div(kblocks, s);
    p.splits = (int)ceil_div(kblocks, p.kb_per_split);
    return p;
  }
  int64_t ntotal = 0, cols256 = 0, cols128 = 0;  // tile columns 256 and 128 wide
  for (int i = 0; i < nproj; ++i) {
    ntotal += Ns[i];
    cols256 += ceil_div(Ns[i], 256);
    cols128 += ceil_div(Ns[i], 128);
  }
  const int64_t t128x256 = ceil_div(M, 128) * cols256;     // 128x256 tiles
  const int64_t t128 = ceil_div(M, 128) * cols128;         // 128x128 tiles
  if (!int4 && M <= 2048) {  // M >= 65 here
    GemmPlan kgp;
    if (plan_two_k_groups(M, Ns, nproj, K, cus, t128, kgp)) return kgp;
    if (plan_long_k_two_groups(M, Ns, nproj, K, cus, kgp)) return kgp;
  }
  GemmPlan p;
  if (M < 128) {
    p.cfg = kV3M64N256;
  } else if (t128 <= 6LL * cus) {
    // Up to six 128x128 tiles per CU the tiles a CU gets decide the time:
    // a launch takes ceil(tiles / CUs) tile times, a 128x256 tile costing
    // two 128x128 ones.  The cheaper shape wins; on a tie 128x128 when it
    // lands one to two tiles per CU (the interleaved schedule below), else
    // 128x256.  (Measured over the Qwen3-8B and Qwen3-VL-32B projections at
    // M 128..4096 on MI355X: e.g. fused q/k/v 10240 x 5120 at M 1024 / 2048
    // 100.6 / 171 us instead of 110.5 / 187 us with 128x256.)  Exception:
    // at two to three 128x128 tiles per CU and at least 1.5 128x256 tiles
    // per CU, both shapes finish in one round and the 128x256 tile, with its
    // B strips in registers, does more work per cycle; so there 128x256 wins
    // unless K is long enough for the K split below (gate/up 24576 x 4096 at
    // M 512: 92.8 instead of 95.1 us; fused q/k/v 6144 x 4096 at M 2048: 83.5
    // instead of 86.9 us; 12288 x 4096 at M 1024: 83.0 instead of 86.8 us).
    // With fewer 128x256 tiles the CUs holding two of them decide, and the
    // results scatter (-6..+8%), so the rule stays as it was.
    const int64_t r256 = ceil_div(t128x256, cus) * 2, r128 = ceil_div(t128, cus);
    const bool one_round = t128 > 2LL * cus && t128 <= 3LL * cus && 2 * t128x256 >= 3LL * cus &&
                           ceil_div(K, 64) < 192;
    const bool use128 =
        !one_round && (r128 < r256 || (r128 == r256 && t128 > cus && t128 <= 2LL * cus));
    p.cfg = !use128 ? kV3M128N256
                    : (M < 1024 && t128 <= 2LL * cus) ? kV3M128N128S3 : kV3M128N128;
  } else if (M >= 1024) {
    // Beyond six 128x128 tiles per CU: 128x256 with B in registers, also on
    // whole rounds of 256x256 tiles and below N 8192 (4096^3 109 us against
    // 111 us with 256x256; 8192 x 4096 x 4096 206 us against 216 us with
    // 256x256 and 231 us with 128x128).
    p.cfg = kV3M128N256;
  } else {
    p.cfg = ntotal >= 16384 ? kV3M128N256 : kV3M128N128S3;
  }
  set_tiles(p, M, Ns, nproj);
  const int kblocks = (int)ceil_div(K, 64);
  const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
  const int64_t slots = (int64_t)cus * kGemmTile[p.cfg][2];
  p.splits = 1;
  p.kb_per_split = kblocks;
  int s = 1;
  if (tiles < cus && tiles <= kMaxSplitTiles) {
    // Below one tile per CU: split K up to the chip's workgroup slots, each
    // split keeping >= 16 K blocks while the launch has at most one
    // workgroup per CU and >= 24 beyond that (shorter splits cost more in
    // partial round trips than they gain: 512 x 4096 x 4096, 128 tiles:
    // 26.5 us with 2 splits, 28.6 us with 4).
    s = (int)(slots / tiles);
    s = s < kMaxGemmSplits ? s : kMaxGemmSplits;
    while (s > 1 && kblocks < s * ((tiles * s <= cus) ? 16 : 24)) --s;
  } else if ((p.cfg == kV3M128N128 || p.cfg == kV3M128N128S3) && kblocks >= 192 &&
             tiles <= 3LL * cus) {
    // Long K (>= 12288) at one tile per CU, or 1.25..1.75 / 2.25..2.75 per
    // CU: two K splits even out the CUs' share (and give one-per-CU launches
    // two waves per SIMD): 1024 x 4096 x 12288 97 us instead of 105 us,
    // 1024 / 2048 x 5120 x 25600 262 / 445 us instead of 290 / 497 us.
    const int64_t q4 = (tiles % cus) * 4;  // fractional tiles per CU, x 4 CUs
    if (tiles == cus || (q4 >= cus && q4 <= 3 * cus)) s = 2;
  }
  if (s >= 2) {
    p.kb_per_split = (int)ceil_div(kblocks, s);
    p.splits = (int)ceil_div(kblocks, p.kb_per_split);  // no empty split
    // A split count sized for the 3-stage tile (two workgroups per CU) that
    // leaves more than one workgroup per CU runs faster on the 2-stage tile
    // with B in registers, except for int8 at long K, where the third stage
    // hides more of the weights' HBM latency.  (Four rotated weight copies:
    // Qwen3-VL-32B o at M 512, 160 tiles in three splits, 46.5 instead of
    // 51.1 us; 12288 x 4096 at M 256 and 4096 x 4096 at M 768 +6%; int4
    // +4..8.5% including K 12288..25600; int8 4096 x 12288 at M 512 -3.8%.)
    // The split count stays the 3-stage tile's: sized for three workgroups
    // per CU it would be four, 131 instead of 118 us on VL down.
    if (p.cfg == kV3M128N128S3 && tiles * p.splits > cus && (int4 || kblocks < 192))
      p.cfg = kV3M128N128;
  }
  // 128x128 tiles that leave one to two workgroups (two wavefronts per SIMD)
  // on a CU: the interleaved schedule (+8..16% on 384 and 512 tiles of
  // M 1024..4096, K 4096..12288, and +20% on the fused Qwen3-VL-32B q/k/v at
  // M = 512; -1..3% at one tile per CU or 2.5..3 per CU, where the plain
  // schedule stays).  Int4 alike: per-channel +6..32% (Qwen3-8B / VL-32B
  // q/k/v and o at M 512..2048), group-wise +14% below M 1024.
  if ((p.cfg == kV3M128N128 || p.cfg == kV3M128N128S3) && p.splits == 1 && tiles > cus &&
      tiles <= 2LL * cus)
    p.cfg = kV3M128N128IL;
  return p;
}

bool gemm_offsets_fit(const GemmPlan& p, int64_t ldx, int K, bool int4) {
  if (p.cfg == kDmaM128N128) return true;  // full per-lane addresses
  GemmKernelArgs ka;
  ka.ldx = ldx;
  ka.kblocks = (int)ceil_div(K, 64);
  ka.wtiles = int4 ? (int)ceil_div(K, kTileK4) : ka.kblocks;
  return v3_offsets_fit(ka, p.bm, p.bn);
}

// The v3 kernels address a tile with 32-bit offsets from its first row /
// strip (row stride ldx); an int8 plan whose offsets could overflow runs the
// 64-bit-address kernel, unsplit.  int4 plans are returned as they are (the
// caller refuses them: there is no int4 64-bit-address kernel).
GemmPlan gemm_plan_for_stride(const GemmPlan& plan, int M, const int* Ns, int nproj, int64_t ldx,
                              int K, bool int4) {
  GemmPlan p = plan;
  if (int4 || gemm_offsets_fit(p, ldx, K, false)) return p;
  p.cfg = kDmaM128N128;
  set_tiles(p, M, Ns, nproj);
  p.splits = 1;
  p.kb_per_split = (int)ceil_div(K, 64);
  return p;
}

size_t gemm_workspace_bytes(const GemmPlan& p) {
  if (p.splits <= 1) return 0;
  return (size_t)p.splits * (size_t)p.tiles_m * (size_t)p.tiles_n * (size_t)p.bm * (size_t)p.bn *
         sizeof(float);
}

hipError_t launch_gemm(const LinearProblem& pr, const GemmPlan& plan, void* workspace,
                       hipStream_t stream) {
  GemmPlan p = plan;
  if (pr.nproj < 1 || pr.nproj > kMaxProj) return hipErrorInvalidValue;
  int ns[kMaxProj];
  for (int i = 0; i < pr.nproj; ++i) ns[i] = pr.proj[i].N;

  GemmKernelArgs ka;
  ka.x = pr.x;
  ka.ldx = pr.ldx;
  ka.M = pr.M;
  ka.K = pr.K;
  ka.kblocks = (int)ceil_div(pr.K, 64);
  ka.wtiles = pr.wf ? (int)ceil_div(pr.K, kTileK4) : ka.kblocks;
  ka.gshift = pr.gshift;
  ka.nproj = pr.nproj;
  auto fill = [&](const GemmPlan& q) {
    ka.tiles_m = q.tiles_m;
    ka.tiles_n = q.tiles_n;
    ka.group_m = q.group_m;
    int tn0 = 0;
    for (int i = 0; i < kMaxProj; ++i) {
      GemmProj& d = ka.proj[i];
      if (i < pr.nproj) {
        const Projection& s = pr.proj[i];
        d.w = s.w;
        d.scale = s.scale;
        d.bias = s.bias;
        d.y = s.y;
        d.ldy = s.ldy;
        d.N = s.N;
        d.nstrips = (int)ceil_div(s.N, 16);
        d.tn0 = tn0;
        tn0 += (int)ceil_div(s.N, q.bn);
      } else {
        d = ka.proj[0];
        d.tn0 = 0x7fffffff;
      }
    }
    ka.splits = q.splits;
    ka.kb_per_split = q.kb_per_split;
    ka.partial = nullptr;
    ka.counters = nullptr;
    if (q.splits > 1) {
      ka.counters = static_cast<uint32_t*>(workspace);
      ka.partial = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + RF_W8A16_WS_COUNTER_BYTES);
    }
  };
  // 64-bit addressing where the v3 kernels' 32-bit tile offsets could
  // overflow (int8; int4 has no such kernel and its callers refuse first).
  if (!gemm_offsets_fit(p, pr.ldx, pr.K, pr.wf != kWfInt8)) {
    if (pr.wf != kWfInt8) return hipErrorInvalidValue;
    p = gemm_plan_for_stride(p, pr.M, ns, pr.nproj, pr.ldx, pr.K, false);
  }
  fill(p);
  if (p.splits > 1 && (!workspace || (int64_t)p.tiles_m * p.tiles_n > kMaxSplitTiles ||
                       gemm_workspace_bytes(p) >= (1ull << 31)))
    return hipErrorInvalidValue;
  if (pr.wf == kWfInt4) return launch_gemm4<kWfInt4>(p.cfg, ka, stream);
  if (pr.wf == kWfInt4Grp) return launch_gemm4<kWfInt4Grp>(p.cfg, ka, stream);
  switch (p.cfg) {
    case kV3M128N256: return launch_v3_t<128, 256, 1, 4, 2, 2, kWfInt8, false, true>(ka, stream);
    case kV3M128N128: return launch_v3_t<128, 128, 1, 4, 2, 3, kWfInt8, false, true>(ka, stream);
    case kV3M128N128S3: return launch_v3_t<128, 128, 1, 4, 3, 2>(ka, stream);
    case kV3M64N256: return launch_v3_t<64, 256, 1, 4, 3, 2>(ka, stream);
    case kDmaM128N128: return launch_dma_t<128, 128, 1, 4, 3>(ka, stream);
    case kV3M32N64: return launch_v3_t<32, 64, 1, 4, 3, 4>(ka, stream);
    case kV3M64N64: return launch_v3_t<64, 64, 1, 4, 4, 4>(ka, stream);
    case kV3M128N128IL: return launch_v3_t<128, 128, 1, 4, 2, 3, kWfInt8, true>(ka, stream);
    case kV3M32N128: return launch_v3_t<32, 128, 1, 4, 4, 3>(ka, stream);
    case kV3M32N256: return launch_v3_t<32, 256, 1, 4, 3, 2>(ka, stream);
    case kV3M128N128KG: return launch_v3_t<128, 128, 1, 4, 3, 1, kWfInt8, false, false, 2>(ka, stream);
    case kV3M64N128KG: return launch_v3_t<64, 128, 1, 4, 3, 1, kWfInt8, false, false, 2>(ka, stream);
    case kV3M64N64KG: return launch_v3_t<64, 64, 1, 4, 4, 1, kWfInt8, false, false, 2>(ka, stream);
    case kV3M128N256KG: return launch_v3_t<128, 256, 1, 4, 2, 1, kWfInt8, false, true, 2>(ka, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rf
