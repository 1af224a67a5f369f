// Prefill GEMM for W8A16 (gfx950): LDS-staged INT8 weight tiles dequantized
// into fp16 MFMA operands, fp32 accumulation.
//
// Workgroup tile BM x BN, WAVES_M x WAVES_N wavefronts, each owning a
// (BM/WAVES_M) x (BN/WAVES_N) block of 16x16 v_mfma_f32_16x16x32_f16
// accumulators.
//   * operands move global -> LDS with global_load_lds_dwordx4 (no VGPR
//     staging), STAGES ring buffers of KS 64-wide K blocks each, so up to
//     STAGES-1 K steps are in flight while one is multiplied;
//   * A (activations, fp16) rows are 128 bytes per K block, chunk-swizzled
//     (a_swizzle) so fragment reads are free of LDS bank conflicts;
//   * B (weights) stays INT8 in LDS (half the LDS bytes and half the
//     global->LDS traffic of an fp16 tile): TILE16X64 tiles are copied
//     verbatim and each lane's 16 bytes are exactly its two MFMA B operands,
//     dequantized in registers right before the MFMAs (exact, v_perm +
//     v_pk_add);
//   * tiles are ordered so that the workgroups one XCD runs at the same time
//     (the hardware deals workgroup ids round-robin over the 8 XCDs) cover a
//     compact block of output tiles and share A and B rows in their L2;
//   * the per-channel scale and bias are applied in the fp32 epilogue.
#include "w8a16_common.h"
#include "w8a16_internal.h"

namespace rf {
namespace {

constexpr int kXcds = 8;

struct GemmKernelArgs {
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
  int tiles_m, tiles_n;
  int group_m;  // output-tile rows per scheduling group
};

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

// ---------------------------------------------------------------------------
// Direct-to-LDS variant: global_load_lds_dwordx4 writes each wavefront's
// 64 x 16 bytes straight into LDS (lane-contiguous), so no VGPRs stage the
// tiles and STAGES K steps can be in flight.  A rows are unpadded (128 B)
// and chunk-swizzled instead (a_swizzle): LDS slot p of row r holds global
// chunk p ^ a_swizzle(r).  Rows past M and strips past N load clamped (valid)
// addresses; their results are never stored.  Columns past K (the last K
// step when K % 64 != 0) are zeroed in LDS after their load lands.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) uint8_t lds_u8;

// One global_load_lds_dwordx4: every lane reads 16 bytes at `g`, the
// wavefront's 64 x 16 bytes land lane-contiguously at LDS byte address
// `lds` (wave-uniform, passed in M0).  Written as inline asm so the
// compiler does not serialise every later LDS read behind it (it cannot
// tell which LDS bytes a DMA writes); the kernel orders the LDS traffic
// itself with explicit s_waitcnt vmcnt + s_barrier.  Nothing else in these
// kernels uses M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Chunk swizzle of the LDS A tile: 16-byte chunk c of row r is stored in
// slot c ^ a_swizzle(r).  An MFMA A-fragment read has 16 lanes on rows
// r0..r0+15 (r0 % 16 == 0) at one chunk, and the next 16 lanes on the same
// rows at chunk ^ 2; with this swizzle the accesses of every 8-, 16- and
// 32-lane group cover distinct LDS banks (64 or 128 banks of 4 bytes).
__device__ __forceinline__ int a_swizzle(int r) { return (r & 7) ^ (((r >> 3) & 1) * 5); }

// Workgroup barrier without the memory fences __syncthreads() implies (a
// release fence would wait for every DMA in flight).  The caller has
// already waited for the loads whose data the other wavefronts read.
__device__ __forceinline__ void barrier_lds() {
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int KS>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64) void w8a16_gemm_dma_kernel(GemmKernelArgs a) {
  constexpr int NT = WAVES_M * WAVES_N * 64;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int A_KB = BM * 128;                  // A bytes of one 64-wide K block
  constexpr int B_TILES = BN / 16;
  constexpr int B_KB = B_TILES * kTileBytes;      // B bytes of one K block
  constexpr int A_BYTES = A_KB * KS, B_BYTES = B_KB * KS;
  constexpr int STAGE = A_BYTES + B_BYTES;        // KS K blocks per stage
  constexpr int A_LOADS = A_BYTES / (NT * 16);    // per thread per stage
  constexpr int B_LOADS = B_BYTES / (NT * 16);
  constexpr int ROWBLKS = BM / 8;                 // 1 KB (8-row) blocks per A K block
  static_assert(A_LOADS >= 1 && B_LOADS >= 1 && A_LOADS * NT * 16 == A_BYTES &&
                    B_LOADS * NT * 16 == B_BYTES,
                "tile does not split into whole 1 KB wavefront loads");
  static_assert(STAGES >= 2 && STAGES <= 4, "2..4 stages");
  static_assert(TM >= 1 && TN >= 1, "wavefront tile");

  __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  int tile_m, tile_n;
  tile_of(blockIdx.x, a, tile_m, tile_n);
  const int m0 = tile_m * BM;
  const int strip0 = tile_n * B_TILES;
  const int nk = a.kblocks;
  const int nstage = (nk + KS - 1) / KS;

  // A load i of this thread: 1 KB block j = wave*A_LOADS + i of the stage,
  // K block kk = j / ROWBLKS, LDS slot p = (j % ROWBLKS)*64 + lane, row
  // p/8, global chunk (p%8) ^ ((row>>1)&7).
  const _Float16* asrc[A_LOADS];
  int acol[A_LOADS];  // column offset inside the stage's KS*64 columns
#pragma unroll
  for (int i = 0; i < A_LOADS; ++i) {
    const int j = wave * A_LOADS + i;
    const int kk = j / ROWBLKS;
    const int p = (j % ROWBLKS) * 64 + lane;
    const int row = p >> 3;
    const int chunk = (p & 7) ^ a_swizzle(row);
    acol[i] = kk * 64 + chunk * 8;
    const int m = min(m0 + row, a.M - 1);
    asrc[i] = a.x + (int64_t)m * a.ldx + acol[i];
  }
  // B load i: 1 KB block j = K block kk = j / B_TILES, tile t = j % B_TILES.
  const uint8_t* bsrc[B_LOADS];
  int bkk[B_LOADS];
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i) {
    const int j = wave * B_LOADS + i;
    bkk[i] = j / B_TILES;
    const int strip = min(strip0 + j % B_TILES, a.nstrips - 1);
    bsrc[i] = a.w + (int64_t)strip * a.kblocks * kTileBytes + lane * 16;
  }
  const bool k_tail = (a.K & 63) != 0 || (nk % KS) != 0;

  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_u8*)smem;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  auto issue = [&](int st_idx) {
    const uint32_t st = lds0 + (st_idx % STAGES) * STAGE;
    const int kcol = st_idx * KS * 64;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      // Columns past K would read past the row: load column 0 instead and
      // zero the slot once it has landed (fix_tail).
      const _Float16* src = kcol + acol[i] < a.K ? asrc[i] + kcol : asrc[i] - acol[i];
      dma16(src, st + (wave_u * A_LOADS + i) * 1024);
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      // K blocks past the weight's last one are clamped; A is zero there.
      const int kb = min(st_idx * KS + bkk[i], nk - 1);
      dma16(bsrc[i] + (int64_t)kb * kTileBytes, st + A_BYTES + (wave_u * B_LOADS + i) * 1024);
    }
  };
  auto fix_tail = [&](int st_idx) {
    uint8_t* st = smem + (st_idx % STAGES) * STAGE;
    const int kcol = st_idx * KS * 64;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i)
      if (kcol + acol[i] >= a.K)
        *reinterpret_cast<uint4*>(st + (wave * A_LOADS + i) * 1024 + lane * 16) = make_uint4(0, 0, 0, 0);
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

  auto compute = [&](int st_idx) {
    const uint8_t* st = smem + (st_idx % STAGES) * STAGE;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const uint8_t* sa = st + kk * A_KB;
      const uint8_t* sb = st + A_BYTES + kk * B_KB;
      uint4 braw[TN];
#pragma unroll
      for (int j = 0; j < TN; ++j)
        braw[j] = *reinterpret_cast<const uint4*>(sb + (wn * TN + j) * kTileBytes + lane * 16);
#pragma unroll
      for (int step = 0; step < 2; ++step) {
        half8 af[TM], bf[TN];
        const int aoff = step == 0 ? aoff0 : aoff1;
#pragma unroll
        for (int i = 0; i < TM; ++i)
          af[i] = *reinterpret_cast<const half8*>(sa + aoff + i * 16 * 128);
#pragma unroll
        for (int j = 0; j < TN; ++j)
          bf[j] = step == 0 ? dequant8(braw[j].x, braw[j].y) : dequant8(braw[j].z, braw[j].w);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32(af[i], bf[j], acc[i][j]);
      }
    }
  };

  // Prologue: STAGES-1 stages in flight.
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < nstage) issue(s);
  for (int sidx = 0; sidx < nstage; ++sidx) {
    // Wait for this thread's loads of stage sidx (later stages may stay in
    // flight), then for everyone's.
    const int ahead = min(STAGES - 2, nstage - 1 - sidx);  // stages issued after sidx
    if (ahead >= 2) __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * (A_LOADS + B_LOADS)) : "memory");
    else if (ahead == 1) __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(A_LOADS + B_LOADS) : "memory");
    else __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (k_tail && sidx == nstage - 1) fix_tail(sidx);
    barrier_lds();
    // Everyone is past compute(sidx-1): its stage can be refilled.
    if (sidx + STAGES - 1 < nstage) issue(sidx + STAGES - 1);
    compute(sidx);
  }

  // Epilogue: lane l holds D[4*(l/16) + r][l%16] of each 16x16 tile.
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = (strip0 + wn * TN + j) * 16 + (lane & 15);
    if (n >= a.N) continue;
    const float sc = (float)a.scale[n];
    const float bi = a.bias ? (float)a.bias[n] : 0.f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * WM + i * 16 + 4 * (lane >> 4) + r;
        if (m < a.M) a.y[(int64_t)m * a.ldy + n] = (_Float16)__builtin_fmaf(acc[i][j][r], sc, bi);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// v3: the DMA kernel with wave-uniform SGPR bases.  Each DMA is
// global_load_lds_dwordx4 voff, s[base]: the per-lane byte offset from the
// tile's first row / strip is fixed for the whole K loop, and one scalar add
// per K block moves the bases, so the loop issues no vector address math.
// OCC workgroups per CU are requested from the register allocator.
// Offsets are 32-bit: the host checks BM*ldx*2 + 2K and the strip span
// B_TILES*kblocks*1024 fit (launch_v3_t).
// ---------------------------------------------------------------------------
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16s(uint32_t voff, const void* sbase, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int OCC>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64) __attribute__((amdgpu_waves_per_eu(OCC * WAVES_M * WAVES_N / 4, 8)))
void w8a16_gemm_v3_kernel(GemmKernelArgs a) {
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
  static_assert(STAGES >= 2 && STAGES <= 4, "2..4 stages");

  __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  int tile_m, tile_n;
  tile_of(blockIdx.x, a, tile_m, tile_n);
  const int m0 = tile_m * BM;
  const int strip0 = tile_n * B_TILES;
  const int nk = a.kblocks;

  // Wave-uniform bases and per-lane 32-bit offsets.
  const uint8_t* abase = reinterpret_cast<const uint8_t*>(a.x + (int64_t)m0 * a.ldx);
  const uint8_t* bbase = a.w + (int64_t)strip0 * a.kblocks * kTileBytes;
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
  uint32_t boff[B_LOADS];
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i) {
    const int t = min(strip0 + wave * B_LOADS + i, a.nstrips - 1) - strip0;
    boff[i] = (uint32_t)t * (uint32_t)a.kblocks * kTileBytes + lane * 16;
  }
  const bool k_tail = (a.K & 63) != 0;

  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_u8*)smem;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  auto issue = [&](int kb) {
    const uint32_t st = lds0 + (kb % STAGES) * STAGE;
    if (k_tail && kb == nk - 1) {
      // Last block with columns past K: those chunks load column 0 instead
      // and are zeroed after they land (fix_tail).
#pragma unroll
      for (int i = 0; i < A_LOADS; ++i) {
        const uint32_t o = kb * 64 + acol[i] < a.K ? aoff[i] + kb * 128 : arow_off[i];
        dma16s(o, abase, st + (wave_u * A_LOADS + i) * 1024);
      }
    } else {
      const uint8_t* ab = abase + kb * 128;
#pragma unroll
      for (int i = 0; i < A_LOADS; ++i) dma16s(aoff[i], ab, st + (wave_u * A_LOADS + i) * 1024);
    }
    const uint8_t* bb = bbase + (int64_t)kb * kTileBytes;
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) dma16s(boff[i], bb, st + A_BYTES + (wave_u * B_LOADS + i) * 1024);
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
  const int sw = a_swizzle(arow);  // same for arow + 16*i
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
      for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const half8*>(st + ao + i * 16 * 128);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const half8 b = step == 0 ? dequant8(braw[j].x, braw[j].y) : dequant8(braw[j].z, braw[j].w);
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i][j] = mfma16x16x32(af[i], b, acc[i][j]);
      }
    }
  };

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < nk) issue(s);
  for (int kb = 0; kb < nk; ++kb) {
    const int ahead = min(STAGES - 2, nk - 1 - kb);  // blocks issued after kb
    if (ahead >= 2) __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * LOADS) : "memory");
    else if (ahead == 1) __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(LOADS) : "memory");
    else __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (k_tail && kb == nk - 1) fix_tail(kb);
    barrier_lds();
    if (kb + STAGES - 1 < nk) issue(kb + STAGES - 1);
    compute(kb);
  }

  // Epilogue: lane l holds D[4*(l/16) + r][l%16] of each 16x16 tile; row
  // offsets are uniform, so a full tile stores without per-element checks.
  const int nl = (strip0 + wn * TN) * 16 + (lane & 15);
  const int ml = m0 + wm * WM + 4 * (lane >> 4);
  _Float16* yl = a.y + (int64_t)ml * a.ldy + nl;
  float sc[TN], bi[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = nl + j * 16;
    sc[j] = n < a.N ? (float)a.scale[n] : 0.f;
    bi[j] = (a.bias && n < a.N) ? (float)a.bias[n] : 0.f;
  }
  const bool full = m0 + BM <= a.M && (strip0 + B_TILES) * 16 <= a.N;
  if (full) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        _Float16* yr = yl + (int64_t)(i * 16 + r) * a.ldy;
#pragma unroll
        for (int j = 0; j < TN; ++j) yr[j * 16] = (_Float16)__builtin_fmaf(acc[i][j][r], sc[j], bi[j]);
      }
  } else {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (ml + i * 16 + r >= a.M) continue;
        _Float16* yr = yl + (int64_t)(i * 16 + r) * a.ldy;
#pragma unroll
        for (int j = 0; j < TN; ++j)
          if (nl + j * 16 < a.N) yr[j * 16] = (_Float16)__builtin_fmaf(acc[i][j][r], sc[j], bi[j]);
      }
  }
}

// True when the 32-bit DMA offsets of w8a16_gemm_v3_kernel cannot overflow.
inline bool v3_offsets_fit(const GemmKernelArgs& ka, int bm, int bn) {
  const uint64_t a_span = (uint64_t)bm * (uint64_t)ka.ldx * 2 + (uint64_t)ka.kblocks * 128;
  const uint64_t b_span = (uint64_t)(bn / 16) * (uint64_t)ka.kblocks * kTileBytes;
  return a_span < (1ull << 32) && b_span < (1ull << 32);
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int OCC>
hipError_t launch_v3_t(const GemmKernelArgs& ka, hipStream_t stream) {
  const int64_t blocks = (int64_t)ka.tiles_m * ka.tiles_n;
  if (blocks <= 0 || blocks > 0x7fffffff || !v3_offsets_fit(ka, BM, BN)) return hipErrorInvalidValue;
  hipLaunchKernelGGL((w8a16_gemm_v3_kernel<BM, BN, WAVES_M, WAVES_N, STAGES, OCC>),
                     dim3((unsigned)blocks), dim3(WAVES_M * WAVES_N * 64), 0, stream, ka);
  return hipGetLastError();
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int KS>
hipError_t launch_dma_t(const GemmKernelArgs& ka, hipStream_t stream) {
  const int64_t blocks = (int64_t)ka.tiles_m * ka.tiles_n;
  if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((w8a16_gemm_dma_kernel<BM, BN, WAVES_M, WAVES_N, STAGES, KS>),
                     dim3((unsigned)blocks), dim3(WAVES_M * WAVES_N * 64), 0, stream, ka);
  return hipGetLastError();
}

GemmKernelArgs make_args(const LinearArgs& a, const GemmPlan& p) {
  GemmKernelArgs ka;
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
  ka.tiles_m = p.tiles_m;
  ka.tiles_n = p.tiles_n;
  ka.group_m = p.group_m;
  return ka;
}

}  // namespace

// Tile configurations (measured on MI355X over the BASELINE prefill shapes).
enum GemmCfgId {
  kV3M128N256,    // 4 wavefronts 1x4, 2 stages, 2 workgroups/CU: wide N
  kV3M128N128,    // 4 wavefronts 1x4, 2 stages, 3 workgroups/CU: M >= 1024, N < 8192
  kV3M128N128S3,  // 4 wavefronts 1x4, 3 stages, 2 workgroups/CU: moderate M and N
  kV3M64N256,     // 4 wavefronts 1x4, 3 stages, 2 workgroups/CU: small M
  kDmaM128N128,   // 64-bit addresses: when the v3 32-bit offsets could overflow
  kGemmCfgCount
};

constexpr int kGemmTile[kGemmCfgCount][2] = {{128, 256}, {128, 128}, {128, 128}, {64, 256}, {128, 128}};

// Kernel choice per shape: the analogue of the reference's W8A16 tile
// tables (src/ops/rpu_linear_tiling.h:69-127, selectors :544-595), as rules
// over (M, N) tuned on MI355X.
GemmPlan plan_gemm(int M, int N, int /*K*/, const DeviceInfo& /*dev*/) {
  GemmPlan p;
  int cfg;
  if (M < 128) {
    cfg = kV3M64N256;
  } else if (M >= 1024) {
    cfg = N >= 8192 ? kV3M128N256 : kV3M128N128;
  } else {
    cfg = N >= 16384 ? kV3M128N256 : kV3M128N128S3;
  }
  p.cfg = cfg;
  p.bm = kGemmTile[cfg][0];
  p.bn = kGemmTile[cfg][1];
  p.tiles_m = (int)ceil_div(M, p.bm);
  p.tiles_n = (int)ceil_div(N, p.bn);
  p.group_m = p.tiles_m < 4 ? p.tiles_m : 4;
  return p;
}

hipError_t launch_gemm(const LinearArgs& a, const GemmPlan& plan, hipStream_t stream) {
  GemmPlan p = plan;
  GemmKernelArgs ka = make_args(a, p);
  // The v3 kernels address a tile with 32-bit offsets from its first row /
  // strip (row stride ldx); fall back to 64-bit addressing when those could
  // overflow.
  if (p.cfg != kDmaM128N128 && !v3_offsets_fit(ka, p.bm, p.bn)) {
    p.cfg = kDmaM128N128;
    p.bm = p.bn = 128;
    p.tiles_m = (int)ceil_div(a.M, 128);
    p.tiles_n = (int)ceil_div(a.N, 128);
    p.group_m = p.tiles_m < 4 ? p.tiles_m : 4;
    ka = make_args(a, p);
  }
  switch (p.cfg) {
    case kV3M128N256: return launch_v3_t<128, 256, 1, 4, 2, 2>(ka, stream);
    case kV3M128N128: return launch_v3_t<128, 128, 1, 4, 2, 3>(ka, stream);
    case kV3M128N128S3: return launch_v3_t<128, 128, 1, 4, 3, 2>(ka, stream);
    case kV3M64N256: return launch_v3_t<64, 256, 1, 4, 3, 2>(ka, stream);
    case kDmaM128N128: return launch_dma_t<128, 128, 1, 4, 3, 1>(ka, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rf
