// Prefill GEMM for W8A16 (gfx950): LDS-staged INT8 weight tiles dequantized
// into fp16 MFMA operands, fp32 accumulation.
//
// Workgroup tile BM x BN x 64 (K), 256 threads = 2 x 2 wavefronts, each
// wavefront owns a (BM/2) x (BN/2) block of 16x16 MFMA accumulators.
//   * A (activations, fp16) is staged row-major in LDS with a 144-byte row
//     pitch, so the 16 rows read by one 16-lane group land on distinct banks;
//   * B (weights) is staged in LDS still as INT8 (half the LDS bytes and
//     half the global->LDS traffic of an fp16 tile): the TILE16X64 tiles are
//     copied verbatim, and each lane's 16 bytes are exactly its two MFMA B
//     operands, dequantized in registers right before the MFMAs;
//   * double-buffered: the next K step's global loads are issued before the
//     current step's MFMAs and written to the other LDS buffer afterwards;
//   * the per-channel scale and bias are applied in the fp32 epilogue.
#include "w8a16_common.h"
#include "w8a16_internal.h"

namespace rf {
namespace {

constexpr int kThreads = 256;
constexpr int kApitch = 72;  // halves per A row in LDS (64 + 8 pad)

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
  int tiles_n;
};

template <int BM, int BN>
__global__ __launch_bounds__(kThreads) void w8a16_gemm_kernel(GemmKernelArgs a) {
  constexpr int WM = BM / 2, WN = BN / 2;       // wavefront tile
  constexpr int TM = WM / 16, TN = WN / 16;     // MFMA tiles per wavefront
  constexpr int A_CHUNKS = BM * 8 / kThreads;   // 16-byte chunks of A per thread
  constexpr int B_TILES = BN / 16;
  constexpr int B_CHUNKS = B_TILES * 64 / kThreads;
  static_assert(A_CHUNKS >= 1 && B_CHUNKS >= 1, "tile too small for 256 threads");

  __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * kApitch];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[2][B_TILES * kTileBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tile_m = blockIdx.x / a.tiles_n;
  const int tile_n = blockIdx.x % a.tiles_n;
  const int m0 = tile_m * BM;
  const int strip0 = tile_n * B_TILES;

  uint4 areg[A_CHUNKS], breg[B_CHUNKS];

  auto gload = [&](int kb) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int c = tid + kThreads * i;
      const int row = c >> 3, col = (c & 7) * 8;
      const int m = m0 + row, k = kb * 64 + col;
      areg[i] = (m < a.M && k < a.K) ? load_u4(a.x + (int64_t)m * a.ldx + k) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      const int c = tid + kThreads * i;
      const int t = c >> 6, l = c & 63;
      const int strip = strip0 + t;
      breg[i] = strip < a.nstrips
                    ? load_u4_stream(a.w + ((int64_t)strip * a.kblocks + kb) * kTileBytes + l * 16)
                    : make_uint4(0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int c = tid + kThreads * i;
      const int row = c >> 3, col = (c & 7) * 8;
      *reinterpret_cast<uint4*>(&As[buf][row * kApitch + col]) = areg[i];
    }
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      const int c = tid + kThreads * i;
      *reinterpret_cast<uint4*>(&Bs[buf][c * 16]) = breg[i];
    }
  };

  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  gload(0);
  sstore(0);
  __syncthreads();

  const int arow = wm * WM + (lane & 15);
  const int acol = 16 * (lane >> 4);
  for (int kb = 0; kb < a.kblocks; ++kb) {
    const int buf = kb & 1;
    const bool more = kb + 1 < a.kblocks;
    if (more) gload(kb + 1);

    half8 bf[TN][2];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const uint4 v = *reinterpret_cast<const uint4*>(&Bs[buf][(wn * TN + j) * kTileBytes + lane * 16]);
      bf[j][0] = dequant8(v.x, v.y);
      bf[j][1] = dequant8(v.z, v.w);
    }
#pragma unroll
    for (int step = 0; step < 2; ++step) {
      half8 af[TM];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const half8*>(&As[buf][(arow + 16 * i) * kApitch + acol + 8 * step]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32(af[i], bf[j][step], acc[i][j]);
    }

    if (more) {
      sstore(buf ^ 1);
      __syncthreads();
    }
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

}  // namespace

GemmPlan plan_gemm(int M, int N, int /*K*/, const DeviceInfo& /*dev*/) {
  GemmPlan p;
  p.bm = 128;
  p.bn = 128;
  p.tiles_m = (int)ceil_div(M, p.bm);
  p.tiles_n = (int)ceil_div(N, p.bn);
  return p;
}

hipError_t launch_gemm(const LinearArgs& a, const GemmPlan& p, hipStream_t stream) {
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
  ka.tiles_n = p.tiles_n;
  const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n;
  if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidValue;
  if (p.bm == 128 && p.bn == 128) {
    hipLaunchKernelGGL((w8a16_gemm_kernel<128, 128>), dim3((unsigned)blocks), dim3(kThreads), 0,
                       stream, ka);
    return hipGetLastError();
  }
  return hipErrorInvalidValue;
}

}  // namespace rf
