/*
 * rhinoforge_amd -- W8A16 weight-only quantized linear for MI355X (gfx950).
 *
 * C ABI of the drop-in boundary.  Plain pointers and sizes only: no torch or
 * HIP types appear in the signatures (a HIP stream is passed as `void*`,
 * NULL = the null stream).  Every entry point returns an rf_w8a16_status;
 * nothing is ever silently computed on the CPU.
 *
 * Operation:  y[M,N] = x[M,K] . (s[N] (.) q[N,K])^T (+ b[N])
 *   x, y, s, b : fp16 (IEEE binary16, little-endian), y accumulated in fp32
 *   q          : int8 per-output-channel weights, packed by rf_w8a16_pack_weight
 *
 * Reference interfaces (paths relative to the RhinoForge tree):
 *   - W8A16 launchers: src/ops/rpu_linear.cpp:1047-1209 (tiled GEMM branch,
 *     declared src/core/rpu_kernel_decls.h:1083-1101) and
 *     src/ops/rpu_linear_gemv.cpp:46-202 (llama_gemv_wint8, declared
 *     src/core/rpu_kernel_decls.h:1120-1127);
 *   - weight swizzle: python/rpu_backend/runtime/weights.py:150-233 and its
 *     C++ twin src/ops/rpu_linear.cpp:67-131;
 *   - tile / kernel selection: src/ops/rpu_linear_tiling.h:544-595 and the
 *     M==1 GEMV hand-off src/ops/rpu_linear.cpp:1094-1103.
 */
#ifndef RHINOFORGE_AMD_W8A16_H_
#define RHINOFORGE_AMD_W8A16_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 4: rf_w8a16_plan applies the compute entry points' refusals (EALIGN,
 * EKERNEL) and their GEMV -> GEMM fallback; the torch boundary's packed
 * weight tensors are 3-D tiles [ceil(N/16), ceil(K/64 or 128), 1024]. */
#define RF_W8A16_ABI_VERSION 4

/* Status codes.  The torch op maps each to a RuntimeError with the message
 * from rf_w8a16_status_str (the reference raises TORCH_CHECK before any
 * launch, e.g. src/ops/rpu_linear.cpp:1120-1134). */
typedef enum rf_w8a16_status {
  RF_W8A16_OK = 0,
  RF_W8A16_EINVAL = 1,      /* bad shape, size or null pointer            */
  RF_W8A16_EALIGN = 2,      /* pointer or leading-dimension alignment     */
  RF_W8A16_ELAYOUT = 3,     /* weight layout tag not accepted             */
  RF_W8A16_EWORKSPACE = 4,  /* workspace missing or too small             */
  RF_W8A16_EHIP = 5,        /* HIP runtime error (launch or query)        */
  RF_W8A16_EDEVICE = 6,     /* current device is not gfx950               */
  RF_W8A16_EKERNEL = 7,     /* requested kernel cannot run this shape     */
  RF_W8A16_ESCRATCH = 8     /* shape needs more scratch than the
                               no-allocation entry point holds            */
} rf_w8a16_status;

/* Weight layout tags (the analogue of the reference's `partition` record,
 * python/rpu_backend/runtime/weights.py:33-51, 386-408).
 *
 * RF_W8A16_LAYOUT_ROWMAJOR: q[N,K] int8 row-major, the on-disk checkpoint
 *   format written by quant/convert_qwen3.py:65-100.  Never accepted by the
 *   compute entry point: pack it first.
 * RF_W8A16_LAYOUT_TILE16X64: the CDNA4 tile order.  With Np = ceil(N/16)*16
 *   and Kp = ceil(K/64)*64 the buffer holds Np*Kp bytes as 1024-byte tiles,
 *   tile (nb, kb) at byte offset (nb*(Kp/64) + kb)*1024; inside a tile the
 *   16 bytes at offset 16*l (l = 0..63) are
 *       q[16*nb + l%16][64*kb + 16*(l/16) + j] XOR 0x80,   j = 0..15
 *   (XOR 0x80 stores q+128 as an unsigned byte); padding rows/columns hold
 *   q = 0.  One tile is exactly one wavefront-wide 128-bit load, and the 16
 *   bytes of lane l are that lane's two fp16 MFMA B operands.
 */
#define RF_W8A16_LAYOUT_ROWMAJOR 0
#define RF_W8A16_LAYOUT_TILE16X64 1

/* Kernel choice (the analogue of `force_gemm`, rpu_linear.cpp:1094-1103). */
#define RF_W8A16_KERNEL_AUTO 0
#define RF_W8A16_KERNEL_GEMV 1 /* decode GEMV / skinny GEMM, M <= 64 (AUTO: M <= 16, M <= 24
                                  with N*K < 2^25, M <= 28 with N*K <= 2^24,
                                  M <= 32 with N*K <= 2^23 or N <= 2048 and
                                  N*K <= 2^24; W4A16: M <= 64)                */
#define RF_W8A16_KERNEL_GEMM 2 /* prefill GEMM: x tiles staged in LDS by DMA, int8 weight
                                  tiles dequantized into fp16 MFMA operands (from
                                  registers on the large tiles, from LDS on the others) */

/* Human-readable text for a status code; never NULL. */
const char* rf_w8a16_status_str(int status);

/* ABI version of the loaded library (RF_W8A16_ABI_VERSION). */
int rf_w8a16_abi_version(void);

/* Bytes of a TILE16X64-packed weight for an [N,K] matrix; 0 if N<1 or K<1. */
size_t rf_w8a16_packed_bytes(int64_t N, int64_t K);

/* Host repack: row-major q[N,K] (row stride ldq >= K bytes) -> TILE16X64.
 * Replaces tp_col_swizzle_mc_weight / tp_row_swizzle_mc_weight /
 * transform_linear_weight (runtime/weights.py:150-233; rpu_linear.cpp:67-131).
 * Exact and invertible (see rf_w8a16_unpack_weight). */
int rf_w8a16_pack_weight(const int8_t* q, int64_t N, int64_t K, int64_t ldq,
                         void* dst, size_t dst_bytes);

/* Host inverse of rf_w8a16_pack_weight (tests and checkpoint export). */
int rf_w8a16_unpack_weight(const void* packed, int64_t N, int64_t K,
                           int8_t* q, int64_t ldq);

/* Device repack on `stream`: q_dev row-major in device memory -> dst_dev.
 * Same result as rf_w8a16_pack_weight; used at load time so multi-hundred-MB
 * weights (e.g. a 151936x5120 lm_head) never round-trip through the host. */
int rf_w8a16_pack_weight_device(const int8_t* q_dev, int64_t N, int64_t K,
                                int64_t ldq, void* dst_dev, size_t dst_bytes,
                                void* stream);

/* Kernel the AUTO policy runs for this shape on the current device
 * (RF_W8A16_KERNEL_GEMV or RF_W8A16_KERNEL_GEMM), or a negative status. */
int rf_w8a16_select_kernel(int64_t M, int64_t N, int64_t K);

/* Launch plan of one call (host only, nothing is launched): the analogue of
 * the reference's tile selection select_tile_acc16 / select_tile_acc32
 * (src/ops/rpu_linear_tiling.h:544-595), which maps (M, local_n, local_k) to
 * an (m_tile, n_tile) pair. */
typedef struct rf_w8a16_plan_info {
  int32_t kernel;           /* RF_W8A16_KERNEL_GEMV or RF_W8A16_KERNEL_GEMM */
  int32_t tile_m;           /* activation rows per workgroup (GEMV: 16 per m-tile) */
  int32_t tile_n;           /* output channels per workgroup, per projection */
  int32_t splits;           /* K splits across workgroups (1: no workspace use) */
  int32_t waves;            /* wavefronts per workgroup */
  int32_t workgroups;       /* workgroups of the launch, all splits */
  uint64_t workspace_bytes; /* workspace the launch uses past the counter region */
  char name[48];            /* configuration, e.g. "gemm 128x256 B-in-registers" */
} rf_w8a16_plan_info;

/* Weight formats of rf_w8a16_plan. */
#define RF_W8A16_FORMAT_INT8 0      /* TILE16X64 int8, per-channel scale        */
#define RF_W8A16_FORMAT_INT4 1      /* TILE16X128_I4, per-channel scale          */
#define RF_W8A16_FORMAT_INT4_GROUP 2 /* TILE16X128_I4, group-wise scales        */

/* Plan of a call with `count` projections of widths Ns sharing (M, K) and a
 * contiguous x (ldx = K), for `kernel` (AUTO / GEMV / GEMM) and weight
 * `format`, on a part with `cus` compute units (0: the current device's).
 * The plan is the one the compute entry points run for that call, with the
 * same refusals: RF_W8A16_EINVAL (bad sizes; int4 with N % 16 or K % 64
 * nonzero), RF_W8A16_EALIGN (int8 with K % 8 nonzero), RF_W8A16_EKERNEL
 * (a forced GEMV at M > 64 or at a row stride ldx = K its 32-bit offsets
 * cannot address -- AUTO then plans the GEMM, as the compute entry points
 * run it -- or an int4 GEMM whose tile offsets overflow), else RF_W8A16_OK. */
int rf_w8a16_plan(int64_t M, const int64_t* Ns, int32_t count, int64_t K, int32_t kernel,
                  int32_t format, int32_t cus, rf_w8a16_plan_info* out);

/* Up to this many projections share one rf_w8a16_linear_multi launch. */
#define RF_W8A16_MAX_PROJ 4

/* One projection of rf_w8a16_linear_multi. */
typedef struct rf_w8a16_proj {
  const void* w_packed; /* rf_w8a16_packed_bytes(N, K) bytes, layout TILE16X64 */
  const void* scale;    /* fp16 [N] */
  const void* bias;     /* fp16 [N] or NULL */
  void* y;              /* fp16 [M, ldy], ldy >= N */
  int64_t ldy;
  int64_t N;
} rf_w8a16_proj;

/* Workspace bytes rf_w8a16_linear needs for (M,N,K) with any kernel choice
 * on the current device (fp32 split-K partials of the GEMV or the GEMM).
 * The first RF_W8A16_WS_COUNTER_BYTES bytes are split-K arrival counters:
 * they must be zero before the first call that uses the buffer, and every
 * successful call leaves them zero again.  The bytes after them are scratch. */
size_t rf_w8a16_workspace_bytes(int64_t M, int64_t N, int64_t K);
#define RF_W8A16_WS_COUNTER_BYTES 65536

/* Workspace bytes rf_w8a16_linear_multi needs for `count` projections with
 * output widths Ns[0..count) sharing (M, K); same counter-region contract. */
size_t rf_w8a16_workspace_bytes_multi(int64_t M, const int64_t* Ns, int32_t count, int64_t K);

/* y = x . dequant(w)^T (+ bias), on `stream` (asynchronous).
 *   x        : fp16 [M, ldx], 16-byte aligned, ldx % 8 == 0, ldx >= K
 *   w_packed : rf_w8a16_packed_bytes(N,K) bytes in `layout` (TILE16X64)
 *   scale    : fp16 [N], per-output-channel scale
 *   bias     : fp16 [N] or NULL; added once after the K reduction
 *              (rpu_linear.cpp:279-283, 796-808)
 *   y        : fp16 [M, ldy], ldy >= N
 *   M >= 1, N >= 1, K >= 8, K % 8 == 0
 *   kernel   : RF_W8A16_KERNEL_AUTO / _GEMV / _GEMM.  The GEMV addresses a
 *              16-row span of x with 32-bit offsets: it returns
 *              RF_W8A16_EKERNEL when (min(M,16) - 1) * ldx * 2 + 256 >= 2^32
 *              (AUTO then runs the GEMM, which has a 64-bit-address kernel)
 *   workspace: device buffer of >= rf_w8a16_workspace_bytes(M,N,K) bytes,
 *              counters zeroed as described above; calls that share one
 *              workspace must be ordered (same stream).
 * Replaces rpu_launch_linear_spm_to_spm_acc16_kernel (rpu_linear.cpp:1047)
 * and rpu_launch_gemv_spm_to_spm_kernel (rpu_linear_gemv.cpp:46). */
int rf_w8a16_linear(const void* x, int64_t ldx, const void* w_packed,
                    int32_t layout, const void* scale, const void* bias,
                    void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                    int32_t kernel, void* workspace, size_t workspace_bytes,
                    void* stream);

/* y_i = x . dequant(w_i)^T (+ b_i) for i < count (1..RF_W8A16_MAX_PROJ),
 * all sharing x [M, ldx] and K (same constraints as rf_w8a16_linear).  All
 * projections run in ONE launch of the chosen kernel (GEMV or GEMM), so the
 * launch ramp and the last partial round of workgroups are paid once (q/k/v
 * or gate/up of a decoder layer).  Replaces the fused Q/K/V W8A16
 * launcher `qkv_parallel_w8a16_multibase` (src/ops/rpu_linear.cpp:1546-1674),
 * which runs one launch over three weight and scale bases. */
int rf_w8a16_linear_multi(const void* x, int64_t ldx, int32_t layout, const rf_w8a16_proj* projs,
                          int32_t count, int64_t M, int64_t K, int32_t kernel, void* workspace,
                          size_t workspace_bytes, void* stream);

/* No-allocation variant of rf_w8a16_linear_multi.  It has no counterpart in
 * the reference: it is for callers that cannot allocate device memory --
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  Same arguments and results as rf_w8a16_linear_multi without
 * the workspace: the split-K counters and fp32 partials of both kernels live
 * in a library-owned device array of RF_W8A16_NOALLOC_SCRATCH_BYTES bytes per
 * GPU (its first RF_W8A16_WS_COUNTER_BYTES bytes the counters), looked up on
 * the first call on each device and held until the process ends.  It
 * allocates nothing and calls no allocating routine.
 *   - A shape whose plan needs more scratch returns RF_W8A16_ESCRATCH before
 *     any launch (e.g. K-split prefill launches of hundreds of 128x128
 *     tiles); rf_w8a16_linear_multi with a workspace runs those.
 *   - Every call on one GPU shares that GPU's array.  Calls that overlap in
 *     time on one GPU (two streams, two host threads, two graphs replayed
 *     concurrently) race and must be ordered by the caller.
 *   - The counters start at zero (the array is zero-initialized when the
 *     library's code object loads; a first call on a device outside graph
 *     capture also clears them with a fill kernel on its stream) and every
 *     call leaves them zero.  A first call under graph capture records no
 *     fill, so replays never reset counters other calls rely on. */
#define RF_W8A16_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int rf_w8a16_linear_multi_noalloc(const void* x, int64_t ldx, int32_t layout,
                                  const rf_w8a16_proj* projs, int32_t count, int64_t M, int64_t K,
                                  int32_t kernel, void* stream);

/* Greedy-decode lm_head: index[m] = argmax_n fp16(y[m][n]) of
 * y = x . dequant(w)^T (+ bias), int32, the lowest n among equal maxima (NaN
 * counts as the largest value, -0 equals +0), for 1 <= M <= 64 (the decode
 * GEMV).  The per-row argmax is folded into the GEMV epilogue, so the
 * logits need not be written or read again; `y` (fp16 [M, ldy], ldy >= N)
 * may be NULL, otherwise the logits are stored as by rf_w8a16_linear.
 *   workspace: >= rf_w8a16_workspace_bytes_argmax(M,N,K) bytes, counter
 *              region zeroed as for rf_w8a16_linear.  Two launches: the GEMV
 *              leaves each workgroup's best per-row key in the workspace, a
 *              second kernel reduces them.
 * Other arguments as rf_w8a16_linear.  Returns RF_W8A16_EKERNEL for M > 64
 * and for row strides the GEMV cannot address (see rf_w8a16_linear).
 * Replaces the decode lm_head GEMM + argmax pair (src/fused/rpu_qwen3_model.h:
 * 3653-3690 writes the logits; src/ops/rpu_argmax.cpp:485-640 reduces them,
 * int32 result, first index among ties). */
int rf_w8a16_linear_argmax(const void* x, int64_t ldx, const void* w_packed, int32_t layout,
                           const void* scale, const void* bias, void* y, int64_t ldy,
                           int32_t* index, int64_t M, int64_t N, int64_t K, void* workspace,
                           size_t workspace_bytes, void* stream);
size_t rf_w8a16_workspace_bytes_argmax(int64_t M, int64_t N, int64_t K);

/* ---------------------------------------------------------------------------
 * W4A16: packed int4 weights, per-channel or group-wise fp16 scales, on the
 * same two kernel families.  Replaces the reference's packed-int4 branch of
 * the launcher (src/ops/rpu_linear.cpp:1211-1489: a uint8 [N, K/2] weight;
 * a 1-D scale [N] selects per-channel, a 2-D scale the group-wise "pgrp"
 * family) and its packers (python/rpu_backend/quant/int4_pack.py:21-58,
 * int4_pgrp_pack.py:33-162).
 *
 * Operation:  y[M,N] = x[M,K] . W^T (+ b[N]), fp32 accumulation, with
 *   per-channel (group_size 0):  W[n][k] = s[n] * q[n][k]   (s applied to the
 *                                fp32 sum, as in the int8 path)
 *   group-wise (32, 64 or 128):  W[n][k] = RN_fp16(s[k / group_size][n] * q[n][k])
 *                                (the reference's fp16 dequantization,
 *                                int4_pgrp_pack.py:63-70)
 *   q[n][k] in [-8, 7] (int8 containers, quant/int4_pgrp_pack.py:33-60);
 *   s fp16: [N], or [K/group_size][N] row-major (N contiguous) -- the logical
 *   scale of int4_pgrp_pack.py:59, not the RPU's controller-striped payload.
 *
 * Shape rules, as the reference's int4 packers require (int4_pack.py:31-40,
 * convert_qwen3_w4a16.py:65-76): N % 16 == 0, K % 64 == 0, and
 * K % group_size == 0.
 *
 * RF_W8A16_LAYOUT_TILE16X128_I4: with Np = ceil(N/16)*16 and
 *   Kp = ceil(K/128)*128 the buffer holds Np*Kp/2 bytes as 1024-byte tiles of
 *   16 channels x 128 positions, tile (nb, kt) at byte offset
 *   (nb*(Kp/128) + kt)*1024.  The 16 bytes at offset 16*l hold channel
 *   16*nb + l%16, positions 128*kt + 32*(l/16) + 8*j + i (dword j = 0..3 of
 *   the 16 bytes, i = 0..7); position i of a dword sits in nibble i/2 if i is
 *   even and nibble 4 + i/2 if odd, as u = q + 8 (0..15).  Padding holds
 *   q = 0.  Lane l of a wavefront loads exactly its four MFMA operands. */
#define RF_W8A16_LAYOUT_TILE16X128_I4 2

/* Bytes of a packed int4 weight (0 on bad sizes). */
size_t rf_w4a16_packed_bytes(int64_t N, int64_t K);
/* Host pack of q[N,K] (row stride ldq, values in [-8, 7]; others: EINVAL). */
int rf_w4a16_pack_weight(const int8_t* q, int64_t N, int64_t K, int64_t ldq, void* dst,
                         size_t dst_bytes);
/* Inverse of rf_w4a16_pack_weight (host). */
int rf_w4a16_unpack_weight(const void* packed, int64_t N, int64_t K, int8_t* q, int64_t ldq);
/* Device pack (device pointers, async on `stream`); values are taken mod 16
 * as two's-complement nibbles, so only [-8, 7] round-trips. */
int rf_w4a16_pack_weight_device(const int8_t* q_dev, int64_t N, int64_t K, int64_t ldq,
                                void* dst_dev, size_t dst_bytes, void* stream);
/* Workspace a W4A16 call needs (counter region + split-K partials). */
size_t rf_w4a16_workspace_bytes(int64_t M, int64_t N, int64_t K);
/* Workspace of rf_w4a16_linear_multi for `count` projections of widths Ns. */
size_t rf_w4a16_workspace_bytes_multi(int64_t M, const int64_t* Ns, int32_t count, int64_t K);
/* y = x . W^T (+ b) with a TILE16X128_I4 weight.  group_size: 0 (per-channel
 * scale [N]) or 32 / 64 / 128 (scale [K/group_size][N], 16-byte aligned).
 * kernel, workspace and stream as for rf_w8a16_linear; the int4 GEMM has no
 * 64-bit-address kernel and returns RF_W8A16_EKERNEL where a tile's rows
 * (up to 128 rows of ldx halves) span 4 GB or more. */
int rf_w4a16_linear(const void* x, int64_t ldx, const void* w_packed, const void* scale,
                    int32_t group_size, const void* bias, void* y, int64_t ldy, int64_t M,
                    int64_t N, int64_t K, int32_t kernel, void* workspace, size_t workspace_bytes,
                    void* stream);
/* y_i = x . W_i^T (+ b_i) for i < count (1..RF_W8A16_MAX_PROJ) TILE16X128_I4
 * weights sharing x [M, ldx], K and group_size, in ONE launch of the chosen
 * kernel (q/k/v or gate/up of a decoder layer), as rf_w8a16_linear_multi
 * does for int8.  projs[i].w_packed is the packed int4 weight and
 * projs[i].scale its scale ([N_i], or [K/group_size][N_i], 16-byte aligned);
 * every N_i % 16 == 0.  The reference has no fused int4 launcher: its
 * packed-int4 branch (src/ops/rpu_linear.cpp:1211-1489) runs one weight per
 * call; this is the int4 form of its fused Q/K/V W8A16 launcher
 * (rpu_linear.cpp:1546-1674). */
int rf_w4a16_linear_multi(const void* x, int64_t ldx, const rf_w8a16_proj* projs, int32_t count,
                          int32_t group_size, int64_t M, int64_t K, int32_t kernel,
                          void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* RHINOFORGE_AMD_W8A16_H_ */
