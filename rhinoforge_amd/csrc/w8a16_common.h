// Device-side building blocks shared by the W8A16 kernels (gfx950 / CDNA4).
//
// Weight tiles use the TILE16X64 layout declared in include/w8a16.h: one
// 1024-byte tile = 16 output channels x 64 input channels, lane l of a
// wavefront owns the 16 bytes at offset 16*l, holding q+128 for channel
// l%16 and input positions 16*(l/16) .. 16*(l/16)+15 of the tile.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rf {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kTileN = 16;       // output channels per tile
constexpr int kTileK = 64;       // input channels per tile
constexpr int kTileBytes = 1024; // kTileN * kTileK
constexpr int kWave = 64;

// Exact int8 -> fp16 for the four bytes of `d` (each byte u = q + 128).
//
// v_perm_b32 places each byte u under the fp16 exponent byte 0x64, giving
// the fp16 number 1024 + u (exact: integers up to 2048 are representable);
// one packed fp16 subtraction of 1152 = 1024 + 128 then yields q exactly.
// This is the "magic number" conversion (Kim et al. 2022, "Who says
// elephants can't run", int8 -> fp16 via exponent bias), written for
// v_perm_b32 + v_pk_add_f16.  Four VALU ops per four weights.
__device__ __forceinline__ half4 dequant4(uint32_t d) {
  const uint32_t exp_bytes = 0x64646464u;
  // perm selector bytes: 0..3 pick bytes of `d`, 4..7 pick bytes of exp_bytes
  const uint32_t lo = __builtin_amdgcn_perm(exp_bytes, d, 0x04010400u);  // [u0 | 0x64, u1 | 0x64]
  const uint32_t hi = __builtin_amdgcn_perm(exp_bytes, d, 0x04030402u);  // [u2 | 0x64, u3 | 0x64]
  const half2v off = {(_Float16)1152.0f, (_Float16)1152.0f};
  const half2v a = __builtin_bit_cast(half2v, lo) - off;
  const half2v b = __builtin_bit_cast(half2v, hi) - off;
  return __builtin_shufflevector(a, b, 0, 1, 2, 3);
}

// Eight weights (two dwords, in memory order) -> one fp16 MFMA operand.
__device__ __forceinline__ half8 dequant8(uint32_t d0, uint32_t d1) {
  return __builtin_shufflevector(dequant4(d0), dequant4(d1), 0, 1, 2, 3, 4, 5, 6, 7);
}

// Packed int4 (TILE16X128_I4, include/w8a16.h): one tile = 16 output
// channels x 128 input channels in 1024 bytes; lane l owns the 16 bytes at
// 16*l: channel l%16, input positions 32*(l/16) .. +31 of the tile, as four
// dwords of eight positions each.  Within a dword, nibble p (bits 4p..4p+3)
// holds position 2p (p < 4) or 2(p-4)+1 (p >= 4), stored as u = q + 8.
constexpr int kTileK4 = 128;

// (a & m) | c in one VALU op.  CDNA3/4 VOP3 encodings take no literal
// constants, so without this the compiler splits it into v_and + v_or.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(c));
  return r;
}

// Exact int4 -> fp16 of one dword (eight positions, in position order), with
// the magic-number conversion (Kim et al. 2022) applied to two nibbles per
// fp16 pair:
//   (d & 0x000F000F) | 0x64006400  = (1024 + u_lo, 1024 + u_hi) for nibbles
//                                    p, p+4 at bits 0..3 of each half;
//   (d & 0x00F000F0) | 0x64006400  = (1024 + 16 u, ...) for nibbles p+1, p+5;
// subtracting 1032, or scaling by 1/16 and subtracting 72 (one fused op:
// 64 + u - 72, all exact in fp16), gives q = u - 8; d >> 8 repeats this for
// nibbles 2, 6 and 3, 7.  Nine VALU ops per eight weights.
__device__ __forceinline__ half8 dequant8_i4(uint32_t d) {
  const uint32_t e = 0x64006400u;
  const uint32_t lo = and_or(d, 0x000F000Fu, e), hi = and_or(d, 0x00F000F0u, e);
  const uint32_t d8 = d >> 8;
  const uint32_t lo8 = and_or(d8, 0x000F000Fu, e), hi8 = and_or(d8, 0x00F000F0u, e);
  const half2v off = {(_Float16)1032.0f, (_Float16)1032.0f};
  const half2v k16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  const half2v b72 = {(_Float16)-72.0f, (_Float16)-72.0f};
  const half2v p0 = __builtin_bit_cast(half2v, lo) - off;                             // 0, 1
  const half2v p1 = __builtin_elementwise_fma(__builtin_bit_cast(half2v, hi), k16, b72);  // 2, 3
  const half2v p2 = __builtin_bit_cast(half2v, lo8) - off;                            // 4, 5
  const half2v p3 = __builtin_elementwise_fma(__builtin_bit_cast(half2v, hi8), k16, b72); // 6, 7
  return __builtin_shufflevector(__builtin_shufflevector(p0, p1, 0, 1, 2, 3),
                                 __builtin_shufflevector(p2, p3, 0, 1, 2, 3), 0, 1, 2, 3, 4, 5,
                                 6, 7);
}

// The same with a group scale applied: RN_fp16(q * s) per weight (the
// product of an integer |q| <= 8 and an fp16 scale, rounded once, as the
// reference's fp16 dequantization computes it).
__device__ __forceinline__ half8 dequant8_i4_scaled(uint32_t d, _Float16 s) {
  const half8 sv = {s, s, s, s, s, s, s, s};
  return dequant8_i4(d) * sv;
}

// Weight formats of a launch: the kernels are templated on it.
enum WeightFormat : int {
  kWfInt8 = 0,     // TILE16X64, per-channel scale [N] (epilogue)
  kWfInt4 = 1,     // TILE16X128_I4, per-channel scale [N] (epilogue)
  kWfInt4Grp = 2,  // TILE16X128_I4, group scale [K/gs][N] applied at dequant
};

// D(16x16, fp32) += A(16x32, fp16) * B(32x16, fp16).
// Lane l supplies A row l%16 and B column l%16, each for the 8 K positions
// of k-group l/16; the product pairs A and B slots with the same (group,
// slot), so any consistent K assignment of the operands gives the same sum.
// Result: lane l, element r holds D[4*(l/16) + r][l%16].
__device__ __forceinline__ floatx4 mfma16x16x32(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint4 load_u4(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}

// Streaming (read-once) 128-bit load: weights are touched exactly once per
// call, so they are marked non-temporal to keep L2 for activations/partials.
__device__ __forceinline__ uint4 load_u4_stream(const void* p) {
  const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(q));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

typedef __attribute__((address_space(3))) uint8_t lds_u8;

// One global_load_lds_dwordx4: every lane reads 16 bytes at `g`, the
// wavefront's 64 x 16 bytes land lane-contiguously at LDS byte address
// `lds` (wave-uniform, passed in M0).  Written as inline asm so the
// compiler does not serialise every later LDS read behind it (it cannot
// tell which LDS bytes a DMA writes); the kernels order the LDS traffic
// themselves with explicit s_waitcnt vmcnt + s_barrier.  Nothing else in
// these kernels uses M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Workgroup barrier without the memory fences __syncthreads() implies (a
// release fence would wait for every DMA in flight).  The caller has
// already waited for the loads whose data the other wavefronts read.
__device__ __forceinline__ void barrier_lds() {
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}


__device__ __forceinline__ half8 as_half8(uint4 v) {
  return __builtin_bit_cast(half8, v);
}

}  // namespace rf
