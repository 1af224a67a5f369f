// Host-side checks of the C ABI, built with AddressSanitizer and
// UndefinedBehaviorSanitizer on the host code by tests/test_host_sanitizers.py:
// every entry point that runs on the host without a GPU, over edge shapes,
// exact-size buffers (an overrun by one byte trips ASan) and refusals.
// Nothing here launches a kernel or passes a host pointer to a compute entry
// point that could reach the device: the refusals used are the ones taken
// before any device query.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "w8a16.h"

static int failures = 0;
#define CHECK(cond)                                                            \
  do {                                                                         \
    if (!(cond)) {                                                             \
      std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);             \
      ++failures;                                                              \
    }                                                                          \
  } while (0)

// int8 TILE16X64: pack then unpack into a row stride wider than K; the
// columns past K must keep their sentinel.
static void int8_round_trip(std::mt19937& rng, int64_t N, int64_t K, int64_t pad) {
  const int64_t ldq = K + pad;
  std::vector<int8_t> q((size_t)(N * ldq));
  for (auto& v : q) v = (int8_t)(rng() & 0xff);
  const size_t bytes = rf_w8a16_packed_bytes(N, K);
  CHECK(bytes == (size_t)((N + 15) / 16 * 16) * (size_t)((K + 63) / 64 * 64));
  std::vector<uint8_t> packed(bytes);
  CHECK(rf_w8a16_pack_weight(q.data(), N, K, ldq, packed.data(), bytes) == RF_W8A16_OK);
  CHECK(rf_w8a16_pack_weight(q.data(), N, K, ldq, packed.data(), bytes - 1) == RF_W8A16_EINVAL);
  std::vector<int8_t> back((size_t)(N * ldq), (int8_t)0x5a);
  CHECK(rf_w8a16_unpack_weight(packed.data(), N, K, back.data(), ldq) == RF_W8A16_OK);
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < ldq; ++k)
      CHECK(back[n * ldq + k] == (k < K ? q[n * ldq + k] : (int8_t)0x5a));
}

// int4 TILE16X128_I4: values in [-8, 7] round-trip; one value outside is
// refused before anything is written.
static void int4_round_trip(std::mt19937& rng, int64_t N, int64_t K) {
  std::vector<int8_t> q((size_t)(N * K));
  for (auto& v : q) v = (int8_t)((int)(rng() % 16) - 8);
  const size_t bytes = rf_w4a16_packed_bytes(N, K);
  CHECK(bytes == (size_t)((N + 15) / 16 * 16) * (size_t)((K + 127) / 128 * 128) / 2);
  std::vector<uint8_t> packed(bytes, 0xa5);
  CHECK(rf_w4a16_pack_weight(q.data(), N, K, K, packed.data(), bytes) == RF_W8A16_OK);
  std::vector<int8_t> back((size_t)(N * K));
  CHECK(rf_w4a16_unpack_weight(packed.data(), N, K, back.data(), K) == RF_W8A16_OK);
  CHECK(back == q);
  std::vector<uint8_t> untouched(bytes, 0x3c);
  q[(size_t)(N * K / 2)] = 8;
  CHECK(rf_w4a16_pack_weight(q.data(), N, K, K, untouched.data(), bytes) == RF_W8A16_EINVAL);
  for (uint8_t b : untouched) CHECK(b == 0x3c);
}

// rf_w8a16_plan over a grid of shapes, formats and CU counts (no device
// query when cus > 0): every plan is consistent and its name terminated.
static void plans() {
  const int64_t Ms[] = {1, 2, 3, 4, 5, 8, 9, 12, 13, 16, 17, 24, 28, 32, 33, 48, 64, 65, 128,
                        200, 512, 1024, 2048, 4096};
  const int64_t Ks[] = {8, 64, 1000, 1024, 4096, 5120, 12288, 25600};
  const int64_t Nsets[][4] = {{16, 0, 0, 0},          {1000, 0, 0, 0},      {4096, 1024, 1024, 0},
                              {12288, 12288, 0, 0},   {151936, 0, 0, 0},    {9000, 9000, 9000, 0},
                              {25600, 25600, 0, 0},   {16, 32, 48, 64},     {8200, 0, 0, 0}};
  const int32_t cuss[] = {256, 80, 304};
  int checked = 0;
  for (int64_t M : Ms)
    for (int64_t K : Ks)
      for (const auto& set : Nsets) {
        int32_t count = 0;
        while (count < 4 && set[count] > 0) ++count;
        for (int32_t cus : cuss)
          for (int32_t kernel : {RF_W8A16_KERNEL_AUTO, RF_W8A16_KERNEL_GEMV, RF_W8A16_KERNEL_GEMM})
            for (int32_t fmt : {RF_W8A16_FORMAT_INT8, RF_W8A16_FORMAT_INT4, RF_W8A16_FORMAT_INT4_GROUP}) {
              rf_w8a16_plan_info info;
              std::memset(&info, 0x77, sizeof(info));
              const int st = rf_w8a16_plan(M, set, count, K, kernel, fmt, cus, &info);
              // int4 packing needs N % 16 == 0 and K % 64 == 0 (rf_w4a16_linear[_multi])
              bool n16 = true;
              for (int32_t i = 0; i < count; ++i) n16 = n16 && set[i] % 16 == 0;
              if (fmt != RF_W8A16_FORMAT_INT8 && (!n16 || K % 64 != 0)) {
                CHECK(st == RF_W8A16_EINVAL);
                continue;
              }
              if (kernel == RF_W8A16_KERNEL_GEMV && M > 64) {
                CHECK(st == RF_W8A16_EKERNEL);
                continue;
              }
              CHECK(st == RF_W8A16_OK);
              if (st != RF_W8A16_OK) continue;
              CHECK(info.kernel == RF_W8A16_KERNEL_GEMV || info.kernel == RF_W8A16_KERNEL_GEMM);
              CHECK(info.tile_m >= 16 && info.tile_n >= 16 && info.splits >= 1);
              CHECK(info.workgroups >= 1 && info.waves >= 1);
              CHECK((info.splits > 1) == (info.workspace_bytes > 0));
              CHECK(std::memchr(info.name, 0, sizeof(info.name)) != nullptr);
              ++checked;
            }
      }
  CHECK(checked > 1000);
  // the compute entry points' other refusals and fallbacks, at ldx = K
  {
    rf_w8a16_plan_info info;
    const int64_t n64 = 64;
    // GEMV offsets over 16 rows of x overflow 32 bits: AUTO plans the GEMM,
    // a forced GEMV is refused
    const int64_t kgemv = (int64_t)1 << 28;  // 15 rows * 2^28 * 2 bytes > 2^32
    CHECK(rf_w8a16_plan(16, &n64, 1, kgemv, RF_W8A16_KERNEL_AUTO, RF_W8A16_FORMAT_INT8, 256, &info) ==
          RF_W8A16_OK);
    CHECK(info.kernel == RF_W8A16_KERNEL_GEMM);
    CHECK(rf_w8a16_plan(16, &n64, 1, kgemv, RF_W8A16_KERNEL_GEMV, RF_W8A16_FORMAT_INT8, 256, &info) ==
          RF_W8A16_EKERNEL);
    // ... which fits at M = 1 (no row offsets) and at M = 16 with K = 2^27
    CHECK(rf_w8a16_plan(1, &n64, 1, kgemv, RF_W8A16_KERNEL_AUTO, RF_W8A16_FORMAT_INT8, 256, &info) ==
          RF_W8A16_OK);
    CHECK(info.kernel == RF_W8A16_KERNEL_GEMV);
    const int64_t kbig = (int64_t)1 << 27;
    CHECK(rf_w8a16_plan(16, &n64, 1, kbig, RF_W8A16_KERNEL_AUTO, RF_W8A16_FORMAT_INT8, 256, &info) ==
          RF_W8A16_OK);
    CHECK(info.kernel == RF_W8A16_KERNEL_GEMV);
    // int8 GEMM tile offsets overflow (128 rows * 2^27 * 2 bytes): the
    // 64-bit-address kernel, unsplit
    CHECK(rf_w8a16_plan(2048, &n64, 1, kbig, RF_W8A16_KERNEL_GEMM, RF_W8A16_FORMAT_INT8, 256, &info) ==
          RF_W8A16_OK);
    CHECK(std::strstr(info.name, "64-bit") != nullptr && info.splits == 1);
    // int4 has no such kernel: refused
    CHECK(rf_w8a16_plan(2048, &n64, 1, kbig, RF_W8A16_KERNEL_GEMM, RF_W8A16_FORMAT_INT4, 256, &info) ==
          RF_W8A16_EKERNEL);
    // int8 K % 8 != 0: EALIGN, as rf_w8a16_linear; int4 N % 16 / K % 64: EINVAL
    CHECK(rf_w8a16_plan(1, &n64, 1, 100, RF_W8A16_KERNEL_AUTO, RF_W8A16_FORMAT_INT8, 256, &info) ==
          RF_W8A16_EALIGN);
    const int64_t n40 = 40;
    CHECK(rf_w8a16_plan(1, &n40, 1, 128, RF_W8A16_KERNEL_AUTO, RF_W8A16_FORMAT_INT4, 256, &info) ==
          RF_W8A16_EINVAL);
    CHECK(rf_w8a16_plan(1, &n64, 1, 96, RF_W8A16_KERNEL_AUTO, RF_W8A16_FORMAT_INT4_GROUP, 256, &info) ==
          RF_W8A16_EINVAL);
  }
  // refusals
  rf_w8a16_plan_info info;
  const int64_t n1 = 64, n0 = 0;
  CHECK(rf_w8a16_plan(1, &n1, 1, 64, RF_W8A16_KERNEL_AUTO, RF_W8A16_FORMAT_INT8, 256, nullptr) == RF_W8A16_EINVAL);
  CHECK(rf_w8a16_plan(1, nullptr, 1, 64, RF_W8A16_KERNEL_AUTO, RF_W8A16_FORMAT_INT8, 256, &info) == RF_W8A16_EINVAL);
  CHECK(rf_w8a16_plan(1, &n0, 1, 64, RF_W8A16_KERNEL_AUTO, RF_W8A16_FORMAT_INT8, 256, &info) == RF_W8A16_EINVAL);
  CHECK(rf_w8a16_plan(0, &n1, 1, 64, RF_W8A16_KERNEL_AUTO, RF_W8A16_FORMAT_INT8, 256, &info) == RF_W8A16_EINVAL);
  CHECK(rf_w8a16_plan(1, &n1, 5, 64, RF_W8A16_KERNEL_AUTO, RF_W8A16_FORMAT_INT8, 256, &info) == RF_W8A16_EINVAL);
  CHECK(rf_w8a16_plan(1, &n1, 1, 64, 7, RF_W8A16_FORMAT_INT8, 256, &info) == RF_W8A16_EINVAL);
  CHECK(rf_w8a16_plan(1, &n1, 1, 64, RF_W8A16_KERNEL_AUTO, 9, 256, &info) == RF_W8A16_EINVAL);
}

// Refusals the compute entry points take before any device query.
static void refusals() {
  alignas(16) static uint16_t x[64], y[64], scale[64];
  alignas(16) static uint8_t w[1024];
  rf_w8a16_proj p{w, scale, nullptr, y, 64, 64};
  CHECK(rf_w8a16_linear_multi(nullptr, 64, RF_W8A16_LAYOUT_TILE16X64, &p, 1, 1, 64,
                              RF_W8A16_KERNEL_AUTO, nullptr, 0, nullptr) == RF_W8A16_EINVAL);
  CHECK(rf_w8a16_linear_multi(x, 32, RF_W8A16_LAYOUT_TILE16X64, &p, 1, 1, 64,  // ldx < K
                              RF_W8A16_KERNEL_AUTO, nullptr, 0, nullptr) == RF_W8A16_EINVAL);
  CHECK(rf_w8a16_linear_multi(x, 64, 12345, &p, 1, 1, 64, RF_W8A16_KERNEL_AUTO, nullptr, 0,
                              nullptr) == RF_W8A16_ELAYOUT);
  CHECK(rf_w8a16_linear_multi(x, 64, RF_W8A16_LAYOUT_TILE16X64, &p, 0, 1, 64,
                              RF_W8A16_KERNEL_AUTO, nullptr, 0, nullptr) == RF_W8A16_EINVAL);
  CHECK(rf_w8a16_linear_multi(x, 64, RF_W8A16_LAYOUT_TILE16X64, &p, 1, 1, 60,  // K % 8
                              RF_W8A16_KERNEL_AUTO, nullptr, 0, nullptr) == RF_W8A16_EALIGN);
  CHECK(rf_w8a16_linear_multi(reinterpret_cast<uint8_t*>(x) + 2, 64, RF_W8A16_LAYOUT_TILE16X64, &p,
                              1, 1, 64, RF_W8A16_KERNEL_AUTO, nullptr, 0, nullptr) == RF_W8A16_EALIGN);
  rf_w8a16_proj bad = p;
  bad.ldy = 32;  // ldy < N
  CHECK(rf_w8a16_linear_multi(x, 64, RF_W8A16_LAYOUT_TILE16X64, &bad, 1, 1, 64,
                              RF_W8A16_KERNEL_AUTO, nullptr, 0, nullptr) == RF_W8A16_EINVAL);
  CHECK(rf_w8a16_linear(x, 64, w, RF_W8A16_LAYOUT_TILE16X64, scale, nullptr, y, 64, 0, 64, 64,
                        RF_W8A16_KERNEL_AUTO, nullptr, 0, nullptr) == RF_W8A16_EINVAL);
  CHECK(rf_w4a16_linear(x, 64, w, scale, 48, nullptr, y, 64, 1, 64, 64, RF_W8A16_KERNEL_AUTO,
                        nullptr, 0, nullptr) == RF_W8A16_EINVAL);  // group size
  CHECK(rf_w4a16_linear(x, 64, w, scale, 0, nullptr, y, 64, 1, 40, 64, RF_W8A16_KERNEL_AUTO,
                        nullptr, 0, nullptr) == RF_W8A16_EINVAL);  // N % 16
  CHECK(rf_w8a16_linear_argmax(x, 64, w, RF_W8A16_LAYOUT_TILE16X64, scale, nullptr, y, 64,
                               nullptr, 1, 64, 64, nullptr, 0, nullptr) == RF_W8A16_EINVAL);
  // the fused int4 launch: the same refusals per projection, before any device query
  rf_w8a16_proj p4[2] = {p, p};
  CHECK(rf_w4a16_linear_multi(x, 64, p4, 2, 48, 1, 64, RF_W8A16_KERNEL_AUTO, nullptr, 0,
                              nullptr) == RF_W8A16_EINVAL);  // group size
  p4[1].N = 40;
  CHECK(rf_w4a16_linear_multi(x, 64, p4, 2, 0, 1, 64, RF_W8A16_KERNEL_AUTO, nullptr, 0,
                              nullptr) == RF_W8A16_EINVAL);  // N % 16 on the second projection
  p4[1] = p;
  CHECK(rf_w4a16_linear_multi(x, 64, p4, 5, 0, 1, 64, RF_W8A16_KERNEL_AUTO, nullptr, 0,
                              nullptr) == RF_W8A16_EINVAL);  // count
  CHECK(rf_w4a16_linear_multi(x, 64, p4, 2, 0, 1, 96, RF_W8A16_KERNEL_AUTO, nullptr, 0,
                              nullptr) == RF_W8A16_EINVAL);  // K % 64
  p4[1].scale = reinterpret_cast<uint8_t*>(scale) + 2;
  CHECK(rf_w4a16_linear_multi(x, 64, p4, 2, 32, 1, 64, RF_W8A16_KERNEL_AUTO, nullptr, 0,
                              nullptr) == RF_W8A16_EALIGN);  // group-wise scale 16-byte aligned
  const int64_t ns4[2] = {64, 32};
  CHECK(rf_w4a16_workspace_bytes_multi(1, ns4, 2, 64) >= RF_W8A16_WS_COUNTER_BYTES);
  CHECK(rf_w4a16_workspace_bytes_multi(1, ns4, 0, 64) == 0);
  int8_t q[64];
  std::memset(q, 0, sizeof(q));
  CHECK(rf_w8a16_pack_weight(q, 0, 64, 64, w, sizeof(w)) == RF_W8A16_EINVAL);
  CHECK(rf_w8a16_pack_weight(q, 1, 64, 32, w, sizeof(w)) == RF_W8A16_EINVAL);
  CHECK(rf_w8a16_pack_weight(nullptr, 1, 64, 64, w, sizeof(w)) == RF_W8A16_EINVAL);
  CHECK(rf_w8a16_unpack_weight(w, 1, 64, nullptr, 64) == RF_W8A16_EINVAL);
  CHECK(rf_w8a16_packed_bytes(0, 64) == 0 && rf_w8a16_packed_bytes(64, -1) == 0);
  CHECK(rf_w8a16_packed_bytes((int64_t)1 << 31, 64) == 0);
  for (int s = -3; s < 16; ++s) CHECK(rf_w8a16_status_str(s) != nullptr);
  CHECK(rf_w8a16_abi_version() == RF_W8A16_ABI_VERSION);
}

int main() {
  std::mt19937 rng(20261202);
  const int64_t shapes[][2] = {{1, 1},   {1, 8},   {15, 63},   {16, 64},    {17, 65},
                               {48, 200}, {100, 1000}, {33, 4097}, {1024, 128}, {7, 1}};
  for (const auto& s : shapes)
    for (int64_t pad : {0, 5}) int8_round_trip(rng, s[0], s[1], pad);
  const int64_t shapes4[][2] = {{16, 64}, {16, 128}, {32, 192}, {48, 1000}, {5, 7}, {1024, 256}};
  for (const auto& s : shapes4) int4_round_trip(rng, s[0], s[1]);
  plans();
  refusals();
  std::printf("%s: %d failure(s)\n", failures ? "FAILED" : "OK", failures);
  return failures ? 1 : 0;
}
