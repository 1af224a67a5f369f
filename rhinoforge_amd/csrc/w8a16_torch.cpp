// Thin torch-library op over the rf_w8a16 C ABI (PyTorch-ROCm).
//
// Schemas (namespace `w8a16`):
//   linear(Tensor input, Tensor weight, Tensor weight_scale, Tensor? bias=None,
//          int layout=1, int kernel=0) -> Tensor
//   linear_into(Tensor input, Tensor weight, Tensor weight_scale, Tensor? bias,
//               Tensor(a!) out, int layout=1, int kernel=0) -> ()
//   linear_multi(Tensor input, Tensor[] weights, Tensor[] weight_scales,
//                Tensor?[] biases, int layout=1, int kernel=0) -> Tensor[]
//   pack_weight(Tensor q) -> Tensor
//   unpack_weight(Tensor packed, int N, int K) -> Tensor
//   select_kernel(int M, int N, int K) -> int
// and (namespace `w4a16`, packed int4 weights, rf_w4a16_* in the C ABI):
//   linear(Tensor input, Tensor weight, Tensor weight_scale, Tensor? bias=None,
//          int kernel=0) -> Tensor
//   linear_multi(Tensor input, Tensor[] weights, Tensor[] weight_scales,
//                Tensor?[] biases, int kernel=0) -> Tensor[]
//   pack_weight(Tensor q) -> Tensor
//   unpack_weight(Tensor packed, int N, int K) -> Tensor
//
// These mirror the reference's eager FP16 `linear_into` (schema at
// src/core/rpu_dispatch_registrations.inc:19-20, checks at
// src/ops/rpu_linear.cpp:664-731) with the fp16 per-channel scale carried
// next to the int8 weight as in `causal_decoder_set_lm_head`
// (registrations :46): input [..., K] is flattened to [M, K]
// (rpu_linear.cpp:596-613), weight is int8 in the packed layout (3-D tiles
// [ceil(N/16), ceil(K/64), 1024]: a row-major [N, K] is refused), scale fp16
// [N], bias fp16 [N] added once after the reduction.  Invalid input raises;
// there is no CPU compute path and no silent fallback (the reference also
// refuses to run swizzled weights on the CPU, rpu_linear.cpp:193-196).
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "../../include/w8a16.h"

namespace {

void check_status(int st, const char* what) {
  TORCH_CHECK(st == RF_W8A16_OK, what, ": ", rf_w8a16_status_str(st), " (status ", st, ")");
}

int64_t ceil_to(int64_t a, int64_t b) { return (a + b - 1) / b * b; }
int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
// Symbolic sizes (FakeTensor tracing with dynamic shapes) round the same way.
c10::SymInt ceil_div(const c10::SymInt& a, int64_t b) { return (a + (b - 1)) / b; }

// Packed weight shapes: [tiles along N, tiles along K, 1024 bytes].
std::vector<int64_t> packed_sizes_int8(int64_t N, int64_t K) {
  return {ceil_div(N, 16), ceil_div(K, 64), 1024};
}
std::vector<int64_t> packed_sizes_int4(int64_t N, int64_t K) {
  return {ceil_div(N, 16), ceil_div(K, 128), 1024};
}

// Refuses anything but the packed tiles of an [N, K] weight (by rank and
// sizes: a row-major or reference-packed 2-D matrix is never accepted).
void check_packed(const at::Tensor& packed, at::ScalarType dtype,
                  const std::vector<int64_t>& want, const char* op) {
  TORCH_CHECK(packed.scalar_type() == dtype, op, ": packed must be ", dtype, ", got ",
              packed.scalar_type());
  TORCH_CHECK(packed.sizes() == at::IntArrayRef(want), op, ": packed must have shape ", want,
              ", got ", packed.sizes());
}

// Workspace per (device, stream): allocated through torch's caching
// allocator, zero-filled once (fill kernel), at least kMinWorkspace bytes.
// The C ABI leaves its counter region zero after every call, and calls on
// one stream are ordered, so one buffer per stream is safe to reuse.  A
// buffer that has to grow is retired, never freed: a HIP graph captured
// earlier on that stream may still reference it.
constexpr int64_t kMinWorkspace = 16 << 20;

struct WorkspaceCache {
  std::mutex mu;
  std::map<std::pair<int, void*>, at::Tensor> bufs;
  std::vector<at::Tensor> retired;

  at::Tensor get(const at::Device& dev, void* stream, size_t bytes) {
    std::lock_guard<std::mutex> g(mu);
    auto key = std::make_pair((int)dev.index(), stream);
    auto it = bufs.find(key);
    if (it != bufs.end() && (size_t)it->second.numel() >= bytes) return it->second;
    if (it != bufs.end()) retired.push_back(it->second);
    const int64_t sz = ceil_to(std::max<int64_t>((int64_t)bytes, kMinWorkspace), 1 << 20);
    at::Tensor t = at::zeros({sz}, at::TensorOptions().dtype(at::kByte).device(dev));
    bufs[key] = t;
    return t;
  }
};

WorkspaceCache& workspace_cache() {
  static WorkspaceCache* c = new WorkspaceCache();  // lives until process exit
  return *c;
}

// Runs call(workspace, bytes) with the stream's cached workspace.  The C ABI
// refuses a workspace that is too small with RF_W8A16_EWORKSPACE before it
// launches anything; only then is the size the shape needs queried (a second
// launch plan), the buffer grown and the call repeated.
template <typename Call, typename Need>
int with_workspace(const at::Device& dev, void* stream, const char* op, Call call, Need need) {
  WorkspaceCache& wc = workspace_cache();
  at::Tensor ws = wc.get(dev, stream, 0);
  int st = call(ws.data_ptr(), (size_t)ws.numel());
  if (st == RF_W8A16_EWORKSPACE) {
    const size_t bytes = need();
    TORCH_CHECK(bytes > 0, op, ": ", rf_w8a16_status_str(RF_W8A16_EINVAL));
    ws = wc.get(dev, stream, bytes);
    st = call(ws.data_ptr(), (size_t)ws.numel());
  }
  return st;
}

struct Checked {
  at::Tensor x2;  // [M, K] view/copy with 16-byte aligned rows
  int64_t M, N, K;
};

// Rows ldx >= 2^24 elements (32 MB) apart are further apart than the kernels'
// 32-bit per-lane offsets reach over a tile's rows (the C ABI refuses the GEMV
// for them and the GEMM takes a slower 64-bit-address kernel); such views are
// copied, as misaligned or non-unit-stride ones are.
constexpr int64_t kMaxRowStride = (int64_t)1 << 24;

// x2 itself when its rows are 16-byte aligned, unit-stride and at most
// kMaxRowStride apart, else a fresh contiguous copy (allocator-aligned).
at::Tensor compact_rows(const at::Tensor& x2) {
  const bool ok = x2.stride(1) == 1 && x2.stride(0) % 8 == 0 &&
                  (x2.size(0) <= 1 || x2.stride(0) < kMaxRowStride) &&
                  (reinterpret_cast<uintptr_t>(x2.data_ptr()) % 16) == 0;
  if (ok) return x2;
  return x2.is_contiguous() ? x2.clone() : x2.contiguous();
}

// Dtype, shape and layout checks (no device checks): shared by the HIP
// kernels and the Meta (shape inference) kernels.  Returns {N, K}.  Sizes are
// read as SymInts so that the Meta kernels also trace symbolic shapes (each
// comparison then guards on the value); on real tensors they are plain ints.
std::pair<c10::SymInt, c10::SymInt> check_shapes(const at::Tensor& input, const at::Tensor& weight,
                                                 const at::Tensor& scale,
                                                 const c10::optional<at::Tensor>& bias,
                                                 int64_t layout, const char* op) {
  TORCH_CHECK(input.scalar_type() == at::kHalf, op, ": input must be float16, got ",
              input.scalar_type());
  TORCH_CHECK(weight.scalar_type() == at::kChar, op,
              ": weight must be int8 (W8A16 packed weight), got ", weight.scalar_type());
  TORCH_CHECK(scale.scalar_type() == at::kHalf, op, ": weight_scale must be float16, got ",
              scale.scalar_type());
  TORCH_CHECK(input.dim() >= 1, op, ": input must have at least one dimension");
  TORCH_CHECK(layout == RF_W8A16_LAYOUT_TILE16X64, op, ": layout ", layout,
              " not accepted: ", rf_w8a16_status_str(RF_W8A16_ELAYOUT));
  TORCH_CHECK(scale.dim() == 1 && scale.is_contiguous(), op,
              ": weight_scale must be a contiguous 1-D [N] tensor, got ", scale.sizes());
  const c10::SymInt N = scale.sym_size(0);
  const c10::SymInt K = input.sym_size(-1);
  TORCH_CHECK(N >= 1, op, ": N (weight_scale.numel()) must be >= 1");
  TORCH_CHECK(K >= 8 && K % 8 == 0, op, ": in_features K=", K, " is zero or not a multiple of 8");
  // The packed form is 3-D (one 1024-byte tile per 16 channels and 64 input
  // positions); a row-major [N, K] matrix never has that rank, so one passed
  // in its place is refused here instead of being read as tiles.
  TORCH_CHECK(weight.is_contiguous() && weight.dim() == 3 &&
                  weight.sym_size(0) == ceil_div(N, 16) && weight.sym_size(1) == ceil_div(K, 64) &&
                  weight.sym_size(2) == 1024,
              op, ": weight must be the packed int8 tiles [", ceil_div(N, 16), ", ",
              ceil_div(K, 64), ", 1024] of an [N=", N, ", K=", K,
              "] weight (use w8a16.pack_weight on the row-major int8 weight), got ",
              weight.sym_sizes());
  if (bias.has_value() && bias->defined()) {
    const at::Tensor& b = *bias;
    TORCH_CHECK(b.scalar_type() == at::kHalf, op, ": bias must be float16");
    TORCH_CHECK(b.dim() == 1 && b.sym_size(0) == N && b.is_contiguous(), op,
                ": bias must be a contiguous vector with ", N, " elements, got shape ",
                b.sym_sizes());
  }
  return {N, K};
}

void check_devices(const at::Tensor& input, const at::Tensor& weight, const at::Tensor& scale,
                   const c10::optional<at::Tensor>& bias, const char* op) {
  TORCH_CHECK(input.is_cuda() && weight.is_cuda() && scale.is_cuda(), op,
              ": input, weight and weight_scale must be on a HIP device (there is no CPU "
              "implementation)");
  TORCH_CHECK(input.device() == weight.device() && input.device() == scale.device(), op,
              ": input, weight and weight_scale must be on the same device");
  if (bias.has_value() && bias->defined())
    TORCH_CHECK(bias->is_cuda() && bias->device() == input.device(), op,
                ": bias must be on the input's device");
}

Checked check_args(const at::Tensor& input, const at::Tensor& weight, const at::Tensor& scale,
                   const c10::optional<at::Tensor>& bias, int64_t layout, const char* op) {
  const auto nk = check_shapes(input, weight, scale, bias, layout, op);
  check_devices(input, weight, scale, bias, op);
  Checked c;
  c.N = nk.first.expect_int();
  c.K = nk.second.expect_int();
  c.M = input.numel() / c.K;
  c.x2 = compact_rows(input.dim() == 2 ? input : input.reshape({c.M, c.K}));
  return c;
}

// Shape of an output [..., N] for input [..., K].
std::vector<int64_t> out_sizes(const at::Tensor& input, int64_t N) {
  std::vector<int64_t> shape = input.sizes().vec();
  shape.back() = N;
  return shape;
}

// y: contiguous [..., N], so its rows are N elements apart.
void launch(const Checked& c, const at::Tensor& weight, const at::Tensor& scale,
            const c10::optional<at::Tensor>& bias, at::Tensor& y, int64_t layout,
            int64_t kernel, const char* op) {
  if (c.M == 0) return;
  c10::DeviceGuard guard(c.x2.device());
  void* stream = c10::hip::getCurrentHIPStream(c.x2.device().index()).stream();
  const void* bptr = (bias.has_value() && bias->defined()) ? bias->data_ptr() : nullptr;
  const int st = with_workspace(
      c.x2.device(), stream, op,
      [&](void* ws, size_t ws_bytes) {
        return rf_w8a16_linear(c.x2.data_ptr(), c.x2.stride(0), weight.data_ptr(), (int32_t)layout,
                               scale.data_ptr(), bptr, y.data_ptr(), c.N, c.M, c.N, c.K,
                               (int32_t)kernel, ws, ws_bytes, stream);
      },
      [&] { return rf_w8a16_workspace_bytes(c.M, c.N, c.K); });
  check_status(st, op);
}

at::Tensor linear_hip(const at::Tensor& input, const at::Tensor& weight, const at::Tensor& scale,
                      const c10::optional<at::Tensor>& bias, int64_t layout, int64_t kernel) {
  RECORD_FUNCTION("w8a16::linear", {});
  Checked c = check_args(input, weight, scale, bias, layout, "w8a16::linear");
  at::Tensor y = at::empty(out_sizes(input, c.N), input.options());  // contiguous: rows N apart
  launch(c, weight, scale, bias, y, layout, kernel, "w8a16::linear");
  return y;
}

void linear_into_hip(const at::Tensor& input, const at::Tensor& weight, const at::Tensor& scale,
                     const c10::optional<at::Tensor>& bias, at::Tensor& out, int64_t layout,
                     int64_t kernel) {
  RECORD_FUNCTION("w8a16::linear_into", {});
  Checked c = check_args(input, weight, scale, bias, layout, "w8a16::linear_into");
  TORCH_CHECK(out.scalar_type() == at::kHalf, "w8a16::linear_into: out must be float16");
  TORCH_CHECK(out.is_cuda() && out.device() == input.device(),
              "w8a16::linear_into: out must be on the input's device");
  const std::vector<int64_t> shape = out_sizes(input, c.N);
  TORCH_CHECK(out.sizes() == shape, "w8a16::linear_into: out shape must be ", shape, ", got ",
              out.sizes());
  TORCH_CHECK(out.is_contiguous(), "w8a16::linear_into: out must be contiguous");
  launch(c, weight, scale, bias, out, layout, kernel, "w8a16::linear_into");
}

// Several projections sharing the input (q/k/v, gate/up): one GEMV launch
// for decode-sized M.  Outputs are fresh tensors [..., N_i].
std::vector<at::Tensor> linear_multi_hip(const at::Tensor& input, at::TensorList weights,
                                         at::TensorList scales,
                                         const c10::List<c10::optional<at::Tensor>>& biases,
                                         int64_t layout, int64_t kernel) {
  RECORD_FUNCTION("w8a16::linear_multi", {});
  const char* op = "w8a16::linear_multi";
  const int64_t count = (int64_t)weights.size();
  TORCH_CHECK(count >= 1 && count <= RF_W8A16_MAX_PROJ, op, ": between 1 and ",
              RF_W8A16_MAX_PROJ, " projections, got ", count);
  TORCH_CHECK((int64_t)scales.size() == count, op, ": ", count, " weights but ", scales.size(),
              " weight_scales");
  TORCH_CHECK(biases.size() == 0 || (int64_t)biases.size() == count, op, ": ", count,
              " weights but ", biases.size(), " biases");
  std::vector<c10::optional<at::Tensor>> b(count);
  for (int64_t i = 0; i < (int64_t)biases.size(); ++i) b[i] = biases.get(i);
  // The shared input is checked and flattened once; each further projection
  // has its own weight, scale and bias checked against the same K.
  const Checked c0 = check_args(input, weights[0], scales[0], b[0], layout, op);
  std::vector<at::Tensor> outs(count);
  rf_w8a16_proj projs[RF_W8A16_MAX_PROJ];
  int64_t Ns[RF_W8A16_MAX_PROJ];
  std::vector<int64_t> shape = input.sizes().vec();
  for (int64_t i = 0; i < count; ++i) {
    int64_t N = c0.N;
    if (i > 0) {
      N = check_shapes(input, weights[i], scales[i], b[i], layout, op).first.expect_int();
      check_devices(input, weights[i], scales[i], b[i], op);
    }
    shape.back() = N;
    outs[i] = at::empty(shape, input.options());  // contiguous: rows N apart
    projs[i].w_packed = weights[i].data_ptr();
    projs[i].scale = scales[i].data_ptr();
    projs[i].bias = (b[i].has_value() && b[i]->defined()) ? b[i]->data_ptr() : nullptr;
    projs[i].y = outs[i].data_ptr();
    projs[i].ldy = N;
    projs[i].N = N;
    Ns[i] = N;
  }
  if (c0.M > 0) {
    c10::DeviceGuard guard(c0.x2.device());
    void* stream = c10::hip::getCurrentHIPStream(c0.x2.device().index()).stream();
    const int st = with_workspace(
        c0.x2.device(), stream, op,
        [&](void* ws, size_t ws_bytes) {
          return rf_w8a16_linear_multi(c0.x2.data_ptr(), c0.x2.stride(0), (int32_t)layout, projs,
                                       (int32_t)count, c0.M, c0.K, (int32_t)kernel, ws, ws_bytes,
                                       stream);
        },
        [&] { return rf_w8a16_workspace_bytes_multi(c0.M, Ns, (int32_t)count, c0.K); });
    check_status(st, op);
  }
  return outs;
}

std::vector<at::Tensor> linear_multi_meta(const at::Tensor& input, at::TensorList weights,
                                          at::TensorList scales,
                                          const c10::List<c10::optional<at::Tensor>>& biases,
                                          int64_t layout, int64_t kernel);

// CPU tensors: the same argument checks as the device path (so a row-major
// weight is named as such), then a refusal -- there is no CPU compute.
std::vector<at::Tensor> linear_multi_cpu(const at::Tensor& input, at::TensorList weights,
                                         at::TensorList scales,
                                         const c10::List<c10::optional<at::Tensor>>& biases,
                                         int64_t layout, int64_t kernel) {
  linear_multi_meta(input, weights, scales, biases, layout, kernel);
  TORCH_CHECK(false, "w8a16::linear_multi: tensors are on the CPU; the W8A16 kernels run on a "
              "HIP device (gfx950) only and there is no CPU implementation");
}

// ---- Meta kernels: output shapes and dtypes (FakeTensor, torch.compile
// tracing), after the same dtype / shape / layout checks as the HIP kernels.
std::vector<c10::SymInt> out_shape(const at::Tensor& input, const c10::SymInt& N) {
  std::vector<c10::SymInt> shape = input.sym_sizes().vec();
  shape.back() = N;
  return shape;
}

at::Tensor linear_meta(const at::Tensor& input, const at::Tensor& weight, const at::Tensor& scale,
                       const c10::optional<at::Tensor>& bias, int64_t layout, int64_t kernel) {
  const auto nk = check_shapes(input, weight, scale, bias, layout, "w8a16::linear");
  return at::empty_symint(out_shape(input, nk.first), input.options());
}

void linear_into_meta(const at::Tensor& input, const at::Tensor& weight, const at::Tensor& scale,
                      const c10::optional<at::Tensor>& bias, at::Tensor& out, int64_t layout,
                      int64_t kernel) {
  const auto nk = check_shapes(input, weight, scale, bias, layout, "w8a16::linear_into");
  TORCH_CHECK(out.scalar_type() == at::kHalf, "w8a16::linear_into: out must be float16");
  const std::vector<c10::SymInt> shape = out_shape(input, nk.first);
  TORCH_CHECK(out.sym_sizes() == c10::SymIntArrayRef(shape),
              "w8a16::linear_into: out shape must be ", c10::SymIntArrayRef(shape), ", got ",
              out.sym_sizes());
}

std::vector<at::Tensor> linear_multi_meta(const at::Tensor& input, at::TensorList weights,
                                          at::TensorList scales,
                                          const c10::List<c10::optional<at::Tensor>>& biases,
                                          int64_t layout, int64_t kernel) {
  const char* op = "w8a16::linear_multi";
  const int64_t count = (int64_t)weights.size();
  TORCH_CHECK(count >= 1 && count <= RF_W8A16_MAX_PROJ, op, ": between 1 and ",
              RF_W8A16_MAX_PROJ, " projections, got ", count);
  TORCH_CHECK((int64_t)scales.size() == count &&
                  (biases.size() == 0 || (int64_t)biases.size() == count),
              op, ": weights, weight_scales and biases differ in length");
  std::vector<at::Tensor> outs;
  for (int64_t i = 0; i < count; ++i) {
    const c10::optional<at::Tensor> b = biases.size() ? biases.get(i) : c10::optional<at::Tensor>();
    const auto nk = check_shapes(input, weights[i], scales[i], b, layout, op);
    outs.push_back(at::empty_symint(out_shape(input, nk.first), input.options()));
  }
  return outs;
}

std::tuple<at::Tensor, at::Tensor> linear_argmax_meta(const at::Tensor& input,
                                                      const at::Tensor& weight,
                                                      const at::Tensor& scale,
                                                      const c10::optional<at::Tensor>& bias,
                                                      bool return_logits, int64_t layout) {
  const char* op = "w8a16::linear_argmax";
  const auto nk = check_shapes(input, weight, scale, bias, layout, op);
  TORCH_CHECK(input.sym_numel() / nk.second <= 64, op,
              ": fused argmax covers decode batches of at most 64 rows");
  std::vector<c10::SymInt> ishape = input.sym_sizes().vec();
  ishape.pop_back();
  at::Tensor index = at::empty_symint(ishape, input.options().dtype(at::kInt));
  at::Tensor logits = return_logits
                          ? at::empty_symint(out_shape(input, nk.first), input.options())
                          : at::empty({0}, input.options());
  return {index, logits};
}

at::Tensor pack_weight_meta(const at::Tensor& q) {
  TORCH_CHECK(q.scalar_type() == at::kChar && q.dim() == 2 && q.sym_size(0) >= 1 &&
                  q.sym_size(1) >= 1,
              "w8a16::pack_weight: q must be a non-empty int8 [N, K] tensor");
  return at::empty_symint({ceil_div(q.sym_size(0), 16), ceil_div(q.sym_size(1), 64), 1024},
                          q.options());
}

at::Tensor unpack_weight_meta(const at::Tensor& packed, int64_t N, int64_t K) {
  TORCH_CHECK(N >= 1 && K >= 1, "w8a16::unpack_weight: N and K must be >= 1");
  check_packed(packed, at::kChar, packed_sizes_int8(N, K), "w8a16::unpack_weight");
  return at::empty({N, K}, packed.options());
}

[[noreturn]] void no_cpu(const char* op) {
  TORCH_CHECK(false, op,
              ": tensors are on the CPU; the W8A16 kernels run on a HIP device (gfx950) only "
              "and there is no CPU implementation");
}

at::Tensor linear_cpu(const at::Tensor& input, const at::Tensor& weight, const at::Tensor& scale,
                      const c10::optional<at::Tensor>& bias, int64_t layout, int64_t) {
  check_shapes(input, weight, scale, bias, layout, "w8a16::linear");
  no_cpu("w8a16::linear");
}

std::tuple<at::Tensor, at::Tensor> linear_argmax_cpu(const at::Tensor& input,
                                                     const at::Tensor& weight,
                                                     const at::Tensor& scale,
                                                     const c10::optional<at::Tensor>& bias, bool,
                                                     int64_t layout) {
  check_shapes(input, weight, scale, bias, layout, "w8a16::linear_argmax");
  no_cpu("w8a16::linear_argmax");
}

// Greedy decode: the per-row argmax of the fp16 logits, folded into the GEMV
// epilogue (M <= 64).  Returns (index int32 [...], logits fp16 [..., N] or an
// empty tensor when return_logits is false).
std::tuple<at::Tensor, at::Tensor> linear_argmax_hip(const at::Tensor& input,
                                                     const at::Tensor& weight,
                                                     const at::Tensor& scale,
                                                     const c10::optional<at::Tensor>& bias,
                                                     bool return_logits, int64_t layout) {
  RECORD_FUNCTION("w8a16::linear_argmax", {});
  const char* op = "w8a16::linear_argmax";
  Checked c = check_args(input, weight, scale, bias, layout, op);
  TORCH_CHECK(c.M <= 64, op, ": fused argmax covers decode batches of at most 64 rows, got M=",
              c.M, " (use w8a16::linear and argmax for longer inputs)");
  std::vector<int64_t> ishape = input.sizes().vec();
  ishape.pop_back();
  at::Tensor index = at::empty(ishape, input.options().dtype(at::kInt));
  at::Tensor logits;
  if (return_logits) {
    std::vector<int64_t> lshape = input.sizes().vec();
    lshape.back() = c.N;
    logits = at::empty(lshape, input.options());
  } else {
    logits = at::empty({0}, input.options());
  }
  if (c.M == 0) return {index, logits};
  c10::DeviceGuard dev_guard(c.x2.device());
  void* stream = c10::hip::getCurrentHIPStream(c.x2.device().index()).stream();
  const void* bptr = (bias.has_value() && bias->defined()) ? bias->data_ptr() : nullptr;
  const int st = with_workspace(
      c.x2.device(), stream, op,
      [&](void* ws, size_t ws_bytes) {
        return rf_w8a16_linear_argmax(c.x2.data_ptr(), c.x2.stride(0), weight.data_ptr(),
                                      (int32_t)layout, scale.data_ptr(), bptr,
                                      return_logits ? logits.data_ptr() : nullptr, c.N,
                                      index.data_ptr<int32_t>(), c.M, c.N, c.K, ws, ws_bytes,
                                      stream);
      },
      [&] { return rf_w8a16_workspace_bytes_argmax(c.M, c.N, c.K); });
  check_status(st, op);
  return {index, logits};
}

void linear_into_cpu(const at::Tensor& input, const at::Tensor& weight, const at::Tensor& scale,
                     const c10::optional<at::Tensor>& bias, at::Tensor&, int64_t layout,
                     int64_t) {
  check_shapes(input, weight, scale, bias, layout, "w8a16::linear_into");
  no_cpu("w8a16::linear_into");
}

// Repack a row-major int8 [N, K] weight into the TILE16X64 layout.
// CPU tensors are packed on the host, HIP tensors on the device.
at::Tensor pack_weight(const at::Tensor& q) {
  TORCH_CHECK(q.scalar_type() == at::kChar, "w8a16::pack_weight: q must be int8, got ",
              q.scalar_type());
  TORCH_CHECK(q.dim() == 2, "w8a16::pack_weight: q must be 2-D [N, K], got ", q.sizes());
  const int64_t N = q.size(0), K = q.size(1);
  TORCH_CHECK(N >= 1 && K >= 1, "w8a16::pack_weight: empty weight ", q.sizes());
  at::Tensor qc = q.contiguous();
  at::Tensor out = at::empty(packed_sizes_int8(N, K), q.options());
  const size_t bytes = rf_w8a16_packed_bytes(N, K);
  TORCH_CHECK((size_t)out.numel() == bytes, "w8a16::pack_weight: size mismatch");
  if (q.is_cuda()) {
    c10::DeviceGuard guard(q.device());
    void* stream = c10::hip::getCurrentHIPStream(q.device().index()).stream();
    check_status(rf_w8a16_pack_weight_device(qc.data_ptr<int8_t>(), N, K, K, out.data_ptr(), bytes,
                                             stream),
                 "w8a16::pack_weight");
  } else {
    TORCH_CHECK(q.device().is_cpu(), "w8a16::pack_weight: unsupported device ", q.device());
    check_status(rf_w8a16_pack_weight(qc.data_ptr<int8_t>(), N, K, K, out.data_ptr(), bytes),
                 "w8a16::pack_weight");
  }
  return out;
}

// Inverse of pack_weight (host); returns a CPU int8 [N, K] tensor.
at::Tensor unpack_weight(const at::Tensor& packed, int64_t N, int64_t K) {
  TORCH_CHECK(N >= 1 && K >= 1, "w8a16::unpack_weight: N and K must be >= 1");
  check_packed(packed, at::kChar, packed_sizes_int8(N, K), "w8a16::unpack_weight");
  at::Tensor p = packed.to(at::kCPU).contiguous();
  at::Tensor q = at::empty({N, K}, p.options());
  check_status(rf_w8a16_unpack_weight(p.data_ptr(), N, K, q.data_ptr<int8_t>(), K),
               "w8a16::unpack_weight");
  return q;
}

// ---- W4A16 -------------------------------------------------------------------
// The reference's launcher takes a packed-int4 weight as a uint8 [N, K/2]
// tensor and tells per-channel from group-wise by the scale's rank
// (src/ops/rpu_linear.cpp:1211-1489); so does this op: weight uint8
// TILE16X128_I4 tiles [ceil(N/16), ceil(K/128), 1024], scale fp16 [N] (per-channel) or
// [G, N] (group-wise, group_size = K / G in {32, 64, 128}).
// W4A16 dtype / shape checks (no device checks), shared by the HIP and Meta
// kernels: N, K and the group size (0 = per-channel scale [N]).
struct W4Shape {
  c10::SymInt N, K, group_size;
};

W4Shape w4_check_shapes(const at::Tensor& input, const at::Tensor& weight, const at::Tensor& scale,
                        const c10::optional<at::Tensor>& bias, const char* op) {
  TORCH_CHECK(input.scalar_type() == at::kHalf, op, ": input must be float16, got ",
              input.scalar_type());
  TORCH_CHECK(weight.scalar_type() == at::kByte, op,
              ": weight must be uint8 (packed int4, use w4a16.pack_weight), got ",
              weight.scalar_type());
  TORCH_CHECK(scale.scalar_type() == at::kHalf, op, ": weight_scale must be float16, got ",
              scale.scalar_type());
  TORCH_CHECK(input.dim() >= 1, op, ": input must have at least one dimension");
  TORCH_CHECK((scale.dim() == 1 || scale.dim() == 2) && scale.is_contiguous(), op,
              ": weight_scale must be a contiguous [N] (per-channel) or [K/group_size, N] "
              "(group-wise) tensor, got ", scale.sizes());
  W4Shape r;
  r.K = input.sym_size(-1);
  r.N = scale.sym_size(-1);
  r.group_size = 0;
  if (scale.dim() == 2) {
    const c10::SymInt G = scale.sym_size(0);
    TORCH_CHECK(G >= 1 && r.K % G == 0, op, ": group-wise scale has ", G,
                " rows, which does not divide K=", r.K);
    r.group_size = r.K / G;
    TORCH_CHECK(r.group_size == 32 || r.group_size == 64 || r.group_size == 128, op,
                ": group size K / scale.size(0) = ", r.group_size, " must be 32, 64 or 128");
  }
  TORCH_CHECK(r.N >= 16 && r.N % 16 == 0, op, ": out_features N=", r.N,
              " is zero or not a multiple of 16, which packed int4 needs");
  TORCH_CHECK(r.K >= 64 && r.K % 64 == 0, op, ": in_features K=", r.K,
              " is zero or not a multiple of 64, which packed int4 needs");
  // 3-D packed tiles, never the rank of the reference's nibble-packed [N, K/2].
  TORCH_CHECK(weight.is_contiguous() && weight.dim() == 3 &&
                  weight.sym_size(0) == ceil_div(r.N, 16) &&
                  weight.sym_size(1) == ceil_div(r.K, 128) && weight.sym_size(2) == 1024,
              op, ": weight must be the packed int4 tiles [", ceil_div(r.N, 16), ", ",
              ceil_div(r.K, 128), ", 1024] of an [N=", r.N, ", K=", r.K,
              "] weight (use w4a16.pack_weight), got ", weight.sym_sizes());
  if (bias.has_value() && bias->defined()) {
    const at::Tensor& b = *bias;
    TORCH_CHECK(b.scalar_type() == at::kHalf, op, ": bias must be float16");
    TORCH_CHECK(b.dim() == 1 && b.sym_size(0) == r.N && b.is_contiguous(), op,
                ": bias must be a contiguous vector with ", r.N, " elements, got shape ",
                b.sym_sizes());
  }
  return r;
}

at::Tensor w4_linear_hip(const at::Tensor& input, const at::Tensor& weight, const at::Tensor& scale,
                         const c10::optional<at::Tensor>& bias, int64_t kernel) {
  RECORD_FUNCTION("w4a16::linear", {});
  const char* op = "w4a16::linear";
  const W4Shape sh = w4_check_shapes(input, weight, scale, bias, op);
  const int64_t N = sh.N.expect_int(), K = sh.K.expect_int(), group_size = sh.group_size.expect_int();
  TORCH_CHECK(input.is_cuda() && weight.is_cuda() && scale.is_cuda(), op,
              ": input, weight and weight_scale must be on a HIP device (there is no CPU "
              "implementation)");
  TORCH_CHECK(input.device() == weight.device() && input.device() == scale.device(), op,
              ": input, weight and weight_scale must be on the same device");
  if (bias.has_value() && bias->defined())
    TORCH_CHECK(bias->is_cuda() && bias->device() == input.device(), op,
                ": bias must be on the input's device");
  const int64_t M = input.numel() / K;
  at::Tensor y = at::empty(out_sizes(input, N), input.options());  // contiguous: rows N apart
  if (M == 0) return y;
  const at::Tensor x2 = compact_rows(input.dim() == 2 ? input : input.reshape({M, K}));
  // group-wise scale rows are copied with 16-byte DMAs
  at::Tensor sc = (group_size && reinterpret_cast<uintptr_t>(scale.data_ptr()) % 16) ? scale.clone()
                                                                                      : scale;
  c10::DeviceGuard dev_guard(x2.device());
  void* stream = c10::hip::getCurrentHIPStream(x2.device().index()).stream();
  const void* bptr = (bias.has_value() && bias->defined()) ? bias->data_ptr() : nullptr;
  const int st = with_workspace(
      x2.device(), stream, op,
      [&](void* ws, size_t ws_bytes) {
        return rf_w4a16_linear(x2.data_ptr(), x2.stride(0), weight.data_ptr(), sc.data_ptr(),
                               (int32_t)group_size, bptr, y.data_ptr(), N, M, N, K,
                               (int32_t)kernel, ws, ws_bytes, stream);
      },
      [&] { return rf_w4a16_workspace_bytes(M, N, K); });
  check_status(st, op);
  return y;
}

at::Tensor w4_linear_cpu(const at::Tensor& input, const at::Tensor& weight,
                         const at::Tensor& scale, const c10::optional<at::Tensor>& bias, int64_t) {
  w4_check_shapes(input, weight, scale, bias, "w4a16::linear");
  TORCH_CHECK(false, "w4a16::linear: tensors are on the CPU; the W4A16 kernels run on a HIP "
              "device (gfx950) only and there is no CPU implementation");
}

at::Tensor w4_linear_meta(const at::Tensor& input, const at::Tensor& weight, const at::Tensor& scale,
                          const c10::optional<at::Tensor>& bias, int64_t kernel) {
  const W4Shape sh = w4_check_shapes(input, weight, scale, bias, "w4a16::linear");
  return at::empty_symint(out_shape(input, sh.N), input.options());
}

// Several packed-int4 projections sharing the input (q/k/v, gate/up) in one
// launch, as w8a16::linear_multi for int8.  All weight_scales have the same
// rank (per-channel [N_i] or group-wise [K/gs, N_i] with one group size).
// Returns the checked shapes (N_i) and the shared group size.
std::pair<std::vector<c10::SymInt>, c10::SymInt> w4_check_multi(
    const at::Tensor& input, at::TensorList weights, at::TensorList scales,
    const c10::List<c10::optional<at::Tensor>>& biases, const char* op) {
  const int64_t count = (int64_t)weights.size();
  TORCH_CHECK(count >= 1 && count <= RF_W8A16_MAX_PROJ, op, ": between 1 and ",
              RF_W8A16_MAX_PROJ, " projections, got ", count);
  TORCH_CHECK((int64_t)scales.size() == count, op, ": ", count, " weights but ", scales.size(),
              " weight_scales");
  TORCH_CHECK(biases.size() == 0 || (int64_t)biases.size() == count, op, ": ", count,
              " weights but ", biases.size(), " biases");
  std::vector<c10::SymInt> Ns;
  c10::SymInt gs0 = 0;
  for (int64_t i = 0; i < count; ++i) {
    const c10::optional<at::Tensor> b = biases.size() ? biases.get(i) : c10::optional<at::Tensor>();
    const W4Shape sh = w4_check_shapes(input, weights[i], scales[i], b, op);
    if (i == 0) gs0 = sh.group_size;
    TORCH_CHECK(sh.group_size == gs0, op, ": every projection needs the same scale form and "
                "group size (projection 0: ", gs0, ", projection ", i, ": ", sh.group_size, ")");
    Ns.push_back(sh.N);
  }
  return {Ns, gs0};
}

std::vector<at::Tensor> w4_linear_multi_hip(const at::Tensor& input, at::TensorList weights,
                                            at::TensorList scales,
                                            const c10::List<c10::optional<at::Tensor>>& biases,
                                            int64_t kernel) {
  RECORD_FUNCTION("w4a16::linear_multi", {});
  const char* op = "w4a16::linear_multi";
  const auto chk = w4_check_multi(input, weights, scales, biases, op);
  const int64_t count = (int64_t)weights.size();
  const int64_t K = input.size(-1), group_size = chk.second.expect_int();
  const int64_t M = input.numel() / K;
  std::vector<at::Tensor> outs(count), keep(count);
  rf_w8a16_proj projs[RF_W8A16_MAX_PROJ];
  int64_t Ns[RF_W8A16_MAX_PROJ];
  std::vector<int64_t> shape = input.sizes().vec();
  for (int64_t i = 0; i < count; ++i) {
    const c10::optional<at::Tensor> b = biases.size() ? biases.get(i) : c10::optional<at::Tensor>();
    check_devices(input, weights[i], scales[i], b, op);
    const int64_t N = chk.first[i].expect_int();
    shape.back() = N;
    outs[i] = at::empty(shape, input.options());  // contiguous: rows N apart
    // group-wise scale rows are copied with 16-byte DMAs
    keep[i] = (group_size && reinterpret_cast<uintptr_t>(scales[i].data_ptr()) % 16)
                  ? scales[i].clone() : scales[i];
    projs[i].w_packed = weights[i].data_ptr();
    projs[i].scale = keep[i].data_ptr();
    projs[i].bias = (b.has_value() && b->defined()) ? b->data_ptr() : nullptr;
    projs[i].y = outs[i].data_ptr();
    projs[i].ldy = N;
    projs[i].N = N;
    Ns[i] = N;
  }
  if (M == 0) return outs;
  const at::Tensor x2 = compact_rows(input.dim() == 2 ? input : input.reshape({M, K}));
  c10::DeviceGuard dev_guard(x2.device());
  void* stream = c10::hip::getCurrentHIPStream(x2.device().index()).stream();
  const int st = with_workspace(
      x2.device(), stream, op,
      [&](void* ws, size_t ws_bytes) {
        return rf_w4a16_linear_multi(x2.data_ptr(), x2.stride(0), projs, (int32_t)count,
                                     (int32_t)group_size, M, K, (int32_t)kernel, ws, ws_bytes,
                                     stream);
      },
      [&] { return rf_w4a16_workspace_bytes_multi(M, Ns, (int32_t)count, K); });
  check_status(st, op);
  return outs;
}

std::vector<at::Tensor> w4_linear_multi_meta(const at::Tensor& input, at::TensorList weights,
                                             at::TensorList scales,
                                             const c10::List<c10::optional<at::Tensor>>& biases,
                                             int64_t kernel) {
  const auto chk = w4_check_multi(input, weights, scales, biases, "w4a16::linear_multi");
  std::vector<at::Tensor> outs;
  for (const c10::SymInt& N : chk.first)
    outs.push_back(at::empty_symint(out_shape(input, N), input.options()));
  return outs;
}

std::vector<at::Tensor> w4_linear_multi_cpu(const at::Tensor& input, at::TensorList weights,
                                            at::TensorList scales,
                                            const c10::List<c10::optional<at::Tensor>>& biases,
                                            int64_t) {
  w4_check_multi(input, weights, scales, biases, "w4a16::linear_multi");
  TORCH_CHECK(false, "w4a16::linear_multi: tensors are on the CPU; the W4A16 kernels run on a "
              "HIP device (gfx950) only and there is no CPU implementation");
}

at::Tensor w4_pack_weight_meta(const at::Tensor& q) {
  TORCH_CHECK(q.scalar_type() == at::kChar && q.dim() == 2 && q.sym_size(0) >= 1 &&
                  q.sym_size(1) >= 1,
              "w4a16::pack_weight: q must be a non-empty int8 [N, K] tensor");
  return at::empty_symint({ceil_div(q.sym_size(0), 16), ceil_div(q.sym_size(1), 128), 1024},
                          q.options().dtype(at::kByte));
}

at::Tensor w4_unpack_weight_meta(const at::Tensor& packed, int64_t N, int64_t K) {
  TORCH_CHECK(N >= 1 && K >= 1, "w4a16::unpack_weight: N and K must be >= 1");
  check_packed(packed, at::kByte, packed_sizes_int4(N, K), "w4a16::unpack_weight");
  return at::empty({N, K}, packed.options().dtype(at::kChar));
}

// Int8 containers [N, K] holding int4 values in [-8, 7] -> TILE16X128_I4
// (uint8).  CPU tensors are packed (and range-checked) on the host, HIP
// tensors on the device.
at::Tensor w4_pack_weight(const at::Tensor& q) {
  TORCH_CHECK(q.scalar_type() == at::kChar, "w4a16::pack_weight: q must be int8 (int4 values), got ",
              q.scalar_type());
  TORCH_CHECK(q.dim() == 2, "w4a16::pack_weight: q must be 2-D [N, K], got ", q.sizes());
  const int64_t N = q.size(0), K = q.size(1);
  TORCH_CHECK(N >= 1 && K >= 1, "w4a16::pack_weight: empty weight ", q.sizes());
  at::Tensor qc = q.contiguous();
  at::Tensor out = at::empty(packed_sizes_int4(N, K), q.options().dtype(at::kByte));
  const size_t bytes = rf_w4a16_packed_bytes(N, K);
  TORCH_CHECK((size_t)out.numel() == bytes, "w4a16::pack_weight: size mismatch");
  if (q.is_cuda()) {
    c10::DeviceGuard dev_guard(q.device());
    void* stream = c10::hip::getCurrentHIPStream(q.device().index()).stream();
    check_status(rf_w4a16_pack_weight_device(qc.data_ptr<int8_t>(), N, K, K, out.data_ptr(), bytes,
                                             stream),
                 "w4a16::pack_weight");
  } else {
    TORCH_CHECK(q.device().is_cpu(), "w4a16::pack_weight: unsupported device ", q.device());
    const int st = rf_w4a16_pack_weight(qc.data_ptr<int8_t>(), N, K, K, out.data_ptr(), bytes);
    TORCH_CHECK(st == RF_W8A16_OK, "w4a16::pack_weight: ", rf_w8a16_status_str(st),
                " (int4 values must lie in [-8, 7])");
  }
  return out;
}

at::Tensor w4_unpack_weight(const at::Tensor& packed, int64_t N, int64_t K) {
  TORCH_CHECK(N >= 1 && K >= 1, "w4a16::unpack_weight: N and K must be >= 1");
  check_packed(packed, at::kByte, packed_sizes_int4(N, K), "w4a16::unpack_weight");
  at::Tensor p = packed.to(at::kCPU).contiguous();
  at::Tensor q = at::empty({N, K}, p.options().dtype(at::kChar));
  check_status(rf_w4a16_unpack_weight(p.data_ptr(), N, K, q.data_ptr<int8_t>(), K),
               "w4a16::unpack_weight");
  return q;
}

int64_t select_kernel(int64_t M, int64_t N, int64_t K) {
  const int k = rf_w8a16_select_kernel(M, N, K);
  TORCH_CHECK(k > 0, "w8a16::select_kernel: ", rf_w8a16_status_str(-k));
  return k;
}

}  // namespace

TORCH_LIBRARY(w8a16, m) {
  m.def("linear(Tensor input, Tensor weight, Tensor weight_scale, Tensor? bias=None, "
        "int layout=1, int kernel=0) -> Tensor");
  m.def("linear_into(Tensor input, Tensor weight, Tensor weight_scale, Tensor? bias, "
        "Tensor(a!) out, int layout=1, int kernel=0) -> ()");
  m.def("linear_multi(Tensor input, Tensor[] weights, Tensor[] weight_scales, Tensor?[] biases, "
        "int layout=1, int kernel=0) -> Tensor[]");
  m.def("linear_argmax(Tensor input, Tensor weight, Tensor weight_scale, Tensor? bias=None, "
        "bool return_logits=False, int layout=1) -> (Tensor, Tensor)");
  m.def("pack_weight(Tensor q) -> Tensor");
  m.def("unpack_weight(Tensor packed, int N, int K) -> Tensor");
  m.def("select_kernel(int M, int N, int K) -> int", TORCH_FN(select_kernel));
}

// HIP tensors carry the CUDA dispatch key on PyTorch-ROCm.
TORCH_LIBRARY_IMPL(w8a16, CUDA, m) {
  m.impl("linear", TORCH_FN(linear_hip));
  m.impl("linear_into", TORCH_FN(linear_into_hip));
  m.impl("linear_multi", TORCH_FN(linear_multi_hip));
  m.impl("linear_argmax", TORCH_FN(linear_argmax_hip));
  m.impl("pack_weight", TORCH_FN(pack_weight));
  m.impl("unpack_weight", TORCH_FN(unpack_weight));
}

TORCH_LIBRARY_IMPL(w8a16, Meta, m) {
  m.impl("linear", TORCH_FN(linear_meta));
  m.impl("linear_into", TORCH_FN(linear_into_meta));
  m.impl("linear_multi", TORCH_FN(linear_multi_meta));
  m.impl("linear_argmax", TORCH_FN(linear_argmax_meta));
  m.impl("pack_weight", TORCH_FN(pack_weight_meta));
  m.impl("unpack_weight", TORCH_FN(unpack_weight_meta));
}

TORCH_LIBRARY_IMPL(w8a16, CPU, m) {
  m.impl("linear", TORCH_FN(linear_cpu));
  m.impl("linear_into", TORCH_FN(linear_into_cpu));
  m.impl("linear_multi", TORCH_FN(linear_multi_cpu));
  m.impl("linear_argmax", TORCH_FN(linear_argmax_cpu));
  m.impl("pack_weight", TORCH_FN(pack_weight));
  m.impl("unpack_weight", TORCH_FN(unpack_weight));
}

// The ops are not differentiable (int8 weights; no backward kernels).  As the
// reference does for its W8A16 schemas (src/core/rpu_dispatch_registrations.inc:
// 1043-1068, AutogradPrivateUse1 fallthroughs), autograd falls through to the
// backend kernel: inputs that require grad are accepted and the outputs do not
// require grad.
TORCH_LIBRARY_IMPL(w8a16, Autograd, m) {
  for (const char* op : {"linear", "linear_into", "linear_multi", "linear_argmax", "pack_weight",
                         "unpack_weight"})
    m.impl(op, torch::CppFunction::makeFallthrough());
}

TORCH_LIBRARY(w4a16, m) {
  m.def("linear(Tensor input, Tensor weight, Tensor weight_scale, Tensor? bias=None, "
        "int kernel=0) -> Tensor");
  m.def("linear_multi(Tensor input, Tensor[] weights, Tensor[] weight_scales, Tensor?[] biases, "
        "int kernel=0) -> Tensor[]");
  m.def("pack_weight(Tensor q) -> Tensor");
  m.def("unpack_weight(Tensor packed, int N, int K) -> Tensor");
}

TORCH_LIBRARY_IMPL(w4a16, CUDA, m) {
  m.impl("linear", TORCH_FN(w4_linear_hip));
  m.impl("linear_multi", TORCH_FN(w4_linear_multi_hip));
  m.impl("pack_weight", TORCH_FN(w4_pack_weight));
  m.impl("unpack_weight", TORCH_FN(w4_unpack_weight));
}
TORCH_LIBRARY_IMPL(w4a16, Meta, m) {
  m.impl("linear", TORCH_FN(w4_linear_meta));
  m.impl("linear_multi", TORCH_FN(w4_linear_multi_meta));
  m.impl("pack_weight", TORCH_FN(w4_pack_weight_meta));
  m.impl("unpack_weight", TORCH_FN(w4_unpack_weight_meta));
}
TORCH_LIBRARY_IMPL(w4a16, CPU, m) {
  m.impl("linear", TORCH_FN(w4_linear_cpu));
  m.impl("linear_multi", TORCH_FN(w4_linear_multi_cpu));
  m.impl("pack_weight", TORCH_FN(w4_pack_weight));
  m.impl("unpack_weight", TORCH_FN(w4_unpack_weight));
}
TORCH_LIBRARY_IMPL(w4a16, Autograd, m) {
  for (const char* op : {"linear", "linear_multi", "pack_weight", "unpack_weight"})
    m.impl(op, torch::CppFunction::makeFallthrough());
}
