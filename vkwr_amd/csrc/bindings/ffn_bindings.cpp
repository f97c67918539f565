// The channel-mix (FFN) ops of namespace vkwr_v1_mix, registered as a
// fragment of the same namespace and linked into the same module (_v1_mix_C)
// as mix_bindings.cpp.  Schemas byte-identical to the reference
// (csrc/v1/mix/torch_bindings.cpp:326-345), checks as there (:149-244).
//
// Function (reference csrc/v1/mix/mix_ops.cu:296-863, 1109-1278):
//   act = fp16(relu(mix(x, shift_state, x_k) . key_fc^T)^2),  out = act . value_fc,
// with key_fc, value_fc [F,C] and shift_state := x[:, T-1].  The reference
// evaluates the up projection as a dot product per output and the down
// projection as a sparse sum over the nonzero activations with fp16 atomics.
// Here both are dense fp16 GEMMs with fp32 accumulation on the matrix cores
// (the zero activations contribute exact zeros, so the function is the same);
// the mixed input is rounded to fp16 by the token-shift op before the product.
#include "vk_torch.h"

using namespace vkt;

namespace {

uint16_t* h(const at::Tensor& t) { return ptr<uint16_t>(t); }

void check_fc(const at::Tensor& t, int64_t F, int64_t C, const char* name) {
  check_half_cuda_contig(t, name);
  TORCH_CHECK(t.dim() == 2 && t.size(0) == F && t.size(1) == C, name, " must have shape [F,C]");
}

void check_cf(int64_t C, int64_t F, int cdiv, int fdiv) {
  TORCH_CHECK((C % cdiv) == 0, "C must be divisible by ", cdiv);
  TORCH_CHECK((F % fdiv) == 0, "F must be divisible by ", fdiv);
}

// out [rows, C] = act_in(a [rows, F]) . value_fc [F,C]
void down(const at::Tensor& a, const at::Tensor& value_fc, at::Tensor& out, int64_t rows, int64_t C, int64_t F,
          int act, const char* what) {
  if (rows == 0 || C == 0) return;
  std::vector<vkwr_gemm_problem> p{gemm_problem(a, value_fc, out, rows, C, F, VKWR_GEMM_B_KN, act)};
  run_gemm(p, a, what);
}

at::Tensor sparse_full(int64_t B, int64_t T, int64_t C, int64_t F, const at::Tensor& x, at::Tensor& shift_state,
                       const at::Tensor& x_k, const at::Tensor& key_fc, const at::Tensor& value_fc,
                       std::vector<int64_t> out_shape, const char* what) {
  check_fits_int(B, "B");
  check_fits_int(T, "T");
  check_fits_int(C, "C");
  check_fits_int(F, "F");
  check_device(x, "x");
  const int64_t rows = B * T;
  auto mixed = at::empty_like(x);
  auto act = at::empty({rows, F}, x.options());
  auto out = at::empty(out_shape, x.options());
  const uint16_t* mp[1] = {h(x_k)};
  uint16_t* op[1] = {h(mixed)};
  check_status(vkwr_token_shift_mix_f16((int)B, (int)T, (int)C, h(x), h(shift_state), 1, mp, op, 0, stream()),
               what);
  if (rows > 0 && F > 0) {
    std::vector<vkwr_gemm_problem> up{gemm_problem(mixed, key_fc, act, rows, F, C, VKWR_GEMM_B_NK,
                                                   VKWR_GEMM_ACT_NONE, VKWR_GEMM_EPI_RELU_SQUARE)};
    run_gemm(up, x, what);
  }
  if (F > 0) {
    down(act, value_fc, out, rows, C, F, VKWR_GEMM_ACT_NONE, what);
  } else if (out.numel() > 0) {
    out.zero_();
  }
  return out;
}

at::Tensor cmix_sparse_one(int64_t C, int64_t F, at::Tensor x, at::Tensor shift_state, at::Tensor x_k,
                           at::Tensor key_fc, at::Tensor value_fc) {
  check_3d(x, 1, 1, C, "x");
  check_half_cuda_contig(shift_state, "shift_state");
  TORCH_CHECK(shift_state.dim() == 2 && shift_state.size(0) == 1 && shift_state.size(1) == C,
              "shift_state must have shape [1,C]");
  check_vec(x_k, C, "x_k");
  check_fc(key_fc, F, C, "key_fc");
  check_fc(value_fc, F, C, "value_fc");
  check_cf(C, F, 256, 128);
  return sparse_full(1, 1, C, F, x, shift_state, x_k, key_fc, value_fc, {1, 1, C}, "cmix_sparse_one");
}

at::Tensor cmix_sparse_rows(int64_t B, int64_t T, int64_t C, int64_t F, at::Tensor x, at::Tensor shift_state,
                            at::Tensor x_k, at::Tensor key_fc, at::Tensor value_fc) {
  check_3d(x, B, T, C, "x");
  check_half_cuda_contig(shift_state, "shift_state");
  TORCH_CHECK(shift_state.dim() == 2 && shift_state.size(0) == B && shift_state.size(1) == C,
              "shift_state must have shape [B,C]");
  check_vec(x_k, C, "x_k");
  check_fc(key_fc, F, C, "key_fc");
  check_fc(value_fc, F, C, "value_fc");
  check_cf(C, F, 256, 128);
  return sparse_full(B, T, C, F, x, shift_state, x_k, key_fc, value_fc, {B, T, C}, "cmix_sparse_rows");
}

at::Tensor down_op(int64_t B, int64_t T, int64_t C, int64_t F, const at::Tensor& a, const at::Tensor& value_fc,
                   int act, std::vector<int64_t> shape, const char* what) {
  check_fits_int(C, "C");
  check_fits_int(F, "F");
  check_device(a, "act");
  auto out = at::empty(shape, a.options());
  down(a, value_fc, out, B * T, C, F, act, what);
  return out;
}

at::Tensor cmix_sparse_down_one(int64_t C, int64_t F, at::Tensor act, at::Tensor value_fc) {
  check_half_cuda_contig(act, "act");
  TORCH_CHECK(act.dim() == 1 && act.size(0) == F, "act must have shape [F]");
  check_fc(value_fc, F, C, "value_fc");
  check_cf(C, F, 256, 128);
  return down_op(1, 1, C, F, act, value_fc, VKWR_GEMM_ACT_NONE, {1, 1, C}, "cmix_sparse_down_one");
}

at::Tensor cmix_sparse_down_rows(int64_t B, int64_t T, int64_t C, int64_t F, at::Tensor act, at::Tensor value_fc) {
  check_3d(act, B, T, F, "act");
  check_fc(value_fc, F, C, "value_fc");
  check_cf(C, F, 256, 128);
  return down_op(B, T, C, F, act, value_fc, VKWR_GEMM_ACT_NONE, {B, T, C}, "cmix_sparse_down_rows");
}

at::Tensor cmix_sparse_down_relu_one(int64_t C, int64_t F, at::Tensor preact, at::Tensor value_fc) {
  check_half_cuda_contig(preact, "preact");
  TORCH_CHECK(preact.dim() == 1 && preact.size(0) == F, "preact must have shape [F]");
  check_fc(value_fc, F, C, "value_fc");
  check_cf(C, F, 256, 128);
  return down_op(1, 1, C, F, preact, value_fc, VKWR_GEMM_ACT_RELU_SQUARE, {1, 1, C},
                 "cmix_sparse_down_relu_one");
}

at::Tensor cmix_sparse_down_relu_rows(int64_t B, int64_t T, int64_t C, int64_t F, at::Tensor preact,
                                      at::Tensor value_fc) {
  check_3d(preact, B, T, F, "preact");
  check_fc(value_fc, F, C, "value_fc");
  check_cf(C, F, 256, 128);
  return down_op(B, T, C, F, preact, value_fc, VKWR_GEMM_ACT_RELU_SQUARE, {B, T, C},
                 "cmix_sparse_down_relu_rows");
}

at::Tensor cmix_sparse_down_relu_rows_t512(int64_t B, int64_t T, int64_t C, int64_t F, at::Tensor preact,
                                           at::Tensor value_fc) {
  check_3d(preact, B, T, F, "preact");
  check_fc(value_fc, F, C, "value_fc");
  check_cf(C, F, 512, 512);
  return down_op(B, T, C, F, preact, value_fc, VKWR_GEMM_ACT_RELU_SQUARE, {B, T, C},
                 "cmix_sparse_down_relu_rows_t512");
}

}  // namespace

TORCH_LIBRARY_FRAGMENT(vkwr_v1_mix, m) {
  m.def("cmix_sparse_one(int C, int F, Tensor x, Tensor(a!) shift_state, Tensor x_k, Tensor key_fc, Tensor value_fc) -> Tensor");
  m.impl("cmix_sparse_one", c10::kCUDA, &cmix_sparse_one);

  m.def("cmix_sparse_rows(int B, int T, int C, int F, Tensor x, Tensor(a!) shift_state, Tensor x_k, Tensor key_fc, Tensor value_fc) -> Tensor");
  m.impl("cmix_sparse_rows", c10::kCUDA, &cmix_sparse_rows);

  m.def("cmix_sparse_down_one(int C, int F, Tensor act, Tensor value_fc) -> Tensor");
  m.impl("cmix_sparse_down_one", c10::kCUDA, &cmix_sparse_down_one);

  m.def("cmix_sparse_down_rows(int B, int T, int C, int F, Tensor act, Tensor value_fc) -> Tensor");
  m.impl("cmix_sparse_down_rows", c10::kCUDA, &cmix_sparse_down_rows);

  m.def("cmix_sparse_down_relu_one(int C, int F, Tensor preact, Tensor value_fc) -> Tensor");
  m.impl("cmix_sparse_down_relu_one", c10::kCUDA, &cmix_sparse_down_relu_one);

  m.def("cmix_sparse_down_relu_rows(int B, int T, int C, int F, Tensor preact, Tensor value_fc) -> Tensor");
  m.impl("cmix_sparse_down_relu_rows", c10::kCUDA, &cmix_sparse_down_relu_rows);

  m.def("cmix_sparse_down_relu_rows_t512(int B, int T, int C, int F, Tensor preact, Tensor value_fc) -> Tensor");
  m.impl("cmix_sparse_down_relu_rows_t512", c10::kCUDA, &cmix_sparse_down_relu_rows_t512);
}
