// torch ops of namespace vkwr_v1_rank (module _v1_rank_C): the RWKV-7
// low-rank adapters, with byte-identical schemas (reference
// csrc/v1/rank/torch_bindings.cpp:103-122) and input checks (:8-101).
//
// rank-in:  {w1, a1, g1, (v1)} = x_{w,a,g,(v)} . {W1, A1, G1, (V1)}^T
// rank-out: w = tanh(w1) . W2^T, a = a1 . A2^T, g = sigmoid(g1) . G2^T,
//           (v = v + (v_first - v) * sigmoid(v0 + v1 . V2^T))
// (reference csrc/v1/rank/rank_ops.cu:16-333).  Each op is one batched GEMM
// launch (3 or 4 problems) on the matrix cores; the rank-out activations are
// applied to the A operand as it is staged and rounded to fp16 there (the
// reference keeps them in fp32 inside its CUDA-core dot products).
#include "vk_torch.h"

using namespace vkt;

namespace {

void check_mat(const at::Tensor& t, int64_t r, int64_t c, const char* name, const char* msg) {
  check_half_cuda_contig(t, name);
  TORCH_CHECK(t.dim() == 2 && t.size(0) == r && t.size(1) == c, msg);
}

std::vector<at::Tensor> rank_in(int64_t M, int64_t K, const std::vector<int64_t>& R,
                                const std::vector<at::Tensor>& xs, const std::vector<at::Tensor>& ws,
                                const char* what) {
  TORCH_CHECK(M >= 0 && K >= 0 && M <= INT32_MAX && K <= INT32_MAX, what, " size out of range");
  check_device(xs[0], "xw");
  std::vector<at::Tensor> outs;
  std::vector<vkwr_gemm_problem> probs;
  for (size_t i = 0; i < xs.size(); ++i) {
    outs.push_back(at::empty({M, R[i]}, xs[i].options()));
    if (M > 0 && R[i] > 0) probs.push_back(gemm_problem(xs[i], ws[i], outs[i], M, R[i], K, VKWR_GEMM_B_NK));
  }
  if (!probs.empty()) run_gemm(probs, xs[0], what);
  return outs;
}

std::vector<at::Tensor> linear_wag_rank_in_f16(int64_t M, int64_t K, int64_t Rw, int64_t Ra, int64_t Rg,
                                               at::Tensor xw, at::Tensor xa, at::Tensor xg,
                                               at::Tensor w1_t, at::Tensor a1_t, at::Tensor g1_t) {
  check_mat(xw, M, K, "xw", "xw shape mismatch");
  check_mat(xa, M, K, "xa", "xa shape mismatch");
  check_mat(xg, M, K, "xg", "xg shape mismatch");
  check_mat(w1_t, Rw, K, "w1_t", "w1_t shape mismatch");
  check_mat(a1_t, Ra, K, "a1_t", "a1_t shape mismatch");
  check_mat(g1_t, Rg, K, "g1_t", "g1_t shape mismatch");
  return rank_in(M, K, {Rw, Ra, Rg}, {xw, xa, xg}, {w1_t, a1_t, g1_t}, "linear_wag_rank_in_f16");
}

std::vector<at::Tensor> linear_wagv_rank_in_f16(int64_t M, int64_t K, int64_t Rw, int64_t Ra, int64_t Rg,
                                                int64_t Rv, at::Tensor xw, at::Tensor xa, at::Tensor xg,
                                                at::Tensor xv, at::Tensor w1_t, at::Tensor a1_t,
                                                at::Tensor g1_t, at::Tensor v1_t) {
  check_mat(xw, M, K, "xw", "xw shape mismatch");
  check_mat(xa, M, K, "xa", "xa shape mismatch");
  check_mat(xg, M, K, "xg", "xg shape mismatch");
  check_mat(xv, M, K, "xv", "xv shape mismatch");
  check_mat(w1_t, Rw, K, "w1_t", "w1_t shape mismatch");
  check_mat(a1_t, Ra, K, "a1_t", "a1_t shape mismatch");
  check_mat(g1_t, Rg, K, "g1_t", "g1_t shape mismatch");
  check_mat(v1_t, Rv, K, "v1_t", "v1_t shape mismatch");
  return rank_in(M, K, {Rw, Ra, Rg, Rv}, {xw, xa, xg, xv}, {w1_t, a1_t, g1_t, v1_t}, "linear_wagv_rank_in_f16");
}

std::vector<at::Tensor> rank_out(int64_t M, int64_t C, const std::vector<int64_t>& Ks,
                                 const std::vector<at::Tensor>& xs, const std::vector<at::Tensor>& ws,
                                 const at::Tensor* v, const at::Tensor* v_first, const at::Tensor* v0,
                                 const char* what) {
  TORCH_CHECK(M >= 0 && C >= 0 && M <= INT32_MAX && C <= INT32_MAX, what, " size out of range");
  check_device(xs[0], "w1");
  static const int acts[4] = {VKWR_GEMM_ACT_TANH, VKWR_GEMM_ACT_NONE, VKWR_GEMM_ACT_SIGMOID, VKWR_GEMM_ACT_NONE};
  std::vector<at::Tensor> outs;
  std::vector<vkwr_gemm_problem> probs;
  for (size_t i = 0; i < xs.size(); ++i) {
    outs.push_back(at::empty({M, C}, xs[i].options()));
    if (M == 0 || C == 0) continue;
    const bool vres = i == 3;
    auto p = gemm_problem(xs[i], ws[i], outs[i], M, C, Ks[i], VKWR_GEMM_B_NK, acts[i],
                          vres ? VKWR_GEMM_EPI_VALUE_RESIDUAL : VKWR_GEMM_EPI_NONE);
    if (vres) {
      p.v = ptr<uint16_t>(*v);
      p.v_first = ptr<uint16_t>(*v_first);
      p.v0 = ptr<uint16_t>(*v0);
    }
    probs.push_back(p);
  }
  if (!probs.empty()) run_gemm(probs, xs[0], what);
  return outs;
}

std::vector<at::Tensor> linear_wag_rank_out_f16(int64_t M, int64_t C, int64_t Kw, int64_t Ka, int64_t Kg,
                                                at::Tensor w1, at::Tensor a1, at::Tensor g1,
                                                at::Tensor w2_t, at::Tensor a2_t, at::Tensor g2_t) {
  check_mat(w1, M, Kw, "w1", "w1 shape mismatch");
  check_mat(a1, M, Ka, "a1", "a1 shape mismatch");
  check_mat(g1, M, Kg, "g1", "g1 shape mismatch");
  check_mat(w2_t, C, Kw, "w2_t", "w2_t shape mismatch");
  check_mat(a2_t, C, Ka, "a2_t", "a2_t shape mismatch");
  check_mat(g2_t, C, Kg, "g2_t", "g2_t shape mismatch");
  return rank_out(M, C, {Kw, Ka, Kg}, {w1, a1, g1}, {w2_t, a2_t, g2_t}, nullptr, nullptr, nullptr,
                  "linear_wag_rank_out_f16");
}

std::vector<at::Tensor> linear_wagv_rank_out_f16(int64_t M, int64_t C, int64_t Kw, int64_t Ka, int64_t Kg,
                                                 int64_t Kv, at::Tensor w1, at::Tensor a1, at::Tensor g1,
                                                 at::Tensor v1, at::Tensor w2_t, at::Tensor a2_t,
                                                 at::Tensor g2_t, at::Tensor v2_t, at::Tensor v,
                                                 at::Tensor v_first, at::Tensor v0) {
  check_mat(w1, M, Kw, "w1", "w1 shape mismatch");
  check_mat(a1, M, Ka, "a1", "a1 shape mismatch");
  check_mat(g1, M, Kg, "g1", "g1 shape mismatch");
  check_mat(v1, M, Kv, "v1", "v1 shape mismatch");
  check_mat(w2_t, C, Kw, "w2_t", "w2_t shape mismatch");
  check_mat(a2_t, C, Ka, "a2_t", "a2_t shape mismatch");
  check_mat(g2_t, C, Kg, "g2_t", "g2_t shape mismatch");
  check_mat(v2_t, C, Kv, "v2_t", "v2_t shape mismatch");
  check_mat(v, M, C, "v", "v shape mismatch");
  check_mat(v_first, M, C, "v_first", "v_first shape mismatch");
  check_half_cuda_contig(v0, "v0");
  TORCH_CHECK(v0.dim() == 1 && v0.size(0) == C, "v0 shape mismatch");
  return rank_out(M, C, {Kw, Ka, Kg, Kv}, {w1, a1, g1, v1}, {w2_t, a2_t, g2_t, v2_t}, &v, &v_first, &v0,
                  "linear_wagv_rank_out_f16");
}

}  // namespace

TORCH_LIBRARY(vkwr_v1_rank, m) {
  m.def("linear_wag_rank_in_f16(int M, int K, int Rw, int Ra, int Rg, "
      "Tensor xw, Tensor xa, Tensor xg, Tensor w1_t, Tensor a1_t, Tensor g1_t) -> Tensor[]");
  m.impl("linear_wag_rank_in_f16", c10::kCUDA, &linear_wag_rank_in_f16);

  m.def("linear_wagv_rank_in_f16(int M, int K, int Rw, int Ra, int Rg, int Rv, "
      "Tensor xw, Tensor xa, Tensor xg, Tensor xv, "
      "Tensor w1_t, Tensor a1_t, Tensor g1_t, Tensor v1_t) -> Tensor[]");
  m.impl("linear_wagv_rank_in_f16", c10::kCUDA, &linear_wagv_rank_in_f16);

  m.def("linear_wag_rank_out_f16(int M, int C, int Kw, int Ka, int Kg, "
      "Tensor w1, Tensor a1, Tensor g1, Tensor w2_t, Tensor a2_t, Tensor g2_t) -> Tensor[]");
  m.impl("linear_wag_rank_out_f16", c10::kCUDA, &linear_wag_rank_out_f16);

  m.def("linear_wagv_rank_out_f16(int M, int C, int Kw, int Ka, int Kg, int Kv, "
      "Tensor w1, Tensor a1, Tensor g1, Tensor v1, "
      "Tensor w2_t, Tensor a2_t, Tensor g2_t, Tensor v2_t, "
      "Tensor v, Tensor v_first, Tensor v0) -> Tensor[]");
  m.impl("linear_wagv_rank_out_f16", c10::kCUDA, &linear_wagv_rank_out_f16);
}

VKT_PYMODULE(_v1_rank_C)
