// torch ops of namespace vkwr_v1_linear (module _v1_linear_C): the reference's
// 17 fp16 linear ops with byte-identical schemas (reference
// csrc/v1/linear/torch_bindings.cpp:174-225) and input checks
// (torch_bindings.cpp:8-172, csrc/v1/linear/linear_ops.cu:973-1833).
//
// Every op computes the same function on gfx950 -- an fp16 GEMM with fp32
// accumulation on the matrix cores (vkwr_gemm_f16) -- whatever kernel family
// the reference dispatched to (cuBLAS, cuBLASLt, CUDA-core tiles, WMMA, split-K
// GEMV).  The tuning arguments (row_tile, out_tile, threads, use4, chunk_k,
// tile_cols, workspace_mb, algo_index) are validated against the same accepted
// sets as the reference, so a call that fails there fails here with the same
// message; they do not change the result.
#include <algorithm>
#include <set>
#include <tuple>

#include "vk_torch.h"

using namespace vkt;

namespace {

std::vector<int64_t> out_sizes(const at::Tensor& x, int64_t n) {
  std::vector<int64_t> s(x.sizes().begin(), x.sizes().end());
  s.back() = n;
  return s;
}

// y[..., N] = x[..., K] . W with W [K,N] (kn) or [N,K] (nk).
at::Tensor linear(const at::Tensor& x, const at::Tensor& w, int layout, const char* what,
                  int a_act = VKWR_GEMM_ACT_NONE) {
  const int64_t K = x.size(-1);
  const int64_t N = layout == VKWR_GEMM_B_KN ? w.size(1) : w.size(0);
  TORCH_CHECK(K <= INT32_MAX && N <= INT32_MAX, what, " K/N too large");
  const int64_t M = K > 0 ? x.numel() / K : 0;
  TORCH_CHECK(M <= INT32_MAX, what, " M too large");
  check_device(x, "x");
  auto y = at::empty(out_sizes(x, N), x.options());
  if (M == 0 || N == 0) return y;
  std::vector<vkwr_gemm_problem> p{gemm_problem(x, w, y, M, N, K, layout, a_act)};
  run_gemm(p, x, what);
  return y;
}

void check_kn(const at::Tensor& x, const at::Tensor& weight, const char* fn) {
  check_half_cuda_contig(x, "x");
  check_half_cuda_contig(weight, "weight");
  TORCH_CHECK(x.dim() >= 2, "x must have at least 2 dims");
  TORCH_CHECK(weight.dim() == 2, "weight must have shape [K, N]");
  TORCH_CHECK(x.size(-1) == weight.size(0), fn, " shape mismatch");
}

void check_nk(const at::Tensor& x, const at::Tensor& w, const char* wname, const char* fn) {
  check_half_cuda_contig(x, "x");
  check_half_cuda_contig(w, wname);
  TORCH_CHECK(x.dim() >= 2, "x must have at least 2 dims");
  TORCH_CHECK(w.dim() == 2, wname, " must have shape [N, K]");
  TORCH_CHECK(x.size(-1) == w.size(1), fn, " shape mismatch");
}

at::Tensor linear_f16(at::Tensor x, at::Tensor weight) {
  check_kn(x, weight, "linear_f16");
  return linear(x, weight, VKWR_GEMM_B_KN, "linear_f16");
}

at::Tensor linear_f16_orig(at::Tensor x, at::Tensor weight_orig) {
  check_nk(x, weight_orig, "weight_orig", "linear_f16_orig");
  return linear(x, weight_orig, VKWR_GEMM_B_NK, "linear_f16_orig");
}

at::Tensor linear_orig_rows_f16(at::Tensor x, at::Tensor weight_orig, int64_t row_tile, int64_t out_tile) {
  check_nk(x, weight_orig, "weight_orig", "linear_orig_rows_f16");
  // Accepted (row_tile, out_tile) pairs (reference linear_ops.cu:1105-1125).
  static const std::set<std::pair<int64_t, int64_t>> ok = {
      {1, 2}, {1, 4}, {1, 8}, {1, 16}, {2, 2}, {2, 4}, {2, 8}, {3, 2}, {3, 4}, {3, 8},
      {4, 2}, {4, 4}, {4, 8}, {8, 2}, {8, 4}, {16, 1}, {16, 2}, {16, 4}};
  TORCH_CHECK(ok.count({row_tile, out_tile}), "unsupported linear_orig_rows_f16 row_tile/out_tile");
  return linear(x, weight_orig, VKWR_GEMM_B_NK, "linear_orig_rows_f16");
}

at::Tensor linear_orig_rows_cfg_f16(at::Tensor x, at::Tensor weight_orig, int64_t threads, int64_t row_tile,
                                    int64_t out_tile) {
  check_nk(x, weight_orig, "weight_orig", "linear_orig_rows_cfg_f16");
  // Accepted (threads, row_tile, out_tile) (reference linear_ops.cu:1127-1148).
  static const std::set<std::tuple<int64_t, int64_t, int64_t>> ok = {
      {64, 1, 4}, {64, 1, 8}, {128, 1, 8}, {256, 1, 1}, {32, 4, 4}, {64, 4, 4}, {96, 4, 4},
      {32, 4, 8}, {64, 4, 8}, {32, 8, 4}, {64, 8, 4}, {32, 2, 4}, {64, 2, 2}, {64, 2, 4},
      {32, 3, 4}, {64, 3, 4}, {96, 3, 4}, {32, 3, 8}, {64, 3, 8}};
  TORCH_CHECK(ok.count({threads, row_tile, out_tile}),
              "unsupported linear_orig_rows_cfg_f16 threads/row_tile/out_tile");
  return linear(x, weight_orig, VKWR_GEMM_B_NK, "linear_orig_rows_cfg_f16");
}

at::Tensor linear_orig_rows_exact_f16(at::Tensor x, at::Tensor weight_orig, int64_t threads, int64_t out_tile,
                                      bool use4) {
  check_nk(x, weight_orig, "weight_orig", "linear_orig_rows_exact_f16");
  // Accepted row counts / configurations (reference linear_ops.cu:1151-1212).
  const int64_t rows = x.numel() / x.size(-1);
  const bool ok1 = rows == 1 && threads == 128 && out_tile == 2;
  const bool ok2 = rows == 2 && ((use4 && threads == 64 && out_tile == 2) ||
                                 (use4 && threads == 256 && out_tile == 1) ||
                                 (!use4 && threads == 128 && out_tile == 2));
  TORCH_CHECK(ok1 || ok2, "unsupported linear_orig_rows_exact_f16 rows/threads/out_tile/use4");
  const char* fn = rows == 1 ? "linear_orig_row1_exact_f16" : "linear_orig_row2_exact_f16";
  TORCH_CHECK((weight_orig.size(0) % out_tile) == 0, fn, " requires N divisible by out_tile");
  TORCH_CHECK((x.size(-1) % (use4 ? 4 : 2)) == 0, fn, " unsupported K alignment");
  return linear(x, weight_orig, VKWR_GEMM_B_NK, fn);
}

at::Tensor linear_orig_wmma16_f16(at::Tensor x, at::Tensor weight_orig) {
  check_nk(x, weight_orig, "weight_orig", "linear_orig_wmma16_f16");
  TORCH_CHECK((x.size(-1) % 16) == 0 && (weight_orig.size(0) % 16) == 0,
              "linear_orig_wmma16_f16 requires K/N multiple of 16");
  return linear(x, weight_orig, VKWR_GEMM_B_NK, "linear_orig_wmma16_f16");
}

at::Tensor linear_f16_orig_lt(at::Tensor x, at::Tensor weight_orig) {
  check_nk(x, weight_orig, "weight_orig", "linear_f16_orig_lt");
  return linear(x, weight_orig, VKWR_GEMM_B_NK, "linear_f16_orig_lt");
}

at::Tensor linear_f16_orig_lt_cfg(at::Tensor x, at::Tensor weight_orig, int64_t workspace_mb, int64_t algo_index) {
  check_nk(x, weight_orig, "weight_orig", "linear_f16_orig_lt_cfg");
  TORCH_CHECK(workspace_mb >= 0 && workspace_mb <= 1024, "workspace_mb out of range");
  TORCH_CHECK(algo_index >= 0 && algo_index < 64, "algo_index out of range");
  return linear(x, weight_orig, VKWR_GEMM_B_NK, "linear_f16_orig_lt_cfg");
}

at::Tensor linear_f16_lt(at::Tensor x, at::Tensor weight) {
  check_kn(x, weight, "linear_f16_lt");
  return linear(x, weight, VKWR_GEMM_B_KN, "linear_f16_lt");
}

// ---- M = 1 split-K GEMV family (reference linear_ops.cu:1394-1692)

const std::set<int64_t>& m1_cfg_chunks() {
  static const std::set<int64_t> s = {64, 96, 112, 128, 144, 152, 160, 168, 176, 184, 192,
                                      208, 224, 256, 384, 512, 640, 768, 896, 1024, 2048, 4096};
  return s;
}

at::Tensor m1_linear(const at::Tensor& x, const at::Tensor& weight, const char* fn) {
  TORCH_CHECK(weight.size(1) % 64 == 0, "linear_f16_m1_splitk requires N multiple of 64");
  return linear(x, weight, VKWR_GEMM_B_KN, fn);
}

void check_m1(const at::Tensor& x, const at::Tensor& weight, const char* fn) {
  check_kn(x, weight, fn);
  TORCH_CHECK(x.numel() == x.size(-1), fn, " requires M=1");
}

at::Tensor linear_f16_m1_splitk(at::Tensor x, at::Tensor weight) {
  check_m1(x, weight, "linear_f16_m1_splitk");
  return m1_linear(x, weight, "linear_f16_m1_splitk");
}

at::Tensor linear_f16_m1_splitk_cfg(at::Tensor x, at::Tensor weight, int64_t chunk_k) {
  check_m1(x, weight, "linear_f16_m1_splitk_cfg");
  TORCH_CHECK(m1_cfg_chunks().count(chunk_k), "unsupported chunk_k");
  return m1_linear(x, weight, "linear_f16_m1_splitk_cfg");
}

at::Tensor linear_f16_m1_splitk_tile(at::Tensor x, at::Tensor weight, int64_t chunk_k, int64_t tile_cols) {
  check_m1(x, weight, "linear_f16_m1_splitk_tile");
  static const std::set<int64_t> t64 = {64, 96, 112, 128, 144, 152, 160, 168, 176, 184,
                                        192, 208, 224, 256, 384, 512, 640, 768, 896};
  if (tile_cols == 64) {
    TORCH_CHECK(t64.count(chunk_k), "unsupported chunk_k");
  } else if (tile_cols == 128) {
    TORCH_CHECK(t64.count(chunk_k) || chunk_k == 1024, "unsupported chunk_k");
  } else {
    TORCH_CHECK(tile_cols == 256, "unsupported tile_cols");
    TORCH_CHECK(m1_cfg_chunks().count(chunk_k), "unsupported chunk_k");
  }
  return m1_linear(x, weight, "linear_f16_m1_splitk_tile");
}

at::Tensor linear_f16_m1_splitk_warpred_tile(at::Tensor x, at::Tensor weight, int64_t chunk_k, int64_t tile_cols) {
  check_m1(x, weight, "linear_f16_m1_splitk_warpred_tile");
  static const std::set<int64_t> ok = {64, 96, 112, 128, 144, 152, 160, 168, 176, 184, 192, 208, 224, 256};
  if (tile_cols != 64 && tile_cols != 128) TORCH_CHECK(tile_cols == 256, "unsupported warpred tile_cols");
  TORCH_CHECK(ok.count(chunk_k), "unsupported warpred chunk_k");
  return m1_linear(x, weight, "linear_f16_m1_splitk_warpred_tile");
}

at::Tensor linear_f16_rows_splitk(at::Tensor x, at::Tensor weight, int64_t chunk_k) {
  check_kn(x, weight, "linear_f16_rows_splitk");
  TORCH_CHECK(chunk_k == 128 || chunk_k == 256 || chunk_k == 512 || chunk_k == 1024, "unsupported chunk_k");
  TORCH_CHECK(weight.size(1) % 64 == 0, "linear_f16_rows_splitk requires N multiple of 64");
  return linear(x, weight, VKWR_GEMM_B_KN, "linear_f16_rows_splitk");
}

// ---- weight_t [N,K] family (reference linear_ops.cu:1738-1833)

at::Tensor linear_t_f16(at::Tensor x, at::Tensor weight_t) {
  check_nk(x, weight_t, "weight_t", "linear_t_f16");
  return linear(x, weight_t, VKWR_GEMM_B_NK, "linear_t_f16");
}

// The reference implements these two only for small-rank rank-out shapes.
void check_small_rank(const at::Tensor& x, const at::Tensor& weight_t, const char* fn) {
  const int64_t K = x.size(-1), N = weight_t.size(0);
  const int64_t M = K > 0 ? x.numel() / K : 0;
  if (M == 0 || N == 0 || K == 0) return;
  TORCH_CHECK(K <= 512 && N >= 1024 && M <= 4, fn, " currently supports only small-rank rank-out");
}

at::Tensor linear_t_act_f16(at::Tensor x, at::Tensor weight_t, int64_t act) {
  check_nk(x, weight_t, "weight_t", "linear_t_act_f16");
  TORCH_CHECK(act == 1 || act == 2, "act must be 1=tanh or 2=sigmoid");
  check_small_rank(x, weight_t, "linear_t_act_f16");
  return linear(x, weight_t, VKWR_GEMM_B_NK, "linear_t_act_f16",
                act == 1 ? VKWR_GEMM_ACT_TANH : VKWR_GEMM_ACT_SIGMOID);
}

at::Tensor linear_t_vres_f16(at::Tensor x, at::Tensor weight_t, at::Tensor v, at::Tensor v_first, at::Tensor v0) {
  check_half_cuda_contig(x, "x");
  check_half_cuda_contig(weight_t, "weight_t");
  check_half_cuda_contig(v, "v");
  check_half_cuda_contig(v_first, "v_first");
  check_half_cuda_contig(v0, "v0");
  TORCH_CHECK(x.dim() >= 2, "x must have at least 2 dims");
  TORCH_CHECK(weight_t.dim() == 2, "weight_t must have shape [N, K]");
  TORCH_CHECK(x.size(-1) == weight_t.size(1), "linear_t_vres_f16 shape mismatch");
  TORCH_CHECK(v.sizes() == v_first.sizes(), "v/v_first shape mismatch");
  TORCH_CHECK(v.dim() >= 2 && v.size(-1) == weight_t.size(0), "v shape mismatch");
  TORCH_CHECK(v0.dim() == 1 && v0.size(0) == weight_t.size(0), "v0 shape mismatch");
  const int64_t K = x.size(-1), N = weight_t.size(0);
  TORCH_CHECK(K <= INT32_MAX && N <= INT32_MAX, "linear_t_vres_f16 K/N too large");
  const int64_t M = K > 0 ? x.numel() / K : 0;
  TORCH_CHECK(v.numel() == M * N, "v shape mismatch");
  check_device(x, "x");
  auto y = at::empty_like(v);
  if (M == 0 || N == 0 || K == 0) return y;
  TORCH_CHECK(K <= 512 && N >= 1024 && M <= 4, "linear_t_vres_f16 currently supports only small-rank rank-out");
  auto p = gemm_problem(x, weight_t, y, M, N, K, VKWR_GEMM_B_NK, VKWR_GEMM_ACT_NONE,
                        VKWR_GEMM_EPI_VALUE_RESIDUAL);
  p.v = ptr<uint16_t>(v);
  p.v_first = ptr<uint16_t>(v_first);
  p.v0 = ptr<uint16_t>(v0);
  std::vector<vkwr_gemm_problem> probs{p};
  run_gemm(probs, x, "linear_t_vres_f16");
  return y;
}

}  // namespace

TORCH_LIBRARY(vkwr_v1_linear, m) {
  m.def("linear_f16(Tensor x, Tensor weight) -> Tensor");
  m.impl("linear_f16", c10::kCUDA, &linear_f16);

  m.def("linear_f16_orig(Tensor x, Tensor weight_orig) -> Tensor");
  m.impl("linear_f16_orig", c10::kCUDA, &linear_f16_orig);

  m.def("linear_orig_rows_f16(Tensor x, Tensor weight_orig, int row_tile, int out_tile) -> Tensor");
  m.impl("linear_orig_rows_f16", c10::kCUDA, &linear_orig_rows_f16);

  m.def("linear_orig_rows_cfg_f16(Tensor x, Tensor weight_orig, int threads, int row_tile, int out_tile) -> Tensor");
  m.impl("linear_orig_rows_cfg_f16", c10::kCUDA, &linear_orig_rows_cfg_f16);

  m.def("linear_orig_rows_exact_f16(Tensor x, Tensor weight_orig, int threads, int out_tile, bool use4) -> Tensor");
  m.impl("linear_orig_rows_exact_f16", c10::kCUDA, &linear_orig_rows_exact_f16);

  m.def("linear_orig_wmma16_f16(Tensor x, Tensor weight_orig) -> Tensor");
  m.impl("linear_orig_wmma16_f16", c10::kCUDA, &linear_orig_wmma16_f16);

  m.def("linear_f16_orig_lt(Tensor x, Tensor weight_orig) -> Tensor");
  m.impl("linear_f16_orig_lt", c10::kCUDA, &linear_f16_orig_lt);

  m.def("linear_f16_orig_lt_cfg(Tensor x, Tensor weight_orig, int workspace_mb, int algo_index) -> Tensor");
  m.impl("linear_f16_orig_lt_cfg", c10::kCUDA, &linear_f16_orig_lt_cfg);

  m.def("linear_f16_lt(Tensor x, Tensor weight) -> Tensor");
  m.impl("linear_f16_lt", c10::kCUDA, &linear_f16_lt);

  m.def("linear_f16_m1_splitk(Tensor x, Tensor weight) -> Tensor");
  m.impl("linear_f16_m1_splitk", c10::kCUDA, &linear_f16_m1_splitk);

  m.def("linear_f16_m1_splitk_cfg(Tensor x, Tensor weight, int chunk_k) -> Tensor");
  m.impl("linear_f16_m1_splitk_cfg", c10::kCUDA, &linear_f16_m1_splitk_cfg);

  m.def("linear_f16_m1_splitk_tile(Tensor x, Tensor weight, int chunk_k, int tile_cols) -> Tensor");
  m.impl("linear_f16_m1_splitk_tile", c10::kCUDA, &linear_f16_m1_splitk_tile);

  m.def("linear_f16_m1_splitk_warpred_tile(Tensor x, Tensor weight, int chunk_k, int tile_cols) -> Tensor");
  m.impl("linear_f16_m1_splitk_warpred_tile", c10::kCUDA, &linear_f16_m1_splitk_warpred_tile);

  m.def("linear_f16_rows_splitk(Tensor x, Tensor weight, int chunk_k) -> Tensor");
  m.impl("linear_f16_rows_splitk", c10::kCUDA, &linear_f16_rows_splitk);

  m.def("linear_t_f16(Tensor x, Tensor weight_t) -> Tensor");
  m.impl("linear_t_f16", c10::kCUDA, &linear_t_f16);

  m.def("linear_t_act_f16(Tensor x, Tensor weight_t, int act) -> Tensor");
  m.impl("linear_t_act_f16", c10::kCUDA, &linear_t_act_f16);

  m.def("linear_t_vres_f16(Tensor x, Tensor weight_t, Tensor v, Tensor v_first, Tensor v0) -> Tensor");
  m.impl("linear_t_vres_f16", c10::kCUDA, &linear_t_vres_f16);
}

VKT_PYMODULE(_v1_linear_C)
