// torch ops of namespace vkwr_v1_mix (module _v1_mix_C) with byte-identical
// schemas (reference csrc/v1/mix/torch_bindings.cpp:302-366) and its input
// checks (torch_bindings.cpp:8-300).  Outputs are allocated here, as the
// reference's host functions do (csrc/v1/mix/mix_ops.cu:867-1378); the work goes
// to the C ABI on the current stream.  The `threads` / `vec` arguments of the
// *_cfg and *_t1_c4096 variants are validated exactly as in the reference and
// then run the same gfx950 kernels; `half_math` selects fp16 lerp arithmetic as
// there.
#include "vk_torch.h"

using namespace vkt;

namespace {

uint16_t* h(const at::Tensor& t) { return ptr<uint16_t>(t); }

void check_shift(const at::Tensor& shift_state, int64_t B, int64_t C, const char* shape) {
  check_half_cuda_contig(shift_state, "shift_state");
  TORCH_CHECK(shift_state.dim() == 2 && shift_state.size(0) == B && shift_state.size(1) == C,
              "shift_state must have shape ", shape);
}

std::vector<at::Tensor> run_shift(int64_t B, int64_t T, int64_t C, const at::Tensor& x,
                                  at::Tensor& shift_state, const std::vector<at::Tensor>& mixv,
                                  bool half_math, const char* what) {
  check_fits_int(B, "B");
  check_fits_int(T, "T");
  check_fits_int(C, "C");
  check_device(x, "x");
  const int n = (int)mixv.size();
  std::vector<at::Tensor> outs;
  const uint16_t* mp[6];
  uint16_t* op[6];
  for (int i = 0; i < n; ++i) {
    outs.push_back(at::empty_like(x));
    mp[i] = h(mixv[i]);
    op[i] = h(outs.back());
  }
  check_status(vkwr_token_shift_mix_f16((int)B, (int)T, (int)C, h(x), h(shift_state), n, mp, op,
                                        half_math ? 1 : 0, stream()),
               what);
  return outs;
}

std::vector<at::Tensor> tmix_mix6(int64_t B, int64_t T, int64_t C, at::Tensor x,
                                  at::Tensor shift_state, at::Tensor x_r, at::Tensor x_w,
                                  at::Tensor x_k, at::Tensor x_v, at::Tensor x_a, at::Tensor x_g) {
  TORCH_CHECK((C % 2) == 0, "C must be even");
  check_3d(x, B, T, C, "x");
  check_shift(shift_state, B, C, "[B,C]");
  check_vec(x_r, C, "x_r");
  check_vec(x_w, C, "x_w");
  check_vec(x_k, C, "x_k");
  check_vec(x_v, C, "x_v");
  check_vec(x_a, C, "x_a");
  check_vec(x_g, C, "x_g");
  return run_shift(B, T, C, x, shift_state, {x_r, x_w, x_k, x_v, x_a, x_g}, false, "tmix_mix6");
}

std::vector<at::Tensor> tmix_mix6_cfg(int64_t B, int64_t T, int64_t C, at::Tensor x,
                                      at::Tensor shift_state, at::Tensor x_r, at::Tensor x_w,
                                      at::Tensor x_k, at::Tensor x_v, at::Tensor x_a,
                                      at::Tensor x_g, int64_t threads) {
  TORCH_CHECK((C % 2) == 0, "C must be even");
  TORCH_CHECK(threads == 128 || threads == 256 || threads == 512 || threads == 1024, "unsupported threads");
  check_3d(x, B, T, C, "x");
  check_shift(shift_state, B, C, "[B,C]");
  check_vec(x_r, C, "x_r");
  check_vec(x_w, C, "x_w");
  check_vec(x_k, C, "x_k");
  check_vec(x_v, C, "x_v");
  check_vec(x_a, C, "x_a");
  check_vec(x_g, C, "x_g");
  return run_shift(B, T, C, x, shift_state, {x_r, x_w, x_k, x_v, x_a, x_g}, false, "tmix_mix6_cfg");
}

std::vector<at::Tensor> tmix_mix6_t1_c4096(int64_t B, at::Tensor x, at::Tensor shift_state,
                                           at::Tensor x_r, at::Tensor x_w, at::Tensor x_k,
                                           at::Tensor x_v, at::Tensor x_a, at::Tensor x_g,
                                           int64_t threads, int64_t vec, bool half_math) {
  TORCH_CHECK(threads == 128 || threads == 256 || threads == 512 || threads == 1024, "unsupported threads");
  TORCH_CHECK(vec == 1 || vec == 2 || vec == 4 || vec == 8, "unsupported vec");
  check_3d(x, B, 1, 4096, "x");
  check_shift(shift_state, B, 4096, "[B,4096]");
  check_vec(x_r, 4096, "x_r");
  check_vec(x_w, 4096, "x_w");
  check_vec(x_k, 4096, "x_k");
  check_vec(x_v, 4096, "x_v");
  check_vec(x_a, 4096, "x_a");
  check_vec(x_g, 4096, "x_g");
  return run_shift(B, 1, 4096, x, shift_state, {x_r, x_w, x_k, x_v, x_a, x_g}, half_math,
                   "tmix_mix6_t1_c4096");
}

std::vector<at::Tensor> run_gate(int64_t B, int64_t T, int64_t C, int64_t H, const at::Tensor& k,
                                 const at::Tensor& k_k, const at::Tensor& a0, const at::Tensor& a12,
                                 const at::Tensor& k_a, const at::Tensor* x, at::Tensor* shift,
                                 const char* what) {
  check_fits_int(B, "B");
  check_fits_int(T, "T");
  check_fits_int(C, "C");
  check_device(k, "k");
  auto new_k = at::empty_like(k);
  auto neg_kk = at::empty_like(k);
  auto kka = at::empty_like(k);
  check_status(vkwr_tmix_kk_a_gate_f16((int)B, (int)T, (int)C, (int)H, h(k), h(k_k), h(a0), h(a12),
                                       h(k_a), x ? h(*x) : nullptr, shift ? h(*shift) : nullptr,
                                       h(new_k), h(neg_kk), h(kka), stream()),
               what);
  return {new_k, neg_kk, kka};
}

std::vector<at::Tensor> tmix_kk_a_gate(int64_t B, int64_t T, int64_t C, int64_t H, at::Tensor k,
                                       at::Tensor k_k, at::Tensor a0, at::Tensor a12, at::Tensor k_a) {
  TORCH_CHECK(C == H * 64, "only head size 64 is supported");
  check_3d(k, B, T, C, "k");
  check_vec(k_k, C, "k_k");
  check_vec(a0, C, "a0");
  check_3d(a12, B, T, C, "a12");
  check_vec(k_a, C, "k_a");
  return run_gate(B, T, C, H, k, k_k, a0, a12, k_a, nullptr, nullptr, "tmix_kk_a_gate");
}

std::vector<at::Tensor> tmix_kk_a_gate_update_shift(int64_t B, int64_t T, int64_t C, int64_t H,
                                                    at::Tensor k, at::Tensor k_k, at::Tensor a0,
                                                    at::Tensor a12, at::Tensor k_a, at::Tensor x,
                                                    at::Tensor shift_state) {
  TORCH_CHECK(T == 1, "tmix_kk_a_gate_update_shift currently requires T=1");
  TORCH_CHECK(C == H * 64, "only head size 64 is supported");
  check_3d(k, B, T, C, "k");
  check_vec(k_k, C, "k_k");
  check_vec(a0, C, "a0");
  check_3d(a12, B, T, C, "a12");
  check_vec(k_a, C, "k_a");
  check_3d(x, B, T, C, "x");
  check_shift(shift_state, B, C, "[B,C]");
  return run_gate(B, T, C, H, k, k_k, a0, a12, k_a, &x, &shift_state, "tmix_kk_a_gate_update_shift");
}

at::Tensor tmix_lnx_rkvres_xg(int64_t B, int64_t T, int64_t C, int64_t H, at::Tensor x,
                              at::Tensor r, at::Tensor k, at::Tensor v, at::Tensor r_k,
                              at::Tensor weight, at::Tensor bias, at::Tensor g) {
  TORCH_CHECK(C == H * 64, "only head size 64 is supported");
  check_3d(x, B, T, C, "x");
  check_3d(r, B, T, C, "r");
  check_3d(k, B, T, C, "k");
  check_3d(v, B, T, C, "v");
  check_3d(g, B, T, C, "g");
  check_vec(r_k, C, "r_k");
  check_vec(weight, C, "weight");
  check_vec(bias, C, "bias");
  check_fits_int(B, "B");
  check_fits_int(T, "T");
  check_device(x, "x");
  auto out = at::empty_like(x);
  check_status(vkwr_tmix_groupnorm_bonus_gate_f16((int)B, (int)T, (int)C, (int)H, h(x), h(r), h(k),
                                                  h(v), h(r_k), h(weight), h(bias), h(g), h(out),
                                                  stream()),
               "tmix_lnx_rkvres_xg");
  return out;
}

at::Tensor tmix_vres_gate(int64_t B, int64_t T, int64_t C, at::Tensor v, at::Tensor v_first,
                          at::Tensor v0, at::Tensor v12) {
  check_3d(v, B, T, C, "v");
  check_3d(v_first, B, T, C, "v_first");
  check_vec(v0, C, "v0");
  check_3d(v12, B, T, C, "v12");
  check_fits_int(C, "C");
  check_device(v, "v");
  auto out = at::empty_like(v);
  if (v.numel() > 0)
    check_status(vkwr_tmix_vres_gate_f16(B * T, (int)C, h(v), h(v_first), h(v0), h(v12), h(out),
                                         stream()),
                 "tmix_vres_gate");
  return out;
}

at::Tensor cmix_mix(int64_t B, int64_t T, int64_t C, at::Tensor x, at::Tensor shift_state,
                    at::Tensor x_k) {
  TORCH_CHECK((C % 2) == 0, "C must be even");
  check_3d(x, B, T, C, "x");
  check_shift(shift_state, B, C, "[B,C]");
  check_vec(x_k, C, "x_k");
  return run_shift(B, T, C, x, shift_state, {x_k}, false, "cmix_mix")[0];
}

at::Tensor cmix_mix_cfg(int64_t B, int64_t T, int64_t C, at::Tensor x, at::Tensor shift_state,
                        at::Tensor x_k, int64_t threads) {
  TORCH_CHECK((C % 2) == 0, "C must be even");
  TORCH_CHECK(threads == 128 || threads == 256 || threads == 512 || threads == 1024, "unsupported threads");
  check_3d(x, B, T, C, "x");
  check_shift(shift_state, B, C, "[B,C]");
  check_vec(x_k, C, "x_k");
  return run_shift(B, T, C, x, shift_state, {x_k}, false, "cmix_mix_cfg")[0];
}

at::Tensor run_act(const at::Tensor& x, int act, const char* what) {
  check_half_cuda_contig(x, "x");
  TORCH_CHECK((x.numel() % 2) == 0, "x.numel() must be even");
  check_device(x, "x");
  auto out = at::empty_like(x);
  check_status(vkwr_activation_f16(act, x.numel(), h(x), h(out), stream()), what);
  return out;
}

at::Tensor relu_square(at::Tensor x) { return run_act(x, VKWR_ACT_RELU_SQUARE, "relu_square"); }
at::Tensor act_tanh(at::Tensor x) { return run_act(x, VKWR_ACT_TANH, "act_tanh"); }
at::Tensor act_sigmoid(at::Tensor x) { return run_act(x, VKWR_ACT_SIGMOID, "act_sigmoid"); }

at::Tensor add_vec(int64_t C, at::Tensor x, at::Tensor vec) {
  check_half_cuda_contig(x, "x");
  check_vec(vec, C, "vec");
  TORCH_CHECK(x.numel() > 0 && (x.numel() % 2) == 0, "x.numel() must be positive and even");
  TORCH_CHECK(x.size(-1) == C, "x last dim must equal C");
  check_fits_int(C, "C");
  check_device(x, "x");
  auto out = at::empty_like(x);
  check_status(vkwr_add_vec_f16(x.numel(), (int)C, h(x), h(vec), h(out), stream()), "add_vec");
  return out;
}

}  // namespace

// The sparse channel-mix (FFN) ops of this namespace are registered by
// ffn_bindings.cpp, linked into this same module (they run on the GEMM kernels).
TORCH_LIBRARY(vkwr_v1_mix, m) {
  m.def("tmix_mix6(int B, int T, int C, Tensor x, Tensor(a!) shift_state, "
      "Tensor x_r, Tensor x_w, Tensor x_k, Tensor x_v, Tensor x_a, Tensor x_g) -> Tensor[]");
  m.impl("tmix_mix6", c10::kCUDA, &tmix_mix6);

  m.def("tmix_mix6_cfg(int B, int T, int C, Tensor x, Tensor(a!) shift_state, "
      "Tensor x_r, Tensor x_w, Tensor x_k, Tensor x_v, Tensor x_a, Tensor x_g, int threads) -> Tensor[]");
  m.impl("tmix_mix6_cfg", c10::kCUDA, &tmix_mix6_cfg);

  m.def("tmix_mix6_t1_c4096(int B, Tensor x, Tensor(a!) shift_state, "
      "Tensor x_r, Tensor x_w, Tensor x_k, Tensor x_v, Tensor x_a, Tensor x_g, int threads, int vec, bool half_math=False) -> Tensor[]");
  m.impl("tmix_mix6_t1_c4096", c10::kCUDA, &tmix_mix6_t1_c4096);

  m.def("tmix_kk_a_gate(int B, int T, int C, int H, Tensor k, Tensor k_k, Tensor a0, Tensor a12, Tensor k_a) -> Tensor[]");
  m.impl("tmix_kk_a_gate", c10::kCUDA, &tmix_kk_a_gate);

  m.def("tmix_kk_a_gate_update_shift(int B, int T, int C, int H, Tensor k, Tensor k_k, Tensor a0, Tensor a12, Tensor k_a, Tensor x, Tensor(a!) shift_state) -> Tensor[]");
  m.impl("tmix_kk_a_gate_update_shift", c10::kCUDA, &tmix_kk_a_gate_update_shift);

  m.def("tmix_lnx_rkvres_xg(int B, int T, int C, int H, Tensor x, Tensor r, Tensor k, Tensor v, "
      "Tensor r_k, Tensor weight, Tensor bias, Tensor g) -> Tensor");
  m.impl("tmix_lnx_rkvres_xg", c10::kCUDA, &tmix_lnx_rkvres_xg);

  m.def("tmix_vres_gate(int B, int T, int C, Tensor v, Tensor v_first, Tensor v0, Tensor v12) -> Tensor");
  m.impl("tmix_vres_gate", c10::kCUDA, &tmix_vres_gate);

  m.def("cmix_mix(int B, int T, int C, Tensor x, Tensor(a!) shift_state, Tensor x_k) -> Tensor");
  m.impl("cmix_mix", c10::kCUDA, &cmix_mix);

  m.def("cmix_mix_cfg(int B, int T, int C, Tensor x, Tensor(a!) shift_state, Tensor x_k, int threads) -> Tensor");
  m.impl("cmix_mix_cfg", c10::kCUDA, &cmix_mix_cfg);

  m.def("relu_square(Tensor x) -> Tensor");
  m.impl("relu_square", c10::kCUDA, &relu_square);

  m.def("act_tanh(Tensor x) -> Tensor");
  m.impl("act_tanh", c10::kCUDA, &act_tanh);

  m.def("act_sigmoid(Tensor x) -> Tensor");
  m.impl("act_sigmoid", c10::kCUDA, &act_sigmoid);

  m.def("add_vec(int C, Tensor x, Tensor vec) -> Tensor");
  m.impl("add_vec", c10::kCUDA, &add_vec);
}

VKT_PYMODULE(_v1_mix_C)
