// torch ops of namespace vkwr_v1_norm (module _v1_norm_C): the reference's 13
// LayerNorm ops with byte-identical schemas (reference
// csrc/v1/norm/torch_bindings.cpp:231-270) and its input checks
// (torch_bindings.cpp:8-229).  Outputs are allocated here, as the reference's
// host functions do (csrc/v1/norm/norm_ops.cu:866-1340); the work goes to the
// C ABI on the current stream.  The `threads` and `_small*` / `_scalar_stats`
// variants are the reference's tuning knobs: they are validated exactly as
// there and then run the same gfx950 kernels (one workgroup per row).
#include "vk_torch.h"

using namespace vkt;

namespace {

uint16_t* h(const at::Tensor& t) { return ptr<uint16_t>(t); }

void check_bf16_cuda_contig(const at::Tensor& x, const char* name) {
  TORCH_CHECK(x.is_cuda(), name, " must be CUDA");
  TORCH_CHECK(x.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(x.scalar_type() == at::kBFloat16, name, " must be bf16");
}

at::Tensor run_ln(const at::Tensor& x, const at::Tensor* residual, const at::Tensor& weight,
                  const at::Tensor& bias, double eps, at::Tensor* x_out, const char* what) {
  check_device(x, "x");
  auto y = at::empty_like(x);
  const int64_t C = x.size(-1);
  const int64_t rows = C > 0 ? x.numel() / C : 0;
  check_status(vkwr_layer_norm_f16(rows, (int)C, h(x), residual ? h(*residual) : nullptr,
                                   h(weight), h(bias), (float)eps, x_out ? h(*x_out) : nullptr,
                                   h(y), stream()),
               what);
  return y;
}

at::Tensor layer_norm_f16(at::Tensor x, at::Tensor weight, at::Tensor bias, double eps) {
  check_half_cuda_contig(x, "x");
  check_half_cuda_contig(weight, "weight");
  check_half_cuda_contig(bias, "bias");
  TORCH_CHECK(x.dim() >= 1, "x must have at least 1 dim");
  const int64_t c = x.size(-1);
  TORCH_CHECK(weight.dim() == 1 && weight.size(0) == c, "weight shape mismatch");
  TORCH_CHECK(bias.dim() == 1 && bias.size(0) == c, "bias shape mismatch");
  TORCH_CHECK(c > 0 && c <= 8192, "unsupported C");
  return run_ln(x, nullptr, weight, bias, eps, nullptr, "layer_norm_f16");
}

at::Tensor layer_norm_f16_small_common(const at::Tensor& x, const at::Tensor& weight,
                                       const at::Tensor& bias, double eps, const char* msg) {
  check_half_cuda_contig(x, "x");
  check_half_cuda_contig(weight, "weight");
  check_half_cuda_contig(bias, "bias");
  TORCH_CHECK(x.dim() >= 1, "x must have at least 1 dim");
  const int64_t c = x.size(-1);
  TORCH_CHECK(c == 4096, msg);
  TORCH_CHECK(weight.dim() == 1 && weight.size(0) == c, "weight shape mismatch");
  TORCH_CHECK(bias.dim() == 1 && bias.size(0) == c, "bias shape mismatch");
  return run_ln(x, nullptr, weight, bias, eps, nullptr, "layer_norm_f16_small");
}

at::Tensor layer_norm_f16_small(at::Tensor x, at::Tensor weight, at::Tensor bias, double eps) {
  return layer_norm_f16_small_common(x, weight, bias, eps, "small LN currently requires C=4096");
}

at::Tensor layer_norm_f16_small512(at::Tensor x, at::Tensor weight, at::Tensor bias, double eps) {
  return layer_norm_f16_small_common(x, weight, bias, eps, "small512 LN currently requires C=4096");
}

at::Tensor emb_ln0_bf16_to_f16(at::Tensor emb, at::Tensor weight, at::Tensor bias, double eps) {
  check_bf16_cuda_contig(emb, "emb");
  check_bf16_cuda_contig(weight, "weight");
  check_bf16_cuda_contig(bias, "bias");
  TORCH_CHECK(emb.dim() == 2, "emb must have shape [V, C]");
  const int64_t c = emb.size(1);
  TORCH_CHECK(weight.dim() == 1 && weight.size(0) == c, "weight shape mismatch");
  TORCH_CHECK(bias.dim() == 1 && bias.size(0) == c, "bias shape mismatch");
  TORCH_CHECK(emb.size(0) <= INT32_MAX && c <= INT32_MAX, "emb shape too large");
  check_device(emb, "emb");
  auto out = at::empty(emb.sizes(), emb.options().dtype(at::kHalf));
  check_status(vkwr_emb_ln0_bf16_to_f16(emb.size(0), (int)c, h(emb), h(weight), h(bias),
                                        (float)eps, h(out), stream()),
               "emb_ln0_bf16_to_f16");
  return out;
}

at::Tensor add_f16(at::Tensor x, at::Tensor y) {
  check_half_cuda_contig(x, "x");
  check_half_cuda_contig(y, "y");
  TORCH_CHECK(x.sizes() == y.sizes(), "add_f16 shape mismatch");
  TORCH_CHECK((x.numel() % 2) == 0, "add_f16 requires even numel");
  check_device(x, "x");
  auto out = at::empty_like(x);
  check_status(vkwr_add_f16(x.numel(), h(x), h(y), h(out), stream()), "add_f16");
  return out;
}

std::vector<at::Tensor> add_layer_norm_f16(at::Tensor x, at::Tensor residual, at::Tensor weight,
                                           at::Tensor bias, double eps) {
  check_half_cuda_contig(x, "x");
  check_half_cuda_contig(residual, "residual");
  check_half_cuda_contig(weight, "weight");
  check_half_cuda_contig(bias, "bias");
  TORCH_CHECK(x.sizes() == residual.sizes(), "add_layer_norm_f16 x/residual shape mismatch");
  TORCH_CHECK(x.dim() >= 1, "x must have at least 1 dim");
  const int64_t c = x.size(-1);
  TORCH_CHECK(weight.dim() == 1 && weight.size(0) == c, "weight shape mismatch");
  TORCH_CHECK(bias.dim() == 1 && bias.size(0) == c, "bias shape mismatch");
  TORCH_CHECK(c > 0 && c <= 8192, "unsupported C");
  auto x_out = at::empty_like(x);
  auto y = run_ln(x, &residual, weight, bias, eps, &x_out, "add_layer_norm_f16");
  return {x_out, y};
}

at::Tensor add_last_layer_norm_f16(at::Tensor x, at::Tensor residual, at::Tensor weight,
                                   at::Tensor bias, double eps) {
  check_half_cuda_contig(x, "x");
  check_half_cuda_contig(residual, "residual");
  check_half_cuda_contig(weight, "weight");
  check_half_cuda_contig(bias, "bias");
  TORCH_CHECK(x.sizes() == residual.sizes(), "add_last_layer_norm_f16 x/residual shape mismatch");
  TORCH_CHECK(x.dim() == 3, "x must have shape [B,T,C]");
  const int64_t c = x.size(2);
  TORCH_CHECK(weight.dim() == 1 && weight.size(0) == c, "weight shape mismatch");
  TORCH_CHECK(bias.dim() == 1 && bias.size(0) == c, "bias shape mismatch");
  TORCH_CHECK(c > 0 && c <= 8192, "unsupported C");
  TORCH_CHECK((c % 2) == 0, "add_last_layer_norm_f16 requires even C");
  check_fits_int(x.size(0), "B");
  check_fits_int(x.size(1), "T");
  check_device(x, "x");
  auto y = at::empty({x.size(0), c}, x.options());
  if (x.size(0) > 0) {
    TORCH_CHECK(x.size(1) > 0, "add_last_layer_norm_f16 requires T >= 1");
    check_status(vkwr_add_last_layer_norm_f16((int)x.size(0), (int)x.size(1), (int)c, h(x),
                                              h(residual), h(weight), h(bias), (float)eps, h(y),
                                              stream()),
                 "add_last_layer_norm_f16");
  }
  return y;
}

// ---- decode fusions: add + LN + token-shift lerp (T == 1)

void check_mix_common(const at::Tensor& x, const at::Tensor& residual, const at::Tensor& shift_state,
                      const at::Tensor& weight, const at::Tensor& bias, const char* fn) {
  check_half_cuda_contig(x, "x");
  check_half_cuda_contig(residual, "residual");
  check_half_cuda_contig(shift_state, "shift_state");
  check_half_cuda_contig(weight, "weight");
  check_half_cuda_contig(bias, "bias");
  TORCH_CHECK(x.sizes() == residual.sizes(), fn, " x/residual shape mismatch");
}

void check_mix_tail(const at::Tensor& x, const at::Tensor& shift_state, const at::Tensor& weight,
                    const at::Tensor& bias, int64_t c) {
  TORCH_CHECK(shift_state.dim() == 2 && shift_state.size(0) == x.size(0) && shift_state.size(1) == c,
              "shift_state shape mismatch");
  TORCH_CHECK(weight.dim() == 1 && weight.size(0) == c, "weight shape mismatch");
  TORCH_CHECK(bias.dim() == 1 && bias.size(0) == c, "bias shape mismatch");
}

std::vector<at::Tensor> run_mix(const at::Tensor& x, const at::Tensor& residual,
                                at::Tensor& shift_state, const at::Tensor& weight,
                                const at::Tensor& bias, const std::vector<at::Tensor>& mixv,
                                double eps, const char* what) {
  check_device(x, "x");
  const int64_t C = x.size(2);
  const int n = (int)mixv.size();
  std::vector<at::Tensor> outs;
  outs.push_back(at::empty_like(x));  // x_out
  const uint16_t* mp[6];
  uint16_t* op[6];
  for (int i = 0; i < n; ++i) {
    outs.push_back(at::empty_like(x));
    mp[i] = h(mixv[i]);
    op[i] = h(outs.back());
  }
  check_status(vkwr_add_layer_norm_mix_f16(x.size(0), (int)C, h(x), h(residual), h(shift_state),
                                           h(weight), h(bias), n, mp, (float)eps, h(outs[0]), op,
                                           nullptr, nullptr, 0, 0, stream()),
               what);
  return outs;
}

std::vector<at::Tensor> cmix_common(at::Tensor x, at::Tensor residual, at::Tensor shift_state,
                                    at::Tensor weight, at::Tensor bias, at::Tensor x_k, double eps,
                                    bool c4096, const char* fn) {
  check_mix_common(x, residual, shift_state, weight, bias, fn);
  check_half_cuda_contig(x_k, "x_k");
  int64_t c;
  if (c4096) {
    TORCH_CHECK(x.dim() == 3 && x.size(1) == 1 && x.size(2) == 4096, fn, " requires shape [B,1,4096]");
    c = 4096;
  } else {
    TORCH_CHECK(x.dim() == 3 && x.size(1) == 1, fn, " requires shape [B,1,C]");
    c = x.size(2);
    TORCH_CHECK((c % 2) == 0 && c > 0 && c <= 8192, "unsupported C");
  }
  check_mix_tail(x, shift_state, weight, bias, c);
  TORCH_CHECK(x_k.dim() == 1 && x_k.size(0) == c, "x_k shape mismatch");
  return run_mix(x, residual, shift_state, weight, bias, {x_k}, eps, fn);
}

std::vector<at::Tensor> add_layer_norm_cmix_mix_f16(at::Tensor x, at::Tensor residual,
                                                    at::Tensor shift_state, at::Tensor weight,
                                                    at::Tensor bias, at::Tensor x_k, double eps) {
  return cmix_common(x, residual, shift_state, weight, bias, x_k, eps, false,
                     "add_layer_norm_cmix_mix_f16");
}

std::vector<at::Tensor> add_layer_norm_cmix_mix_f16_cfg(at::Tensor x, at::Tensor residual,
                                                        at::Tensor shift_state, at::Tensor weight,
                                                        at::Tensor bias, at::Tensor x_k, double eps,
                                                        int64_t threads) {
  TORCH_CHECK(threads == 256 || threads == 512 || threads == 1024, "threads must be 256, 512, or 1024");
  return cmix_common(x, residual, shift_state, weight, bias, x_k, eps, true,
                     "add_layer_norm_cmix_mix_f16_cfg");
}

std::vector<at::Tensor> add_layer_norm_cmix_mix_f16_scalar_stats(at::Tensor x, at::Tensor residual,
                                                                 at::Tensor shift_state,
                                                                 at::Tensor weight, at::Tensor bias,
                                                                 at::Tensor x_k, double eps) {
  return cmix_common(x, residual, shift_state, weight, bias, x_k, eps, true,
                     "add_layer_norm_cmix_mix_f16_scalar_stats");
}

std::vector<at::Tensor> tmix_common(at::Tensor x, at::Tensor residual, at::Tensor shift_state,
                                    at::Tensor weight, at::Tensor bias, at::Tensor x_r,
                                    at::Tensor x_w, at::Tensor x_k, at::Tensor x_v, at::Tensor x_a,
                                    at::Tensor x_g, double eps, bool c4096, const char* fn) {
  check_mix_common(x, residual, shift_state, weight, bias, fn);
  check_half_cuda_contig(x_r, "x_r");
  check_half_cuda_contig(x_w, "x_w");
  check_half_cuda_contig(x_k, "x_k");
  check_half_cuda_contig(x_v, "x_v");
  check_half_cuda_contig(x_a, "x_a");
  check_half_cuda_contig(x_g, "x_g");
  int64_t c;
  if (c4096) {
    TORCH_CHECK(x.dim() == 3 && x.size(1) == 1 && x.size(2) == 4096, fn, " requires shape [B,1,4096]");
    c = 4096;
  } else {
    TORCH_CHECK(x.dim() == 3 && x.size(1) == 1, fn, " requires shape [B,1,C]");
    c = x.size(2);
    TORCH_CHECK((c % 2) == 0 && c > 0 && c <= 8192, "unsupported C");
  }
  check_mix_tail(x, shift_state, weight, bias, c);
  TORCH_CHECK(x_r.numel() == c && x_w.numel() == c && x_k.numel() == c && x_v.numel() == c &&
                  x_a.numel() == c && x_g.numel() == c,
              "mix vector shape mismatch");
  return run_mix(x, residual, shift_state, weight, bias, {x_r, x_w, x_k, x_v, x_a, x_g}, eps, fn);
}

std::vector<at::Tensor> add_layer_norm_tmix_mix6_f16(at::Tensor x, at::Tensor residual,
                                                     at::Tensor shift_state, at::Tensor weight,
                                                     at::Tensor bias, at::Tensor x_r, at::Tensor x_w,
                                                     at::Tensor x_k, at::Tensor x_v, at::Tensor x_a,
                                                     at::Tensor x_g, double eps) {
  return tmix_common(x, residual, shift_state, weight, bias, x_r, x_w, x_k, x_v, x_a, x_g, eps,
                     false, "add_layer_norm_tmix_mix6_f16");
}

std::vector<at::Tensor> add_layer_norm_tmix_mix6_f16_cfg(at::Tensor x, at::Tensor residual,
                                                         at::Tensor shift_state, at::Tensor weight,
                                                         at::Tensor bias, at::Tensor x_r,
                                                         at::Tensor x_w, at::Tensor x_k,
                                                         at::Tensor x_v, at::Tensor x_a,
                                                         at::Tensor x_g, double eps, int64_t threads) {
  TORCH_CHECK(threads == 256 || threads == 512 || threads == 1024, "threads must be 256, 512, or 1024");
  return tmix_common(x, residual, shift_state, weight, bias, x_r, x_w, x_k, x_v, x_a, x_g, eps,
                     true, "add_layer_norm_tmix_mix6_f16_cfg");
}

std::vector<at::Tensor> add_layer_norm_tmix_mix6_f16_scalar_stats(
    at::Tensor x, at::Tensor residual, at::Tensor shift_state, at::Tensor weight, at::Tensor bias,
    at::Tensor x_r, at::Tensor x_w, at::Tensor x_k, at::Tensor x_v, at::Tensor x_a, at::Tensor x_g,
    double eps) {
  return tmix_common(x, residual, shift_state, weight, bias, x_r, x_w, x_k, x_v, x_a, x_g, eps,
                     true, "add_layer_norm_tmix_mix6_f16_scalar_stats");
}

}  // namespace

TORCH_LIBRARY(vkwr_v1_norm, m) {
  m.def("layer_norm_f16(Tensor x, Tensor weight, Tensor bias, float eps=1e-5) -> Tensor");
  m.impl("layer_norm_f16", c10::kCUDA, &layer_norm_f16);

  m.def("layer_norm_f16_small(Tensor x, Tensor weight, Tensor bias, float eps=1e-5) -> Tensor");
  m.impl("layer_norm_f16_small", c10::kCUDA, &layer_norm_f16_small);

  m.def("layer_norm_f16_small512(Tensor x, Tensor weight, Tensor bias, float eps=1e-5) -> Tensor");
  m.impl("layer_norm_f16_small512", c10::kCUDA, &layer_norm_f16_small512);

  m.def("emb_ln0_bf16_to_f16(Tensor emb, Tensor weight, Tensor bias, float eps=1e-5) -> Tensor");
  m.impl("emb_ln0_bf16_to_f16", c10::kCUDA, &emb_ln0_bf16_to_f16);

  m.def("add_f16(Tensor x, Tensor y) -> Tensor");
  m.impl("add_f16", c10::kCUDA, &add_f16);

  m.def("add_layer_norm_f16(Tensor x, Tensor residual, Tensor weight, Tensor bias, float eps=1e-5) -> Tensor[]");
  m.impl("add_layer_norm_f16", c10::kCUDA, &add_layer_norm_f16);

  m.def("add_last_layer_norm_f16(Tensor x, Tensor residual, Tensor weight, Tensor bias, float eps=1e-5) -> Tensor");
  m.impl("add_last_layer_norm_f16", c10::kCUDA, &add_last_layer_norm_f16);

  m.def("add_layer_norm_cmix_mix_f16(Tensor x, Tensor residual, Tensor(a!) shift_state, Tensor weight, Tensor bias, Tensor x_k, float eps=1e-5) -> Tensor[]");
  m.impl("add_layer_norm_cmix_mix_f16", c10::kCUDA, &add_layer_norm_cmix_mix_f16);

  m.def("add_layer_norm_cmix_mix_f16_cfg(Tensor x, Tensor residual, Tensor(a!) shift_state, Tensor weight, Tensor bias, Tensor x_k, float eps, int threads) -> Tensor[]");
  m.impl("add_layer_norm_cmix_mix_f16_cfg", c10::kCUDA, &add_layer_norm_cmix_mix_f16_cfg);

  m.def("add_layer_norm_cmix_mix_f16_scalar_stats(Tensor x, Tensor residual, Tensor(a!) shift_state, Tensor weight, Tensor bias, Tensor x_k, float eps=1e-5) -> Tensor[]");
  m.impl("add_layer_norm_cmix_mix_f16_scalar_stats", c10::kCUDA, &add_layer_norm_cmix_mix_f16_scalar_stats);

  m.def("add_layer_norm_tmix_mix6_f16(Tensor x, Tensor residual, Tensor(a!) shift_state, Tensor weight, Tensor bias, Tensor x_r, Tensor x_w, Tensor x_k, Tensor x_v, Tensor x_a, Tensor x_g, float eps=1e-5) -> Tensor[]");
  m.impl("add_layer_norm_tmix_mix6_f16", c10::kCUDA, &add_layer_norm_tmix_mix6_f16);

  m.def("add_layer_norm_tmix_mix6_f16_cfg(Tensor x, Tensor residual, Tensor(a!) shift_state, Tensor weight, Tensor bias, Tensor x_r, Tensor x_w, Tensor x_k, Tensor x_v, Tensor x_a, Tensor x_g, float eps, int threads) -> Tensor[]");
  m.impl("add_layer_norm_tmix_mix6_f16_cfg", c10::kCUDA, &add_layer_norm_tmix_mix6_f16_cfg);

  m.def("add_layer_norm_tmix_mix6_f16_scalar_stats(Tensor x, Tensor residual, Tensor(a!) shift_state, Tensor weight, Tensor bias, Tensor x_r, Tensor x_w, Tensor x_k, Tensor x_v, Tensor x_a, Tensor x_g, float eps=1e-5) -> Tensor[]");
  m.impl("add_layer_norm_tmix_mix6_f16_scalar_stats", c10::kCUDA, &add_layer_norm_tmix_mix6_f16_scalar_stats);
}

VKT_PYMODULE(_v1_norm_C)
