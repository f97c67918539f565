// torch ops of namespace vkwr_rwkv7 (module _rwkv7_C), schemas byte-identical
// to the reference (csrc/rwkv7/torch_bindings.cpp:36-50).
//
// The reference binds these without input validation beyond C == 64*H
// (csrc/rwkv7/state_fwd_fp16.cu:308,313).  Here dtype, device, contiguity and
// element counts are also checked, because a mis-sized tensor would otherwise
// fault the GPU; any shape with the right element count is accepted (the
// reference's own tests pass the state as [1,C,64]).  Both ops run on the
// current stream (the reference's forward_seq used the default stream).
#include "vk_torch.h"

using namespace vkt;

namespace {

void check_legacy(const char* fn, int64_t B, int64_t T, int64_t C, int64_t H,
                  const at::Tensor& state, const at::Tensor& r, const at::Tensor& w,
                  const at::Tensor& k, const at::Tensor& v, const at::Tensor& a,
                  const at::Tensor& b, const at::Tensor& y, const at::Tensor& elapsed_t) {
  TORCH_CHECK(H * 64 == C, fn, ": expected C == H * _N_, got C=", C, " H=", H, " _N_=", 64);
  check_fits_int(B, "B");
  check_fits_int(T, "T");
  check_fits_int(C, "C");
  check_half_cuda_contig(state, "state");
  TORCH_CHECK(state.numel() == B * H * 64 * 64, "state must hold B*H*64*64 elements");
  const at::Tensor* io[] = {&r, &w, &k, &v, &a, &b, &y};
  const char* names[] = {"r", "w", "k", "v", "a", "b", "y"};
  for (int i = 0; i < 7; ++i) {
    check_half_cuda_contig(*io[i], names[i]);
    TORCH_CHECK(io[i]->numel() == B * T * C, names[i], " must hold B*T*C elements");
  }
  check_i32_cuda_contig(elapsed_t, "elapsed_t");
  TORCH_CHECK(elapsed_t.numel() >= B, "elapsed_t must hold at least B elements");
  check_device(state, "state");
}

void forward_seq(int64_t B, int64_t T, int64_t C, int64_t H, at::Tensor state, at::Tensor r,
                 at::Tensor w, at::Tensor k, at::Tensor v, at::Tensor a, at::Tensor b,
                 at::Tensor y, at::Tensor elapsed_t) {
  check_legacy("forward_seq", B, T, C, H, state, r, w, k, v, a, b, y, elapsed_t);
  check_status(vkwr_rwkv7_forward((int)B, (int)T, (int)C, (int)H, ptr<uint16_t>(state),
                                  ptr<uint16_t>(r), ptr<uint16_t>(w), ptr<uint16_t>(k),
                                  ptr<uint16_t>(v), ptr<uint16_t>(a), ptr<uint16_t>(b),
                                  ptr<uint16_t>(y), ptr<int32_t>(elapsed_t), stream()),
               "forward_seq");
}

void forward_one(int64_t B, int64_t C, int64_t H, at::Tensor state, at::Tensor r, at::Tensor w,
                 at::Tensor k, at::Tensor v, at::Tensor a, at::Tensor b, at::Tensor y,
                 at::Tensor elapsed_t) {
  check_legacy("forward_one", B, 1, C, H, state, r, w, k, v, a, b, y, elapsed_t);
  check_status(vkwr_rwkv7_forward((int)B, 1, (int)C, (int)H, ptr<uint16_t>(state),
                                  ptr<uint16_t>(r), ptr<uint16_t>(w), ptr<uint16_t>(k),
                                  ptr<uint16_t>(v), ptr<uint16_t>(a), ptr<uint16_t>(b),
                                  ptr<uint16_t>(y), ptr<int32_t>(elapsed_t), stream()),
               "forward_one");
}

void spmv_forward(int64_t D, int64_t C, at::Tensor vec, at::Tensor mat, at::Tensor out) {
  (void)D;
  (void)C;
  (void)vec;
  (void)mat;
  (void)out;
  TORCH_CHECK_NOT_IMPLEMENTED(false,
                              "vkwr_rwkv7::spmv_forward is not part of the MI355X build; use "
                              "vkwr_v1_mix::cmix_sparse_down_one");
}

}  // namespace

TORCH_LIBRARY(vkwr_rwkv7, m) {
  m.def("forward_seq(int B, int T, int C, int H, "
        "Tensor(a!) state, Tensor r, Tensor w, Tensor k, Tensor v, "
        "Tensor a, Tensor b, Tensor(a!) y, Tensor(a!) elapsed_t) -> ()");
  m.impl("forward_seq", c10::kCUDA, &forward_seq);

  m.def("forward_one(int B, int C, int H, "
        "Tensor(a!) state, Tensor r, Tensor w, Tensor k, Tensor v, "
        "Tensor a, Tensor b, Tensor(a!) y, Tensor(a!) elapsed_t) -> ()");
  m.impl("forward_one", c10::kCUDA, &forward_one);

  m.def("spmv_forward(int D, int C, "
        "Tensor vec, Tensor mat, Tensor(a!) out) -> ()");
  m.impl("spmv_forward", c10::kCUDA, &spmv_forward);
}

VKT_PYMODULE(_rwkv7_C)
