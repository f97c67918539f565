// torch ops of namespace vkwr_v1_wkv (module _v1_wkv_C): the reference's nine
// WKV ops with byte-identical schemas (reference csrc/v1/wkv/torch_bindings.cpp:
// 231-258) plus the slot-pool op wkv_forward_slots_fp32, which has no
// reference counterpart (it fuses the caller's gather/scatter).
#include "vk_torch.h"

using namespace vkt;

namespace {

// fp16-state checks (reference torch_bindings.cpp:15-59).
void check_wkv_fp16_common(int64_t B, int64_t C, int64_t H, const at::Tensor& state,
                           const at::Tensor& r, const at::Tensor& w, const at::Tensor& k,
                           const at::Tensor& v, const at::Tensor& a, const at::Tensor& b) {
  TORCH_CHECK(C == H * 64, "only head size 64 is supported");
  check_half_cuda_contig(r, "r");
  check_half_cuda_contig(w, "w");
  check_half_cuda_contig(k, "k");
  check_half_cuda_contig(v, "v");
  check_half_cuda_contig(a, "a");
  check_half_cuda_contig(b, "b");
  TORCH_CHECK(r.sizes() == w.sizes() && r.sizes() == k.sizes() && r.sizes() == v.sizes() &&
                  r.sizes() == a.sizes() && r.sizes() == b.sizes(),
              "r,w,k,v,a,b shape mismatch");
  TORCH_CHECK(state.dim() == 4 && state.size(0) == B && state.size(1) == H && state.size(2) == 64 &&
                  state.size(3) == 64,
              "state must have shape [B,H,64,64]");
  TORCH_CHECK(state.scalar_type() == at::kHalf, "state must be fp16");
  TORCH_CHECK(state.is_cuda() && state.is_contiguous(), "state must be CUDA contiguous");
}

void check_elapsed(const at::Tensor& elapsed_t, int64_t B) {
  TORCH_CHECK(elapsed_t.dim() == 1 && elapsed_t.size(0) == B, "elapsed_t must have shape [B]");
  TORCH_CHECK(elapsed_t.scalar_type() == at::kInt, "elapsed_t must be int32");
  TORCH_CHECK(elapsed_t.is_cuda() && elapsed_t.is_contiguous(), "elapsed_t must be CUDA contiguous");
}

void check_w0(const at::Tensor& w0, int64_t C) {
  check_half_cuda_contig(w0, "w0");
  // The reference reads w0[c] for c < C without a size check
  // (wkv_fp16_v2.cu:32-39); reading past the end would fault here.
  TORCH_CHECK(w0.numel() >= C, "w0 must hold at least C elements");
}

void run_fp16(int64_t B, int64_t T, int64_t C, int64_t H, at::Tensor& state, const at::Tensor& r,
              const at::Tensor& w, const at::Tensor* w0, const at::Tensor& k, const at::Tensor& v,
              const at::Tensor& a, const at::Tensor& b, at::Tensor& y, const at::Tensor& elapsed_t,
              const char* what) {
  check_fits_int(B, "B");
  check_fits_int(T, "T");
  check_fits_int(C, "C");
  check_device(state, "state");
  const int st = vkwr_wkv7_fp16_forward(
      (int)B, (int)T, (int)C, (int)H, ptr<uint16_t>(state), ptr<uint16_t>(r), ptr<uint16_t>(w),
      w0 ? ptr<uint16_t>(*w0) : nullptr, ptr<uint16_t>(k), ptr<uint16_t>(v), ptr<uint16_t>(a),
      ptr<uint16_t>(b), ptr<uint16_t>(y), ptr<int32_t>(elapsed_t), stream());
  check_status(st, what);
}

void wkv_seq_fp16(int64_t B, int64_t T, int64_t C, int64_t H, at::Tensor state, at::Tensor r,
                  at::Tensor w, at::Tensor k, at::Tensor v, at::Tensor a, at::Tensor b,
                  at::Tensor y, at::Tensor elapsed_t) {
  check_wkv_fp16_common(B, C, H, state, r, w, k, v, a, b);
  TORCH_CHECK(r.dim() == 3 && r.size(0) == B && r.size(1) == T && r.size(2) == C,
              "r must have shape [B,T,C]");
  check_half_cuda_contig(y, "y");
  TORCH_CHECK(y.dim() == 3 && y.size(0) == B && y.size(1) == T && y.size(2) == C,
              "y must have shape [B,T,C]");
  check_elapsed(elapsed_t, B);
  run_fp16(B, T, C, H, state, r, w, nullptr, k, v, a, b, y, elapsed_t, "wkv_seq_fp16");
}

void wkv_seq_w0_fp16(int64_t B, int64_t T, int64_t C, int64_t H, at::Tensor state, at::Tensor r,
                     at::Tensor w, at::Tensor w0, at::Tensor k, at::Tensor v, at::Tensor a,
                     at::Tensor b, at::Tensor y, at::Tensor elapsed_t) {
  check_wkv_fp16_common(B, C, H, state, r, w, k, v, a, b);
  TORCH_CHECK(r.dim() == 3 && r.size(0) == B && r.size(1) == T && r.size(2) == C,
              "r must have shape [B,T,C]");
  check_w0(w0, C);
  check_half_cuda_contig(y, "y");
  TORCH_CHECK(y.dim() == 3 && y.size(0) == B && y.size(1) == T && y.size(2) == C,
              "y must have shape [B,T,C]");
  check_elapsed(elapsed_t, B);
  run_fp16(B, T, C, H, state, r, w, &w0, k, v, a, b, y, elapsed_t, "wkv_seq_w0_fp16");
}

void wkv_one_fp16(int64_t B, int64_t C, int64_t H, at::Tensor state, at::Tensor r, at::Tensor w,
                  at::Tensor k, at::Tensor v, at::Tensor a, at::Tensor b, at::Tensor y,
                  at::Tensor elapsed_t) {
  check_wkv_fp16_common(B, C, H, state, r, w, k, v, a, b);
  TORCH_CHECK(r.dim() == 2 && r.size(0) == B && r.size(1) == C, "r must have shape [B,C]");
  check_half_cuda_contig(y, "y");
  TORCH_CHECK(y.dim() == 2 && y.size(0) == B && y.size(1) == C, "y must have shape [B,C]");
  check_elapsed(elapsed_t, B);
  run_fp16(B, 1, C, H, state, r, w, nullptr, k, v, a, b, y, elapsed_t, "wkv_one_fp16");
}

void wkv_one_w0_fp16(int64_t B, int64_t C, int64_t H, at::Tensor state, at::Tensor r,
                     at::Tensor w, at::Tensor w0, at::Tensor k, at::Tensor v, at::Tensor a,
                     at::Tensor b, at::Tensor y, at::Tensor elapsed_t) {
  check_wkv_fp16_common(B, C, H, state, r, w, k, v, a, b);
  TORCH_CHECK(r.dim() == 2 && r.size(0) == B && r.size(1) == C, "r must have shape [B,C]");
  check_w0(w0, C);
  check_half_cuda_contig(y, "y");
  TORCH_CHECK(y.dim() == 2 && y.size(0) == B && y.size(1) == C, "y must have shape [B,C]");
  check_elapsed(elapsed_t, B);
  run_fp16(B, 1, C, H, state, r, w, &w0, k, v, a, b, y, elapsed_t, "wkv_one_w0_fp16");
}

// fp32-state checks (reference torch_bindings.cpp:141-174).
void check_fp32_io(const at::Tensor& x, const char* name) {
  TORCH_CHECK(x.is_cuda(), name, " must be CUDA");
  TORCH_CHECK(x.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(x.scalar_type() == at::kHalf, name, " must be fp16");
}

void check_wkv_fp32_io(int64_t B, int64_t T, int64_t C, int64_t H, const at::Tensor& r,
                       const at::Tensor& w, const at::Tensor& k, const at::Tensor& v,
                       const at::Tensor& a, const at::Tensor& b, const at::Tensor& y) {
  TORCH_CHECK(C == H * 64, "only head size 64 is supported");
  check_fp32_io(r, "r");
  check_fp32_io(w, "w");
  check_fp32_io(k, "k");
  check_fp32_io(v, "v");
  check_fp32_io(a, "a");
  check_fp32_io(b, "b");
  check_fp32_io(y, "y");
  TORCH_CHECK(r.sizes() == w.sizes() && r.sizes() == k.sizes() && r.sizes() == v.sizes() &&
                  r.sizes() == a.sizes() && r.sizes() == b.sizes() && r.sizes() == y.sizes(),
              "r,w,k,v,a,b,y shape mismatch");
  TORCH_CHECK(r.dim() == 3 && r.size(0) == B && r.size(1) == T && r.size(2) == C,
              "r must have shape [B,T,C]");
  check_fits_int(B, "B");
  check_fits_int(T, "T");
  check_fits_int(C, "C");
}

void wkv_fp32_mode(int64_t B, int64_t T, int64_t C, int64_t H, at::Tensor& state,
                   const at::Tensor& r, const at::Tensor& w, const at::Tensor& k,
                   const at::Tensor& v, const at::Tensor& a, const at::Tensor& b, at::Tensor& y,
                   int mode, const char* what) {
  TORCH_CHECK(C == H * 64, "only head size 64 is supported");
  TORCH_CHECK(state.is_cuda(), "state", " must be CUDA");
  TORCH_CHECK(state.is_contiguous(), "state", " must be contiguous");
  TORCH_CHECK(state.scalar_type() == at::kFloat, "state", " must be fp32");
  check_wkv_fp32_io(B, T, C, H, r, w, k, v, a, b, y);
  TORCH_CHECK(state.dim() == 4 && state.size(0) == B && state.size(1) == H && state.size(2) == 64 &&
                  state.size(3) == 64,
              "state must have shape [B,H,64,64]");
  check_device(state, "state");
  const int st = vkwr_wkv7_fp32_forward(
      (int)B, (int)T, (int)C, (int)H, mode, ptr<float>(state), ptr<uint16_t>(r), ptr<uint16_t>(w),
      ptr<uint16_t>(k), ptr<uint16_t>(v), ptr<uint16_t>(a), ptr<uint16_t>(b), ptr<uint16_t>(y),
      stream());
  check_status(st, what);
}

void wkv_forward_fp32(int64_t B, int64_t T, int64_t C, int64_t H, at::Tensor state, at::Tensor r,
                      at::Tensor w, at::Tensor k, at::Tensor v, at::Tensor a, at::Tensor b,
                      at::Tensor y) {
  wkv_fp32_mode(B, T, C, H, state, r, w, k, v, a, b, y, 0, "wkv_forward_fp32");
}
void wkv_forward_seq_fp32(int64_t B, int64_t T, int64_t C, int64_t H, at::Tensor state,
                          at::Tensor r, at::Tensor w, at::Tensor k, at::Tensor v, at::Tensor a,
                          at::Tensor b, at::Tensor y) {
  wkv_fp32_mode(B, T, C, H, state, r, w, k, v, a, b, y, 1, "wkv_forward_seq_fp32");
}
void wkv_forward_small_fp32(int64_t B, int64_t T, int64_t C, int64_t H, at::Tensor state,
                            at::Tensor r, at::Tensor w, at::Tensor k, at::Tensor v, at::Tensor a,
                            at::Tensor b, at::Tensor y) {
  wkv_fp32_mode(B, T, C, H, state, r, w, k, v, a, b, y, 2, "wkv_forward_small_fp32");
}
void wkv_forward_block_fp32(int64_t B, int64_t T, int64_t C, int64_t H, at::Tensor state,
                            at::Tensor r, at::Tensor w, at::Tensor k, at::Tensor v, at::Tensor a,
                            at::Tensor b, at::Tensor y) {
  wkv_fp32_mode(B, T, C, H, state, r, w, k, v, a, b, y, 3, "wkv_forward_block_fp32");
}

// Slot-pool variant: state_pool [P,H,64,64] fp32, slots [B] int32 (distinct, in
// [0,P)); r..y [B,T,C].  Slot values are checked on the device (an out-of-range
// slot leaves the pool untouched and yields NaN rows); distinctness is the
// caller's contract (see the Python wrapper's validate option).
void wkv_forward_slots_fp32(int64_t B, int64_t T, int64_t C, int64_t H, at::Tensor state_pool,
                            at::Tensor slots, at::Tensor r, at::Tensor w, at::Tensor k,
                            at::Tensor v, at::Tensor a, at::Tensor b, at::Tensor y) {
  TORCH_CHECK(C == H * 64, "only head size 64 is supported");
  TORCH_CHECK(state_pool.is_cuda(), "state_pool", " must be CUDA");
  TORCH_CHECK(state_pool.is_contiguous(), "state_pool", " must be contiguous");
  TORCH_CHECK(state_pool.scalar_type() == at::kFloat, "state_pool", " must be fp32");
  TORCH_CHECK(state_pool.dim() == 4 && state_pool.size(1) == H && state_pool.size(2) == 64 &&
                  state_pool.size(3) == 64,
              "state_pool must have shape [P,H,64,64]");
  check_i32_cuda_contig(slots, "slots");
  TORCH_CHECK(slots.dim() == 1 && slots.size(0) == B, "slots must have shape [B]");
  check_wkv_fp32_io(B, T, C, H, r, w, k, v, a, b, y);
  check_fits_int(state_pool.size(0), "pool size");
  check_device(state_pool, "state_pool");
  const int st = vkwr_wkv7_fp32_forward_slots(
      (int)B, (int)T, (int)C, (int)H, ptr<float>(state_pool), (int)state_pool.size(0),
      ptr<int32_t>(slots), ptr<uint16_t>(r), ptr<uint16_t>(w), ptr<uint16_t>(k), ptr<uint16_t>(v),
      ptr<uint16_t>(a), ptr<uint16_t>(b), ptr<uint16_t>(y), stream());
  check_status(st, "wkv_forward_slots_fp32");
}

// advance_i32 (reference torch_bindings.cpp:224-228, advance_i32_ops.cu:15-25).
void advance_i32(at::Tensor x, int64_t amount) {
  check_i32_cuda_contig(x, "x");
  TORCH_CHECK(x.dim() == 1, "x must have shape [B]");
  TORCH_CHECK(amount >= INT32_MIN && amount <= INT32_MAX, "advance_i32 amount out of int range");
  check_device(x, "x");
  check_status(vkwr_advance_i32(ptr<int32_t>(x), x.numel(), (int32_t)amount, stream()),
               "advance_i32");
}

}  // namespace

TORCH_LIBRARY(vkwr_v1_wkv, m) {
  m.def("wkv_seq_fp16(int B, int T, int C, int H, Tensor(a!) state, Tensor r, Tensor w, Tensor k, Tensor v, Tensor a, Tensor b, Tensor(a!) y, Tensor(a!) elapsed_t) -> ()");
  m.impl("wkv_seq_fp16", c10::kCUDA, &wkv_seq_fp16);

  m.def("wkv_seq_w0_fp16(int B, int T, int C, int H, Tensor(a!) state, Tensor r, Tensor w, Tensor w0, Tensor k, Tensor v, Tensor a, Tensor b, Tensor(a!) y, Tensor(a!) elapsed_t) -> ()");
  m.impl("wkv_seq_w0_fp16", c10::kCUDA, &wkv_seq_w0_fp16);

  m.def("wkv_one_fp16(int B, int C, int H, Tensor(a!) state, Tensor r, Tensor w, Tensor k, Tensor v, Tensor a, Tensor b, Tensor(a!) y, Tensor(a!) elapsed_t) -> ()");
  m.impl("wkv_one_fp16", c10::kCUDA, &wkv_one_fp16);

  m.def("wkv_one_w0_fp16(int B, int C, int H, Tensor(a!) state, Tensor r, Tensor w, Tensor w0, Tensor k, Tensor v, Tensor a, Tensor b, Tensor(a!) y, Tensor(a!) elapsed_t) -> ()");
  m.impl("wkv_one_w0_fp16", c10::kCUDA, &wkv_one_w0_fp16);

  m.def("wkv_forward_fp32(int B, int T, int C, int H, Tensor(a!) state, Tensor r, Tensor w, Tensor k, Tensor v, Tensor a, Tensor b, Tensor(a!) y) -> ()");
  m.impl("wkv_forward_fp32", c10::kCUDA, &wkv_forward_fp32);

  m.def("wkv_forward_seq_fp32(int B, int T, int C, int H, Tensor(a!) state, Tensor r, Tensor w, Tensor k, Tensor v, Tensor a, Tensor b, Tensor(a!) y) -> ()");
  m.impl("wkv_forward_seq_fp32", c10::kCUDA, &wkv_forward_seq_fp32);

  m.def("wkv_forward_small_fp32(int B, int T, int C, int H, Tensor(a!) state, Tensor r, Tensor w, Tensor k, Tensor v, Tensor a, Tensor b, Tensor(a!) y) -> ()");
  m.impl("wkv_forward_small_fp32", c10::kCUDA, &wkv_forward_small_fp32);

  m.def("wkv_forward_block_fp32(int B, int T, int C, int H, Tensor(a!) state, Tensor r, Tensor w, Tensor k, Tensor v, Tensor a, Tensor b, Tensor(a!) y) -> ()");
  m.impl("wkv_forward_block_fp32", c10::kCUDA, &wkv_forward_block_fp32);

  m.def("advance_i32(Tensor(a!) x, int amount) -> ()");
  m.impl("advance_i32", c10::kCUDA, &advance_i32);

  m.def("wkv_forward_slots_fp32(int B, int T, int C, int H, Tensor(a!) state_pool, Tensor slots, Tensor r, Tensor w, Tensor k, Tensor v, Tensor a, Tensor b, Tensor(a!) y) -> ()");
  m.impl("wkv_forward_slots_fp32", c10::kCUDA, &wkv_forward_slots_fp32);
}

VKT_PYMODULE(_v1_wkv_C)
