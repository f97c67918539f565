// Shared helpers of the thin torch extension modules.
//
// Input checks repeat the reference's messages (csrc/v1/common/v1_check.h:5-32)
// so callers see the same RuntimeError text.  Device work is delegated to the
// C ABI (include/vkwr_amd.h) on torch's current HIP stream.
#pragma once

#include <Python.h>
#include <ATen/ATen.h>
#include <c10/hip/HIPFunctions.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <vector>

#include "vkwr_amd.h"

namespace vkt {

inline void check_half_cuda_contig(const at::Tensor& x, const char* name) {
  TORCH_CHECK(x.is_cuda(), name, " must be CUDA");
  TORCH_CHECK(x.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(x.scalar_type() == at::kHalf, name, " must be fp16");
}

inline void check_i32_cuda_contig(const at::Tensor& x, const char* name) {
  TORCH_CHECK(x.is_cuda(), name, " must be CUDA");
  TORCH_CHECK(x.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(x.scalar_type() == at::kInt, name, " must be int32");
}

inline void check_f32_cuda_contig(const at::Tensor& x, const char* name) {
  TORCH_CHECK(x.is_cuda(), name, " must be CUDA");
  TORCH_CHECK(x.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(x.scalar_type() == at::kFloat, name, " must be fp32");
}

inline void check_3d(const at::Tensor& x, int64_t B, int64_t T, int64_t C, const char* name) {
  check_half_cuda_contig(x, name);
  TORCH_CHECK(x.dim() == 3, name, " must have shape [B,T,C]");
  TORCH_CHECK(x.size(0) == B && x.size(1) == T && x.size(2) == C, name, " shape mismatch");
}

inline void check_vec(const at::Tensor& x, int64_t C, const char* name) {
  check_half_cuda_contig(x, name);
  TORCH_CHECK(x.dim() == 1 && x.size(0) == C, name, " must have shape [C]");
}

inline void check_fits_int(int64_t v, const char* name) {
  TORCH_CHECK(v >= 0 && v <= 0x7fffffff, name, " out of range");
}

inline void* stream() { return (void*)c10::hip::getCurrentHIPStream().stream(); }

// All tensors of one call must live on the current device (the launch goes to
// the current device's stream).
inline void check_device(const at::Tensor& x, const char* name) {
  TORCH_CHECK(x.device().index() == c10::hip::current_device(), name,
              " must be on the current device");
}

inline void check_status(int st, const char* what) {
  TORCH_CHECK(st == VKWR_OK, what, ": ", vkwr_status_string(st), ": ", vkwr_last_error());
}

template <typename T>
inline T* ptr(const at::Tensor& x) {
  return reinterpret_cast<T*>(x.data_ptr());
}

// Runs a batch of GEMMs (include/vkwr_amd.h vkwr_gemm_f16) on the current
// stream, with the K-split workspace taken from torch's caching allocator.
inline void run_gemm(std::vector<vkwr_gemm_problem>& probs, const at::Tensor& like, const char* what) {
  const int64_t ws = vkwr_gemm_f16_workspace_bytes((int)probs.size(), probs.data());
  check_status(ws < 0 ? VKWR_ERR_INVALID : VKWR_OK, what);
  at::Tensor w;
  if (ws > 0) w = at::empty({ws}, like.options().dtype(at::kByte));
  check_status(vkwr_gemm_f16((int)probs.size(), probs.data(), ws > 0 ? w.data_ptr() : nullptr, ws,
                             stream()),
               what);
}

inline vkwr_gemm_problem gemm_problem(const at::Tensor& a, const at::Tensor& b, at::Tensor& c,
                                      int64_t m, int64_t n, int64_t k, int b_layout,
                                      int a_act = VKWR_GEMM_ACT_NONE,
                                      int epilogue = VKWR_GEMM_EPI_NONE) {
  vkwr_gemm_problem p{};
  p.a = reinterpret_cast<const uint16_t*>(a.data_ptr());
  p.b = reinterpret_cast<const uint16_t*>(b.data_ptr());
  p.c = reinterpret_cast<uint16_t*>(c.data_ptr());
  p.m = m;
  p.n = n;
  p.k = k;
  p.b_layout = b_layout;
  p.a_act = a_act;
  p.epilogue = epilogue;
  return p;
}

}  // namespace vkt

// Empty Python module object so the .so can be imported by name
// (the ops register through TORCH_LIBRARY static initialisers).
#define VKT_PYMODULE(NAME)                                                           \
  PyMODINIT_FUNC PyInit_##NAME(void) {                                               \
    static struct PyModuleDef def = {PyModuleDef_HEAD_INIT, #NAME, nullptr, 0, nullptr}; \
    return PyModule_Create(&def);                                                    \
  }
