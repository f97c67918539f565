/*
 * vkwr_amd -- C ABI of the MI355X (gfx950) RWKV-7 hot-path kernels.
 *
 * Plain pointers and sizes only.  fp16 tensors are passed as `uint16_t*`
 * (IEEE binary16 bit patterns), fp32 as `float*`, integer tables as
 * `int32_t*`.  Every pointer is a device pointer of the current HIP device
 * unless stated otherwise.  `stream` is a `hipStream_t` (NULL = the legacy
 * default stream); every entry point only enqueues work on it and returns
 * without synchronising.
 *
 * Return value: VKWR_OK (0) or an error code; on error nothing was enqueued
 * and vkwr_last_error() describes the failure (thread-local).
 *
 * Each entry point names the reference interface (szxysdt/VKWR, paths relative
 * to its root) whose device work it replaces.  The reference exposes those
 * through torch ops; the torch extension modules of this repository
 * (vkwr_amd/_v1_*_C, vkwr_amd/_rwkv7_C) register the same op names and
 * schemas and call these functions.
 */
#ifndef VKWR_AMD_H
#define VKWR_AMD_H

#include <stdint.h>

#if defined(__GNUC__)
#define VKWR_EXPORT __attribute__((visibility("default")))
#else
#define VKWR_EXPORT
#endif

#ifdef __cplusplus
extern "C" {
#endif

enum {
  VKWR_OK = 0,
  VKWR_ERR_INVALID = 1, /* bad argument: shape, null pointer, unsupported size */
  VKWR_ERR_LAUNCH = 2   /* the HIP runtime refused the launch */
};

/* Name of a status code. */
VKWR_EXPORT const char* vkwr_status_string(int status);
/* Message of the last failure on this thread ("" if none). */
VKWR_EXPORT const char* vkwr_last_error(void);

/* ------------------------------------------------------------------ WKV-7 */

/* fp32-state WKV-7 over T tokens, dense state.
 *   state [B,H,64,64] fp32, updated in place; r,w,k,v,a,b,y [B,T,C] fp16, C = 64*H.
 *   w is the raw (pre-activation) decay input; the kernel applies
 *   d = exp(-e^{-1/2} * sigmoid(w)).
 * Replaces wkv_fp32_v2_cuda (csrc/v1/wkv/wkv_fp32_v2.cu:230-288), reached from
 * vkwr_v1_wkv::wkv_forward_fp32 / _seq_fp32 / _small_fp32 / _block_fp32
 * (csrc/v1/wkv/torch_bindings.cpp:179-221).  `mode` (0..3) is the reference's
 * dispatch selector; all modes compute the same function on gfx950. */
VKWR_EXPORT int vkwr_wkv7_fp32_forward(int B, int T, int C, int H, int mode, float* state,
                           const uint16_t* r, const uint16_t* w, const uint16_t* k,
                           const uint16_t* v, const uint16_t* a, const uint16_t* b,
                           uint16_t* y, void* stream);

/* fp32-state WKV-7 over T tokens with the state gathered from, and scattered
 * back to, a slot pool in one pass: sequence i uses pool[slots[i]].
 *   pool [n_slots,H,64,64] fp32 (in place); slots [B] int32, distinct, each in
 *   [0, n_slots); r..y as above.  Pool entries not named by `slots` are not
 *   touched.  A slot outside [0, n_slots) is skipped and its y rows are set to
 *   NaN; duplicate slots race (the caller guarantees distinctness).
 * No single reference function: replaces the caller-side sequence
 * index_select -> vkwr_v1_wkv::wkv_forward_fp32 -> index_copy_
 * (csrc/v1/wkv/torch_bindings.cpp:179-188 plus ATen gather/scatter). */
VKWR_EXPORT int vkwr_wkv7_fp32_forward_slots(int B, int T, int C, int H, float* pool, int n_slots,
                                 const int32_t* slots, const uint16_t* r,
                                 const uint16_t* w, const uint16_t* k, const uint16_t* v,
                                 const uint16_t* a, const uint16_t* b, uint16_t* y,
                                 void* stream);

/* fp16-state WKV-7 with the dither decay delta.
 *   state [B,H,64,64] fp16 (in place); r..y [B,T,C] fp16; w0 NULL or >= C fp16
 *   values added to w per channel; elapsed_t [B] int32 (read only).
 * Replaces wkv_seq_v2_cuda / wkv_seq_w0_v2_cuda / wkv_one_v2_cuda /
 * wkv_one_w0_v2_cuda (csrc/v1/wkv/wkv_fp16_v2.cu:702-768), reached from
 * vkwr_v1_wkv::wkv_{seq,one}{,_w0}_fp16 (csrc/v1/wkv/torch_bindings.cpp:64-136). */
VKWR_EXPORT int vkwr_wkv7_fp16_forward(int B, int T, int C, int H, uint16_t* state,
                           const uint16_t* r, const uint16_t* w, const uint16_t* w0,
                           const uint16_t* k, const uint16_t* v, const uint16_t* a,
                           const uint16_t* b, uint16_t* y, const int32_t* elapsed_t,
                           void* stream);

/* Legacy fp16-state WKV-7 (per-token dither phase, separately rounded ops).
 *   Same layout as vkwr_wkv7_fp16_forward without w0.
 * Replaces cuda_forward_seq / cuda_forward_one (csrc/rwkv7/state_fwd_fp16.cu:307-316),
 * reached from vkwr_rwkv7::forward_seq / forward_one (csrc/rwkv7/torch_bindings.cpp:11-29). */
VKWR_EXPORT int vkwr_rwkv7_forward(int B, int T, int C, int H, uint16_t* state, const uint16_t* r,
                       const uint16_t* w, const uint16_t* k, const uint16_t* v,
                       const uint16_t* a, const uint16_t* b, uint16_t* y,
                       const int32_t* elapsed_t, void* stream);

/* x[i] += amount (int32 wrap-around), i < n.
 * Replaces advance_i32_cuda (csrc/v1/wkv/advance_i32_ops.cu:15-25), reached from
 * vkwr_v1_wkv::advance_i32 (csrc/v1/wkv/torch_bindings.cpp:224-228). */
VKWR_EXPORT int vkwr_advance_i32(int32_t* x, int64_t n, int32_t amount, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VKWR_AMD_H */
