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
 * (vkwr/_v1_*_C, vkwr/_rwkv7_C, vkwr/_sampling_C) register the same op names and
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

/* One decode step (T = 1) of vkwr_wkv7_fp32_forward_slots with the dot products in the
 * row-split order of the prefill kernels (eight 8-term FMA chains per state row, combined
 * pairwise) instead of one 64-term chain, and no LDS: it can run on a second stream beside
 * the chunked prefill kernel, which holds most of each CU's LDS.  Same arguments and slot
 * semantics (out-of-range slot: NaN y rows, pool untouched); pool and v 16-byte aligned,
 * r, w, k, a, b 8-byte aligned.  No counterpart in the reference (its T = 1 op is
 * wkv_forward_fp32, csrc/v1/wkv/torch_bindings.cpp:179-188, in one-chain order); for
 * mixed prefill + decode batches. */
VKWR_EXPORT int vkwr_wkv7_fp32_step_rows_slots(int B, int C, int H, float* pool, int n_slots,
                                               const int32_t* slots, const uint16_t* r, const uint16_t* w,
                                               const uint16_t* k, const uint16_t* v, const uint16_t* a,
                                               const uint16_t* b, uint16_t* y, void* stream);

/* Layouts of an fp32 64x64 WKV state block (16 KiB) in a pool.
 *   VKWR_WKV_STATE_STD: row-major S[i][j] at float 64 i + j (the reference's
 *     [.., H, 64, 64] layout; every other entry point uses it).
 *   VKWR_WKV_STATE_ILV: interleaved, S[i][4q + e] at float (64 q + i) * 4 + e:
 *     column chunk q of all 64 rows is one contiguous kilobyte, which the fused
 *     decode kernel streams straight into registers (lane i = row i). */
enum { VKWR_WKV_STATE_STD = 0, VKWR_WKV_STATE_ILV = 1 };

/* Converts n_blocks state blocks from src to dst (not aliased) into layout
 * to_layout (from the other one).  No counterpart in the reference. */
VKWR_EXPORT int vkwr_wkv7_state_layout_f32(int64_t n_blocks, const float* src, float* dst, int to_layout,
                                           void* stream);

/* Fused time-mix decode step (T = 1) on a slot pool, one pass per (sequence, head):
 *   kk = normalize_head(k * k_k), a = sigmoid(a0 + a12),
 *   new_k = k * (a * k_a + 1 - k_a), then the WKV-7 update of pool[slots[b]]
 *   with (r, w, new_k, v, -kk, kk * a) as in vkwr_wkv7_fp32_forward_slots,
 *   then out = ((y - mean_h) * rstd_h * ln_w + ln_b + (sum_h r * new_k * r_k) * v) * g
 *   (GroupNorm eps 64e-5), with the fp16 roundings of the unfused sequence
 *   vkwr_tmix_kk_a_gate_f16 -> vkwr_wkv7_fp32_forward_slots ->
 *   vkwr_tmix_groupnorm_bonus_gate_f16, so the result is bit-identical to it.
 *   r, w, k, v, a12, g [B, C] fp16; k_k, a0, k_a, r_k, ln_w, ln_b [C];
 *   out [B, C] row-major, or a frag matrix [B, C] when out_frag = 1
 *   (C % 128 == 0).  pool [n_slots, H] blocks in state_layout (VKWR_WKV_STATE_*).
 *   A slot outside [0, n_slots) leaves the pool untouched and writes NaN to
 *   that sequence's out row.
 * No single reference function: fuses tmix_kk_a_gate (csrc/v1/mix/mix_ops.cu:
 * 1015-1049), the fp32 WKV (csrc/v1/wkv/wkv_fp32_v2.cu:230-288) with the
 * caller's slot gather/scatter, and tmix_lnx_rkvres_xg (mix_ops.cu:1051-1083). */
VKWR_EXPORT int vkwr_wkv7_decode_fused_f16(int B, int C, int H, float* pool, int n_slots,
                                           int state_layout, const int32_t* slots, const uint16_t* r, const uint16_t* w,
                                           const uint16_t* k, const uint16_t* v, const uint16_t* a12,
                                           const uint16_t* g, const uint16_t* k_k, const uint16_t* a0,
                                           const uint16_t* k_a, const uint16_t* r_k, const uint16_t* ln_w,
                                           const uint16_t* ln_b, uint16_t* out, int out_frag,
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

/* ------------------------------------------------------------- LayerNorm */

/* Row LayerNorm, fp16 in/out, fp32 statistics (two passes over the row held
 * in registers), y = (v - mean) * rstd * weight + bias with
 * rstd = 1/sqrt(var + eps), var the biased variance.
 *   x, y [rows, C]; residual NULL or [rows, C]: v = x + residual (fp32), and
 *   then x_out (if not NULL) receives fp16(v); the statistics use the fp32 v.
 *   0 < C <= 8192.
 * Replaces layer_norm_f16_cuda / _small_cuda / _small512_cuda and
 * add_layer_norm_f16_cuda (csrc/v1/norm/norm_ops.cu:878-954, 975-1012), reached
 * from vkwr_v1_norm::layer_norm_f16{,_small,_small512}, add_layer_norm_f16
 * (csrc/v1/norm/torch_bindings.cpp:8-40, 64-77). */
VKWR_EXPORT int vkwr_layer_norm_f16(int64_t rows, int C, const uint16_t* x,
                                    const uint16_t* residual, const uint16_t* weight,
                                    const uint16_t* bias, float eps, uint16_t* x_out,
                                    uint16_t* y, void* stream);

/* LayerNorm of the last token of each sequence: y[b] = LN(x[b,T-1] + residual[b,T-1]).
 *   x, residual [B,T,C]; y [B,C].
 * Replaces add_last_layer_norm_f16_cuda (csrc/v1/norm/norm_ops.cu:1014-1043),
 * reached from vkwr_v1_norm::add_last_layer_norm_f16 (torch_bindings.cpp:79-91). */
VKWR_EXPORT int vkwr_add_last_layer_norm_f16(int B, int T, int C, const uint16_t* x,
                                             const uint16_t* residual, const uint16_t* weight,
                                             const uint16_t* bias, float eps, uint16_t* y,
                                             void* stream);

/* LayerNorm of a bf16 embedding table into fp16: out [V,C] = LN(emb [V,C]) with
 * bf16 weight/bias.
 * Replaces emb_ln0_bf16_to_f16_cuda (csrc/v1/norm/norm_ops.cu:956-973), reached
 * from vkwr_v1_norm::emb_ln0_bf16_to_f16 (torch_bindings.cpp:42-52). */
VKWR_EXPORT int vkwr_emb_ln0_bf16_to_f16(int64_t V, int C, const uint16_t* emb,
                                         const uint16_t* weight, const uint16_t* bias,
                                         float eps, uint16_t* out, void* stream);

/* Decode-step fused residual add + LayerNorm + token-shift lerp (T = 1).
 *   x, residual [rows, C] (residual may be NULL: zero); shift_state [*, C]
 *   (in place); n_mix = 1 or 6 mix vectors mix[i] [C]; outputs
 *   x_out [rows, C] = fp16(x + residual) and out[i] [rows, C] =
 *   fp16(y + (prev - y) * mix[i]), where y = fp16(LN(x + residual)) and prev is
 *   the shift_state row at entry; then that shift_state row = y.
 *   x_rows (may be NULL) gathers x: row r reads x[x_rows[r]] (an embedding
 *   lookup; x has n_x rows); shift_slots (may be NULL) maps row r to
 *   shift_state[shift_slots[r]] (a per-sequence slot pool of n_shift rows).
 *   shift_slots must be distinct.  A row whose x_rows or shift_slots entry
 *   lies outside [0, n_x) / [0, n_shift) gets NaN in x_out and out[], and no
 *   shift row is read or written for it (checked on the device; the host does
 *   not read the index arrays).  n_x / n_shift are ignored when the matching
 *   index array is NULL.
 * Replaces add_layer_norm_cmix_mix_f16{,_cfg,_scalar_stats}_cuda and
 * add_layer_norm_tmix_mix6_f16{,_cfg,_scalar_stats}_cuda
 * (csrc/v1/norm/norm_ops.cu:1045-1340), reached from the vkwr_v1_norm ops of the
 * same names (torch_bindings.cpp:93-229). */
VKWR_EXPORT int vkwr_add_layer_norm_mix_f16(int64_t rows, int C, const uint16_t* x,
                                            const uint16_t* residual, uint16_t* shift_state,
                                            const uint16_t* weight, const uint16_t* bias,
                                            int n_mix, const uint16_t* const* mix, float eps,
                                            uint16_t* x_out, uint16_t* const* out,
                                            const int32_t* x_rows, const int32_t* shift_slots,
                                            int64_t n_x, int64_t n_shift, void* stream);

/* out = x + y elementwise (fp32 add, fp16 round), n elements.
 * Replaces add_f16_cuda (csrc/v1/norm/norm_ops.cu:866-876), reached from
 * vkwr_v1_norm::add_f16 (torch_bindings.cpp:54-62). */
VKWR_EXPORT int vkwr_add_f16(int64_t n, const uint16_t* x, const uint16_t* y, uint16_t* out,
                             void* stream);

/* ----------------------------------------------------------- token shift */

/* Token-shift lerp over T tokens: for each output i,
 * out[i][b,t,c] = fp16(x + (prev - x) * mix[i][c]) where prev is shift_state[b]
 * at t = 0 (its value at entry) and x[b,t-1] after; then shift_state[b] = x[b,T-1].
 *   x [B,T,C]; shift_state [B,C] (in place); n_mix = 1 or 6 vectors mix[i] [C];
 *   out[i] [B,T,C].  half_math = 1 evaluates the lerp in fp16 (subtract, then
 *   fused multiply-add), as the reference's half_math option does.
 * Replaces tmix_mix6{,_cfg,_t1_c4096}_cuda and cmix_mix{,_cfg}_cuda
 * (csrc/v1/mix/mix_ops.cu:867-1013, 1280-1324), reached from vkwr_v1_mix::
 * tmix_mix6{,_cfg,_t1_c4096} and cmix_mix{,_cfg} (mix/torch_bindings.cpp:8-74,
 * 246-276).  Unlike the reference (which reads shift_state at t = 0 and writes
 * it at t = T-1 from different threads), prev at t = 0 is always the entry value. */
VKWR_EXPORT int vkwr_token_shift_mix_f16(int B, int T, int C, const uint16_t* x,
                                         uint16_t* shift_state, int n_mix,
                                         const uint16_t* const* mix, uint16_t* const* out,
                                         int half_math, void* stream);

/* Token-shift lerp of T tokens for B sequences whose shift rows live in a slot
 * pool of n_slots rows: sequence b's shift row is shift_pool[shift_slots[b]]
 * (slots distinct); otherwise identical to vkwr_token_shift_mix_f16.  A slot
 * outside [0, n_slots) gives that sequence NaN outputs and leaves the pool
 * untouched (checked on the device).  No single reference function: replaces gathering
 * the shift rows, tmix_mix6 / cmix_mix (csrc/v1/mix/mix_ops.cu:42-160,
 * 432-462) and scattering them back, for the mixed prefill + decode step. */
VKWR_EXPORT int vkwr_token_shift_mix_slots_f16(int B, int T, int C, const uint16_t* x, uint16_t* shift_pool,
                                               int64_t n_slots, const int32_t* shift_slots, int n_mix,
                                               const uint16_t* const* mix, uint16_t* const* out,
                                               int half_math, void* stream);

/* Per-head key normalisation and in-context learning-rate gate of RWKV-7 time mix:
 *   u = k * k_k; kk = u / max(||u||_2 over the head, 1e-12); a = sigmoid(a0 + a12);
 *   new_k = k * (a * k_a + (1 - k_a)); neg_kk = -kk; kka = kk * a.
 *   k, a12, new_k, neg_kk, kka [B,T,C]; k_k, a0, k_a [C]; C = 64 H.
 *   If shift_state is not NULL (T must be 1): shift_state [B,C] = x [B,1,C].
 * Replaces tmix_kk_a_gate_cuda (csrc/v1/mix/mix_ops.cu:1015-1049), reached from
 * vkwr_v1_mix::tmix_kk_a_gate{,_update_shift} (mix/torch_bindings.cpp:76-115). */
VKWR_EXPORT int vkwr_tmix_kk_a_gate_f16(int B, int T, int C, int H, const uint16_t* k,
                                        const uint16_t* k_k, const uint16_t* a0,
                                        const uint16_t* a12, const uint16_t* k_a,
                                        const uint16_t* x, uint16_t* shift_state,
                                        uint16_t* new_k, uint16_t* neg_kk, uint16_t* kka,
                                        void* stream);

/* Per-head GroupNorm of the WKV output plus the r.k bonus and the output gate:
 *   out = ((x - mean_h) * rstd_h * weight + bias + (sum_h r*k*r_k) * v) * g,
 *   statistics over the 64 channels of each head, eps = 64e-5.
 *   x, r, k, v, g, out [B,T,C]; r_k, weight, bias [C]; C = 64 H.
 * Replaces tmix_lnx_rkvres_xg_cuda (csrc/v1/mix/mix_ops.cu:1051-1083), reached
 * from vkwr_v1_mix::tmix_lnx_rkvres_xg (mix/torch_bindings.cpp:117-135). */
VKWR_EXPORT int vkwr_tmix_groupnorm_bonus_gate_f16(int B, int T, int C, int H,
                                                   const uint16_t* x, const uint16_t* r,
                                                   const uint16_t* k, const uint16_t* v,
                                                   const uint16_t* r_k, const uint16_t* weight,
                                                   const uint16_t* bias, const uint16_t* g,
                                                   uint16_t* out, void* stream);

/* Value-residual gate: out = v + (v_first - v) * sigmoid(v0 + v12).
 *   v, v_first, v12, out [rows, C]; v0 [C].
 * Replaces tmix_vres_gate_cuda (csrc/v1/mix/mix_ops.cu:1085-1104), reached from
 * vkwr_v1_mix::tmix_vres_gate (mix/torch_bindings.cpp:137-147). */
VKWR_EXPORT int vkwr_tmix_vres_gate_f16(int64_t rows, int C, const uint16_t* v,
                                        const uint16_t* v_first, const uint16_t* v0,
                                        const uint16_t* v12, uint16_t* out, void* stream);

enum {
  VKWR_ACT_RELU_SQUARE = 0, /* max(x, 0)^2 */
  VKWR_ACT_TANH = 1,
  VKWR_ACT_SIGMOID = 2
};

/* out = act(x) elementwise, n elements, fp32 math.
 * Replaces relu_square_cuda / act_tanh_cuda / act_sigmoid_cuda
 * (csrc/v1/mix/mix_ops.cu:1326-1363), reached from vkwr_v1_mix::relu_square,
 * act_tanh, act_sigmoid (mix/torch_bindings.cpp:278-300). */
VKWR_EXPORT int vkwr_activation_f16(int act, int64_t n, const uint16_t* x, uint16_t* out,
                                    void* stream);

/* out[i] = x[i] + vec[i mod C], n elements (n a multiple of C).
 * Replaces add_vec_cuda (csrc/v1/mix/mix_ops.cu:1365-1378), reached from
 * vkwr_v1_mix::add_vec (mix/torch_bindings.cpp:302-309). */
VKWR_EXPORT int vkwr_add_vec_f16(int64_t n, int C, const uint16_t* x, const uint16_t* vec,
                                 uint16_t* out, void* stream);

/* ------------------------------------------------------------------ GEMM */

enum {
  VKWR_GEMM_B_NK = 0, /* B is [N,K] row-major (nn.Linear weight): y = x . B^T */
  VKWR_GEMM_B_KN = 1  /* B is [K,N] row-major:                      y = x . B   */
};
enum {
  VKWR_GEMM_ACT_NONE = 0,
  VKWR_GEMM_ACT_TANH = 1,   /* applied to A elementwise (rounded to fp16) before the product */
  VKWR_GEMM_ACT_SIGMOID = 2,
  VKWR_GEMM_ACT_RELU_SQUARE = 3
};
enum {
  VKWR_GEMM_EPI_NONE = 0,
  VKWR_GEMM_EPI_RELU_SQUARE = 1,    /* y = max(acc, 0)^2 */
  VKWR_GEMM_EPI_VALUE_RESIDUAL = 2, /* y = v + (v_first - v) * sigmoid(v0[n] + acc) */
  VKWR_GEMM_EPI_BIAS = 3,           /* y = acc + v0[n] */
  VKWR_GEMM_EPI_TANH = 4,           /* y = tanh(acc) (same value as VKWR_FRAG_EPI_TANH) */
  VKWR_GEMM_EPI_SIGMOID = 5         /* y = sigmoid(acc) (same value as VKWR_FRAG_EPI_SIGMOID) */
};

/* One GEMM of a batch: c[m,n] = epilogue(sum_k act(a[m,k]) * B(k,n)), fp16
 * operands and output, fp32 accumulation.  a [m,k], c [m,n] and B are
 * contiguous row-major; v, v_first [m,n] and v0 [n] are read by the
 * value-residual epilogue, v0 [n] by the bias epilogue. */
typedef struct vkwr_gemm_problem {
  const uint16_t* a;
  const uint16_t* b;
  uint16_t* c;
  int64_t m, n, k;
  int b_layout;
  int a_act;
  int epilogue;
  const uint16_t* v;
  const uint16_t* v_first;
  const uint16_t* v0;
} vkwr_gemm_problem;

/* Bytes of device workspace vkwr_gemm_f16 needs for this batch (fp32 partial
 * sums: K splits of small-M problems, or the k-parts of a large-M batch's last
 * round of 256x256 tiles; 0 when nothing is split), or -1 on invalid arguments.
 * The plan depends on the current device's CU count: ask on that device. */
VKWR_EXPORT int64_t vkwr_gemm_f16_workspace_bytes(int n_problems, const vkwr_gemm_problem* problems);

/* Runs 1..8 independent GEMMs in one launch on the gfx950 matrix cores.
 * `problems` is a host array; `workspace` is device memory of at least
 * vkwr_gemm_f16_workspace_bytes(...) bytes (may be NULL when that is 0).
 * Replaces the device work of every vkwr_v1_linear op -- cublasGemmEx /
 * cublasLtMatmul (csrc/v1/linear/linear_ops.cu:973-1057, 1237-1392), the
 * CUDA-core, WMMA and split-K GEMV/GEMM kernels (:46-969, 1059-1833) -- and of
 * the vkwr_v1_rank adapters (csrc/v1/rank/rank_ops.cu:16-482), reached from
 * csrc/v1/linear/torch_bindings.cpp:8-225 and csrc/v1/rank/torch_bindings.cpp:8-122. */
VKWR_EXPORT int vkwr_gemm_f16(int n_problems, const vkwr_gemm_problem* problems, void* workspace,
                              int64_t workspace_bytes, void* stream);

/* vkwr_gemm_f16 without a workspace argument and without any allocation: the K-split /
 * stream-K partials go to a scratch array of vkwr_gemm_f16_noalloc_max_bytes() bytes
 * (32 MiB) that the library holds in device memory, one copy per device, for the life of
 * the process.  Same plan, same kernels, same results bit for bit as vkwr_gemm_f16 with a
 * workspace.  A batch whose plan needs more scratch (vkwr_gemm_f16_workspace_bytes) than
 * that is rejected with VKWR_ERR_INVALID before any GPU work; every GEMM batch of the
 * 1.5B-shape decode step (C = 2048) at up to 256 rows fits.  It calls no hipMalloc / hipFree.  Calls that overlap on
 * one device (concurrent streams, or host threads) share that device's scratch and race:
 * serialise them.  The first call on a device looks the array's device address up once
 * (hipGetSymbolAddress): make one call on each device before capturing it into a HIP graph
 * -- any call does, even a batch of one empty problem (m = 0); captured calls then only
 * enqueue kernels.
 * No counterpart in the reference: it is for callers that cannot allocate device memory,
 * e.g. code under HIP graph capture, tight serving loops, or harnesses that forbid it. */
VKWR_EXPORT int vkwr_gemm_f16_noalloc(int n_problems, const vkwr_gemm_problem* problems, void* stream);

/* The scratch size of vkwr_gemm_f16_noalloc in bytes (its limit). */
VKWR_EXPORT int64_t vkwr_gemm_f16_noalloc_max_bytes(void);

/* Frag-output variants of three producers: identical arithmetic to
 * vkwr_add_layer_norm_mix_f16, vkwr_add_last_layer_norm_f16 and
 * vkwr_tmix_groupnorm_bonus_gate_f16, but out[] / y / out are written as frag
 * matrices [rows, C] (the layout defined below; C % 128 == 0, x_out and the
 * shift state stay row-major), ready to be the activation of
 * vkwr_frag_gemm_f16.  Rows pad and columns need no pad (C % 128 == 0); rows
 * beyond `rows` are not written.  No counterpart in the reference: they let
 * the decode executor feed its projections without a layout pass. */
VKWR_EXPORT int vkwr_add_layer_norm_mix_frag_f16(int64_t rows, int C, const uint16_t* x,
                                                 const uint16_t* residual, uint16_t* shift_state,
                                                 const uint16_t* weight, const uint16_t* bias,
                                                 int n_mix, const uint16_t* const* mix, float eps,
                                                 uint16_t* x_out, uint16_t* const* out,
                                                 const int32_t* x_rows, const int32_t* shift_slots,
                                                 int64_t n_x, int64_t n_shift, void* stream);

/* vkwr_add_layer_norm_mix_frag_f16 whose x is the unreduced output of
 * vkwr_frag_gemm_splitk_parts_f16: x[r, c] = fp16(sum over q < n_parts of
 * x_parts[q * part_stride + r * C + c]), the parts added in q order -- the
 * same values vkwr_frag_gemm_splitk_f16 would have stored, so the result is
 * bit-identical to reducing first.  n_parts 2, 4 or 8; C % 128 == 0,
 * C <= 4096; no x_rows gather.  No counterpart in the reference: it removes
 * the reduce launch between the decode step's FFN value GEMM and the next
 * layer's LayerNorm. */
VKWR_EXPORT int vkwr_add_layer_norm_mix_parts_frag_f16(int64_t rows, int C, const float* x_parts,
                                                       int n_parts, int64_t part_stride,
                                                       const uint16_t* residual, uint16_t* shift_state,
                                                       const uint16_t* weight, const uint16_t* bias,
                                                       int n_mix, const uint16_t* const* mix, float eps,
                                                       uint16_t* x_out, uint16_t* const* out,
                                                       const int32_t* shift_slots, int64_t n_shift,
                                                       void* stream);

/* A group of rows of a mixed prefill + decode batch: B sequences of T consecutive rows each,
 * starting at row row0, sequence b's shift row at shift_state[slots[b]]. */
typedef struct vkwr_ln_shift_group {
  int64_t row0;
  int32_t B, T;
  const int32_t* slots;
} vkwr_ln_shift_group;

/* Residual add + LayerNorm + token-shift lerp over the row groups of a mixed batch, in one
 * launch: x_out = fp16(x + residual) (residual may be NULL), y = LN(x + residual), and for
 * row t of a sequence out[i] = lerp(y, prev, mix[i]) with prev the y of row t - 1, or for
 * t = 0 the sequence's shift row, which then takes the y of the sequence's last row.  The
 * same bits as vkwr_layer_norm_f16 followed, per group, by vkwr_token_shift_mix_slots_f16
 * (the reference's add_layer_norm_f16 and tmix_mix6 / cmix_mix, csrc/v1/norm/norm_ops.cu
 * and csrc/v1/mix/mix_ops.cu:42-160, run back to back).  The groups cover rows 0 .. rows-1 in
 * order (1..8 of them); C % 8 == 0, C <= 4096; n_mix 1 or 6; every tensor 16-byte aligned;
 * slots distinct across the call; x_out and out[] must not overlap x or residual (a row's
 * lerp reads the previous row, so no update in place; an overlap is rejected).  A slot outside 0 .. n_shift-1 makes its rows' x_out and
 * outputs NaN and leaves the pool untouched.  No counterpart in the reference: it is the
 * mixed step's fusion of those two ops. */
VKWR_EXPORT int vkwr_add_layer_norm_shift_rows_f16(int64_t rows, int C, const uint16_t* x,
                                                   const uint16_t* residual, const uint16_t* weight,
                                                   const uint16_t* bias, float eps, uint16_t* x_out,
                                                   int n_mix, const uint16_t* const* mix,
                                                   uint16_t* const* out, uint16_t* shift_state,
                                                   int64_t n_shift, int n_groups,
                                                   const vkwr_ln_shift_group* groups, void* stream);
VKWR_EXPORT int vkwr_add_last_layer_norm_frag_f16(int B, int T, int C, const uint16_t* x,
                                                  const uint16_t* residual, const uint16_t* weight,
                                                  const uint16_t* bias, float eps, uint16_t* y,
                                                  void* stream);
VKWR_EXPORT int vkwr_tmix_groupnorm_bonus_gate_frag_f16(int B, int T, int C, int H, const uint16_t* x,
                                                        const uint16_t* r, const uint16_t* k,
                                                        const uint16_t* v, const uint16_t* r_k,
                                                        const uint16_t* weight, const uint16_t* bias,
                                                        const uint16_t* g, uint16_t* out, void* stream);

/* ------------------------------------------------- fragment-layout GEMM
 *
 * Decode-step GEMMs (m <= a few hundred rows) are bound by streaming the
 * weights once from HBM.  The fragment ("frag") layout stores a matrix X[R,K]
 * (R = rows of the activation or output columns of the weight, K = the
 * reduction dimension) in the operand order of v_mfma_f32_32x32x16_f16, so
 * every wave-wide 16-byte-per-lane load is one contiguous kilobyte:
 *   R_pad = roundup(R, 128), K_pad = roundup(K, 128), zero padded;
 *   element (r, k) at half index
 *     (((r / 32) * (K_pad / 16) + k / 16) * 64 + ((k / 8) % 2) * 32 + r % 32) * 8 + k % 8.
 * No counterpart in the reference (it streams row-major weights through
 * cuBLAS / its split-K kernels, csrc/v1/linear/linear_ops.cu:46-1833); the
 * model executor packs its weights once at load and its producers write the
 * activations feeding each projection directly in this layout. */

#define VKWR_FRAG_PAD 128

enum {
  VKWR_FRAG_EPI_TANH = 4,   /* y = tanh(acc) (frag GEMM only) */
  VKWR_FRAG_EPI_SIGMOID = 5 /* y = sigmoid(acc) (frag GEMM only) */
};

/* Packs src into frag layout: src is [rows, k] row-major (src_layout
 * VKWR_GEMM_B_NK) or [k, rows] row-major (VKWR_GEMM_B_KN); dst holds
 * roundup(rows,128) * roundup(k,128) halfs, pads written as zero. */
VKWR_EXPORT int vkwr_frag_pack_f16(int64_t rows, int64_t k, const uint16_t* src, int src_layout,
                                   uint16_t* dst, void* stream);

/* Inverse of vkwr_frag_pack_f16 for the [rows, k] row-major case. */
VKWR_EXPORT int vkwr_frag_unpack_f16(int64_t rows, int64_t k, const uint16_t* src, uint16_t* dst,
                                     void* stream);

/* One problem of a frag GEMM batch: c = epilogue(a . b^T) with a the frag
 * activation [m, k], b the frag weight [n, k], fp32 accumulation.  c is
 * row-major [m, n] (c_frag = 0) or a frag matrix [m, n] (c_frag = 1, ready to
 * feed the next frag GEMM as its activation; the pad columns n..n_pad-1 are
 * written too, as epilogue(0), and rows >= m are not written).  Epilogues:
 * VKWR_GEMM_EPI_* (value residual and bias need c_frag = 0) or
 * VKWR_FRAG_EPI_TANH / _SIGMOID. */
typedef struct vkwr_frag_gemm_problem {
  const uint16_t* a;
  const uint16_t* b;
  uint16_t* c;
  int64_t m, n, k;
  int epilogue;
  int c_frag;
  const uint16_t* v;
  const uint16_t* v_first;
  const uint16_t* v0;
} vkwr_frag_gemm_problem;

/* Runs 1..8 frag GEMMs in one launch (no workspace: the K split is inside
 * each workgroup, reduced through LDS in a fixed order, so results are
 * deterministic).  All pointers 16-byte aligned; n a multiple of 8 for
 * row-major c.  No counterpart in the reference (see above). */
VKWR_EXPORT int vkwr_frag_gemm_f16(int n_problems, const vkwr_frag_gemm_problem* problems,
                                   void* stream);

/* One frag GEMM with K split over `splits` workgroups per 64 x 64 output
 * tile: the parts write fp32 partial tiles to `workspace`, and a second
 * kernel adds them in increasing K order and applies the epilogue (same
 * epilogues and layouts as vkwr_frag_gemm_f16).  For long-K decode GEMMs
 * (the FFN value, K = 4 F) whose untiled form reads the activations once per
 * 32-column tile.  Deterministic.  frag_pad(k) must be a multiple of
 * 256 * splits; splits in 1..16; workspace 16-byte aligned, at least
 * vkwr_frag_gemm_splitk_workspace_bytes(m, n, splits) bytes.  Calls that share
 * a workspace must not overlap.  No counterpart in the reference (see above). */
VKWR_EXPORT int64_t vkwr_frag_gemm_splitk_workspace_bytes(int64_t m, int64_t n, int splits);
VKWR_EXPORT int vkwr_frag_gemm_splitk_f16(const vkwr_frag_gemm_problem* problem, int splits,
                                          void* workspace, int64_t workspace_bytes, void* stream);

/* The first half of vkwr_frag_gemm_splitk_f16 alone: writes the `splits` fp32
 * partial planes to workspace (plane q at q * roundup(m, 64) * frag_pad(n)
 * floats, row stride frag_pad(n)) and leaves the reduction to a consumer that
 * reads them (vkwr_add_layer_norm_mix_parts_frag_f16).  epilogue must be NONE,
 * c_frag 0; c is not used.  No counterpart in the reference (see above). */
VKWR_EXPORT int vkwr_frag_gemm_splitk_parts_f16(const vkwr_frag_gemm_problem* problem, int splits,
                                                void* workspace, int64_t workspace_bytes, void* stream);

/* ---- token sampling (reference csrc/sampling/, ops vkwr_sampling::*) ----
 *
 * Per batch row b, on the logits of its last token (logits [B,T,V] fp32, row
 * b*T + T-1; V a multiple of 4, at most 1048576):
 *   u_i = sf((sf(l_i) - pen_i) log2(e) / temperature), p = base-2 softmax of u,
 *   tau = the largest p value v with #{p >= v} >= top_k or mass{p >= v} >= top_p,
 *   kept_i = p_i (p_i > tau), p_i * comp (p_i == tau), 0 (p_i < tau), where comp
 *   spends exactly the top_k / top_p budget left on the entries equal to tau,
 *   out[b] = inverse CDF of kept (vocabulary order) at one Philox uniform in (0,1].
 * sf() maps NaN to 0 and +-inf to +-FLT_MAX.  top_k <= 0 or > V means V;
 * top_p outside [0,1] means 1; top_p == 0 means top_k = 1 (greedy up to ties).
 * temperature must lie in [0.001, 1000].  Every reduction has a fixed order,
 * so a call is run-to-run deterministic for a given state.
 * The random stream is Philox4x32-10 (counter-based; one 128-bit block per
 * draw) and is not the curand stream of the reference: draws agree in law,
 * not value by value. */
#define VKWR_SAMPLING_STATE_BYTES 32 /* per batch row: key[2], counter[4], 2 reserved words */

/* states [B] (B * VKWR_SAMPLING_STATE_BYTES bytes, device): key = seed, counter =
 * (0, 0, b, 0) -- row b draws from its own counter subsequence.
 * Replaces setup_rand_impl / setup_rand_kernel (csrc/sampling/sampling.cu:123-132),
 * op vkwr_sampling::setup_rand (csrc/sampling/torch_bindings.cpp:37-38). */
VKWR_EXPORT int vkwr_sampling_setup_rand(int64_t seed, int B, void* states, void* stream);

/* out [B] int32.  scratch: B*V floats of device memory, required only when
 * V > 65536 (smaller vocabularies stay in registers), else may be NULL.
 * Replaces sampling_temperature_topk_topp_impl and its two kernels
 * (csrc/sampling/sampling.cu:438-646, 648-835, 842-915), op
 * vkwr_sampling::temperature_topk_topp (torch_bindings.cpp:40-42). */
VKWR_EXPORT int vkwr_sampling_temperature_topk_topp(int B, int T, int V, const float* logits, void* states,
                                                    int32_t* out, float* scratch, double temperature,
                                                    int top_k, double top_p, void* stream);

/* As above with per-row penalties [B,V] fp32 subtracted from the logits, then
 * updated in place after the draw:
 *   pen_i <- pen_i * decay + (i == out[b] ? (pen_i == 0 ? presence : repetition) : 0)
 * (fused multiply-add).  Replaces sampling_repetition_topk_topp_impl
 * (csrc/sampling/sampling.cu:134-359, 361-436), op vkwr_sampling::repetition_topk_topp
 * (torch_bindings.cpp:44-47). */
VKWR_EXPORT int vkwr_sampling_repetition_topk_topp(int B, int T, int V, const float* logits, float* penalties,
                                                   void* states, int32_t* out, float* scratch,
                                                   double presence_penalty, double repetition_penalty,
                                                   double penalty_decay, double temperature, int top_k,
                                                   double top_p, void* stream);

/* Host-side Philox4x32-10 block (the generator the sampling kernels run), for
 * checking it against published known-answer vectors.  No counterpart in the
 * reference (which calls curand). */
VKWR_EXPORT void vkwr_sampling_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

#ifdef __cplusplus
}
#endif

#endif /* VKWR_AMD_H */
