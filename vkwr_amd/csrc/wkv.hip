// RWKV-7 WKV (generalised delta rule) kernels for gfx950.
//
// Work decomposition: one 64-lane wavefront (one workgroup) per (sequence,
// head).  Lane i owns row i of the head's 64x64 state in VGPRs for the whole
// call, so the two per-token dot products
//     sa_i = sum_j S_ij a_j        y_i = sum_j S'_ij r_j
// are lane-local FMA chains in j order, exactly the reference's per-thread
// loop (csrc/v1/wkv/wkv_fp32_v2.cu:103-117), and need no cross-lane traffic.
// The per-token channel vectors (r, decay, k, a, b) are produced one channel
// per lane, staged in LDS and read back as broadcasts (uniform-address
// ds_read_b128).
//
// State I/O: the row-per-lane layout would make lane i touch bytes
// [256 i, 256 i + 256) of the head -- a 256-byte lane stride, uncoalesced.
// Instead each lane issues 16-byte direct-to-LDS loads (global_load_lds_dwordx4)
// whose addresses cover whole 128-byte lines.  The fp32 state (16 KiB per head)
// goes through an 8 KiB LDS tile in two phases, one column half (128 bytes of
// every row) per phase: chunk q (16 bytes) of row i's half lands at LDS slot
// i*8 + (q ^ (i & 7)), so the row-per-lane reads that follow hit 8 distinct
// 16-byte bank groups per 8 lanes.  The write-back is the mirror image (LDS
// transpose, then 128-byte-line global stores), again one half at a time.
// Halving the tile from 16 to 8 KiB doubles the waves an MI355X CU can hold
// (160 KiB LDS): a 128-sequence x 32-head decode step (4096 waves) is then
// resident in one round instead of 1.6, which measured 21.9 us against
// 26.1 us per step for a single 16 KiB phase.
// The fp16-state family stages its 8 KiB head in one phase (128-byte rows, 8
// chunks per row, slot i*8 + (q ^ ((i >> 1) & 7))).

#include "vk_capi.h"
#include "vk_common.cuh"

namespace vk {
namespace {

struct Fp32Args {
  int T, C, H, n_slots;
  float* state;
  const int32_t* slots;
  const _Float16 *r, *w, *k, *v, *a, *b;
  _Float16* y;
};

// ---- fp32 state staging: HBM <-> LDS (swizzled) <-> VGPRs, one column half
// per phase (see the State I/O note above).  `st` is the 8 KiB tile.
__device__ __forceinline__ void load_state_fp32(const float* S, f4* st, float* s, int lane) {
  const int sub = lane & 7;
#pragma unroll
  for (int ph = 0; ph < 2; ++ph) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int row = 8 * c + (lane >> 3);
      dma16(S + row * kHead + ph * 32 + (sub ^ (row & 7)) * 4, &st[c * 64]);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const f4 x = st[lane * 8 + (q ^ sub)];
      const int j = ph * 32 + 4 * q;
      s[j + 0] = x.x;
      s[j + 1] = x.y;
      s[j + 2] = x.z;
      s[j + 3] = x.w;
    }
    __syncthreads();
  }
}

__device__ __forceinline__ void store_state_fp32(float* S, f4* st, const float* s, int lane) {
  const int sub = lane & 7;
  __syncthreads();
#pragma unroll
  for (int ph = 0; ph < 2; ++ph) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int j = ph * 32 + 4 * q;
      st[lane * 8 + (q ^ sub)] = f4{s[j + 0], s[j + 1], s[j + 2], s[j + 3]};
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int row = 8 * c + (lane >> 3);
      *reinterpret_cast<f4*>(S + row * kHead + ph * 32 + (sub ^ (row & 7)) * 4) = st[c * 64 + lane];
    }
    __syncthreads();
  }
}

// One token of the fp32-state recurrence for row `lane` (state row in s[]).
// vb: 5*64 floats of LDS for the token's channel vectors (r, decay, k, a, b),
// written here one channel per lane and read back as broadcasts.
__device__ __forceinline__ _Float16 token_fp32(float* s, float* vb, int lane, _Float16 xr,
                                               _Float16 xw, _Float16 xk, _Float16 xv,
                                               _Float16 xa, _Float16 xb) {
  vb[lane] = (float)xr;
  vb[kHead + lane] = decay((float)xw);
  vb[2 * kHead + lane] = (float)xk;
  vb[3 * kHead + lane] = (float)xa;
  vb[4 * kHead + lane] = (float)xb;
  const float vi = (float)xv;
  __syncthreads();
  const f4* R4 = reinterpret_cast<const f4*>(vb);
  const f4* D4 = R4 + 16;
  const f4* K4 = R4 + 32;
  const f4* A4 = R4 + 48;
  const f4* B4 = R4 + 64;

  float sa = 0.0f;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const f4 a4 = A4[q];
    sa = __builtin_fmaf(s[4 * q + 0], a4.x, sa);
    sa = __builtin_fmaf(s[4 * q + 1], a4.y, sa);
    sa = __builtin_fmaf(s[4 * q + 2], a4.z, sa);
    sa = __builtin_fmaf(s[4 * q + 3], a4.w, sa);
  }
  float acc = 0.0f;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const f4 d4 = D4[q], b4 = B4[q], k4 = K4[q], r4 = R4[q];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float x = s[4 * q + e] * d4[e];
      x = __builtin_fmaf(sa, b4[e], x);
      x = __builtin_fmaf(k4[e], vi, x);
      s[4 * q + e] = x;
      acc = __builtin_fmaf(x, r4[e], acc);
    }
  }
  // Keep acc an fp32 value: without this the compiler may fold fma + cvt into
  // v_fma_mixlo_f16, which rounds once instead of f32-then-f16.
  asm volatile("" : "+v"(acc));
  return (_Float16)acc;
}

// Resolves the state block of (sequence bi, head h); with slots, an entry
// outside [0, n_slots) yields nullptr (the caller writes NaN rows, skips the pool).
template <bool kSlots>
__device__ __forceinline__ float* state_block(const Fp32Args& p, int bi, int h) {
  size_t sidx = (size_t)bi;
  if constexpr (kSlots) {
    const int sl = p.slots[bi];
    if (sl < 0 || sl >= p.n_slots) return nullptr;
    sidx = (size_t)sl;
  }
  return p.state + (sidx * p.H + h) * (kHead * kHead);
}

// Decode step (T == 1).  At most 128 VGPRs (4 waves per SIMD, 16 per CU):
// with the 8 KiB LDS tile a 4096-wave step then fits on the 256 CUs in one
// round.  The token's inputs are loaded before the state so that their
// latency overlaps the state transfer.
template <bool kSlots>
__global__ __launch_bounds__(64, 4) void wkv7_fp32_step_kernel(Fp32Args p) {
  __shared__ f4 st[512];
  const int lane = threadIdx.x;
  const int bh = blockIdx.x;
  const int bi = bh / p.H;
  const int h = bh - bi * p.H;
  const size_t tok = (size_t)bi * p.C + (size_t)h * kHead + lane;
  const _Float16 xr = p.r[tok], xw = p.w[tok], xk = p.k[tok];
  const _Float16 xv = p.v[tok], xa = p.a[tok], xb = p.b[tok];
  float* S = state_block<kSlots>(p, bi, h);
  if (S == nullptr) {
    p.y[tok] = (_Float16)__builtin_nanf("");
    return;
  }
  float s[kHead];
  load_state_fp32(S, st, s, lane);
  p.y[tok] = token_fp32(s, reinterpret_cast<float*>(st), lane, xr, xw, xk, xv, xa, xb);
  store_state_fp32(S, st, s, lane);
}

// T tokens; the next token's inputs are loaded while the current one computes,
// and the token vectors are double-buffered inside the staging tile.
template <bool kSlots>
__global__ __launch_bounds__(64) void wkv7_fp32_seq_kernel(Fp32Args p) {
  __shared__ f4 st[512];
  const int lane = threadIdx.x;
  const int bh = blockIdx.x;
  const int bi = bh / p.H;
  const int h = bh - bi * p.H;
  const size_t tok0 = (size_t)bi * p.T * p.C + (size_t)h * kHead + lane;
  float* S = state_block<kSlots>(p, bi, h);
  if (S == nullptr) {
    for (int t = 0; t < p.T; ++t) p.y[tok0 + (size_t)t * p.C] = (_Float16)__builtin_nanf("");
    return;
  }
  _Float16 xr = p.r[tok0], xw = p.w[tok0], xk = p.k[tok0];
  _Float16 xv = p.v[tok0], xa = p.a[tok0], xb = p.b[tok0];
  float s[kHead];
  load_state_fp32(S, st, s, lane);
  float* vec = reinterpret_cast<float*>(st);
  for (int t = 0; t < p.T; ++t) {
    const _Float16 cr = xr, cw = xw, ck = xk, cv = xv, ca = xa, cb = xb;
    if (t + 1 < p.T) {
      const size_t o = tok0 + (size_t)(t + 1) * p.C;
      xr = p.r[o];
      xw = p.w[o];
      xk = p.k[o];
      xv = p.v[o];
      xa = p.a[o];
      xb = p.b[o];
    }
    p.y[tok0 + (size_t)t * p.C] =
        token_fp32(s, vec + (t & 1) * (5 * kHead), lane, cr, cw, ck, cv, ca, cb);
  }
  store_state_fp32(S, st, s, lane);
}

template <bool kSlots>
void launch_fp32(const Fp32Args& p, int B, hipStream_t stream) {
  if (p.T == 1) {
    hipLaunchKernelGGL(wkv7_fp32_step_kernel<kSlots>, dim3(B * p.H), dim3(64), 0, stream, p);
  } else {
    hipLaunchKernelGGL(wkv7_fp32_seq_kernel<kSlots>, dim3(B * p.H), dim3(64), 0, stream, p);
  }
}

struct Fp16Args {
  int T, C, H;
  _Float16* state;
  const _Float16 *r, *w, *w0, *k, *v, *a, *b;
  _Float16* y;
  const int32_t* elapsed;
};

// fp16-state recurrence.  kLegacy = false: vkwr_v1_wkv::wkv_*_fp16 semantics
// (wkv_fp16_v2.cu:259-291): hfma2 nesting s = fma(s, wd, fma(k, v, fma(sa, b, s))),
// dither phase elapsed + channel + t, optional w0.  kLegacy = true:
// vkwr_rwkv7::forward_* (state_fwd_fp16.cu:57-83): s += s*wd + k*v + sa*b with
// separately rounded fp16 operations, dither phase elapsed + t.
template <bool kLegacy>
__global__ __launch_bounds__(64) void wkv7_fp16_kernel(Fp16Args p) {
  __shared__ f4 st[512];  // one head's fp16 state (8 KiB); reused for token vectors
  const int lane = threadIdx.x;
  const int bh = blockIdx.x;
  const int bi = bh / p.H;
  const int h = bh - bi * p.H;
  const size_t tok0 = (size_t)bi * p.T * p.C + (size_t)h * kHead + lane;
  _Float16* S = p.state + (size_t)bh * (kHead * kHead);

  const int sub = lane & 7;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int row = 8 * c + (lane >> 3);
    const int q = sub ^ ((row >> 1) & 7);
    dma16(S + row * kHead + q * 8, &st[c * 64]);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const int sw = (lane >> 1) & 7;
  h2 s[32];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const f4 x = st[lane * 8 + (q ^ sw)];
    const h2* hx = reinterpret_cast<const h2*>(&x);
    s[4 * q + 0] = hx[0];
    s[4 * q + 1] = hx[1];
    s[4 * q + 2] = hx[2];
    s[4 * q + 3] = hx[3];
  }
  __syncthreads();

  const uint32_t el = (uint32_t)p.elapsed[bi];
  const uint32_t chan = (uint32_t)(h * kHead + lane);
  float w0f = 0.0f;
  if (!kLegacy && p.w0 != nullptr) w0f = (float)p.w0[chan];

  _Float16* vec = reinterpret_cast<_Float16*>(st);
  _Float16 xr = p.r[tok0], xw = p.w[tok0], xk = p.k[tok0];
  _Float16 xv = p.v[tok0], xa = p.a[tok0], xb = p.b[tok0];
  for (int t = 0; t < p.T; ++t) {
    _Float16* vb = vec + (t & 1) * (5 * kHead);
    float wf = (float)xw;
    uint32_t phase;
    if constexpr (kLegacy) {
      phase = el + (uint32_t)t;
    } else {
      if (p.w0 != nullptr) wf = wf + w0f;
      phase = el + chan + (uint32_t)t;
    }
    vb[lane] = xr;
    vb[kHead + lane] = w_delta(wf, phase);
    vb[2 * kHead + lane] = xk;
    vb[3 * kHead + lane] = xa;
    vb[4 * kHead + lane] = xb;
    const _Float16 vi = xv;
    if (t + 1 < p.T) {
      const size_t o = tok0 + (size_t)(t + 1) * p.C;
      xr = p.r[o];
      xw = p.w[o];
      xk = p.k[o];
      xv = p.v[o];
      xa = p.a[o];
      xb = p.b[o];
    }
    __syncthreads();
    const h2* R2 = reinterpret_cast<const h2*>(vb);
    const h2* W2 = R2 + 32;
    const h2* K2 = R2 + 64;
    const h2* A2 = R2 + 96;
    const h2* B2 = R2 + 128;

    h2 sa2 = {(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
    for (int m = 0; m < 32; ++m) {
      if constexpr (kLegacy) {
        sa2 = sa2 + A2[m] * s[m];
      } else {
        sa2 = __builtin_elementwise_fma(A2[m], s[m], sa2);
      }
    }
    const _Float16 sa = sa2.x + sa2.y;
    const h2 sav = {sa, sa};
    const h2 vv = {vi, vi};
    h2 y2 = {(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
    for (int m = 0; m < 32; ++m) {
      if constexpr (kLegacy) {
        const h2 t1 = s[m] * W2[m];
        const h2 t2 = K2[m] * vv;
        const h2 t3 = t1 + t2;
        const h2 t4 = sav * B2[m];
        const h2 t5 = t3 + t4;
        s[m] = s[m] + t5;
        y2 = y2 + s[m] * R2[m];
      } else {
        const h2 in1 = __builtin_elementwise_fma(sav, B2[m], s[m]);
        const h2 in2 = __builtin_elementwise_fma(K2[m], vv, in1);
        s[m] = __builtin_elementwise_fma(s[m], W2[m], in2);
        y2 = __builtin_elementwise_fma(s[m], R2[m], y2);
      }
    }
    p.y[tok0 + (size_t)t * p.C] = y2.x + y2.y;
  }

  __syncthreads();
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    f4 x;
    h2* hx = reinterpret_cast<h2*>(&x);
    hx[0] = s[4 * q + 0];
    hx[1] = s[4 * q + 1];
    hx[2] = s[4 * q + 2];
    hx[3] = s[4 * q + 3];
    st[lane * 8 + (q ^ sw)] = x;
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int row = 8 * c + (lane >> 3);
    const int q = sub ^ ((row >> 1) & 7);
    *reinterpret_cast<f4*>(S + row * kHead + q * 8) = st[c * 64 + lane];
  }
}

__global__ __launch_bounds__(256) void advance_i32_kernel(int32_t* x, int64_t n, int32_t amount) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = (int32_t)((uint32_t)x[i] + (uint32_t)amount);
}

int check_wkv_dims(const char* fn, int B, int T, int C, int H) {
  VK_REQUIRE(B >= 0 && T >= 0 && H >= 0, "%s: negative size (B=%d T=%d H=%d)", fn, B, T, H);
  VK_REQUIRE(C == H * kHead, "%s: only head size 64 is supported (C=%d H=%d)", fn, C, H);
  VK_REQUIRE((int64_t)B * H <= 0x7fffffff, "%s: B*H too large", fn);
  return VKWR_OK;
}

}  // namespace
}  // namespace vk

using namespace vk;

extern "C" int vkwr_wkv7_fp32_forward(int B, int T, int C, int H, int mode, float* state,
                                      const uint16_t* r, const uint16_t* w, const uint16_t* k,
                                      const uint16_t* v, const uint16_t* a, const uint16_t* b,
                                      uint16_t* y, void* stream) {
  clear_error();
  if (int e = check_wkv_dims("vkwr_wkv7_fp32_forward", B, T, C, H)) return e;
  VK_REQUIRE(mode >= 0 && mode <= 3, "vkwr_wkv7_fp32_forward: mode must be 0..3 (got %d)", mode);
  if (B == 0 || H == 0 || T == 0) return VKWR_OK;
  VK_REQUIRE(state && r && w && k && v && a && b && y, "vkwr_wkv7_fp32_forward: null pointer");
  Fp32Args p{T, C, H, B, state, nullptr,
             reinterpret_cast<const _Float16*>(r), reinterpret_cast<const _Float16*>(w),
             reinterpret_cast<const _Float16*>(k), reinterpret_cast<const _Float16*>(v),
             reinterpret_cast<const _Float16*>(a), reinterpret_cast<const _Float16*>(b),
             reinterpret_cast<_Float16*>(y)};
  launch_fp32<false>(p, B, (hipStream_t)stream);
  return check_launch("vkwr_wkv7_fp32_forward");
}

extern "C" int vkwr_wkv7_fp32_forward_slots(int B, int T, int C, int H, float* pool, int n_slots,
                                            const int32_t* slots, const uint16_t* r,
                                            const uint16_t* w, const uint16_t* k, const uint16_t* v,
                                            const uint16_t* a, const uint16_t* b, uint16_t* y,
                                            void* stream) {
  clear_error();
  if (int e = check_wkv_dims("vkwr_wkv7_fp32_forward_slots", B, T, C, H)) return e;
  VK_REQUIRE(n_slots >= 0, "vkwr_wkv7_fp32_forward_slots: negative pool size");
  if (B == 0 || H == 0 || T == 0) return VKWR_OK;
  VK_REQUIRE(pool && slots && r && w && k && v && a && b && y,
             "vkwr_wkv7_fp32_forward_slots: null pointer");
  Fp32Args p{T, C, H, n_slots, pool, slots,
             reinterpret_cast<const _Float16*>(r), reinterpret_cast<const _Float16*>(w),
             reinterpret_cast<const _Float16*>(k), reinterpret_cast<const _Float16*>(v),
             reinterpret_cast<const _Float16*>(a), reinterpret_cast<const _Float16*>(b),
             reinterpret_cast<_Float16*>(y)};
  launch_fp32<true>(p, B, (hipStream_t)stream);
  return check_launch("vkwr_wkv7_fp32_forward_slots");
}

static int launch_fp16(const char* fn, bool legacy, int B, int T, int C, int H, uint16_t* state,
                       const uint16_t* r, const uint16_t* w, const uint16_t* w0, const uint16_t* k,
                       const uint16_t* v, const uint16_t* a, const uint16_t* b, uint16_t* y,
                       const int32_t* elapsed_t, void* stream) {
  clear_error();
  if (int e = check_wkv_dims(fn, B, T, C, H)) return e;
  if (B == 0 || H == 0 || T == 0) return VKWR_OK;
  VK_REQUIRE(state && r && w && k && v && a && b && y && elapsed_t, "%s: null pointer", fn);
  Fp16Args p{T, C, H, reinterpret_cast<_Float16*>(state),
             reinterpret_cast<const _Float16*>(r), reinterpret_cast<const _Float16*>(w),
             reinterpret_cast<const _Float16*>(w0), reinterpret_cast<const _Float16*>(k),
             reinterpret_cast<const _Float16*>(v), reinterpret_cast<const _Float16*>(a),
             reinterpret_cast<const _Float16*>(b), reinterpret_cast<_Float16*>(y), elapsed_t};
  if (legacy) {
    hipLaunchKernelGGL(wkv7_fp16_kernel<true>, dim3(B * H), dim3(64), 0, (hipStream_t)stream, p);
  } else {
    hipLaunchKernelGGL(wkv7_fp16_kernel<false>, dim3(B * H), dim3(64), 0, (hipStream_t)stream, p);
  }
  return check_launch(fn);
}

extern "C" int vkwr_wkv7_fp16_forward(int B, int T, int C, int H, uint16_t* state,
                                      const uint16_t* r, const uint16_t* w, const uint16_t* w0,
                                      const uint16_t* k, const uint16_t* v, const uint16_t* a,
                                      const uint16_t* b, uint16_t* y, const int32_t* elapsed_t,
                                      void* stream) {
  return launch_fp16("vkwr_wkv7_fp16_forward", false, B, T, C, H, state, r, w, w0, k, v, a, b, y,
                     elapsed_t, stream);
}

extern "C" int vkwr_rwkv7_forward(int B, int T, int C, int H, uint16_t* state, const uint16_t* r,
                                  const uint16_t* w, const uint16_t* k, const uint16_t* v,
                                  const uint16_t* a, const uint16_t* b, uint16_t* y,
                                  const int32_t* elapsed_t, void* stream) {
  return launch_fp16("vkwr_rwkv7_forward", true, B, T, C, H, state, r, w, nullptr, k, v, a, b, y,
                     elapsed_t, stream);
}

extern "C" int vkwr_advance_i32(int32_t* x, int64_t n, int32_t amount, void* stream) {
  clear_error();
  VK_REQUIRE(n >= 0, "vkwr_advance_i32: negative length");
  if (n == 0) return VKWR_OK;
  VK_REQUIRE(x != nullptr, "vkwr_advance_i32: null pointer");
  const int64_t blocks = (n + 255) / 256;
  VK_REQUIRE(blocks <= 0x7fffffff, "vkwr_advance_i32: too many elements");
  hipLaunchKernelGGL(advance_i32_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     x, n, amount);
  return check_launch("vkwr_advance_i32");
}
