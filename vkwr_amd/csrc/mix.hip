// RWKV-7 time-mix / channel-mix glue for gfx950: token-shift lerp (1 or 6
// mix vectors), per-head key normalisation + learning-rate gate, per-head
// GroupNorm with the r.k bonus and output gate, value-residual gate, and the
// elementwise activations.  All HBM-bound.
//
// Token shift.  A lane owns 8 consecutive channels (one 16-byte access) of one
// sequence for a run of up to kTokRun tokens, so x[t-1] is reused from
// registers.  shift_state[b] is read (the previous token at t = 0) and then
// overwritten with x[b,T-1] by the same lane -- the lane whose run starts at
// t = 0 -- so prev at t = 0 is always the value at entry.  Algorithmic bytes
// per token and channel: 2 (x) + 2n (outputs), plus 4 per sequence and
// channel for the shift read and write.
//
// Per-head ops (kk/a gate, GroupNorm) run one wave64 per (sequence, token,
// head), lane = channel; reductions over the head are wave butterflies with a
// broadcast of lane 0's total.

#include "vk_capi.h"
#include "vk_common.cuh"

namespace vk {
namespace {

constexpr int kTokRun = 16;

struct ShiftArgs {
  int B, T, C;
  const _Float16* x;
  _Float16* shift;
  const int32_t* shift_slots;  // may be null: sequence b uses shift row b
  int64_t n_slots;             // rows of the shift pool when shift_slots is given
  const _Float16* mix[6];
  _Float16* out[6];
};

// VW = 8 (16-byte accesses) or 1 (scalar); NMIX = 1 or 6.
template <int VW, int NMIX, bool kHalfMath>
__global__ __launch_bounds__(256) void token_shift_kernel(ShiftArgs p) {
  const int nch = p.C / VW;
  const int runs = (p.T + kTokRun - 1) / kTokRun;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)p.B * runs * nch) return;
  const int ch = (int)(gid % nch);
  const int64_t rest = gid / nch;
  const int run = (int)(rest % runs);
  const int b = (int)(rest / runs);
  const int c0 = ch * VW;
  const int t0 = run * kTokRun;
  const int t1 = min(p.T, t0 + kTokRun);

  _Float16 mu[NMIX][VW];
#pragma unroll
  for (int i = 0; i < NMIX; ++i)
#pragma unroll
    for (int e = 0; e < VW; ++e) mu[i][e] = p.mix[i][c0 + e];

  _Float16 prev[VW];
  const int64_t slot = p.shift_slots ? (int64_t)p.shift_slots[b] : b;
  const int64_t srow = slot * p.C + c0;
  const _Float16* xs = p.x + ((int64_t)b * p.T) * p.C + c0;
  if (p.shift_slots && (slot < 0 || slot >= p.n_slots)) {
    // A slot outside the pool: this sequence's outputs are NaN and no shift row is touched.
    for (int t = t0; t < t1; ++t)
#pragma unroll
      for (int i = 0; i < NMIX; ++i)
#pragma unroll
        for (int e = 0; e < VW; ++e) p.out[i][((int64_t)b * p.T + t) * p.C + c0 + e] = (_Float16)__builtin_nanf("");
    return;
  }
  if (t0 == 0) {
#pragma unroll
    for (int e = 0; e < VW; ++e) prev[e] = p.shift[srow + e];
  } else {
#pragma unroll
    for (int e = 0; e < VW; ++e) prev[e] = xs[(int64_t)(t0 - 1) * p.C + e];
  }
  for (int t = t0; t < t1; ++t) {
    _Float16 cur[VW];
    const int64_t off = (int64_t)t * p.C;
    if constexpr (VW == 8) {
      *reinterpret_cast<h8*>(cur) = ld8(xs + off);
    } else {
      cur[0] = xs[off];
    }
#pragma unroll
    for (int i = 0; i < NMIX; ++i) {
      _Float16 o[VW];
#pragma unroll
      for (int e = 0; e < VW; ++e) {
        if constexpr (kHalfMath) {
          const _Float16 dx = prev[e] - cur[e];
          o[e] = (_Float16)__builtin_fmaf16(dx, mu[i][e], cur[e]);
        } else {
          const float cf = (float)cur[e];
          o[e] = f16_of(__builtin_fmaf((float)prev[e] - cf, (float)mu[i][e], cf));
        }
      }
      _Float16* dst = p.out[i] + ((int64_t)b * p.T + t) * p.C + c0;
      if constexpr (VW == 8) {
        st8(dst, *reinterpret_cast<const h8*>(o));
      } else {
        dst[0] = o[0];
      }
    }
#pragma unroll
    for (int e = 0; e < VW; ++e) prev[e] = cur[e];
  }
  if (t0 == 0) {
    // This lane read shift_state above; it alone writes the new value.
    const _Float16* last = xs + (int64_t)(p.T - 1) * p.C;
#pragma unroll
    for (int e = 0; e < VW; ++e) p.shift[srow + e] = last[e];
  }
}

struct GateArgs {
  int H;
  int64_t heads;  // B * T * H
  const _Float16 *k, *k_k, *a0, *a12, *k_a, *x;
  _Float16* shift;
  _Float16 *new_k, *neg_kk, *kka;
};

// One wave per (b, t, h); 4 waves per workgroup.
__global__ __launch_bounds__(256) void kk_a_gate_kernel(GateArgs p) {
  const int64_t head = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (head >= p.heads) return;  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int h = (int)(head % p.H);
  const int c = h * kHead + lane;
  const int64_t idx = head * kHead + lane;
  const float kv = (float)p.k[idx];
  const float u = kv * (float)p.k_k[c];
  const float total = wave_sum_prod(u, u);
  const float inv = 1.0f / fmaxf(sqrtf(total), kKkEps);
  const float kk = u * inv;
  const float a = sigmoidf((float)p.a0[c] + (float)p.a12[idx]);
  const float ka = (float)p.k_a[c];
  p.new_k[idx] = f16_of(kv * __builtin_fmaf(a, ka, 1.0f - ka));
  p.neg_kk[idx] = (_Float16)(-kk);
  p.kka[idx] = f16_of(kk * a);
  if (p.shift) p.shift[idx] = p.x[idx];  // T == 1: row (b,0) == b
}

struct GnArgs {
  int H;
  int64_t heads;
  const _Float16 *x, *r, *k, *v, *r_k, *w, *b, *g;
  _Float16* out;
  int out_frag;  // out in frag layout (row = token, K = C)
};

__global__ __launch_bounds__(256) void groupnorm_bonus_gate_kernel(GnArgs p) {
  const int64_t head = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (head >= p.heads) return;  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int h = (int)(head % p.H);
  const int c = h * kHead + lane;
  const int64_t idx = head * kHead + lane;
  const float xv = (float)p.x[idx];
  const float mean = wave_sum(xv) * (1.0f / 64.0f);
  const float d = xv - mean;
  const float var = wave_sum_prod(d, d) * (1.0f / 64.0f);
  const float rstd = rsqrtf(var + kGroupNormEps);
  const float rkv = wave_sum_prod((float)p.r[idx] * (float)p.k[idx], (float)p.r_k[c]);
  float y = __builtin_fmaf(d * rstd, (float)p.w[c], (float)p.b[c]);
  y = __builtin_fmaf(rkv, (float)p.v[idx], y);
  const int64_t o = p.out_frag ? frag_index(head / p.H, c, (int64_t)p.H * kHead) : idx;
  p.out[o] = f16_of(y * (float)p.g[idx]);
}

// ---- 16-byte forms of the two kernels above: 8 lanes per (b, t, h), lane g of
// the group holding channels 8g .. 8g + 7 (one 16-byte access per vector), 8
// heads per wave.  head_sum8 adds the 64 channel values in exactly the
// pairwise tree of wave_sum (xor 32, 16, 8, 4, 2, 1 over the channel index):
// channel 8g + e pairs with lane g ^ 4, g ^ 2, g ^ 1 (same e), then with e ^ 4,
// e ^ 2, e ^ 1 inside the lane, so the results are bit-identical to the
// one-channel-per-lane kernels (and to the fused decode kernel).
// The result is the group's lane 0 value, broadcast: with a fused first stage
// the lanes' trees differ (each keeps its own products exact), and wave_sum
// takes lane 0's.
__device__ __forceinline__ float head_sum8_tail(float (&x)[8], int first_m) {
#pragma unroll
  for (int m = 4; m >= 1; m >>= 1)
    if (m <= first_m)
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] += __shfl_xor(x[e], m, 64);
  const float t = ((x[0] + x[4]) + (x[2] + x[6])) + ((x[1] + x[5]) + (x[3] + x[7]));
  return __shfl(t, (int)(threadIdx.x & 56), 64);
}
__device__ __forceinline__ float head_sum8(float (&x)[8]) { return head_sum8_tail(x, 4); }
// head_sum8 of a[e] * b[e] with the first stage fused as in wave_sum_prod
__device__ __forceinline__ float head_sum8_prod(const float (&a)[8], const float (&b)[8]) {
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = __builtin_fmaf(a[e], b[e], __shfl_xor(a[e] * b[e], 4, 64));
  return head_sum8_tail(x, 2);
}

__global__ __launch_bounds__(256) void kk_a_gate_vec_kernel(GateArgs p) {
  const int64_t head = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  const bool live = head < p.heads;
  const int64_t hd = live ? head : p.heads - 1;  // dead lanes join the shuffles on a valid head
  const int g = threadIdx.x & 7;
  const int c0 = (int)(hd % p.H) * kHead + 8 * g;
  const int64_t i0 = hd * kHead + 8 * g;
  const h8 k8 = ld8(p.k + i0), kk8 = ld8(p.k_k + c0), a08 = ld8(p.a0 + c0), a128 = ld8(p.a12 + i0),
           ka8 = ld8(p.k_a + c0);
  float u[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) u[e] = (float)k8.v[e] * (float)kk8.v[e];
  const float total = head_sum8_prod(u, u);
  const float inv = 1.0f / fmaxf(sqrtf(total), kKkEps);
  h8 nk, nkk, kka;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float kv = (float)k8.v[e];
    const float kk = u[e] * inv;
    const float a = sigmoidf((float)a08.v[e] + (float)a128.v[e]);
    const float ka = (float)ka8.v[e];
    nk.v[e] = f16_of(kv * __builtin_fmaf(a, ka, 1.0f - ka));
    nkk.v[e] = (_Float16)(-kk);
    kka.v[e] = f16_of(kk * a);
  }
  if (!live) return;
  st8(p.new_k + i0, nk);
  st8(p.neg_kk + i0, nkk);
  st8(p.kka + i0, kka);
  if (p.shift) st8(p.shift + i0, ld8(p.x + i0));  // T == 1: row (b,0) == b
}

__global__ __launch_bounds__(256) void groupnorm_bonus_gate_vec_kernel(GnArgs p) {
  const int64_t head = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  const bool live = head < p.heads;
  const int64_t hd = live ? head : p.heads - 1;
  const int g = threadIdx.x & 7;
  const int c0 = (int)(hd % p.H) * kHead + 8 * g;
  const int64_t i0 = hd * kHead + 8 * g;
  const h8 x8 = ld8(p.x + i0), r8 = ld8(p.r + i0), k8 = ld8(p.k + i0), rk8 = ld8(p.r_k + c0);
  float t[8], xv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) t[e] = xv[e] = (float)x8.v[e];
  const float mean = head_sum8(t) * (1.0f / 64.0f);
  float d[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) d[e] = xv[e] - mean;
  const float var = head_sum8_prod(d, d) * (1.0f / 64.0f);
  const float rstd = rsqrtf(var + kGroupNormEps);
  float rk[8], rkc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    rk[e] = (float)r8.v[e] * (float)k8.v[e];
    rkc[e] = (float)rk8.v[e];
  }
  const float rkv = head_sum8_prod(rk, rkc);
  const h8 w8 = ld8(p.w + c0), b8 = ld8(p.b + c0), v8 = ld8(p.v + i0), g8 = ld8(p.g + i0);
  h8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float y = __builtin_fmaf(d[e] * rstd, (float)w8.v[e], (float)b8.v[e]);
    y = __builtin_fmaf(rkv, (float)v8.v[e], y);
    o.v[e] = f16_of(y * (float)g8.v[e]);
  }
  if (!live) return;
  const int64_t o0 = p.out_frag ? frag_index(hd / p.H, c0, (int64_t)p.H * kHead) : i0;
  st8(p.out + o0, o);
}

__global__ __launch_bounds__(256) void vres_gate_kernel(int64_t n, int C, const _Float16* v,
                                                        const _Float16* vf, const _Float16* v0,
                                                        const _Float16* v12, _Float16* out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int c = (int)(i % C);
  const float vv = (float)v[i];
  const float gate = sigmoidf((float)v0[c] + (float)v12[i]);
  out[i] = f16_of(__builtin_fmaf((float)vf[i] - vv, gate, vv));
}

template <int ACT>
__device__ __forceinline__ float act_f(float x) {
  if constexpr (ACT == VKWR_ACT_RELU_SQUARE) {
    const float r = fmaxf(x, 0.0f);
    return r * r;
  } else if constexpr (ACT == VKWR_ACT_TANH) {
    return tanhf(x);
  } else {
    return sigmoidf(x);
  }
}

// n8 = number of 8-element vectors handled by the vector path; the scalar tail
// (n - 8*n8 elements) by the same launch.
template <int ACT>
__global__ __launch_bounds__(256) void activation_kernel(int64_t n, int64_t n8, const _Float16* x,
                                                         _Float16* out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n8) {
    const h8 a = ld8(x + i * 8);
    h8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o.v[e] = (_Float16)act_f<ACT>((float)a.v[e]);
    st8(out + i * 8, o);
  } else {
    const int64_t j = n8 * 8 + (i - n8);
    if (j < n) out[j] = (_Float16)act_f<ACT>((float)x[j]);
  }
}

__global__ __launch_bounds__(256) void add_vec_kernel(int64_t n, int C, const _Float16* x,
                                                      const _Float16* vec, _Float16* out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = (_Float16)((float)x[i] + (float)vec[i % C]);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int grid_for(int64_t items, const char* fn, unsigned* blocks) {
  const int64_t b = (items + 255) / 256;
  VK_REQUIRE(b <= 0x7fffffff, "%s: too many elements", fn);
  *blocks = (unsigned)b;
  return VKWR_OK;
}

template <int VW, int NMIX>
void launch_shift(const ShiftArgs& p, bool half, unsigned blocks, hipStream_t s) {
  if (half) hipLaunchKernelGGL((token_shift_kernel<VW, NMIX, true>), dim3(blocks), dim3(256), 0, s, p);
  else hipLaunchKernelGGL((token_shift_kernel<VW, NMIX, false>), dim3(blocks), dim3(256), 0, s, p);
}

}  // namespace
}  // namespace vk

using namespace vk;

namespace {
int token_shift_mix(const char* fn, int B, int T, int C, const uint16_t* x, uint16_t* shift_state,
                    const int32_t* shift_slots, int64_t n_slots, int n_mix, const uint16_t* const* mix,
                    uint16_t* const* out, int half_math, void* stream) {
  VK_REQUIRE(B >= 0 && T >= 0 && C >= 0, "%s: negative size", fn);
  VK_REQUIRE(n_mix == 1 || n_mix == 6, "%s: n_mix must be 1 or 6 (got %d)", fn, n_mix);
  if ((int64_t)B * T * C == 0) return VKWR_OK;
  VK_REQUIRE(x && shift_state && mix && out, "%s: null pointer", fn);
  ShiftArgs p{};
  p.B = B;
  p.T = T;
  p.C = C;
  p.x = reinterpret_cast<const _Float16*>(x);
  p.shift = reinterpret_cast<_Float16*>(shift_state);
  p.shift_slots = shift_slots;
  p.n_slots = n_slots;
  bool vec = (C % 8 == 0) && aligned16(x) && aligned16(shift_state);
  for (int i = 0; i < n_mix; ++i) {
    VK_REQUIRE(mix[i] && out[i], "%s: null pointer", fn);
    p.mix[i] = reinterpret_cast<const _Float16*>(mix[i]);
    p.out[i] = reinterpret_cast<_Float16*>(out[i]);
    vec = vec && aligned16(mix[i]) && aligned16(out[i]);
  }
  const int VW = vec ? 8 : 1;
  const int64_t items = (int64_t)B * ((T + kTokRun - 1) / kTokRun) * (C / VW);
  unsigned blocks;
  if (int e = grid_for(items, fn, &blocks)) return e;
  hipStream_t s = (hipStream_t)stream;
  const bool half = half_math != 0;
  if (vec) {
    if (n_mix == 1) launch_shift<8, 1>(p, half, blocks, s);
    else launch_shift<8, 6>(p, half, blocks, s);
  } else {
    if (n_mix == 1) launch_shift<1, 1>(p, half, blocks, s);
    else launch_shift<1, 6>(p, half, blocks, s);
  }
  return check_launch(fn);
}
}  // namespace

extern "C" int vkwr_token_shift_mix_f16(int B, int T, int C, const uint16_t* x,
                                        uint16_t* shift_state, int n_mix,
                                        const uint16_t* const* mix, uint16_t* const* out,
                                        int half_math, void* stream) {
  clear_error();
  return token_shift_mix("vkwr_token_shift_mix_f16", B, T, C, x, shift_state, nullptr, 0, n_mix, mix, out,
                         half_math, stream);
}

extern "C" int vkwr_token_shift_mix_slots_f16(int B, int T, int C, const uint16_t* x, uint16_t* shift_pool,
                                              int64_t n_slots, const int32_t* shift_slots, int n_mix,
                                              const uint16_t* const* mix, uint16_t* const* out,
                                              int half_math, void* stream) {
  clear_error();
  const char* fn = "vkwr_token_shift_mix_slots_f16";
  VK_REQUIRE((int64_t)B * T * C == 0 || shift_slots, "%s: null shift_slots", fn);
  VK_REQUIRE(n_slots >= 0, "%s: negative n_slots", fn);
  return token_shift_mix(fn, B, T, C, x, shift_pool, shift_slots, n_slots, n_mix, mix, out, half_math, stream);
}

extern "C" int vkwr_tmix_kk_a_gate_f16(int B, int T, int C, int H, const uint16_t* k,
                                       const uint16_t* k_k, const uint16_t* a0,
                                       const uint16_t* a12, const uint16_t* k_a,
                                       const uint16_t* x, uint16_t* shift_state,
                                       uint16_t* new_k, uint16_t* neg_kk, uint16_t* kka,
                                       void* stream) {
  clear_error();
  const char* fn = "vkwr_tmix_kk_a_gate_f16";
  VK_REQUIRE(B >= 0 && T >= 0 && H >= 0, "%s: negative size", fn);
  VK_REQUIRE(C == H * kHead, "%s: only head size 64 is supported (C=%d H=%d)", fn, C, H);
  VK_REQUIRE(shift_state == nullptr || T == 1, "%s: the shift update needs T == 1", fn);
  const int64_t heads = (int64_t)B * T * H;
  if (heads == 0) return VKWR_OK;
  VK_REQUIRE(k && k_k && a0 && a12 && k_a && new_k && neg_kk && kka, "%s: null pointer", fn);
  VK_REQUIRE(shift_state == nullptr || x != nullptr, "%s: null x with a shift update", fn);
  GateArgs p{H, heads,
             reinterpret_cast<const _Float16*>(k), reinterpret_cast<const _Float16*>(k_k),
             reinterpret_cast<const _Float16*>(a0), reinterpret_cast<const _Float16*>(a12),
             reinterpret_cast<const _Float16*>(k_a), reinterpret_cast<const _Float16*>(x),
             reinterpret_cast<_Float16*>(shift_state), reinterpret_cast<_Float16*>(new_k),
             reinterpret_cast<_Float16*>(neg_kk), reinterpret_cast<_Float16*>(kka)};
  const bool vec = aligned16(k) && aligned16(k_k) && aligned16(a0) && aligned16(a12) && aligned16(k_a) &&
                   aligned16(new_k) && aligned16(neg_kk) && aligned16(kka) &&
                   (!shift_state || (aligned16(shift_state) && aligned16(x)));
  const int64_t blocks = vec ? (heads + 31) / 32 : (heads + 3) / 4;
  VK_REQUIRE(blocks <= 0x7fffffff, "%s: too many heads", fn);
  if (vec)
    hipLaunchKernelGGL(kk_a_gate_vec_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL(kk_a_gate_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, p);
  return check_launch(fn);
}

namespace {
int groupnorm_bonus_gate(const char* fn, int B, int T, int C, int H, const uint16_t* x, const uint16_t* r,
                         const uint16_t* k, const uint16_t* v, const uint16_t* r_k, const uint16_t* weight,
                         const uint16_t* bias, const uint16_t* g, uint16_t* out, int frag, void* stream) {
  VK_REQUIRE(B >= 0 && T >= 0 && H >= 0, "%s: negative size", fn);
  VK_REQUIRE(C == H * kHead, "%s: only head size 64 is supported (C=%d H=%d)", fn, C, H);
  const int64_t heads = (int64_t)B * T * H;
  if (heads == 0) return VKWR_OK;
  VK_REQUIRE(x && r && k && v && r_k && weight && bias && g && out, "%s: null pointer", fn);
  GnArgs p{H, heads,
           reinterpret_cast<const _Float16*>(x), reinterpret_cast<const _Float16*>(r),
           reinterpret_cast<const _Float16*>(k), reinterpret_cast<const _Float16*>(v),
           reinterpret_cast<const _Float16*>(r_k), reinterpret_cast<const _Float16*>(weight),
           reinterpret_cast<const _Float16*>(bias), reinterpret_cast<const _Float16*>(g),
           reinterpret_cast<_Float16*>(out), frag};
  VK_REQUIRE(!frag || C % kFragPad == 0, "%s: frag output needs C %% %d == 0", fn, kFragPad);
  const bool vec = aligned16(x) && aligned16(r) && aligned16(k) && aligned16(v) && aligned16(r_k) &&
                   aligned16(weight) && aligned16(bias) && aligned16(g) && aligned16(out);
  const int64_t blocks = vec ? (heads + 31) / 32 : (heads + 3) / 4;
  VK_REQUIRE(blocks <= 0x7fffffff, "%s: too many heads", fn);
  if (vec)
    hipLaunchKernelGGL(groupnorm_bonus_gate_vec_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL(groupnorm_bonus_gate_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, p);
  return check_launch(fn);
}
}  // namespace

extern "C" int vkwr_tmix_groupnorm_bonus_gate_f16(int B, int T, int C, int H, const uint16_t* x,
                                                  const uint16_t* r, const uint16_t* k,
                                                  const uint16_t* v, const uint16_t* r_k,
                                                  const uint16_t* weight, const uint16_t* bias,
                                                  const uint16_t* g, uint16_t* out, void* stream) {
  clear_error();
  return groupnorm_bonus_gate("vkwr_tmix_groupnorm_bonus_gate_f16", B, T, C, H, x, r, k, v, r_k, weight, bias,
                              g, out, 0, stream);
}

extern "C" int vkwr_tmix_groupnorm_bonus_gate_frag_f16(int B, int T, int C, int H, const uint16_t* x,
                                                       const uint16_t* r, const uint16_t* k,
                                                       const uint16_t* v, const uint16_t* r_k,
                                                       const uint16_t* weight, const uint16_t* bias,
                                                       const uint16_t* g, uint16_t* out, void* stream) {
  clear_error();
  return groupnorm_bonus_gate("vkwr_tmix_groupnorm_bonus_gate_frag_f16", B, T, C, H, x, r, k, v, r_k, weight,
                              bias, g, out, 1, stream);
}

extern "C" int vkwr_tmix_vres_gate_f16(int64_t rows, int C, const uint16_t* v,
                                       const uint16_t* v_first, const uint16_t* v0,
                                       const uint16_t* v12, uint16_t* out, void* stream) {
  clear_error();
  const char* fn = "vkwr_tmix_vres_gate_f16";
  VK_REQUIRE(rows >= 0 && C > 0, "%s: bad size", fn);
  const int64_t n = rows * (int64_t)C;
  if (n == 0) return VKWR_OK;
  VK_REQUIRE(v && v_first && v0 && v12 && out, "%s: null pointer", fn);
  unsigned blocks;
  if (int e = grid_for(n, fn, &blocks)) return e;
  hipLaunchKernelGGL(vres_gate_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, n, C,
                     reinterpret_cast<const _Float16*>(v), reinterpret_cast<const _Float16*>(v_first),
                     reinterpret_cast<const _Float16*>(v0), reinterpret_cast<const _Float16*>(v12),
                     reinterpret_cast<_Float16*>(out));
  return check_launch(fn);
}

extern "C" int vkwr_activation_f16(int act, int64_t n, const uint16_t* x, uint16_t* out,
                                   void* stream) {
  clear_error();
  const char* fn = "vkwr_activation_f16";
  VK_REQUIRE(act >= VKWR_ACT_RELU_SQUARE && act <= VKWR_ACT_SIGMOID, "%s: unknown act %d", fn, act);
  VK_REQUIRE(n >= 0, "%s: negative size", fn);
  if (n == 0) return VKWR_OK;
  VK_REQUIRE(x && out, "%s: null pointer", fn);
  const int64_t n8 = (aligned16(x) && aligned16(out)) ? n / 8 : 0;
  unsigned blocks;
  if (int e = grid_for(n8 + (n - 8 * n8), fn, &blocks)) return e;
  const _Float16* xi = reinterpret_cast<const _Float16*>(x);
  _Float16* o = reinterpret_cast<_Float16*>(out);
  hipStream_t s = (hipStream_t)stream;
  if (act == VKWR_ACT_RELU_SQUARE)
    hipLaunchKernelGGL(activation_kernel<VKWR_ACT_RELU_SQUARE>, dim3(blocks), dim3(256), 0, s, n, n8, xi, o);
  else if (act == VKWR_ACT_TANH)
    hipLaunchKernelGGL(activation_kernel<VKWR_ACT_TANH>, dim3(blocks), dim3(256), 0, s, n, n8, xi, o);
  else
    hipLaunchKernelGGL(activation_kernel<VKWR_ACT_SIGMOID>, dim3(blocks), dim3(256), 0, s, n, n8, xi, o);
  return check_launch(fn);
}

extern "C" int vkwr_add_vec_f16(int64_t n, int C, const uint16_t* x, const uint16_t* vec,
                                uint16_t* out, void* stream) {
  clear_error();
  const char* fn = "vkwr_add_vec_f16";
  VK_REQUIRE(n >= 0 && C > 0 && n % C == 0, "%s: n must be a multiple of C", fn);
  if (n == 0) return VKWR_OK;
  VK_REQUIRE(x && vec && out, "%s: null pointer", fn);
  unsigned blocks;
  if (int e = grid_for(n, fn, &blocks)) return e;
  hipLaunchKernelGGL(add_vec_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, n, C,
                     reinterpret_cast<const _Float16*>(x), reinterpret_cast<const _Float16*>(vec),
                     reinterpret_cast<_Float16*>(out));
  return check_launch(fn);
}
