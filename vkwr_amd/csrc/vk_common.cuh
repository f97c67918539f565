// Device helpers shared by the vkwr_amd HIP kernels (gfx950 / CDNA4, wave64).
//
// All floating-point code here is compiled with -ffp-contract=off: every fused
// multiply-add is an explicit __builtin_fmaf / elementwise fma, so results are
// reproducible bit for bit by any implementation that performs the same IEEE
// operations in the same order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vk {

constexpr int kHead = 64;  // RWKV-7 head size (the only one the ops accept)
// Time-mix epsilons (reference csrc/v1/mix/mix_ops.cu:17-18).
constexpr float kKkEps = 1.0e-12f;         // L2-normalisation floor of kk
constexpr float kGroupNormEps = 64.0e-5f;  // GroupNorm eps of the time-mix output

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

// RWKV-7 decay constants: -e^{-1/2}*log2(e) and -log2(e)
// (reference csrc/v1/wkv/wkv_fp32_v2.cu:14-15; model math, not library constants).
constexpr float kDecayC1 = -0.8750387749145276f;
constexpr float kDecayC2 = -1.4426950408889634f;
constexpr float kTwoNeg41 = 4.547473508864641e-13f;

// 2^x from correctly rounded operations only: range reduction by rint, the
// degree-7 Taylor polynomial of 2^f = e^{f ln 2} on |f| <= 1/2 in Horner form
// with FMA, then an exact power-of-two scale.  Max relative error ~6e-8.
// Results below 2^-126 return 0 (the decay only adds them to 1).  Written without
// branches (the special cases are selected at the end, from the same arithmetic
// on a clamped argument), so that it can be scheduled among other work.
__device__ __forceinline__ float exp2_det(float x) {
  const float xc = __builtin_fminf(__builtin_fmaxf(x, -127.0f), 128.0f);  // NaN -> -127 (replaced below)
  const float n = __builtin_rintf(xc);
  const float f = xc - n;
  float p = 1.525273380405984e-05f;
  p = __builtin_fmaf(p, f, 1.5403530393381608e-04f);
  p = __builtin_fmaf(p, f, 1.3333558146428443e-03f);
  p = __builtin_fmaf(p, f, 9.618129107628477e-03f);
  p = __builtin_fmaf(p, f, 5.550410866482158e-02f);
  p = __builtin_fmaf(p, f, 2.402265069591007e-01f);
  p = __builtin_fmaf(p, f, 6.931471805599453e-01f);
  p = __builtin_fmaf(p, f, 1.0f);
  float r = __builtin_ldexpf(p, (int)n);
  r = x < -126.0f ? 0.0f : r;
  r = x >= 128.0f ? __builtin_huge_valf() : r;
  return x != x ? x : r;
}

// Per-channel decay d = exp(-e^{-1/2} * sigmoid(w)), written in the reference's
// exp2 form (wkv_fp32_v2.cu:27-29) with an IEEE division.
__device__ __forceinline__ float decay(float w) {
  const float e = exp2_det(kDecayC2 * w);
  const float den = 1.0f + e;
  const float q = kDecayC1 / den;
  return exp2_det(q);
}

// Dither of the fp16-state family (wkv_fp16_v2.cu:23-25): a Knuth
// multiplicative hash of the phase, wrapped to int32, scaled by 2^-41.
__device__ __forceinline__ float rotator(uint32_t phase) {
  const uint32_t m = 2654435769u * phase;
  return kTwoNeg41 * (float)(int32_t)m;
}

// fp16 decay delta of the fp16-state family (wkv_fp16_v2.cu:27-30):
// fp16_rn((d - 1) + rot).
__device__ __forceinline__ _Float16 w_delta(float w, uint32_t phase) {
  float d = decay(w) - 1.0f;
  d = d + rotator(phase);
  return (_Float16)d;
}

__device__ __forceinline__ float h2f(uint16_t bits) {
  return (float)__builtin_bit_cast(_Float16, bits);
}

// The LDS address space, for the direct global->LDS (DMA) loads of gfx950.
#define VK_LDS __attribute__((address_space(3)))

// One 16-byte-per-lane global->LDS transfer: lane L's 16 bytes at `gsrc` land
// at `lds_base + 16*L`.  `lds_base` must be wave-uniform.
__device__ __forceinline__ void dma16(const void* gsrc, void* lds_base) {
  __builtin_amdgcn_global_load_lds(gsrc, (VK_LDS void*)lds_base, 16, 0, 0);
}
// The same with the non-temporal cache policy (nt): streamed data that will not be
// read again soon is not kept in the caches it passes.
__device__ __forceinline__ void dma16_nt(const void* gsrc, void* lds_base) {
  __builtin_amdgcn_global_load_lds(gsrc, (VK_LDS void*)lds_base, 16, 0, 2);
}

// ---------------------------------------------------------------- reductions

// Sum over the 64 lanes of a wave: xor butterfly, then lane 0's total is
// broadcast so every lane holds bit-identical values (each lane's butterfly
// associates differently).  Fixed order, so run-to-run deterministic.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

// fp16 of an fp32 value computed by a product: the value is first rounded to
// fp32, then to fp16 (as a float -> half conversion of the product does), not
// folded with the product into one mixed-precision FMA that rounds once.
__device__ __forceinline__ _Float16 f16_of(float x) {
  asm volatile("" : "+v"(x));
  return (_Float16)x;
}

// wave_sum(a * b) with the first butterfly stage fused: each lane adds its
// exact product to its xor-32 partner's rounded product, fma(a, b, partner).
// Written out because that is what the compiler makes of wave_sum(a * b)
// under fp contraction, and every kernel that reduces the same quantity (the
// per-head kk norm, GroupNorm variance, the r.k bonus) must agree bit for bit.
__device__ __forceinline__ float wave_sum_prod(float a, float b) {
  float v = __builtin_fmaf(a, b, __shfl_xor(a * b, 32, 64));
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

// Sum over a workgroup of NW waves (NW * 64 threads); `red` is NW floats of LDS.
// Wave totals are added in wave order.  Contains two barriers: every thread of
// the workgroup must call it.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) t += red[w];
  __syncthreads();
  return t;
}

// ---------------------------------------------------------------- vectors

// 8 fp16 values (16 bytes), the unit of the vectorised elementwise kernels.
struct alignas(16) h8 {
  _Float16 v[8];
};

__device__ __forceinline__ h8 ld8(const _Float16* p) { return *reinterpret_cast<const h8*>(p); }
__device__ __forceinline__ void st8(_Float16* p, const h8& x) { *reinterpret_cast<h8*>(p) = x; }

// bf16 bit pattern -> float (exact).
__device__ __forceinline__ float bf16f(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}

__device__ __forceinline__ float sigmoidf(float x) { return 1.0f / (1.0f + __expf(-x)); }

// ---------------------------------------------------------------- frag layout

// Half index of element (r, k) of a matrix stored in the fragment order of
// v_mfma_f32_32x32x16_f16 operands (row blocks of 32, K padded to kpad, a
// multiple of 16): the 64 lanes x 8 halfs of one (row block, 16-k step)
// operand are contiguous, lane = ((k / 8) % 2) * 32 + r % 32.  Eight
// consecutive k starting at a multiple of 8 are contiguous.
__device__ __forceinline__ int64_t frag_index(int64_t r, int64_t k, int64_t kpad) {
  return (((r >> 5) * (kpad >> 4) + (k >> 4)) * 64 + ((k >> 3) & 1) * 32 + (r & 31)) * 8 + (k & 7);
}

constexpr int kFragPad = 128;  // rows and K of frag matrices are padded to multiples of this

__host__ __device__ __forceinline__ int64_t frag_pad(int64_t x) {
  return (x + kFragPad - 1) / kFragPad * kFragPad;
}

}  // namespace vk
