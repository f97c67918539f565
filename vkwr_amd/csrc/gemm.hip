// fp16 GEMM on the gfx950 matrix cores: y[M,N] = act(x)[M,K] . W, fp32
// accumulation, fp16 output, with the RWKV-7 epilogues fused.
//
// One launch runs a batch of up to 8 independent problems (e.g. the r/k/v
// projections and the four low-rank adapter inputs of one layer), each cut
// into BM x BN output tiles and optionally into K splits; the flat workgroup
// index walks problem -> M tile -> N tile -> K split.
//
// Tile loop: 256 lanes (4 waves in a WM x WN grid), K advanced 32 at a time.
// Each stage moves an A tile (BM x 32) and a B tile (BN x 32, stored k-inner)
// global -> VGPRs -> LDS, double buffered: the next stage's global loads are
// issued before the current stage's MFMAs, and one barrier per stage separates
// the LDS writes from the reads.  A wave computes its (BM/WM) x (BN/WN) sub-tile
// as 32x32 blocks with v_mfma_f32_32x32x16_f16; lane l feeds A[l%32][8(l/32)..+7]
// and B[8(l/32)..+7][l%32] (16-byte LDS reads) and receives
// D[8(r/4) + 4(l/32) + r%4][l%32] in accumulator r.
//
// Weights come in either layout of the reference ops: [N,K] (nn.Linear,
// K contiguous: loaded like A) or [K,N] (N contiguous: 16-byte loads along N,
// transposed into the k-inner LDS tile).
//
// K splits: with too few tiles to fill the 256 CUs, each split writes fp32
// partial sums to a workspace; a second kernel adds the splits in index order
// (deterministic) and applies the epilogue.
//
// Roofline: HBM-bound at decode (M <= 128 rows: every weight byte is read
// once, 2 flops per weight element per row); MFMA-bound for large M.

#include <algorithm>
#include <mutex>
#include <numeric>
#include <type_traits>

#include "vk_capi.h"
#include "vk_common.cuh"

namespace vk {
namespace {

typedef _Float16 hv8 __attribute__((ext_vector_type(8)));
typedef float fv16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 32;          // K per stage
constexpr int kLdsK = kBK + 8;   // padded LDS row (halfs): 80-byte rows spread the banks
constexpr int kMaxProblems = 8;

struct Prob {
  const _Float16* a;
  const _Float16* b;
  _Float16* c;
  float* ws;  // split partials [splits][m][n] when splits > 1
  const _Float16 *v, *vf, *v0;  // value-residual epilogue operands
  int m, n, k;
  int b_kn;   // 1: B is [K,N]; 0: B is [N,K]
  int a_act;  // VKWR_GEMM_ACT_*
  int epi;    // VKWR_GEMM_EPI_*
  int vec;    // 16-byte accesses allowed (aligned rows, K and N multiples of 8)
  int vec_out;  // 16-byte epilogue: c (and v, v_first, v0, ws when used) aligned, N a multiple of 8
  int tiles_m, tiles_n, splits, k_per_split;
  int tile_begin;
};

struct Batch {
  int n;
  Prob p[kMaxProblems];
  // Large-M batches of unequal K (whole tiles, every problem's tile count a multiple of 8):
  // each XCD takes an equal share of every problem's tiles, longest K first (order[] holds
  // the problems in decreasing K).  0: the XCD-contiguous tile order.
  int xbal;
  int order[kMaxProblems];
};

// A-operand activations.  Each workgroup applies them to every A element it reads, so a
// batch re-evaluates them once per column tile; they use the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32) instead of the libm forms (tanhf is a few dozen instructions): the
// rank-out batch of a 128-row decode step took 13.1 us with tanhf and 8.6 us with no
// activation.  The result is rounded to fp16 before the product, so their relative error
// (about 2e-6: 1.9e-6 for tanh and 0.9e-6 for sigmoid in a float32 emulation against
// float64, plus an ulp or two of the hardware exp2 and reciprocal) only moves the fp16
// rounding of an activated operand now and then (5e-5 of them in that emulation).
//   tanh(x) = sign(x) (1 - 2 / (1 + e^{2|x|})), and x - x^3/3 + 2x^5/15 for |x| < 1/16 (where
//   the subtraction would cancel; the next term, 17x^7/315, is below 1e-8 relative there);
//   sigmoid(x) = 1 / (1 + e^{-x}).
__device__ __forceinline__ float tanh_act(float x) {
  const float ax = fabsf(x);
  if (ax < 0.0625f) {
    const float x2 = x * x;
    return x * __builtin_fmaf(x2, __builtin_fmaf(x2, 0.13333333333f, -0.33333333333f), 1.0f);
  }
  const float e = __builtin_amdgcn_exp2f(ax * 2.8853900817779268f);  // e^{2|x|}
  return __builtin_copysignf(__builtin_fmaf(-2.0f, __builtin_amdgcn_rcpf(1.0f + e), 1.0f), x);
}

__device__ __forceinline__ float sigmoid_act(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

__device__ __forceinline__ float act_in(float x, int act) {
  if (act == VKWR_GEMM_ACT_TANH) return tanh_act(x);
  if (act == VKWR_GEMM_ACT_SIGMOID) return sigmoid_act(x);
  if (act == VKWR_GEMM_ACT_RELU_SQUARE) {
    const float r = fmaxf(x, 0.0f);
    return r * r;
  }
  return x;
}

__device__ __forceinline__ float epilogue(const Prob& P, float acc, int row, int col) {
  if (P.epi == VKWR_GEMM_EPI_RELU_SQUARE) {
    const float r = fmaxf(acc, 0.0f);
    return r * r;
  }
  if (P.epi == VKWR_GEMM_EPI_VALUE_RESIDUAL) {
    const int64_t i = (int64_t)row * P.n + col;
    const float vv = (float)P.v[i];
    const float gate = sigmoidf((float)P.v0[col] + acc);
    return __builtin_fmaf((float)P.vf[i] - vv, gate, vv);
  }
  if (P.epi == VKWR_GEMM_EPI_BIAS) return acc + (float)P.v0[col];
  if (P.epi == VKWR_GEMM_EPI_TANH) return tanhf(acc);
  if (P.epi == VKWR_GEMM_EPI_SIGMOID) return sigmoidf(acc);
  return acc;
}

// Loads 8 consecutive fp16 values at p[0..7] that lie in a row whose valid
// range is [0, lim) relative to p; invalid elements read as 0 and `act` (the
// A-operand activation) is applied to valid elements only.
__device__ __forceinline__ hv8 load8(const _Float16* p, int lim, bool vec, int act) {
  hv8 r;
  if (vec && lim >= 8) {
    r = *reinterpret_cast<const hv8*>(p);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (!vec && e < lim) ? p[e] : (_Float16)0.0f;
  }
  if (act != VKWR_GEMM_ACT_NONE) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (e < lim) r[e] = (_Float16)act_in((float)r[e], act);
  }
  return r;
}

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(256) void gemm_kernel(Batch bt) {
  constexpr int TM = BM / WM / 32;  // 32x32 blocks per wave along M
  constexpr int TN = BN / WN / 32;
  constexpr int NA = BM * (kBK / 8);  // 16-byte chunks per stage
  constexpr int NB = BN * (kBK / 8);
  constexpr int CA = (NA + 255) / 256;  // per lane
  constexpr int CB = (NB + 255) / 256;
  static_assert(TM >= 1 && TN >= 1 && CA >= 1 && CB >= 1, "tile shape");
  // One LDS block: the A and B stages during the K loop, then the fp32 output
  // tile (half of it at a time) for the vector epilogue.
  __shared__ __attribute__((aligned(16))) _Float16 smem[2 * (BM + BN) * kLdsK];
  auto& As = *reinterpret_cast<_Float16(*)[2][BM * kLdsK]>(smem);
  auto& Bs = *reinterpret_cast<_Float16(*)[2][BN * kLdsK]>(smem + 2 * BM * kLdsK);
  static_assert(BM / WM * BN * 4 <= 2 * (BM + BN) * kLdsK * 2, "epilogue staging must fit the stage buffers");

  // ---- locate problem / tile / split (workgroup-uniform)
  const int t = blockIdx.x;
  int pi = 0;
#pragma unroll
  for (int i = 1; i < kMaxProblems; ++i)
    if (i < bt.n && t >= bt.p[i].tile_begin) pi = i;
  const Prob& P = bt.p[pi];
  int lt = t - P.tile_begin;
  const int split = lt % P.splits;
  lt /= P.splits;
  const int m0 = (lt / P.tiles_n) * BM;
  const int n0 = (lt % P.tiles_n) * BN;
  const int kb = split * P.k_per_split;
  const int ke = min(P.k, kb + P.k_per_split);
  const int nstage = (ke - kb + kBK - 1) / kBK;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const bool vec = P.vec != 0;

  hv8 ra[CA], rb[CB];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      const int c = tid + i * 256;
      const int row = c >> 2, kc = (c & 3) * 8;
      const int gr = m0 + row, gk = k0 + kc;
      const int lim = (c < NA && gr < P.m) ? ke - gk : 0;
      ra[i] = load8(P.a + (int64_t)gr * P.k + gk, lim, vec, P.a_act);
    }
    if (!P.b_kn) {
#pragma unroll
      for (int i = 0; i < CB; ++i) {
        const int c = tid + i * 256;
        const int row = c >> 2, kc = (c & 3) * 8;
        const int gn = n0 + row, gk = k0 + kc;
        const int lim = (c < NB && gn < P.n) ? ke - gk : 0;
        rb[i] = load8(P.b + (int64_t)gn * P.k + gk, lim, vec, VKWR_GEMM_ACT_NONE);
      }
    } else {
      constexpr int NC = BN / 8;  // 8-wide n chunks per k row
#pragma unroll
      for (int i = 0; i < CB; ++i) {
        const int c = tid + i * 256;
        const int kr = c / NC, nc = (c % NC) * 8;
        const int gk = k0 + kr, gn = n0 + nc;
        const int lim = (c < NB && gk < ke) ? P.n - gn : 0;
        rb[i] = load8(P.b + (int64_t)gk * P.n + gn, lim, vec, VKWR_GEMM_ACT_NONE);
      }
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      const int c = tid + i * 256;
      if (c < NA) *reinterpret_cast<hv8*>(&As[buf][(c >> 2) * kLdsK + (c & 3) * 8]) = ra[i];
    }
    if (!P.b_kn) {
#pragma unroll
      for (int i = 0; i < CB; ++i) {
        const int c = tid + i * 256;
        if (c < NB) *reinterpret_cast<hv8*>(&Bs[buf][(c >> 2) * kLdsK + (c & 3) * 8]) = rb[i];
      }
    } else {
      constexpr int NC = BN / 8;
#pragma unroll
      for (int i = 0; i < CB; ++i) {
        const int c = tid + i * 256;
        if (c >= NB) continue;
        const int kr = c / NC, nc = (c % NC) * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) Bs[buf][(nc + e) * kLdsK + kr] = rb[i][e];
      }
    }
  };

  fv16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int arow = wm * (BM / WM) + (lane & 31);
  const int bcol = wn * (BN / WN) + (lane & 31);
  const int koff = (lane >> 5) * 8;

  if (nstage > 0) {
    gload(kb);
    lstore(0);
    __syncthreads();
  }
  for (int s = 0; s < nstage; ++s) {
    const int buf = s & 1;
    if (s + 1 < nstage) gload(kb + (s + 1) * kBK);
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 16) {
      hv8 fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        fa[i] = *reinterpret_cast<const hv8*>(&As[buf][(arow + i * 32) * kLdsK + kk + koff]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        fb[j] = *reinterpret_cast<const hv8*>(&Bs[buf][(bcol + j * 32) * kLdsK + kk + koff]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (s + 1 < nstage) lstore(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue.  With 16-byte rows (P.vec_out) the accumulators go through LDS,
  // one half of the tile (the waves of one wm) at a time, and each thread
  // finishes 8 consecutive columns of a row with 16-byte loads and stores;
  // written straight from the MFMA layout, every store would be 2 bytes per
  // lane.  Same per-element arithmetic either way.
  if (P.vec_out) {
    constexpr int HR = BM / WM;  // rows per half
    float* const stage = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int half = 0; half < WM; ++half) {
      if (wm == half) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int rl = i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
              stage[rl * BN + wn * (BN / WN) + j * 32 + (lane & 31)] = acc[i][j][r];
            }
      }
      __syncthreads();
      for (int g = tid; g < HR * BN / 8; g += 256) {
        const int rl = g / (BN / 8), c8 = (g % (BN / 8)) * 8;
        const int row = m0 + half * HR + rl, col = n0 + c8;
        if (row >= P.m || col >= P.n) continue;
        const float* sp = stage + rl * BN + c8;
        const f4 lo = *reinterpret_cast<const f4*>(sp), hi = *reinterpret_cast<const f4*>(sp + 4);
        const float s8[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        const int64_t idx = (int64_t)row * P.n + col;
        if (P.splits > 1) {
          float* w = P.ws + (int64_t)split * P.m * P.n + idx;
          *reinterpret_cast<f4*>(w) = lo;
          *reinterpret_cast<f4*>(w + 4) = hi;
          continue;
        }
        hv8 o;
        if (P.epi == VKWR_GEMM_EPI_VALUE_RESIDUAL) {
          const hv8 vv = *reinterpret_cast<const hv8*>(P.v + idx), vf = *reinterpret_cast<const hv8*>(P.vf + idx),
                    v0 = *reinterpret_cast<const hv8*>(P.v0 + col);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float x = (float)vv[e];
            float y = __builtin_fmaf((float)vf[e] - x, sigmoidf((float)v0[e] + s8[e]), x);
            asm volatile("" : "+v"(y));
            o[e] = (_Float16)y;
          }
        } else if (P.epi == VKWR_GEMM_EPI_BIAS) {
          const hv8 v0 = *reinterpret_cast<const hv8*>(P.v0 + col);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            float y = s8[e] + (float)v0[e];
            asm volatile("" : "+v"(y));
            o[e] = (_Float16)y;
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            float y = epilogue(P, s8[e], row, col + e);
            asm volatile("" : "+v"(y));
            o[e] = (_Float16)y;
          }
        }
        *reinterpret_cast<hv8*>(P.c + idx) = o;
      }
      __syncthreads();
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + bcol + j * 32;
      if (col >= P.n) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * (BM / WM) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row >= P.m) continue;
        if (P.splits > 1) {
          P.ws[((int64_t)split * P.m + row) * P.n + col] = acc[i][j][r];
        } else {
          float y = epilogue(P, acc[i][j][r], row, col);
          asm volatile("" : "+v"(y));  // round in fp32, then to fp16 (no fused mixed-precision op)
          P.c[(int64_t)row * P.n + col] = (_Float16)y;
        }
      }
    }
  }
}

// Adds the K-split partials of every split problem and applies the epilogue.
// blockIdx.y = problem index.  A workgroup takes 64 consecutive outputs at a time; wave w
// adds the parts [w q, w q + q) (q = ceil(splits / 4)) in part order, with 8 loads in
// flight per step, and the 4 wave sums are added in wave order.  The order is fixed, so
// results are run-to-run identical, and a 64-part split costs two round trips to memory
// instead of 64.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(Batch bt) {
  __shared__ float wsum[4][64];
  const Prob& P = bt.p[blockIdx.y];
  {
    // every field in one round of kernel-argument loads, before the first branch (the
    // compiler otherwise issued them one dependent round at a time, five in all)
    const _Float16 *fv = P.v, *fvf = P.vf, *fv0 = P.v0;
    _Float16* fc = P.c;
    float* fws = P.ws;
    const int f0 = P.m, f1 = P.n, f2 = P.epi, f3 = P.splits;
    asm volatile("" ::"s"(fv), "s"(fvf), "s"(fv0), "s"(fc), "s"(fws), "s"(f0), "s"(f1), "s"(f2), "s"(f3));
  }
  if (P.splits <= 1) return;
  const int64_t mn = (int64_t)P.m * P.n;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int q = (P.splits + 3) / 4;
  const int z0 = min(P.splits, w * q), z1 = min(P.splits, z0 + q);
  for (int64_t i0 = (int64_t)blockIdx.x * 64; i0 < mn; i0 += (int64_t)gridDim.x * 64) {
    const int64_t i = min(i0 + lane, mn - 1);
    float s = 0.0f;
    for (int z = z0; z < z1; z += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = P.ws[(int64_t)min(z + u, z1 - 1) * mn + i];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (z + u < z1) s += v[u];
    }
    wsum[w][lane] = s;
    __syncthreads();
    if (w == 0 && i0 + lane < mn) {
      const float t = ((wsum[0][lane] + wsum[1][lane]) + wsum[2][lane]) + wsum[3][lane];
      const int row = (int)(i / P.n), col = (int)(i % P.n);
      float y = epilogue(P, t, row, col);
      asm volatile("" : "+v"(y));  // round in fp32, then to fp16 (no fused mixed-precision op)
      P.c[i] = (_Float16)y;
    }
    __syncthreads();
  }
}

// Workgroups of splitk_reduce_kernel: one per 64 outputs of the largest split problem,
// at most 1024 (they loop beyond).
int reduce_wgs(const Batch& bt) {
  int64_t mn = 0;
  for (int i = 0; i < bt.n; ++i)
    if (bt.p[i].splits > 1) mn = std::max(mn, (int64_t)bt.p[i].m * bt.p[i].n);
  return (int)std::min<int64_t>(1024, std::max<int64_t>(1, (mn + 63) / 64));
}

// ---- large-M path (prefill / mixed batches): 256x256 output tiles, matrix-core bound.
//
// Eligible batches: A without activation, B as [N,K], K a multiple of 64, 16-byte aligned
// operands, M >= 256 somewhere in the batch.  256 lanes = 4 waves in a 2x2 grid, each wave
// a 128x128 sub-tile of 4x4 v_mfma_f32_32x32x16_f16 blocks (256 fp32 accumulators).  K
// advances 64 per stage through two 64 KiB LDS buffers (A and B tiles of 256 rows x 64):
//   * the next stage's tiles are copied global -> LDS by the DMA form of the vector load
//     (global_load_lds_dwordx4: 16 bytes per lane straight into LDS, no VGPR staging),
//     16 instructions per wave and stage, issued one after every other MFMA of the two
//     k16 groups that follow the barrier freeing its buffer (a burst of them would stall
//     the wave's in-order issue of MFMAs), so two to four groups of MFMAs run before the
//     barrier that waits for them; the lanes of one load instruction cover
//     8 whole 128-byte rows, and row r's 16-byte chunk c lands at LDS slot
//     r*8 + (c ^ ((r >> 1) & 7)), so that the fragment reads below touch 16 distinct
//     16-byte bank groups per 16 lanes (conflict-free);
//   * fragments for the next k16 group are read (ds_read_b128) while the current group's
//     16 MFMAs run, one read after each of the first 8;
//   * one barrier per stage, after the third group: this wave's DMA has landed
//     (vmcnt(0)) and its reads of the current buffer are done (lgkmcnt(0)); after the
//     barrier both hold for every wave, so the next stage's buffer may be read and the
//     current one reloaded.
// The DMA is written as inline assembly: the compiler would otherwise make every LDS read
// wait for all outstanding DMA (it cannot tell the two buffers apart); the waits are placed
// here instead, as described.  Accumulation runs over k16 chunks in increasing order from
// zero, as in gemm_kernel without K splits, so an unsplit tile has the same bits in both.
//
// Work distribution: with G = #CUs, the first D = T - (T % G) of the T tiles run whole
// (gemm_big_kernel, XCD-aware order).  When the remaining R tiles would leave CUs idle
// and the split pays for its traffic, each of them is cut into S equal k-parts, one per
// workgroup of gemm_big_sk_kernel, which store fp32 partial tiles; gemm_big_fixup_kernel
// adds each tile's S partials in increasing k order (deterministic) and applies the
// epilogue.  Where R tiles divide unevenly over the CUs (the 7B FFN value GEMM: 144 tiles
// of 256 stages on 256 CUs) a layered split gives every CU the same number of stages
// instead (Layers below; 293 -> 275 us for that GEMM's split kernel, fixup 24 -> 29 us).
// A split that hands each CU one contiguous range of the tiles laid end to end balances
// the work as well, but its CUs then sit at unrelated k offsets and share no operand
// panels in the L2 (measured 349 us).  The split is chosen by a time model (plan_big).
//
// Workgroup b runs on XCD b % 8; logical tiles are handed out so that each XCD holds a
// contiguous range, walked in groups of 4 tile rows, which keeps the A row blocks and B
// column blocks an XCD needs at once few (its own L2).
// Tiles are BM x 256 (BM = 256, or 192 where 256-row tiles would leave many CUs idle: M =
// 2304 gives 9 rows of 256 but 12 of 192); the LDS buffers are sized for BM = 256.
constexpr int kBigBM = 256, kBigBK = 64, kBigTile = 256 * kBigBK;  // halves per operand tile
constexpr int kBigTileElems = kBigBM * kBigBM;                       // floats per partial tile (BM = 256)

struct BigPlan {
  int bm;        // tile rows: 256 or 192
  int dp_tiles;  // D: tiles computed whole
  int sk_tiles;  // R: tiles split into k-parts
  int parts;     // S: k-parts per split tile (equal split)
  int nst;       // k-stages per tile (all problems, when sk_tiles > 0)
  int wgs;       // W > 0: layered split over W workgroups (below); 0: equal split
  int per;       // layered split: k-stages per workgroup (R nst / W)
  int gran;      // layered split: k-stages per third-layer piece
  float* ws;     // partial tiles: [R][S] (equal split) or one per piece (layered split)
};

// Position of workgroup b among W when the blocks of each XCD (b % 8) take a contiguous
// range of positions (the order gemm_big_kernel hands out tiles in).
__device__ __forceinline__ int xcd_contiguous(int b, int W) {
  const int xb = b & 7, idx = b >> 3, q8 = W >> 3, r8 = W & 7;
  return (xb < r8 ? xb * (q8 + 1) : r8 * (q8 + 1) + (xb - r8) * q8) + idx;
}

// Layered split of R tiles of nst k-stages over W workgroups (R <= W < 2R), each doing
// per = R nst / W stages (per >= nst / 2), so that every CU gets the same work although the
// tiles do not divide evenly over the CUs.  Every piece of one layer covers the same k range,
// so workgroups that share A or B panels stream them through the L2 together:
//   layer 1: workgroup t < R takes stages [0, per) of tile t;
//   layer 2: workgroup R + j (j < W' = W - R) takes [per, nst) of tile j (L = nst - per stages);
//   layer 3: the other R'' = R - W' tiles' [per, nst) ranges, cut into L / g pieces of
//            g = gran stages, in k-major order (piece q: k class q / R'', tile W' + q % R''),
//            b / g consecutive pieces to each layer-2 workgroup (b = per - L).
// Partial slot of a piece: layer 1 t, layer 2 R + j, layer 3 R + W' + q.
struct Layers {
  int R, W2, L, R3, npc, bpw;  // R, W', L, R'', pieces per tile, pieces per workgroup (layer 3)
};
__device__ __host__ inline Layers layers_of(const BigPlan& pl) {
  Layers y;
  y.R = pl.sk_tiles;
  y.W2 = pl.wgs - pl.sk_tiles;
  y.L = pl.nst - pl.per;
  y.R3 = y.R - y.W2;
  y.npc = y.L / pl.gran;
  y.bpw = (pl.per - y.L) / pl.gran;
  return y;
}

__device__ __forceinline__ int big_slot(int row, int c) { return row * 8 + (c ^ ((row >> 1) & 7)); }

// A wave-uniform pointer in scalar registers (the compiler cannot always prove uniformity).
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// 16 bytes per lane: global (base + voff) -> LDS (lds + 16 * lane); base and lds wave-uniform
__device__ __forceinline__ void dma16_m0(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(base)
               : "memory", "m0");
}

// Logical tile L of the batch -> its problem index and tile origin (groups of 4 tile rows,
// column-major inside a group).
template <int BM>
__device__ __forceinline__ int big_tile(const Batch& bt, int L, int& m0, int& n0) {
  int pi = 0;
#pragma unroll
  for (int i = 1; i < kMaxProblems; ++i)
    if (i < bt.n && L >= bt.p[i].tile_begin) pi = i;
  const Prob& P = bt.p[pi];
  const int lt = L - P.tile_begin;
  constexpr int kGroup = 4;
  const int per = kGroup * P.tiles_n, grp = lt / per, in = lt - grp * per;
  const int g0 = grp * kGroup, gs = min(kGroup, P.tiles_m - g0);
  m0 = (g0 + in % gs) * BM;
  n0 = (in / gs) * kBigBM;
  return pi;
}

template <int kEpi>
__device__ __forceinline__ float big_epilogue(const Prob& P, float y, int row, int col) {
  if constexpr (kEpi == VKWR_GEMM_EPI_RELU_SQUARE) {
    y = fmaxf(y, 0.0f);
    return y * y;
  } else if constexpr (kEpi == VKWR_GEMM_EPI_BIAS) {
    return y + (float)P.v0[col];
  } else if constexpr (kEpi == VKWR_GEMM_EPI_NONE) {
    return y;
  } else if constexpr (kEpi == VKWR_GEMM_EPI_TANH) {
    return tanhf(y);
  } else if constexpr (kEpi == VKWR_GEMM_EPI_SIGMOID) {
    return sigmoidf(y);
  } else if constexpr (kEpi == VKWR_GEMM_EPI_VALUE_RESIDUAL) {
    const int64_t i = (int64_t)row * P.n + col;
    const float vv = (float)P.v[i];
    const float gate = sigmoidf((float)P.v0[col] + y);
    return __builtin_fmaf((float)P.vf[i] - vv, gate, vv);
  } else {
    return epilogue(P, y, row, col);
  }
}

// Stores a BM x 256 accumulator tile through epilogue kEpi (fp16, clipped to M x N) via LDS
// (P.vec_out: 16-byte aligned rows, N a multiple of 8).  Wave w walks its (BM / 2) x 128 part
// in BM / 32 strips of 32 x 64 (two horizontally adjacent 32 x 32 accumulator blocks): strip p's
// fp32 sums go to one of two LDS buffers of the wave (32 rows of kBigStRow floats each)
// while strip p - 1 is read back from the other, lane l taking 8 columns (8 (l % 8) .. + 7)
// of rows l / 8 + 8 h, h = 0..3, so that each 16-byte store instruction writes 8 whole
// 128-byte lines; epilogue operands are read the same way.  Written straight from the MFMA
// layout every store would be 2 bytes per lane, and that form kept the accumulator tile in
// scratch memory for the value-residual and mixed-epilogue instances.  Per-column operands
// (bias / v0) are loaded once; the value residual's v and v_first rows one strip ahead.
constexpr int kBigStRow = 68;               // 64 columns + 4 floats of padding
constexpr int kBigStBuf = 32 * kBigStRow;   // floats per strip buffer
template <int BM, int kEpi>
__device__ __forceinline__ void big_store_lds(float* st, const Prob& P, const fv16 (&acc)[BM / 64][4], int m0,
                                              int n0, int wm, int wn, int lane) {
  constexpr int kStrips = 2 * (BM / 64);  // 32 x 64 strips of the wave's (BM / 2) x 128 part
  const int lr = lane & 31, lh = lane >> 5, r8 = lane >> 3, c8 = 8 * (lane & 7);
  // The problem's fields, held in SGPRs for the whole store loop (an asm output cannot be
  // re-derived): left alone the compiler re-reads them from the kernel arguments before each
  // store, and the wait for each such scalar load also waits for every LDS read in flight,
  // which serialised the strips (the epilogue of a 256 x 256 tile took ~11 us).
  // (Global address-space pointers, so the accesses stay global, not flat, ones: a flat
  // access would count against the LDS counter too.)
  typedef _Float16 __attribute__((address_space(1)))* gptr;
  typedef const _Float16 __attribute__((address_space(1)))* gcptr;
  int pm = P.m, pn = P.n;
  gptr pcp = (gptr)P.c;
  gcptr pvp = (gcptr)P.v, pvfp = (gcptr)P.vf, pv0p = (gcptr)P.v0;
  asm("" : "+s"(pm), "+s"(pn), "+s"(pcp), "+s"(pvp), "+s"(pvfp), "+s"(pv0p));
  constexpr bool kVres = kEpi == VKWR_GEMM_EPI_VALUE_RESIDUAL;
  constexpr bool kCol = kVres || kEpi == VKWR_GEMM_EPI_BIAS;  // a per-column operand v0
  const int rowb = m0 + wm * (BM / 2) + r8, colb = n0 + wn * 128 + c8;
  hv8 ov0[2];
  if constexpr (kCol) {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) ov0[jj] = *reinterpret_cast<const __attribute__((address_space(1))) hv8*>(pv0p + min(colb + jj * 64, pn - 8));
  }
  hv8 ov[2][4], ovf[2][4];
  auto load_ops = [&](int p) __attribute__((always_inline)) {
    const int col = colb + (p & 1) * 64;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int row = rowb + (p >> 1) * 32 + 8 * h;
      const bool in = row < pm && col < pn;
      const int64_t idx = in ? (int64_t)row * pn + col : 0;
      ov[p & 1][h] = *reinterpret_cast<const __attribute__((address_space(1))) hv8*>(pvp + idx);
      ovf[p & 1][h] = *reinterpret_cast<const __attribute__((address_space(1))) hv8*>(pvfp + idx);
    }
  };
  auto write_strip = [&](int p) __attribute__((always_inline)) {
    float* sb = st + (p & 1) * kBigStBuf;
    const int i = p >> 1, jj = p & 1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int rl = 8 * (r >> 2) + 4 * lh + (r & 3);
      sb[rl * kBigStRow + lr] = acc[i][2 * jj][r];
      sb[rl * kBigStRow + 32 + lr] = acc[i][2 * jj + 1][r];
    }
  };
  auto finish_strip = [&](int p) __attribute__((always_inline)) {
    const float* sb = st + (p & 1) * kBigStBuf + r8 * kBigStRow + c8;
    f4 v[4][2];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      v[h][0] = *reinterpret_cast<const f4*>(sb + 8 * h * kBigStRow);
      v[h][1] = *reinterpret_cast<const f4*>(sb + 8 * h * kBigStRow + 4);
    }
    const int col = colb + (p & 1) * 64;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int row = rowb + (p >> 1) * 32 + 8 * h;
      const float s8[8] = {v[h][0].x, v[h][0].y, v[h][0].z, v[h][0].w, v[h][1].x, v[h][1].y, v[h][1].z, v[h][1].w};
      hv8 o;
      if constexpr (kVres) {
        const hv8 vv = ov[p & 1][h], vf = ovf[p & 1][h], v0 = ov0[p & 1];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = (float)vv[e];
          float y = __builtin_fmaf((float)vf[e] - x, sigmoidf((float)v0[e] + s8[e]), x);
          asm volatile("" : "+v"(y));
          o[e] = (_Float16)y;
        }
      } else if constexpr (kEpi == VKWR_GEMM_EPI_BIAS) {
        const hv8 v0 = ov0[p & 1];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float y = s8[e] + (float)v0[e];
          asm volatile("" : "+v"(y));
          o[e] = (_Float16)y;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float y = big_epilogue<kEpi>(P, s8[e], row, col + e);
          asm volatile("" : "+v"(y));
          o[e] = (_Float16)y;
        }
      }
      if (row < pm && col < pn) *reinterpret_cast<__attribute__((address_space(1))) hv8*>(pcp + (int64_t)row * pn + col) = o;
    }
  };
  if constexpr (kVres) load_ops(0);
  write_strip(0);
#pragma unroll
  for (int p = 1; p < kStrips; ++p) {
    if constexpr (kVres) load_ops(p);
    write_strip(p);
    finish_strip(p - 1);
  }
  finish_strip(kStrips - 1);
}

// One BM x 256 tile over k-stages [ks, ke): kPartial stores the fp32 sums to part in
// register order -- element ((4 i + j) * 16 + r) * 256 + thread is accumulator r of block
// (i, j) of that thread, so each store is one coalesced kilobyte -- otherwise the
// epilogue's fp16 values (clipped to M x N) to P.c.
template <int BM, bool kPartial, int kEpi>
__device__ __forceinline__ void big_tile_run(_Float16 (&sm)[2][2][kBigTile], const Prob& P, int m0, int n0,
                                             int ks, int ke, float* part) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w >> 1, wn = w & 1;
  const int lr = lane & 31, lh = lane >> 5;
  const int M = P.m, N = P.n, K = P.k;
  constexpr int RB = BM / 64;          // 32-row accumulator blocks per wave
  constexpr int NA = BM / 32, ND = NA + 8;  // DMA instructions per stage: A, A + B
  // DMA instruction j (0..7) of wave w fills slots j*256 + w*64 + lane of a tile
  uint32_t ao[NA], bo[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int sl = j * 256 + w * 64 + lane, row = sl >> 3, c = (sl & 7) ^ ((row >> 1) & 7);
    if (j < NA) ao[j] = (uint32_t)((min(m0 + row, M - 1) * (int64_t)K + c * 8) * 2);
    bo[j] = (uint32_t)((min(n0 + row, N - 1) * (int64_t)K + c * 8) * 2);
  }
  const uint32_t wl = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)&sm[0][0][0] + w * 64 * 16);
  int fra[4][RB], frb[4][4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      if (rb < RB) fra[kk][rb] = big_slot(wm * (BM / 2) + 32 * rb + lr, 2 * kk + lh) * 8;
      frb[kk][rb] = big_slot(wn * 128 + 32 * rb + lr, 2 * kk + lh) * 8;
    }
  fv16 acc[RB][4];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // read once: the DMA statements clobber memory, so P.a / P.b would be reloaded after each
  const _Float16* const pa = (const _Float16*)uniform_ptr(P.a);
  const _Float16* const pb = (const _Float16*)uniform_ptr(P.b);
  // DMA instruction d (0..ND-1) of a stage: A and B rows of instruction d / 2 alternating
  // while both have some (even d: A), then the remaining B ones
  auto dma_one = [&](int d, const void* ab, const void* bb, uint32_t la) __attribute__((always_inline)) {
    if (d >= 2 * NA) dma16_m0(bb, bo[d - NA], la + kBigTile * 2 + (d - NA) * 256 * 16);
    else if (d & 1) dma16_m0(bb, bo[d >> 1], la + kBigTile * 2 + (d >> 1) * 256 * 16);
    else dma16_m0(ab, ao[d >> 1], la + (d >> 1) * 256 * 16);
  };
  auto stage_src = [&](int st, const void*& ab, const void*& bb) __attribute__((always_inline)) {
    const int k0 = min(st, ke - 1) * kBigBK;  // past the range: re-load its last stage (unused)
    ab = uniform_ptr(pa + k0);
    bb = uniform_ptr(pb + k0);
  };
  auto dma = [&](int buf, int st, int d0, int d1) __attribute__((always_inline)) {
    const void *ab, *bb;
    stage_src(st, ab, bb);
    const uint32_t la = wl + (uint32_t)(buf * 2 * kBigTile * 2);
#pragma unroll
    for (int d = 0; d < ND; ++d)
      if (d >= d0 && d < d1) dma_one(d, ab, bb, la);
  };
  hv8 fa[2][RB], fb[2][4];
  auto fread = [&](int buf, int kk, int set) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i < RB) fa[set][i] = *reinterpret_cast<const hv8*>(&sm[buf][0][fra[kk][i]]);
      fb[set][i] = *reinterpret_cast<const hv8*>(&sm[buf][1][frb[kk][i]]);
    }
  };
  // 4 RB MFMAs with the next group's RB + 4 fragment reads interleaved, one after each of the
  // first RB + 4
  auto mfma16 = [&](int set) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[set][i], fb[set][j], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int q = 0; q < RB + 4; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 3 * RB - 4, 0);
  };
  // 4 RB MFMAs with DMA instructions d0 .. d0 + ND / 2 - 1 of stage st (buffer buf) after
  // every other one (any left over after the last): a burst of DMA issues would hold up the
  // wave's in-order issue of the MFMAs
  auto mfma16_dma = [&](int set, int buf, int st, int d0) __attribute__((always_inline)) {
    const void *ab, *bb;
    stage_src(st, ab, bb);
    const uint32_t la = wl + (uint32_t)(buf * 2 * kBigTile * 2);
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[set][i], fb[set][j], acc[i][j], 0, 0, 0);
        const int q = 2 * i + (j >> 1);  // the q-th DMA of this half
        if ((j & 1) == 0 && q < ND / 2) dma_one(d0 + q, ab, bb, la);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
    for (int q = 2 * RB; q < ND / 2; ++q) dma_one(d0 + q, ab, bb, la);
    __builtin_amdgcn_sched_barrier(0);
  };
  dma(0, ks, 0, ND);
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  dma(1, ks + 1, 0, ND / 2);
  fread(0, 0, 0);
  int cb = 0;
  for (int s = ks; s < ke; ++s) {
    const int nb = cb ^ 1;
    fread(cb, 1, 1);
    mfma16_dma(0, nb, s + 1, ND / 2);  // the second half of stage s + 1
    __builtin_amdgcn_sched_barrier(0);
    fread(cb, 2, 0);
    mfma16(1);
    __builtin_amdgcn_sched_barrier(0);
    fread(cb, 3, 1);
    mfma16(0);
    __builtin_amdgcn_sched_barrier(0);
    // stage s + 1 (buffer nb) has landed and buffer cb is read
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    fread(nb, 0, 0);
    mfma16_dma(1, cb, s + 2, 0);  // the first half of stage s + 2, into the buffer just freed
    __builtin_amdgcn_sched_barrier(0);
    cb = nb;
  }
  // every wave's DMA (the last stage's re-load) has landed and its LDS reads are done: the
  // epilogue may reuse the buffers
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  float* const st = reinterpret_cast<float*>(&sm[0][0][0]) + w * 2 * kBigStBuf;

  if constexpr (kPartial) {
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) part[((4 * i + j) * 16 + r) * 256 + tid] = acc[i][j][r];
  } else if constexpr (kEpi >= 0) {
    big_store_lds<BM, kEpi>(st, P, acc, m0, n0, wm, wn, lane);
  } else {
    // a batch of mixed epilogues: one branch per tile to a specialized store loop
    // (a per-element switch would not keep the accumulator tile in registers)
    switch (P.epi) {
      case VKWR_GEMM_EPI_RELU_SQUARE: big_store_lds<BM, VKWR_GEMM_EPI_RELU_SQUARE>(st, P, acc, m0, n0, wm, wn, lane); break;
      case VKWR_GEMM_EPI_VALUE_RESIDUAL:
        big_store_lds<BM, VKWR_GEMM_EPI_VALUE_RESIDUAL>(st, P, acc, m0, n0, wm, wn, lane);
        break;
      case VKWR_GEMM_EPI_BIAS: big_store_lds<BM, VKWR_GEMM_EPI_BIAS>(st, P, acc, m0, n0, wm, wn, lane); break;
      case VKWR_GEMM_EPI_TANH: big_store_lds<BM, VKWR_GEMM_EPI_TANH>(st, P, acc, m0, n0, wm, wn, lane); break;
      case VKWR_GEMM_EPI_SIGMOID: big_store_lds<BM, VKWR_GEMM_EPI_SIGMOID>(st, P, acc, m0, n0, wm, wn, lane); break;
      default: big_store_lds<BM, VKWR_GEMM_EPI_NONE>(st, P, acc, m0, n0, wm, wn, lane); break;
    }
  }
}

// Unequal-K batch (bt.xbal): XCD x (workgroup b runs on XCD b % 8) takes tiles x T_p / 8 ..
// (x + 1) T_p / 8 - 1 of every problem p, the longest-K problem's first.  In the
// XCD-contiguous order each XCD would hold one problem's tiles, and the XCDs holding the
// long-K tiles (the 7B rank-out batch: K = 512 for g2, 128 for the others) would run for
// several times as long as the rest.
__device__ __forceinline__ int big_balanced_tile(const Batch& bt, int b) {
  const int x = b & 7;
  int idx = b >> 3;
  for (int q = 0; q < bt.n; ++q) {
    const Prob& P = bt.p[bt.order[q]];
    const int share = P.tiles_m * P.tiles_n / 8;
    if (idx < share) return P.tile_begin + x * share + idx;
    idx -= share;
  }
  return 0;  // not reached: the grid has one workgroup per tile
}

// Whole tiles: workgroup b takes logical tile (XCD-contiguous order) of the first `tiles`.
// kEpi >= 0: every problem of the batch has that epilogue; -1: each its own.
template <int BM, int kEpi>
__global__ __launch_bounds__(256, 1) void gemm_big_kernel(Batch bt, int tiles) {
  __shared__ __attribute__((aligned(1024))) _Float16 sm[2][2][kBigTile];  // [buffer][A/B]: 128 KiB
  const int L = bt.xbal ? big_balanced_tile(bt, blockIdx.x) : xcd_contiguous(blockIdx.x, tiles);
  int m0, n0;
  const Prob& P = bt.p[big_tile<BM>(bt, L, m0, n0)];
  big_tile_run<BM, false, kEpi>(sm, P, m0, n0, 0, P.k / kBigBK, nullptr);
}

// Split tiles.  Equal split: workgroup b computes part b % S (k-stages [p nst / S, (p+1) nst / S))
// of split tile D + b / S into partial slot b.  Balanced split: the workgroup at position lw
// (XCD-contiguous) computes its stage range, one piece per tile it touches, the piece of tile
// t into slot lw pmax + (t - its first tile); so every CU gets the same number of stages
// even when the split tiles do not divide evenly over the CUs.
template <int BM>
__global__ __launch_bounds__(256, 1) void gemm_big_sk_kernel(Batch bt, BigPlan pl) {
  __shared__ __attribute__((aligned(1024))) _Float16 sm[2][2][kBigTile];
  if (pl.wgs > 0) {
    const Layers y = layers_of(pl);
    const size_t tile = (size_t)BM * kBigBM;
    auto piece = [&](int t, int ks, int ke, int slot) __attribute__((always_inline)) {
      int m0, n0;
      const Prob& P = bt.p[big_tile<BM>(bt, pl.dp_tiles + t, m0, n0)];
      big_tile_run<BM, true, -1>(sm, P, m0, n0, ks, ke, pl.ws + (size_t)slot * tile);
    };
    if ((int)blockIdx.x < y.R) {
      const int t = xcd_contiguous(blockIdx.x, y.R);
      piece(t, 0, pl.per, t);
      return;
    }
    const int j = xcd_contiguous(blockIdx.x - y.R, y.W2);
    piece(j, pl.per, pl.nst, y.R + j);
    for (int q = j * y.bpw; q < (j + 1) * y.bpw; ++q) {
      const int ks = pl.per + (q / y.R3) * pl.gran;
      piece(y.W2 + q % y.R3, ks, ks + pl.gran, y.R + y.W2 + q);
    }
    return;
  }
  const int t = blockIdx.x / pl.parts, p = blockIdx.x - t * pl.parts;
  int m0, n0;
  const Prob& P = bt.p[big_tile<BM>(bt, pl.dp_tiles + t, m0, n0)];
  big_tile_run<BM, true, -1>(sm, P, m0, n0, p * pl.nst / pl.parts, (p + 1) * pl.nst / pl.parts,
                             pl.ws + (size_t)blockIdx.x * (BM * kBigBM));
}

// Fixup: blockIdx.y = split tile t, blockIdx.x = accumulator block (i, j) of the partial
// layout; adds the tile's partials in increasing k order (equal split: its S parts; layered
// split: its layer-1 piece, then its layer-2 piece or its layer-3 pieces in k order), applies
// the epilogue, stores.
template <int BM, int kEpi>
__global__ __launch_bounds__(256) void gemm_big_fixup_kernel(Batch bt, BigPlan pl) {
  const int t = blockIdx.y, blk = blockIdx.x, tid = threadIdx.x;
  int m0, n0;
  const Prob& P = bt.p[big_tile<BM>(bt, pl.dp_tiles + t, m0, n0)];
  const int lane = tid & 63, w = tid >> 6, wm = w >> 1, wn = w & 1, lr = lane & 31, lh = lane >> 5;
  const int i = blk >> 2, j = blk & 3;
  const int col = n0 + wn * 128 + j * 32 + lr;
  if (col >= P.n) return;
  // The 16 values of a part are loaded together (the workspace holds whole
  // tiles, so rows past M are in bounds), then the parts are added in order.
  const size_t in_tile = (size_t)blk * 16 * 256 + tid;
  float acc[16];
  if (pl.wgs > 0) {
    const Layers y = layers_of(pl);
    auto slot = [&](int q) { return pl.ws + (size_t)q * (BM * kBigBM) + in_tile; };
    auto add = [&](const float* bq) __attribute__((always_inline)) {
      float nx[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) nx[r] = bq[r * 256];
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] += nx[r];
    };
    const float* b0 = slot(t);
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = b0[r * 256];
    if (t < y.W2) {
      add(slot(y.R + t));
    } else {
      for (int i = 0; i < y.npc; ++i) add(slot(y.R + y.W2 + i * y.R3 + (t - y.W2)));
    }
  } else {
    const float* base = pl.ws + (size_t)t * pl.parts * (BM * kBigBM) + in_tile;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = base[r * 256];
    for (int q = 1; q < pl.parts; ++q) {
      const float* bq = base + (size_t)q * (BM * kBigBM);
      float nx[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) nx[r] = bq[r * 256];
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] += nx[r];
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = m0 + wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
    if (row >= P.m) continue;
    float y = big_epilogue<kEpi>(P, acc[r], row, col);
    asm volatile("" : "+v"(y));
    P.c[(int64_t)row * P.n + col] = (_Float16)y;
  }
}

// ---- small-M path (decode-sized batches, M <= 128): row-major operands staged through LDS.
//
// At M <= 128 every weight byte is used M times, so the launch streams the weights
// once and is bound by how many bytes each CU keeps in flight.  A workgroup owns a
// (32 TM) x (32 TN) output tile over the whole of K -- or, when the tiles alone leave CUs
// idle (the low-rank input projections, [K,N] weights with long K), over one of `splits`
// K parts, writing fp32 partials that splitk_reduce_kernel adds in part order; its 4
// waves take the 64-deep k blocks w, w + 4, ... (an in-workgroup K split), and each wave
// stages its blocks through two private LDS buffers with the DMA form of the vector
// load (global_load_lds_dwordx4, no VGPR staging): one instruction moves 8 whole
// 128-byte rows (64 k of a row is one cache line), chunk c of row r landing at slot
// r*8 + (c ^ ((r >> 1) & 7)) so that the fragment reads (ds_read_b128, 8 consecutive k
// of one row per lane) are conflict-free.  A [K,N] weight is staged as k-rows of 64
// columns and its fragments read with the transposing LDS read (two per fragment).  The wave
// issues the next block's DMA before computing on the current one; the waits are
// explicit, the DMA being invisible to the compiler.  After the loop the 4 wave
// partials are added in wave order through LDS and each thread finishes 8 consecutive
// columns with the generic epilogue (the A activation is applied to each fragment
// after it is read, rounded to fp16, as gemm_kernel applies it while staging).
// Rows past M and columns past N are read clamped to the last valid row / column and
// discarded; k chunks past K (K % 8 == 0) are zeroed in the A fragment.
constexpr int kRmBK = 64;

// Waves per workgroup: 8 for the 32 x 32 tile (its LDS stages are half the size, so twice
// the waves keep the same bytes in flight), 4 otherwise.
template <int TM, int TN>
constexpr int rm_waves() { return TM * TN == 1 ? 8 : 4; }

// kAct: some problem of the batch has an A-operand activation.  Without one the fragment
// reads of a whole k block have no branch between them and the matrix products, so they are
// all issued before the first product (with the activation's per-element branches in the
// loop, each product waited for its own two reads).
// kMulti: the batch holds more than one problem (the workgroup first finds its own).
template <int TM, int TN, bool kKN, bool kAct, bool kMulti>
__global__ __launch_bounds__((64 * rm_waves<TM, TN>())) void gemm_rm_kernel(Batch bt) {
  constexpr int kRmNW = rm_waves<TM, TN>();
  static_assert(!kKN || TN == 2, "[K,N] weights are staged as 128-byte k rows of 64 columns");
  constexpr int kA = 32 * TM * kRmBK, kB = 32 * TN * kRmBK, kStage = kA + kB;  // halves
  constexpr int kTiles = TM * TN;
  constexpr int kBDma = kKN ? 8 : 4 * TN;           // DMA instructions per B block
  constexpr int kDmaPerStage = 4 * TM + kBDma;
  __shared__ __attribute__((aligned(1024))) _Float16 sm[kRmNW][2][kStage];
  const int t = blockIdx.x;
  int pi = 0;
  if constexpr (kMulti) {
#pragma unroll
    for (int i = 1; i < kMaxProblems; ++i)
      if (i < bt.n && t >= bt.p[i].tile_begin) pi = i;
  }
  const Prob& P = bt.p[pi];
  {
    // Every field of the problem is requested here, in one round of kernel-argument loads
    // (the empty asm pins them above the first branch): left alone the compiler issued them
    // in two dependent rounds after finding the problem, each ~0.3 us before the first
    // operand load.  A one-problem launch (every op-surface linear call) has no search.
    const _Float16 *fa = P.a, *fb = P.b, *fv = P.v, *fvf = P.vf, *fv0 = P.v0;
    _Float16* fc = P.c;
    float* fws = P.ws;
    const int f0 = P.m, f1 = P.n, f2 = P.k, f3 = P.a_act, f4_ = P.epi, f5 = P.vec_out, f6 = P.tiles_m,
              f7 = P.tiles_n, f8 = P.splits, f9 = P.k_per_split, f10 = P.tile_begin;
    asm volatile("" ::"s"(fa), "s"(fb), "s"(fv), "s"(fvf), "s"(fv0), "s"(fc), "s"(fws), "s"(f0), "s"(f1), "s"(f2),
                 "s"(f3), "s"(f4_), "s"(f5), "s"(f6), "s"(f7), "s"(f8), "s"(f9), "s"(f10));
  }
  const int ntiles = P.tiles_m * P.tiles_n;
  const int lt0 = t - P.tile_begin;
  const int split = lt0 / ntiles;  // K part (split-major: the parts of a tile run apart in time)
  const int lt = lt0 - split * ntiles;
  const int m0 = (lt / P.tiles_n) * (32 * TM), n0 = (lt % P.tiles_n) * (32 * TN);
  const int M = P.m, N = P.n, K = P.k, a_act = kAct ? P.a_act : VKWR_GEMM_ACT_NONE;
  // this workgroup's K range [kbeg, kbeg + klen); klen is a multiple of 8
  const int kbeg = split * P.k_per_split;
  const int klen = min(K - kbeg, P.k_per_split);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nkb = (klen + kRmBK - 1) / kRmBK;
  const int nb = nkb > w ? (nkb - w + kRmNW - 1) / kRmNW : 0;  // this wave's k blocks

  // DMA instruction j of a stage fills slots 64 j + lane: row (64 j + lane) >> 3, chunk
  // (slot & 7) ^ swizzle -- byte offsets for k block 0 (32-bit: the host checks that every
  // operand is below 4 GiB).
  uint32_t ao[TM * 4], bo[kBDma];
#pragma unroll
  for (int j = 0; j < TM * 4; ++j) {
    const int sl = 64 * j + lane, r = sl >> 3, c = (sl & 7) ^ ((r >> 1) & 7);
    ao[j] = (uint32_t)(((int64_t)min(m0 + r, M - 1) * K + kbeg + c * 8) * 2);
  }
#pragma unroll
  for (int j = 0; j < kBDma; ++j) {
    const int sl = 64 * j + lane, r = sl >> 3, c = (sl & 7) ^ ((r >> 1) & 7);
    if constexpr (kKN) bo[j] = (uint32_t)(min(n0 + c * 8, N - 8) * 2);  // the k row is added per block
    else bo[j] = (uint32_t)(((int64_t)min(n0 + r, N - 1) * K + kbeg + c * 8) * 2);
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)&sm[w][0][0]);
  const void* const abase = uniform_ptr(P.a);
  const void* const bbase = uniform_ptr(P.b);
  auto dma = [&](int buf, int kb) __attribute__((always_inline)) {
    const uint32_t la = lds0 + (uint32_t)(buf * kStage * 2), lb = la + kA * 2;
    // k past the part's end: the chunk offset is clamped to the part's last chunk (read,
    // then zeroed)
    const int k0 = kb * kRmBK;
#pragma unroll
    for (int j = 0; j < TM * 4; ++j) {
      const int c = ((64 * j + lane) & 7) ^ ((((64 * j + lane) >> 3) >> 1) & 7);
      const int kk = min(k0 + c * 8, klen - 8) - c * 8;
      dma16_m0(abase, ao[j] + (uint32_t)(kk * 2), la + j * 1024);
    }
#pragma unroll
    for (int j = 0; j < kBDma; ++j) {
      if constexpr (kKN) {
        const int r = (64 * j + lane) >> 3;
        dma16_m0(bbase, bo[j] + (uint32_t)((int64_t)(kbeg + min(k0 + r, klen - 1)) * N * 2), lb + j * 1024);
      } else {
        const int c = ((64 * j + lane) & 7) ^ ((((64 * j + lane) >> 3) >> 1) & 7);
        const int kk = min(k0 + c * 8, klen - 8) - c * 8;
        dma16_m0(bbase, bo[j] + (uint32_t)(kk * 2), lb + j * 1024);
      }
    }
  };

  fv16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int lr = lane & 31, lh = lane >> 5;
  auto compute = [&](int buf, int kb) __attribute__((always_inline)) {
    const _Float16* sa = &sm[w][buf][0];
    const _Float16* sb = sa + kA;
    hv8 fa4[4][TM], fb4[4][TN];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int ch = 2 * kk + lh;
      const bool kin = kb * kRmBK + ch * 8 < klen;
      hv8 (&fa)[TM] = fa4[kk];
      hv8 (&fb)[TN] = fb4[kk];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = 32 * i + lr;
        fa[i] = *reinterpret_cast<const hv8*>(sa + (r * 8 + (ch ^ ((r >> 1) & 7))) * 8);
        if (kAct && a_act != VKWR_GEMM_ACT_NONE) {
#pragma unroll
          for (int e = 0; e < 8; ++e) fa[i][e] = (_Float16)act_in((float)fa[i][e], a_act);
        }
        if (!kin) fa[i] = hv8{};
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if constexpr (kKN) {
          // gfx950's transposing LDS read (ds_read_b64_tr_b16): within each 16-lane group,
          // element t of lane j's result is element j % 4 of the 8 bytes that lane 4t + j/4
          // of the group read.  Each lane reads 4 consecutive columns of one k row (lane s of
          // group g: k row k0 + s/4, columns n0 + 4 (s % 4) ..), so lane j receives 4
          // consecutive k of column n0 + j; two reads give the 8 k of an MFMA operand.
          // Group g of the wave: columns n0 = 32 j + 16 (g & 1), k half g >> 1 (the
          // 32x32x16 operand's lane layout).
          const int grp = lane >> 4, sl = lane & 15;
          const int n = 32 * j + 16 * (grp & 1) + 4 * (sl & 3), cn = n >> 3, e0 = n & 7;
          typedef short sv4 __attribute__((ext_vector_type(4)));
          sv4 part[2];
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const int r = 16 * kk + 8 * (grp >> 1) + 4 * hf + (sl >> 2);  // k row of the block
            part[hf] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (VK_LDS sv4*)((VK_LDS _Float16*)sb + (r * 8 + (cn ^ ((r >> 1) & 7))) * 8 + e0));
          }
          // (one shuffle: assigned element by element, the fragment was compiled into copies of
          // element 0 of each read)
          typedef _Float16 hv4 __attribute__((ext_vector_type(4)));
          fb[j] = __builtin_shufflevector(__builtin_bit_cast(hv4, part[0]), __builtin_bit_cast(hv4, part[1]), 0, 1,
                                          2, 3, 4, 5, 6, 7);
        } else {
          const int r = 32 * j + lr;
          fb[j] = *reinterpret_cast<const hv8*>(sb + (r * 8 + (ch ^ ((r >> 1) & 7))) * 8);
        }
      }
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa4[kk][i], fb4[kk][j], acc[i][j], 0, 0, 0);
  };

  if (nb > 0) dma(0, w);
  for (int it = 0; it < nb; ++it) {
    const int buf = it & 1;
    if (it + 1 < nb) {
      // the other buffer was last read in the previous iteration
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      dma(buf ^ 1, w + (it + 1) * kRmNW);
      // only the block just issued may still be in flight
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDmaPerStage) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    compute(buf, w + it * kRmNW);
  }

  // ---- add the wave partials in wave order, then 8 columns per thread
  float* red = reinterpret_cast<float*>(&sm[0][0][0]);
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  __syncthreads();
#pragma unroll
  for (int tt = 0; tt < kTiles; ++tt)
#pragma unroll
    for (int r = 0; r < 16; ++r) red[((w * kTiles + tt) * 16 + r) * 64 + lane] = acc[tt / TN][tt % TN][r];
  __syncthreads();
  for (int g = tid; g < kTiles * 16 * 8; g += 64 * kRmNW) {
    const int tt = g >> 7, r = (g >> 3) & 15, l0 = (g & 7) * 8;
    f4 s0 = *reinterpret_cast<const f4*>(&red[(tt * 16 + r) * 64 + l0]);
    f4 s1 = *reinterpret_cast<const f4*>(&red[(tt * 16 + r) * 64 + l0 + 4]);
#pragma unroll
    for (int ww = 1; ww < kRmNW; ++ww) {
      s0 += *reinterpret_cast<const f4*>(&red[((ww * kTiles + tt) * 16 + r) * 64 + l0]);
      s1 += *reinterpret_cast<const f4*>(&red[((ww * kTiles + tt) * 16 + r) * 64 + l0 + 4]);
    }
    const int i = tt / TN, j = tt % TN;
    const int row = m0 + 32 * i + 8 * (r >> 2) + 4 * (l0 >> 5) + (r & 3);
    const int col = n0 + 32 * j + (l0 & 31);
    if (row >= M || col >= N) continue;
    const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    const int64_t idx = (int64_t)row * N + col;
    if (P.splits > 1) {  // fp32 partial of this K part; splitk_reduce_kernel finishes
      float* const o = P.ws + (int64_t)split * M * N + idx;
      if (P.vec_out && col + 8 <= N) {
        *reinterpret_cast<f4*>(o) = s0;
        *reinterpret_cast<f4*>(o + 4) = s1;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (col + e < N) o[e] = sv[e];
      }
      continue;
    }
    if (P.vec_out && col + 8 <= N) {
      hv8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float y = epilogue(P, sv[e], row, col + e);
        asm volatile("" : "+v"(y));  // round in fp32, then to fp16 (no fused mixed-precision op)
        o[e] = (_Float16)y;
      }
      *reinterpret_cast<hv8*>(P.c + idx) = o;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (col + e >= N) break;
        float y = epilogue(P, sv[e], row, col + e);
        asm volatile("" : "+v"(y));
        P.c[idx + e] = (_Float16)y;
      }
    }
  }
}

// ---- GEMV-shaped path (M <= 4): the weights stream straight into registers.
//
// With one to four activation rows there is no operand reuse worth a matrix tile: every
// weight byte is used M times, so each workgroup streams its weight slice with fully
// coalesced 16-byte loads and does the M dot products on the vector ALU in fp32.  The
// activation rows (at most 64 KiB) are staged once per workgroup in LDS, with the A
// activation applied and rounded to fp16 as gemm_kernel does.
constexpr int kGvMaxM = 4;
constexpr int kGvLdsHalfs = 32768;  // 64 KiB
constexpr int kGvRowsNK = 16;       // [N,K]: weight rows per workgroup (4 per wave)
constexpr int kGvColsKN = 512;      // [K,N]: columns per workgroup (a kilobyte of each k row)
constexpr int kGvRowsKN = 8192;     // [K,N]: most k rows of one workgroup's K part

__device__ __forceinline__ void gv_stage_x(_Float16* xs, const Prob& P, int k0, int kn, int stride) {
  // x[m][k0 .. k0 + kn) -> xs[m * stride + ...], 16 bytes per thread and step (kn % 8 == 0)
  const int nch = kn / 8;
  for (int i = threadIdx.x; i < P.m * nch; i += 256) {
    const int m = i / nch, c = i - m * nch;
    hv8 v = *reinterpret_cast<const hv8*>(P.a + (int64_t)m * P.k + k0 + 8 * c);
    if (P.a_act != VKWR_GEMM_ACT_NONE) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (_Float16)act_in((float)v[e], P.a_act);
    }
    *reinterpret_cast<hv8*>(xs + m * stride + 8 * c) = v;
  }
}

// [N,K] weights: a wave owns 4 rows over the whole of K; lane l reads chunks l, l + 64, ...
// of each row (a kilobyte per instruction), and the (row, m) sums are reduced across the
// wave in a fixed order.
template <int M, bool kMulti>
__global__ __launch_bounds__(256) void gemv_nk_kernel(Batch bt) {
  __shared__ __attribute__((aligned(16))) _Float16 xs[kGvLdsHalfs];
  const int t = blockIdx.x;
  int pi = 0;
  if constexpr (kMulti) {
#pragma unroll
    for (int i = 1; i < kMaxProblems; ++i)
      if (i < bt.n && t >= bt.p[i].tile_begin) pi = i;
  }
  const Prob& P = bt.p[pi];
  {
    // every field in one round of kernel-argument loads, before the first branch (one round
    // in all for a one-problem launch; the compiler otherwise issued dependent rounds)
    const _Float16 *fa = P.a, *fb = P.b, *fv = P.v, *fvf = P.vf, *fv0 = P.v0;
    _Float16* fc = P.c;
    float* fws = P.ws;
    const int f0 = P.m, f1 = P.n, f2 = P.k, f3 = P.a_act, f4_ = P.epi, f5 = P.vec_out, f6 = P.splits,
              f7 = P.k_per_split, f8 = P.tile_begin, f9 = P.vec;
    asm volatile("" ::"s"(fa), "s"(fb), "s"(fv), "s"(fvf), "s"(fv0), "s"(fc), "s"(fws), "s"(f0), "s"(f1), "s"(f2),
                 "s"(f3), "s"(f4_), "s"(f5), "s"(f6), "s"(f7), "s"(f8), "s"(f9));
  }
  const int N = P.n, K = P.k;
  const int nr0 = (t - P.tile_begin) * kGvRowsNK;
  gv_stage_x(xs, P, 0, K, K);
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int nch = K / 8;
  float acc[4][M];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;
  const _Float16* wr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) wr[r] = P.b + (int64_t)min(nr0 + 4 * w + r, N - 1) * K;
  // 4 chunks of each of the 4 rows (16 loads, 16 KiB per wave) in flight per batch; chunks
  // past the row end are read clamped and weighted by zero.
  constexpr int kU = 4;
  for (int c0 = lane; c0 < nch; c0 += 64 * kU) {
    hv8 wv[kU][4];
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        wv[u][r] = *reinterpret_cast<const hv8*>(wr[r] + 8 * min(c0 + 64 * u, nch - 1));
    // every load of the batch is issued before the first use (no branch between them)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int c = min(c0 + 64 * u, nch - 1);
      const bool in = c0 + 64 * u < nch;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        hv8 xv = *reinterpret_cast<const hv8*>(xs + m * K + 8 * c);
        if (!in) xv = hv8{};
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[r][m] = __builtin_fmaf((float)wv[u][r][e], (float)xv[e], acc[r][m]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int n = nr0 + 4 * w + r;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float s = wave_sum(acc[r][m]);
      if (lane == m && n < N && m < P.m) {
        float y = epilogue(P, s, m, n);
        asm volatile("" : "+v"(y));  // round in fp32, then to fp16 (no fused mixed-precision op)
        P.c[(int64_t)m * N + n] = (_Float16)y;
      }
    }
  }
}

// [K,N] weights: a workgroup owns 512 columns (a kilobyte of each k row, lane l the 8
// columns 8 l .. 8 l + 7) over the k rows of its K part, wave w the rows w, w + 4, ...
// Only the k rows where some activation row is nonzero are read: each wave first lists
// its nonzero rows in LDS (a ballot per 64 rows), then streams those weight rows, every
// load instruction one contiguous kilobyte, and each lane accumulates its own columns in
// row order with no cross-lane reduction.  This is the reference's activation-sparse down
// projection (a relu^2 activation is zero for about half of the rows); a zero row adds
// exact zeros, so for finite weights the sum is the dense product's.  The 4 wave partials
// are added in wave order.  With K split over workgroups (P.splits > 1) each part stores
// fp32 sums to the workspace and splitk_reduce_kernel adds the parts and applies the
// epilogue.
template <int M, bool kMulti>
__global__ __launch_bounds__(256) void gemv_kn_kernel(Batch bt) {
  __shared__ __attribute__((aligned(16))) _Float16 xs[M * kGvRowsKN];
  __shared__ __attribute__((aligned(16))) float red[4][M][kGvColsKN];
  __shared__ __attribute__((aligned(16))) unsigned short nz[kGvRowsKN];  // wave w's list at w * q16
  const int t = blockIdx.x;
  int pi = 0;
  if constexpr (kMulti) {
#pragma unroll
    for (int i = 1; i < kMaxProblems; ++i)
      if (i < bt.n && t >= bt.p[i].tile_begin) pi = i;
  }
  const Prob& P = bt.p[pi];
  {
    // every field in one round of kernel-argument loads, before the first branch (one round
    // in all for a one-problem launch; the compiler otherwise issued dependent rounds)
    const _Float16 *fa = P.a, *fb = P.b, *fv = P.v, *fvf = P.vf, *fv0 = P.v0;
    _Float16* fc = P.c;
    float* fws = P.ws;
    const int f0 = P.m, f1 = P.n, f2 = P.k, f3 = P.a_act, f4_ = P.epi, f5 = P.vec_out, f6 = P.splits,
              f7 = P.k_per_split, f8 = P.tile_begin, f9 = P.vec;
    asm volatile("" ::"s"(fa), "s"(fb), "s"(fv), "s"(fvf), "s"(fv0), "s"(fc), "s"(fws), "s"(f0), "s"(f1), "s"(f2),
                 "s"(f3), "s"(f4_), "s"(f5), "s"(f6), "s"(f7), "s"(f8), "s"(f9));
  }
  const int N = P.n, K = P.k;
  int lt = t - P.tile_begin;
  const int part = lt % P.splits;
  lt /= P.splits;
  const int n0 = lt * kGvColsKN;
  const int k0 = part * P.k_per_split, kn = min(K, k0 + P.k_per_split) - k0;
  const int xstride = P.k_per_split;
  gv_stage_x(xs, P, k0, kn, xstride);
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // this wave's rows [r0, r1) of the part, and the nonzero ones among them
  const int q16 = ((kn + 3) / 4 + 15) & ~15;
  const int nw = kn > w ? (kn - w + 3) / 4 : 0;  // this wave's rows w, w + 4, ...
  unsigned short* list = nz + w * q16;
  int cnt = 0;
  for (int jb = 0; jb < nw; jb += 64) {
    const int r = w + 4 * (jb + lane);
    bool on = false;
    if (jb + lane < nw) {
#pragma unroll
      for (int m = 0; m < M; ++m)
        on |= (__builtin_bit_cast(unsigned short, xs[m * xstride + r]) & 0x7fff) != 0;
    }
    const uint64_t msk = __builtin_amdgcn_ballot_w64(on);
    const int at = cnt + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(msk >> 32),
                                                         __builtin_amdgcn_mbcnt_lo((uint32_t)msk, 0u));
    if (on) list[at] = (unsigned short)r;
    cnt += __builtin_popcountll(msk);
  }
  // the list padded to a multiple of 16 with its last row (weighted by zero below), so a
  // batch reads its 16 entries as two 16-byte LDS loads
  if (cnt > 0 && lane < ((16 - (cnt & 15)) & 15)) list[cnt + lane] = list[cnt - 1];
  const bool dense = cnt == nw;  // no zero row: the rows are w, w + 4, ...
  const int col = min(n0 + 8 * lane, N - 8);
  float acc[M][8];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[m][e] = 0.0f;
  const _Float16* wp = P.b + (int64_t)k0 * N + col;
  // 16 listed rows per lane (16 KiB per wave) in flight per batch; entries past the list end
  // read its last row again and are weighted by zero.
  constexpr int kU = 16;
  for (int i0 = 0; i0 < cnt; i0 += kU) {
    int rows[kU];
    hv8 wv[kU];
    if (dense) {
#pragma unroll
      for (int u = 0; u < kU; ++u) rows[u] = w + 4 * min(i0 + u, cnt - 1);
    } else {
      const uint4 l0 = *reinterpret_cast<const uint4*>(list + i0);
      const uint4 l1 = *reinterpret_cast<const uint4*>(list + i0 + 8);
      const unsigned lw[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
#pragma unroll
      for (int u = 0; u < kU; ++u) rows[u] = (lw[u >> 1] >> (16 * (u & 1))) & 0xffff;
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) wv[u] = *reinterpret_cast<const hv8*>(wp + (int64_t)rows[u] * N);
    // every load of the batch is issued before the first use (no branch between them)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const bool in = i0 + u < cnt;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float xm = in ? (float)xs[m * xstride + rows[u]] : 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[m][e] = __builtin_fmaf((float)wv[u][e], xm, acc[m][e]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
    *reinterpret_cast<f4*>(&red[w][m][8 * lane]) = f4{acc[m][0], acc[m][1], acc[m][2], acc[m][3]};
    *reinterpret_cast<f4*>(&red[w][m][8 * lane + 4]) = f4{acc[m][4], acc[m][5], acc[m][6], acc[m][7]};
  }
  __syncthreads();
  for (int i = threadIdx.x; i < P.m * kGvColsKN; i += 256) {
    const int m = i / kGvColsKN, cc = i - m * kGvColsKN, n = n0 + cc;
    if (n >= N) continue;
    const float s = ((red[0][m][cc] + red[1][m][cc]) + red[2][m][cc]) + red[3][m][cc];
    if (P.splits > 1) {
      P.ws[((int64_t)part * P.m + m) * N + n] = s;
    } else {
      float y = epilogue(P, s, m, n);
      asm volatile("" : "+v"(y));
      P.c[(int64_t)m * N + n] = (_Float16)y;
    }
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

struct Config {
  int bm, bn;
  bool big;         // gemm_big_kernel (256x256 tiles, no K splits)
  bool rm = false;  // gemm_rm_kernel (bm x bn tiles, K split over its waves, no workspace)
  bool kn = false;  // ... with [K,N] weights
  int gv = 0;       // gemv_{nk,kn}_kernel<gv> (M <= gv <= 4), 0: not this path
};

// Tile shape from the largest M of the batch (all problems of one launch share it).
Config pick_config(int max_m, int min_n) {
  if (max_m <= 32) return {32, 128, false};
  if (max_m <= 64) return {64, 128, false};
  if (min_n >= 128 && max_m > 256) return {128, 128, false};
  return {128, 64, false};
}

// gemm_big_kernel takes the batch when every non-empty problem has an unactivated A, a
// [N,K] B, K a multiple of 64, 16-byte aligned rows (operands and output, N a multiple of 8),
// 32-bit byte offsets into A and B, and some problem has M >= 256.
bool big_eligible(const Batch& bt, int max_m) {
  if (max_m < kBigBM) return false;
  for (int i = 0; i < bt.n; ++i) {
    const Prob& P = bt.p[i];
    if (P.m == 0 || P.n == 0) continue;
    if (P.b_kn || P.a_act != VKWR_GEMM_ACT_NONE || !P.vec || !P.vec_out || P.k < kBigBK || P.k % kBigBK)
      return false;
    if ((int64_t)std::max(P.m, P.n) * P.k * 2 > 0xFFFF0000LL) return false;
  }
  return true;
}

// gemm_rm_kernel takes a batch of decode-sized problems (M <= 128) when every non-empty
// problem has 16-byte aligned rows with K a multiple of 8 (and N one for [K,N] weights),
// N >= 8, one weight layout, operands below 4 GiB (32-bit DMA offsets), and the batch
// fills the CUs with tiles: it then streams the weights through LDS without a workspace.
// The tile is the largest of 64 x 64, 32 x 64 and 32 x 32 ([K,N]: 64 columns) that
// still gives every CU a workgroup.
constexpr int kRmMaxM = 128;

bool rm_config(const Batch& bt, int max_m, Config& cfg) {
  if (max_m < 1 || max_m > kRmMaxM) return false;
  int kn = -1;
  for (int i = 0; i < bt.n; ++i) {
    const Prob& P = bt.p[i];
    if (P.m == 0 || P.n == 0) continue;
    if (!P.vec || P.n < 8 || (P.k > 0 && P.k < 8)) return false;
    if (kn >= 0 && kn != P.b_kn) return false;
    kn = P.b_kn;
    if ((int64_t)P.m * P.k * 2 >= 0xFFFFFFFFLL || (int64_t)P.n * P.k * 2 >= 0xFFFFFFFFLL) return false;
  }
  if (kn < 0) return false;
  const int cus = device_cus();
  const int shapes[3][2] = {{64, 64}, {32, 64}, {32, 32}};
  int pick = -1;
  for (int c = 0; c < 3; ++c) {
    const int bm = shapes[c][0], bn = shapes[c][1];
    if (bm == 64 && max_m <= 32) continue;
    if (kn && bn != 64) continue;
    int64_t tiles = 0;
    for (int i = 0; i < bt.n; ++i) {
      const Prob& P = bt.p[i];
      if (P.m == 0 || P.n == 0) continue;
      tiles += (int64_t)((P.m + bm - 1) / bm) * ((P.n + bn - 1) / bn);
    }
    if (tiles >= cus) {
      pick = c;
      break;
    }
  }
  if (pick < 0) {
    // Too few tiles for the CUs whole: split K over workgroups (parts of at least one 64-deep
    // block per wave, at most 16 parts).  Take the largest tile shape whose split fills the
    // CUs, else the shape that comes closest.
    int64_t best = 0;
    for (int c = 0; c < 3; ++c) {
      const int bm = shapes[c][0], bn = shapes[c][1];
      if (bm == 64 && max_m <= 32) continue;
      if (kn && bn != 64) continue;
      const int nw = (bm == 32 && bn == 32) ? 8 : 4;
      int64_t wgs = 0;
      for (int i = 0; i < bt.n; ++i) {
        const Prob& P = bt.p[i];
        if (P.m == 0 || P.n == 0) continue;
        const int64_t t = (int64_t)((P.m + bm - 1) / bm) * ((P.n + bn - 1) / bn);
        wgs += t * std::max(1, std::min(16, P.k / (kRmBK * nw)));
      }
      if (wgs >= cus) {
        pick = c;
        break;
      }
      if (wgs > best) {
        best = wgs;
        pick = c;
      }
    }
    if (pick < 0) return false;
  }
  cfg = Config{shapes[pick][0], shapes[pick][1], false, true, kn == 1};
  return true;
}

// The GEMV kernels take a batch of at most 4 rows when every non-empty problem has 16-byte
// aligned rows, K (and N for [K,N]) a multiple of 8, N >= 8 and one weight layout, and
// (for [N,K]) the activation rows fit the 64 KiB staging buffer.
bool gv_config(const Batch& bt, int max_m, Config& cfg) {
  if (max_m < 1 || max_m > kGvMaxM) return false;
  int kn = -1;
  for (int i = 0; i < bt.n; ++i) {
    const Prob& P = bt.p[i];
    if (P.m == 0 || P.n == 0) continue;
    if (!P.vec || P.n < 8 || P.k < 8) return false;
    if (kn >= 0 && kn != P.b_kn) return false;
    kn = P.b_kn;
    if (!P.b_kn && (int64_t)max_m * P.k > kGvLdsHalfs) return false;
  }
  if (kn < 0) return false;
  cfg = Config{1, kn ? kGvColsKN : kGvRowsNK, false, false, kn == 1, max_m <= 2 ? max_m : 4};
  return true;
}

int64_t plan_big(Batch& bt, BigPlan& pl);

// Fills tiling fields and returns the workspace bytes the batch needs.
int64_t plan(Batch& bt, Config cfg, int target_wgs) {
  if (cfg.big) {
    BigPlan pl;
    return plan_big(bt, pl);
  }
  if (cfg.gv) {
    // [K,N]: split K over workgroups until the batch has a workgroup per CU, each part >= 128
    // k rows (a multiple of 32) whose activation slice fits the staging buffer.
    int tiles = 0;
    for (int i = 0; i < bt.n; ++i) {
      Prob& P = bt.p[i];
      const bool empty = P.m == 0 || P.n == 0;
      P.tiles_m = empty ? 0 : 1;
      P.tiles_n = empty ? 0 : (P.n + cfg.bn - 1) / cfg.bn;
      tiles += P.tiles_n;
    }
    int64_t ws = 0;
    int begin = 0;
    for (int i = 0; i < bt.n; ++i) {
      Prob& P = bt.p[i];
      P.splits = 1;
      P.k_per_split = P.k;
      if (cfg.kn && P.tiles_n > 0) {
        const int kmax = kGvRowsKN;  // staging and row-list limit, rows of K
        const int cus = device_cus();
        int s = tiles > 0 ? (cus + tiles - 1) / tiles : 1;
        s = std::max(1, std::min({s, 64, P.k / 128}));
        s = std::max(s, (P.k + kmax - 1) / kmax);
        const int kps = ((P.k + s - 1) / s + 31) / 32 * 32;
        P.splits = (P.k + kps - 1) / kps;
        P.k_per_split = P.splits > 1 ? kps : P.k;
        if (P.splits > 1) ws += (int64_t)P.splits * P.m * P.n * 4;
      }
      P.tile_begin = begin;
      begin += P.tiles_m * P.tiles_n * P.splits;
    }
    return ws;
  }
  if (cfg.rm) {
    // K parts only when the batch's tiles leave CUs idle: enough parts to give every CU a
    // workgroup, each a multiple of 64 deep and at least one 64-deep block per wave.
    const int nw = (cfg.bm == 32 && cfg.bn == 32) ? 8 : 4;
    int tiles = 0;
    for (int i = 0; i < bt.n; ++i) {
      Prob& P = bt.p[i];
      const bool empty = P.m == 0 || P.n == 0;
      P.tiles_m = empty ? 0 : (P.m + cfg.bm - 1) / cfg.bm;
      P.tiles_n = empty ? 0 : (P.n + cfg.bn - 1) / cfg.bn;
      tiles += P.tiles_m * P.tiles_n;
    }
    const int cus = device_cus();
    int64_t ws = 0;
    int begin = 0;
    for (int i = 0; i < bt.n; ++i) {
      Prob& P = bt.p[i];
      P.splits = 1;
      P.k_per_split = P.k;
      if (tiles > 0 && tiles < cus && P.tiles_m * P.tiles_n > 0 && P.k > 0) {
        int s = std::min(16, (cus + tiles - 1) / tiles);
        s = std::max(1, std::min(s, P.k / (kRmBK * nw)));
        const int kps = ((P.k + s - 1) / s + kRmBK - 1) / kRmBK * kRmBK;
        P.splits = (P.k + kps - 1) / kps;
        P.k_per_split = P.splits > 1 ? kps : P.k;
        if (P.splits > 1) ws += (int64_t)P.splits * P.m * P.n * 4;
      }
      P.tile_begin = begin;
      begin += P.tiles_m * P.tiles_n * P.splits;
    }
    return ws;
  }
  int tiles = 0;
  for (int i = 0; i < bt.n; ++i) {
    Prob& P = bt.p[i];
    P.tiles_m = (P.m + cfg.bm - 1) / cfg.bm;
    P.tiles_n = (P.n + cfg.bn - 1) / cfg.bn;
    tiles += P.tiles_m * P.tiles_n;
  }
  int64_t ws = 0;
  for (int i = 0; i < bt.n; ++i) {
    Prob& P = bt.p[i];
    const int base = P.tiles_m * P.tiles_n;
    // Split K only when the whole batch leaves CUs idle; keep >= 8 stages per split.
    // An empty problem (no tiles) or K == 0 (the kernel writes epilogue(0)) is never split.
    int s = 1;
    if (!cfg.big && tiles > 0 && base > 0 && P.k > 0 && tiles < target_wgs && P.m <= 256) {
      s = (target_wgs + tiles - 1) / tiles;
      s = std::min(s, std::max(1, P.k / (8 * kBK)));
      s = std::min(s, 16);
    }
    const int kps = std::max(kBK, ((P.k + s - 1) / s + kBK - 1) / kBK * kBK);
    P.splits = std::max(1, (P.k + kps - 1) / kps);
    P.k_per_split = kps;
    if (P.splits > 1) ws += (int64_t)P.splits * P.m * P.n * 4;
  }
  int begin = 0;
  for (int i = 0; i < bt.n; ++i) {
    bt.p[i].tile_begin = begin;
    begin += bt.p[i].tiles_m * bt.p[i].tiles_n * bt.p[i].splits;
  }
  return ws;
}

// Tiles (256x256) of a large-M batch and its stream-K split; returns the workspace bytes.
// The plan for tile rows BM: tile fields of the batch's problems, and the split of the last
// round; returns its estimated time (us).  Time model: a tile's k-stage ~1.7 us when every CU
// is busy (0.80 of that for 192 rows: 0.77 measured on the 7B FFN key, 768 tiles in three
// whole rounds against 576 in two rounds and a split tail; the operand bytes per MAC are
// higher), plus ~2 stages of prologue and epilogue per workgroup; a split tile costs its S
// fp32 partials written and read back at ~5 TB/s, and a split plan the ramp of its two
// extra launches (~3 us each).  Batches of unequal K (the low-rank outputs: K = 512 and
// 128, their time in the epilogue stores) are scored by how fully the last round of tiles
// fills the CUs instead (returned as a negative fill fraction).
double plan_big_bm(Batch& bt, BigPlan& pl, int BM) {
  int T = 0, k_all = -1;
  bool uniform_k = true;
  for (int i = 0; i < bt.n; ++i) {
    Prob& P = bt.p[i];
    P.splits = 1;
    P.k_per_split = P.k;
    if (P.m == 0 || P.n == 0) {
      P.tiles_m = P.tiles_n = 0;
    } else {
      P.tiles_m = (P.m + BM - 1) / BM;
      P.tiles_n = (P.n + kBigBM - 1) / kBigBM;
      uniform_k = uniform_k && (k_all < 0 || k_all == P.k);
      k_all = P.k;
    }
    P.tile_begin = T;
    T += P.tiles_m * P.tiles_n;
  }
  pl = BigPlan{BM, T, 0, 1, 0, 0, 0, 0, nullptr};
  const int G = device_cus();
  const double stage = 1.7 * (BM == 192 ? 0.80 : 1.0), over = 2.0 * stage, split_launches = 6.0;
  if (!uniform_k) {
    // whole tiles; spread every problem's tiles evenly over the XCDs where the counts allow
    bool even = true;
    for (int i = 0; i < bt.n; ++i) {
      bt.order[i] = i;
      even = even && (bt.p[i].tiles_m * bt.p[i].tiles_n) % 8 == 0;
    }
    std::stable_sort(bt.order, bt.order + bt.n, [&](int a, int b) { return bt.p[a].k > bt.p[b].k; });
    bt.xbal = even ? 1 : 0;
    return -(double)T / ((double)((T + G - 1) / G) * G);
  }
  bt.xbal = 0;
  const int nst = k_all / kBigBK;
  const double rounds_whole = (double)((T + G - 1) / G);
  double best = rounds_whole * (nst * stage + over);
  if (T < 32 || T % G == 0) return best;
  const int R = T % G, D = T - R;
  const double full = (double)(D / G) * (nst * stage + over);
  int best_s = 1;
  for (int S = 2; S <= 8 && nst / S >= 8; ++S) {
    const double rounds = (double)((R * S + G - 1) / G);
    const double t = full + rounds * ((double)nst / S * stage + over) + (double)R * S * 2 * BM * kBigBM * 4 / 5e6 +
                     split_launches;
    if (t < best) {
      best = t;
      best_s = S;
    }
  }
  // Layered split of the R tiles over all G CUs (when its shape conditions hold): R nst / G
  // stages on every CU, in 1 + 1 + b / g pieces at most.
  int lay_per = 0, lay_g = 0;
  if (R <= G && G < 2 * R && ((int64_t)R * nst) % G == 0) {
    const int per = (int)((int64_t)R * nst / G), L = nst - per, b = per - L;
    int g = std::gcd(b, L);
    if (L > 0 && b > 0 && g >= 8) {
      const int R3 = R - (G - R), pieces = R + (G - R) + R3 * (L / g);
      const double t =
          full + per * stage + (2 + b / g) * over + (double)pieces * 2 * BM * kBigBM * 4 / 5e6 + split_launches;
      if (t < best) {
        best = t;
        lay_per = per;
        lay_g = g;
      }
    }
  }
  if (lay_per > 0 || best_s > 1) {
    pl.dp_tiles = D;
    pl.sk_tiles = R;
    pl.parts = lay_per > 0 ? 0 : best_s;
    pl.nst = nst;
    pl.wgs = lay_per > 0 ? G : 0;
    pl.per = lay_per;
    pl.gran = lay_g;
  }
  return best;
}

// Picks the tile rows (256, or 192 when its plan is estimated to be at least 5 % faster -- M =
// 2304 fills 256 CUs with 192 row tiles far better than with 144 -- or, for unequal K, fills
// the last round better) and plans the batch; returns the workspace bytes the plan needs.
int64_t plan_big(Batch& bt, BigPlan& pl) {
  BigPlan p192;
  const double t192 = plan_big_bm(bt, p192, 192);
  const double t256 = plan_big_bm(bt, pl, 256);
  if (t256 < 0 ? t192 < t256 - 0.05 : t192 < 0.95 * t256) plan_big_bm(bt, pl, 192);
  if (pl.sk_tiles == 0) return 0;
  int64_t slots = (int64_t)pl.sk_tiles * pl.parts;
  if (pl.wgs > 0) {
    const Layers y = layers_of(pl);
    slots = (int64_t)y.R + y.W2 + (int64_t)y.R3 * y.npc;
  }
  return slots * pl.bm * kBigBM * 4;
}

int total_wgs(const Batch& bt) {
  int t = 0;
  for (int i = 0; i < bt.n; ++i) t += bt.p[i].tiles_m * bt.p[i].tiles_n * bt.p[i].splits;
  return t;
}

int build_batch(const char* fn, int n, const vkwr_gemm_problem* pr, Batch& bt, Config& cfg) {
  VK_REQUIRE(n >= 1 && n <= kMaxProblems, "%s: 1..%d problems per launch (got %d)", fn, kMaxProblems, n);
  VK_REQUIRE(pr != nullptr, "%s: null problem list", fn);
  bt.n = n;
  bt.xbal = 0;
  int max_m = 0, min_n = 1 << 30;
  for (int i = 0; i < n; ++i) {
    const vkwr_gemm_problem& q = pr[i];
    VK_REQUIRE(q.m >= 0 && q.n >= 0 && q.k >= 0, "%s: negative size in problem %d", fn, i);
    VK_REQUIRE(q.m <= 0x7fffffff && q.n <= 0x7fffffff && q.k <= 0x7fffffff &&
                   q.m * q.n <= ((int64_t)1 << 40),
               "%s: problem %d too large", fn, i);
    VK_REQUIRE(q.b_layout == VKWR_GEMM_B_NK || q.b_layout == VKWR_GEMM_B_KN, "%s: bad b_layout", fn);
    VK_REQUIRE(q.a_act >= VKWR_GEMM_ACT_NONE && q.a_act <= VKWR_GEMM_ACT_RELU_SQUARE, "%s: bad a_act", fn);
    VK_REQUIRE(q.epilogue >= VKWR_GEMM_EPI_NONE && q.epilogue <= VKWR_GEMM_EPI_SIGMOID,
               "%s: bad epilogue", fn);
    const bool empty = q.m == 0 || q.n == 0;
    VK_REQUIRE(empty || (q.a && q.b && q.c), "%s: null pointer in problem %d", fn, i);
    VK_REQUIRE(empty || q.epilogue != VKWR_GEMM_EPI_VALUE_RESIDUAL || (q.v && q.v_first && q.v0),
               "%s: value-residual epilogue needs v, v_first, v0", fn);
    VK_REQUIRE(empty || q.epilogue != VKWR_GEMM_EPI_BIAS || q.v0, "%s: bias epilogue needs v0", fn);
    Prob& P = bt.p[i];
    P = Prob{};
    P.a = reinterpret_cast<const _Float16*>(q.a);
    P.b = reinterpret_cast<const _Float16*>(q.b);
    P.c = reinterpret_cast<_Float16*>(q.c);
    P.v = reinterpret_cast<const _Float16*>(q.v);
    P.vf = reinterpret_cast<const _Float16*>(q.v_first);
    P.v0 = reinterpret_cast<const _Float16*>(q.v0);
    P.m = (int)q.m;
    P.n = (int)q.n;
    P.k = (int)q.k;
    P.b_kn = q.b_layout == VKWR_GEMM_B_KN;
    P.a_act = q.a_act;
    P.epi = q.epilogue;
    P.vec = aligned16(q.a) && aligned16(q.b) && q.k % 8 == 0 && (!P.b_kn || q.n % 8 == 0);
    P.vec_out = aligned16(q.c) && q.n % 8 == 0 &&
                (q.epilogue != VKWR_GEMM_EPI_VALUE_RESIDUAL ||
                 (aligned16(q.v) && aligned16(q.v_first) && aligned16(q.v0))) &&
                (q.epilogue != VKWR_GEMM_EPI_BIAS || aligned16(q.v0));
    if (!empty) {
      max_m = std::max(max_m, P.m);
      min_n = std::min(min_n, P.n);
    }
  }
  cfg = pick_config(max_m, min_n);
  if (big_eligible(bt, max_m)) cfg = Config{kBigBM, kBigBM, true};
  else if (!gv_config(bt, max_m, cfg)) rm_config(bt, max_m, cfg);
  return VKWR_OK;
}

constexpr int kTargetWgs = 512;  // two workgroups per CU on 256 CUs

}  // namespace
}  // namespace vk

using namespace vk;

extern "C" int64_t vkwr_gemm_f16_workspace_bytes(int n_problems, const vkwr_gemm_problem* problems) {
  clear_error();
  Batch bt;
  Config cfg;
  if (build_batch("vkwr_gemm_f16_workspace_bytes", n_problems, problems, bt, cfg)) return -1;
  return plan(bt, cfg, kTargetWgs);
}

// Scratch of vkwr_gemm_f16_noalloc: the K-split / stream-K partials of one launch.  Each
// device that loads the library holds its own copy for the life of the process.  Host code
// reaches it only through the address hipGetSymbolAddress returns for the current device
// (scratch_ptr below); the array's name itself is a host-side stand-in.
static constexpr int64_t kNoAllocScratchBytes = (int64_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

// Launches a planned batch whose workspace (need bytes, checked by the caller) is at
// `workspace`.  Shared by vkwr_gemm_f16 and vkwr_gemm_f16_noalloc.
int gemm_run(const char* fn, Batch& bt, const Config& cfg, void* workspace, void* stream) {
  // Zero-sized problems and K == 0: nothing to tile; K == 0 writes epilogue(0).
  float* ws = reinterpret_cast<float*>(workspace);
  for (int i = 0; i < bt.n; ++i) {
    Prob& P = bt.p[i];
    if (P.m == 0 || P.n == 0) {
      P.tiles_m = P.tiles_n = 0;
    }
    if (P.splits > 1) {
      P.ws = ws;
      ws += (int64_t)P.splits * P.m * P.n;
      if (!aligned16(P.ws)) P.vec_out = 0;
    }
  }
  int begin = 0;
  bool any_split = false;
  for (int i = 0; i < bt.n; ++i) {
    bt.p[i].tile_begin = begin;
    begin += bt.p[i].tiles_m * bt.p[i].tiles_n * bt.p[i].splits;
    any_split = any_split || bt.p[i].splits > 1;
  }
  const int wgs = total_wgs(bt);
  if (wgs == 0) return VKWR_OK;
  hipStream_t s = (hipStream_t)stream;
  if (cfg.gv) {
    if (cfg.kn) {
      auto go_gv = [&](auto multi) {
        constexpr bool kM = decltype(multi)::value;
        if (cfg.gv == 1) hipLaunchKernelGGL((gemv_kn_kernel<1, kM>), dim3(wgs), dim3(256), 0, s, bt);
        else if (cfg.gv == 2) hipLaunchKernelGGL((gemv_kn_kernel<2, kM>), dim3(wgs), dim3(256), 0, s, bt);
        else hipLaunchKernelGGL((gemv_kn_kernel<4, kM>), dim3(wgs), dim3(256), 0, s, bt);
      };
      if (bt.n > 1) go_gv(std::true_type{});
      else go_gv(std::false_type{});
    } else {
      auto go_gv = [&](auto multi) {
        constexpr bool kM = decltype(multi)::value;
        if (cfg.gv == 1) hipLaunchKernelGGL((gemv_nk_kernel<1, kM>), dim3(wgs), dim3(256), 0, s, bt);
        else if (cfg.gv == 2) hipLaunchKernelGGL((gemv_nk_kernel<2, kM>), dim3(wgs), dim3(256), 0, s, bt);
        else hipLaunchKernelGGL((gemv_nk_kernel<4, kM>), dim3(wgs), dim3(256), 0, s, bt);
      };
      if (bt.n > 1) go_gv(std::true_type{});
      else go_gv(std::false_type{});
    }
    if (int e = check_launch(fn)) return e;
    if (any_split) {
      hipLaunchKernelGGL(splitk_reduce_kernel, dim3(reduce_wgs(bt), bt.n), dim3(256), 0, s, bt);
      if (int e = check_launch(fn)) return e;
    }
    return VKWR_OK;
  }
  if (cfg.rm) {
    bool any_act = false;
    for (int i = 0; i < bt.n; ++i) any_act = any_act || bt.p[i].a_act != VKWR_GEMM_ACT_NONE;
    auto go_rm = [&](auto act, auto multi) {
      constexpr bool kAct = decltype(act)::value, kM = decltype(multi)::value;
      if (cfg.kn && cfg.bm == 64)
        hipLaunchKernelGGL((gemm_rm_kernel<2, 2, true, kAct, kM>), dim3(wgs), dim3(256), 0, s, bt);
      else if (cfg.kn) hipLaunchKernelGGL((gemm_rm_kernel<1, 2, true, kAct, kM>), dim3(wgs), dim3(256), 0, s, bt);
      else if (cfg.bm == 64)
        hipLaunchKernelGGL((gemm_rm_kernel<2, 2, false, kAct, kM>), dim3(wgs), dim3(256), 0, s, bt);
      else if (cfg.bn == 64)
        hipLaunchKernelGGL((gemm_rm_kernel<1, 2, false, kAct, kM>), dim3(wgs), dim3(256), 0, s, bt);
      else hipLaunchKernelGGL((gemm_rm_kernel<1, 1, false, kAct, kM>), dim3(wgs), dim3(512), 0, s, bt);
    };
    if (bt.n > 1) {
      if (any_act) go_rm(std::true_type{}, std::true_type{});
      else go_rm(std::false_type{}, std::true_type{});
    } else {
      if (any_act) go_rm(std::true_type{}, std::false_type{});
      else go_rm(std::false_type{}, std::false_type{});
    }
    if (int e = check_launch(fn)) return e;
    if (any_split) {
      hipLaunchKernelGGL(splitk_reduce_kernel, dim3(reduce_wgs(bt), bt.n), dim3(256), 0, s, bt);
      if (int e = check_launch(fn)) return e;
    }
    return VKWR_OK;
  }
  if (cfg.big) {
    BigPlan pl;
    plan_big(bt, pl);  // same plan as above (need)
    pl.ws = reinterpret_cast<float*>(workspace);
    int epi = -2;  // the batch's common epilogue, -1 if they differ
    for (int i = 0; i < bt.n; ++i) {
      if (bt.p[i].m == 0 || bt.p[i].n == 0) continue;
      epi = epi == -2 ? bt.p[i].epi : (epi == bt.p[i].epi ? epi : -1);
    }
    auto go = [&](auto bm_tag, auto whole, auto fix) {
      constexpr int BM = decltype(bm_tag)::value;
      if (pl.dp_tiles > 0) hipLaunchKernelGGL(whole, dim3(pl.dp_tiles), dim3(256), 0, s, bt, pl.dp_tiles);
      if (pl.sk_tiles > 0) {
        const int sk_wgs = pl.wgs > 0 ? pl.wgs : pl.sk_tiles * pl.parts;
        hipLaunchKernelGGL(gemm_big_sk_kernel<BM>, dim3(sk_wgs), dim3(256), 0, s, bt, pl);
        hipLaunchKernelGGL(fix, dim3(4 * (BM / 64), pl.sk_tiles), dim3(256), 0, s, bt, pl);
      }
    };
    auto go_bm = [&](auto bm_tag) {
      constexpr int BM = decltype(bm_tag)::value;
      if (epi == VKWR_GEMM_EPI_NONE)
        go(bm_tag, gemm_big_kernel<BM, VKWR_GEMM_EPI_NONE>, gemm_big_fixup_kernel<BM, VKWR_GEMM_EPI_NONE>);
      else if (epi == VKWR_GEMM_EPI_RELU_SQUARE)
        go(bm_tag, gemm_big_kernel<BM, VKWR_GEMM_EPI_RELU_SQUARE>,
           gemm_big_fixup_kernel<BM, VKWR_GEMM_EPI_RELU_SQUARE>);
      else if (epi == VKWR_GEMM_EPI_BIAS)
        go(bm_tag, gemm_big_kernel<BM, VKWR_GEMM_EPI_BIAS>, gemm_big_fixup_kernel<BM, VKWR_GEMM_EPI_BIAS>);
      else if (epi == VKWR_GEMM_EPI_VALUE_RESIDUAL)
        go(bm_tag, gemm_big_kernel<BM, VKWR_GEMM_EPI_VALUE_RESIDUAL>,
           gemm_big_fixup_kernel<BM, VKWR_GEMM_EPI_VALUE_RESIDUAL>);
      else
        go(bm_tag, gemm_big_kernel<BM, -1>, gemm_big_fixup_kernel<BM, -1>);
    };
    if (pl.bm == 192) go_bm(std::integral_constant<int, 192>{});
    else go_bm(std::integral_constant<int, 256>{});
    return check_launch(fn);
  }
  if (cfg.bm == 32) hipLaunchKernelGGL((gemm_kernel<32, 128, 1, 4>), dim3(wgs), dim3(256), 0, s, bt);
  else if (cfg.bm == 64) hipLaunchKernelGGL((gemm_kernel<64, 128, 2, 2>), dim3(wgs), dim3(256), 0, s, bt);
  else if (cfg.bn == 128) hipLaunchKernelGGL((gemm_kernel<128, 128, 2, 2>), dim3(wgs), dim3(256), 0, s, bt);
  else hipLaunchKernelGGL((gemm_kernel<128, 64, 2, 2>), dim3(wgs), dim3(256), 0, s, bt);
  if (int e = check_launch(fn)) return e;
  if (any_split) {
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(reduce_wgs(bt), bt.n), dim3(256), 0, s, bt);
    if (int e = check_launch(fn)) return e;
  }
  return VKWR_OK;
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device, set on first use

// The device address of the current device's copy of `scratch` (the array's name is a
// host-side stand-in and must never reach a kernel).  Looked up once per device.
int scratch_ptr(const char* fn, void** out) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  VK_REQUIRE(e == hipSuccess && dev >= 0 && dev < kMaxDevices, "%s: no current device (%s)", fn,
             hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    VK_REQUIRE(r == hipSuccess && p, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", fn, dev,
               hipGetErrorString(r));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return VKWR_OK;
}

}  // namespace

extern "C" int vkwr_gemm_f16(int n_problems, const vkwr_gemm_problem* problems, void* workspace,
                             int64_t workspace_bytes, void* stream) {
  clear_error();
  const char* fn = "vkwr_gemm_f16";
  Batch bt;
  Config cfg;
  if (int e = build_batch(fn, n_problems, problems, bt, cfg)) return e;
  const int64_t need = plan(bt, cfg, kTargetWgs);
  VK_REQUIRE(need <= workspace_bytes && (need == 0 || workspace != nullptr),
             "%s: workspace of %lld bytes needed (got %lld)", fn, (long long)need,
             (long long)workspace_bytes);
  return gemm_run(fn, bt, cfg, workspace, stream);
}

extern "C" int64_t vkwr_gemm_f16_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int vkwr_gemm_f16_noalloc(int n_problems, const vkwr_gemm_problem* problems, void* stream) {
  clear_error();
  const char* fn = "vkwr_gemm_f16_noalloc";
  // The scratch address is looked up on every call's device before anything else, so that
  // any first call -- an empty or even an invalid batch -- does it outside a graph capture.
  void* ws = nullptr;
  if (int e = scratch_ptr(fn, &ws)) return e;
  Batch bt;
  Config cfg;
  if (int e = build_batch(fn, n_problems, problems, bt, cfg)) return e;
  const int64_t need = plan(bt, cfg, kTargetWgs);
  VK_REQUIRE(need <= kNoAllocScratchBytes,
             "%s: this batch needs %lld bytes of scratch; the allocation-free entry point holds at most "
             "%lld (use vkwr_gemm_f16 with a workspace)",
             fn, (long long)need, (long long)kNoAllocScratchBytes);
  return gemm_run(fn, bt, cfg, need > 0 ? ws : nullptr, stream);
}
