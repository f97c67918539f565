// Decode-step GEMM on fragment-layout operands: c = epilogue(a . b^T).
//
// At decode the activation a has few rows (one per sequence, m <= a few
// hundred) and every weight byte is used m times, so the GEMM is bound by
// streaming the weights once from HBM.  Two things decide how close to that
// bound a gfx950 kernel gets:
//
//  * Load efficiency.  The A and B operands of v_mfma_f32_32x32x16_f16 give
//    lane l the 8 halfs (row l % 32, k 8*(l / 32)..+7) of a 32 x 16 tile; read
//    from a row-major matrix each wave load touches 32 rows x 32 bytes.  In the
//    frag layout (vk_common.cuh frag_index) that tile is one contiguous
//    kilobyte, so every load is fully coalesced and needs no LDS staging.
//    Weights are packed once at model load; the producers of each projection
//    input write it directly in frag layout.
//
//  * Parallelism without a K-split workspace.  A workgroup owns one
//    (32 TM) x (32 TN) output tile over the whole of K; its NW waves take the
//    16 KS-wide k blocks w, w + NW, ... with a two-deep register pipeline
//    (loads are issued unconditionally inside the loop and the last blocks are
//    peeled, so the compiler's wait counts stay exact), and the NW partial
//    tiles are added through LDS in wave order after one barrier.
//    Deterministic, no second kernel, no fp32 partials in HBM.
//
//  * For long K (the FFN value, K = 4 C) the same kernel can instead give
//    each workgroup one K part of a 64 x 64 tile and write its fp32 partial
//    tile to a caller workspace (vkwr_frag_gemm_splitk_f16): each workgroup
//    then reads half the activation bytes of the unsplit 32 x 32 form, and
//    frag_splitk_reduce_kernel (or the consumer) adds the parts in K order.
//
// A launch runs up to 8 problems, each on its own range of workgroups.  When a
// problem has several row tiles, the row tiles of one column tile are
// given workgroup ids that differ by multiples of 8: gfx950 dispatches
// workgroups round-robin over its 8 XCDs, so they share an L2 and the second
// read of the weight tile hits it.
//
// Roofline: HBM-bound; algorithmic bytes = n*k*2 (weights) + m*k*2 + m*n*2.

#include <algorithm>

#include "vk_capi.h"
#include "vk_common.cuh"

namespace vk {
namespace {

typedef _Float16 hv8 __attribute__((ext_vector_type(8)));
typedef float fv16 __attribute__((ext_vector_type(16)));

constexpr int kMaxFragProblems = 8;

struct FProb {
  const _Float16* a;
  const _Float16* b;
  _Float16* c;
  const _Float16 *v, *vf, *v0;
  int m, n, npad, kpad;
  int epi, c_frag;
  int ncol, nmb;            // column tiles, row tiles
  int wg_begin;             // first workgroup id (multiple of 8)
  float* ws;                // K split: fp32 partial tiles [ksplit][nmb * 32 * TM][npad]
  int ksplit;               // K parts (1: no split)
  int xcd_map;              // row tiles of a column tile share an XCD
};

struct FBatch {
  int n;
  FProb p[kMaxFragProblems];
};

__device__ __forceinline__ float apply_act(int epi, float x) {
  if (epi == VKWR_GEMM_EPI_RELU_SQUARE) {
    const float r = fmaxf(x, 0.0f);
    return r * r;
  }
  if (epi == VKWR_FRAG_EPI_TANH) return tanhf(x);
  if (epi == VKWR_FRAG_EPI_SIGMOID) return sigmoidf(x);
  return x;
}

// Store paths.  kStoreAny branches per tile on the problem's epilogue and
// layout; the two specialised ones hold only their own code, which the decode
// step's single-problem launches (FFN key, FFN value, o projection, head)
// take: the generic path costs them about 0.8 us per launch.
// kStorePartial writes the workgroup's fp32 tile of one K part to the split
// workspace; frag_splitk_reduce_kernel adds the parts and applies the epilogue.
// kStoreActFrag and kStoreRowMajor cover the decode step's two mixed batches
// (projections: plain row-major or frag with none / tanh / sigmoid; low-rank
// outputs: row-major with none / bias / value residual) without the other
// paths' code.
constexpr int kStoreAny = 0, kStorePlain = 1, kStoreReluSqFrag = 2, kStorePartial = 3, kStoreActFrag = 4,
              kStoreRowMajor = 5;

// W consecutive fp16 values, stored or loaded as one access.
template <int W>
struct alignas(2 * W) HW {
  _Float16 v[W];
};

// Epilogue and store of W consecutive output columns (col % W == 0, W = 4 or
// 8: a group never straddles a frag chunk or the row end, n being a multiple
// of 8) of one row.
template <int kStore, int W>
__device__ __forceinline__ void store_cols(const float (&s)[W], int row, int col, int n, int npad, int epi,
                                           int c_frag, _Float16* pc, const _Float16* pv, const _Float16* pvf,
                                           const _Float16* pv0) {
  typedef HW<W> hw;
  hw o;
  if constexpr (kStore == kStoreReluSqFrag) {
#pragma unroll
    for (int e = 0; e < W; ++e) {
      const float x = fmaxf(s[e], 0.0f);
      o.v[e] = (_Float16)(x * x);
    }
    *reinterpret_cast<hw*>(pc + frag_index(row, col, npad)) = o;
    return;
  }
  if constexpr (kStore == kStorePlain) {
    if (col >= n) return;
#pragma unroll
    for (int e = 0; e < W; ++e) o.v[e] = (_Float16)s[e];
    *reinterpret_cast<hw*>(pc + (int64_t)row * n + col) = o;
    return;
  }
  if (kStore != kStoreRowMajor && c_frag) {
#pragma unroll
    for (int e = 0; e < W; ++e) o.v[e] = (_Float16)apply_act(epi, s[e]);
    *reinterpret_cast<hw*>(pc + frag_index(row, col, npad)) = o;
    return;
  }
  if (col >= n) return;
  const int64_t idx = (int64_t)row * n + col;
  if constexpr (kStore == kStoreActFrag) {  // row-major outputs of this batch are plain
#pragma unroll
    for (int e = 0; e < W; ++e) o.v[e] = (_Float16)s[e];
    *reinterpret_cast<hw*>(pc + idx) = o;
    return;
  }
  if (epi == VKWR_GEMM_EPI_VALUE_RESIDUAL) {
    const hw vv = *reinterpret_cast<const hw*>(pv + idx), vf = *reinterpret_cast<const hw*>(pvf + idx),
             v0 = *reinterpret_cast<const hw*>(pv0 + col);
#pragma unroll
    for (int e = 0; e < W; ++e) {
      const float x = (float)vv.v[e];
      const float gate = sigmoidf((float)v0.v[e] + s[e]);
      o.v[e] = f16_of(__builtin_fmaf((float)vf.v[e] - x, gate, x));
    }
  } else if (epi == VKWR_GEMM_EPI_BIAS) {
    const hw v0 = *reinterpret_cast<const hw*>(pv0 + col);
#pragma unroll
    for (int e = 0; e < W; ++e) o.v[e] = (_Float16)(s[e] + (float)v0.v[e]);
  } else if (kStore == kStoreRowMajor) {  // none (activations only come with frag outputs here)
#pragma unroll
    for (int e = 0; e < W; ++e) o.v[e] = (_Float16)s[e];
  } else {
#pragma unroll
    for (int e = 0; e < W; ++e) o.v[e] = (_Float16)apply_act(epi, s[e]);
  }
  *reinterpret_cast<hw*>(pc + idx) = o;
}

template <int TM, int TN, int NW, int KS, int kStore, bool kMulti>
__global__ __launch_bounds__(NW * 64) void frag_gemm_kernel(FBatch bt) {
  constexpr int kTiles = TM * TN;
  __shared__ __attribute__((aligned(16))) float red[NW * kTiles * 1024];

  // ---- problem and tile of this workgroup (uniform).  Every field the
  // workgroup uses is read into a register here, before the first branch (the
  // empty asm pins the loads above it): the compiler otherwise sinks each field
  // load below the branch that precedes its first use, and each dependent
  // kernel-argument round trip delays the first operand load by ~0.3 us.  A
  // single-problem launch needs that one round; a batch first finds its
  // problem among the first-workgroup ids (one more round).  The problems of a
  // batch own consecutive workgroup ranges: with one grid row per problem
  // instead, the small problems' empty slots queue behind the large ones'
  // one-workgroup-per-CU tiles.
  int pi = 0;
  if constexpr (kMulti) {
#pragma unroll
    for (int i = 1; i < kMaxFragProblems; ++i)
      if (i < bt.n && (int)blockIdx.x >= bt.p[i].wg_begin) pi = i;
  }
  const FProb& Pr = bt.p[pi];
  const _Float16* const pa = Pr.a;
  const _Float16* const pb = Pr.b;
  _Float16* const pc = Pr.c;
  const _Float16 *const pv = Pr.v, *const pvf = Pr.vf, *const pv0 = Pr.v0;
  const int m = Pr.m, n = Pr.n, npad = Pr.npad, kpad = Pr.kpad, epi = Pr.epi, c_frag = Pr.c_frag;
  const int ncol = Pr.ncol, nmb = Pr.nmb, xcd_map = Pr.xcd_map, wg_begin = Pr.wg_begin;
  float* const ws = Pr.ws;
  const int ksplit = kStore == kStorePartial ? Pr.ksplit : 1;
  asm volatile("" ::"s"(pa), "s"(pb), "s"(pc), "s"(pv), "s"(pvf), "s"(pv0), "s"(m), "s"(n), "s"(npad), "s"(kpad),
               "s"(epi), "s"(c_frag), "s"(ncol), "s"(nmb), "s"(xcd_map), "s"(wg_begin), "s"(ws), "s"(ksplit));
  const int lt = (int)blockIdx.x - wg_begin;
  if (lt >= ncol * nmb * ksplit) return;  // round-up workgroup
  // Tile and K part.  With the XCD map, the K parts and row tiles of a column
  // tile get ids that differ by multiples of 8 (one L2).
  int cb, mb, part;
  if (xcd_map) {
    const int x = lt & 7, t = lt >> 3;
    part = t % ksplit;
    const int u = t / ksplit;
    cb = (u / nmb) * 8 + x;
    mb = u % nmb;
  } else {
    part = lt % ksplit;
    const int u = lt / ksplit;
    cb = u / nmb;
    mb = u % nmb;
  }

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t kstep = kpad >> 4;             // 16-k steps per 32-row block
  const int64_t k0 = part * (kstep / ksplit);  // first 16-k step of this K part
  const _Float16* ap[TM];
  const _Float16* bp[TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) ap[i] = pa + (((int64_t)(mb * TM + i) * kstep + k0) * 64 + lane) * 8;
#pragma unroll
  for (int j = 0; j < TN; ++j) bp[j] = pb + (((int64_t)(cb * TN + j) * kstep + k0) * 64 + lane) * 8;

  fv16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int nper = kpad / ksplit / (16 * KS * NW);  // k blocks per wave (host guarantees >= 1, exact)
  hv8 fa[2][KS][TM], fb[2][KS][TN];
  auto load = [&](int buf, int j) {
    const int64_t o = (int64_t)(wave + NW * j) * KS * 512;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int jj = 0; jj < TN; ++jj) fb[buf][s][jj] = *reinterpret_cast<const hv8*>(bp[jj] + o + s * 512);
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[buf][s][i] = *reinterpret_cast<const hv8*>(ap[i] + o + s * 512);
    }
  };
  auto compute = [&](int buf) {
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[buf][s][i], fb[buf][s][j], acc[i][j], 0, 0, 0);
  };
  // The scheduling barriers keep each prefetch ahead of the MFMAs that do not
  // need it (left alone, the scheduler sinks the loads below them).
  // Every load inside the loop is unconditional (a conditional prefetch makes
  // the compiler wait for all outstanding loads); the last one or two blocks
  // are peeled after it, so no block is loaded twice.
  load(0, 0);
  int jb = 0;
  for (; jb + 2 < nper; jb += 2) {
    load(1, jb + 1);
    __builtin_amdgcn_sched_barrier(0);
    compute(0);
    __builtin_amdgcn_sched_barrier(0);
    load(0, jb + 2);
    __builtin_amdgcn_sched_barrier(0);
    compute(1);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (jb + 1 < nper) {
    load(1, jb + 1);
    __builtin_amdgcn_sched_barrier(0);
    compute(0);
    __builtin_amdgcn_sched_barrier(0);
    compute(1);
  } else {
    compute(0);
  }

  // ---- reduce the NW partial tiles in wave order, then 8 columns per thread
#pragma unroll
  for (int t = 0; t < kTiles; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) red[((wave * kTiles + t) * 16 + r) * 64 + lane] = acc[t / TN][t % TN][r];
  __syncthreads();
  constexpr int kGroups = kTiles * 16 * 8;
  for (int g = threadIdx.x; g < kGroups; g += NW * 64) {
    const int t = g >> 7, r = (g >> 3) & 15, l0 = (g & 7) * 8;
    // Two 16-byte LDS reads per wave partial, all issued before the adds (read
    // element by element, the compiler split them into dependent 4- and
    // 12-byte reads).
    f4 s0 = *reinterpret_cast<const f4*>(&red[(t * 16 + r) * 64 + l0]);
    f4 s1 = *reinterpret_cast<const f4*>(&red[(t * 16 + r) * 64 + l0 + 4]);
#pragma unroll
    for (int w = 1; w < NW; ++w) {
      s0 += *reinterpret_cast<const f4*>(&red[((w * kTiles + t) * 16 + r) * 64 + l0]);
      s1 += *reinterpret_cast<const f4*>(&red[((w * kTiles + t) * 16 + r) * 64 + l0 + 4]);
    }
    const int i = t / TN, j = t % TN;
    const int row = (mb * TM + i) * 32 + 8 * (r >> 2) + 4 * (l0 >> 5) + (r & 3);
    const int col = (cb * TN + j) * 32 + (l0 & 31);
    if constexpr (kStore == kStorePartial) {
      float* const o = ws + ((int64_t)part * nmb * (32 * TM) + row) * npad + col;
      *reinterpret_cast<f4*>(o) = s0;
      *reinterpret_cast<f4*>(o + 4) = s1;
      continue;
    }
    if (row >= m) continue;
    const float s[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    store_cols<kStore, 8>(s, row, col, n, npad, epi, c_frag, pc, pv, pvf, pv0);
  }
}

// Adds the ksplit fp32 partial planes of a K-split GEMM in increasing K order
// and applies the epilogue: one thread per 4 consecutive columns of a row (a
// 128-row decode batch fills 256 workgroups).
__global__ __launch_bounds__(256) void frag_splitk_reduce_kernel(FProb P, int mrows) {
  const int groups = P.npad >> 2;
  const int g = blockIdx.x * 256 + threadIdx.x;
  if (g >= P.m * groups) return;
  const int row = g / groups, col = (g - row * groups) * 4;
  const int64_t plane = (int64_t)mrows * P.npad;
  const float* p = P.ws + (int64_t)row * P.npad + col;
  f4 a = *reinterpret_cast<const f4*>(p);
  for (int q = 1; q < P.ksplit; ++q) a += *reinterpret_cast<const f4*>(p + q * plane);
  const float s[4] = {a.x, a.y, a.z, a.w};
  store_cols<kStoreAny, 4>(s, row, col, P.n, P.npad, P.epi, P.c_frag, P.c, P.v, P.vf, P.v0);
}

// ---------------------------------------------------------------- packing

__global__ __launch_bounds__(256) void frag_pack_kernel(int64_t rows, int64_t k, const _Float16* src, int kn,
                                                        int64_t kpad, int64_t nchunks, int vec,
                                                        _Float16* dst) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t ci = (int64_t)blockIdx.x * 256 + threadIdx.x; ci < nchunks; ci += stride) {
    const int lane = (int)(ci & 63);
    const int64_t fs = ci >> 6;
    const int64_t rb = fs / (kpad >> 4), ks = fs % (kpad >> 4);
    const int64_t r = rb * 32 + (lane & 31);
    const int64_t k0 = ks * 16 + (lane >> 5) * 8;
    h8 o;
    if (!kn && vec && r < rows && k0 + 8 <= k) {
      o = ld8(src + r * k + k0);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t kk = k0 + e;
        o.v[e] = (r < rows && kk < k) ? (kn ? src[kk * rows + r] : src[r * k + kk]) : (_Float16)0.0f;
      }
    }
    st8(dst + ci * 8, o);
  }
}

__global__ __launch_bounds__(256) void frag_unpack_kernel(int64_t rows, int64_t k, const _Float16* src,
                                                          int64_t kpad, _Float16* dst) {
  const int64_t n = rows * k;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    const int64_t r = i / k, kk = i % k;
    dst[i] = src[frag_index(r, kk, kpad)];
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

unsigned grid_blocks(int64_t work) {
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>((work + 255) / 256, 8192));
}

// ---------------------------------------------------------------- dispatch

struct FragConfig {
  int tm, tn, nw, ks;
};

int tiles_for(const FBatch& bt, int bm, int bn) {
  int t = 0;
  for (int i = 0; i < bt.n; ++i) t += (bt.p[i].m + bm - 1) / bm * (bt.p[i].npad / bn);
  return t;
}

// One configuration per launch.  Large batches of tiles take 128 x 64 tiles;
// medium ones 64 x 64; small ones (fewer than 128 such tiles: too few
// workgroups for 256 CUs) 32 x 32 with more K per block.
FragConfig pick_frag_config(const FBatch& bt) {
  int max_m = 0;
  int64_t kdiv = 0;  // gcd of the padded K
  for (int i = 0; i < bt.n; ++i) {
    max_m = std::max(max_m, bt.p[i].m);
    int64_t a = kdiv, b = bt.p[i].kpad;
    while (b) { const int64_t t = a % b; a = b; b = t; }
    kdiv = a;
  }
  auto ks_for = [&](int nw, int ks_max) {
    int ks = ks_max;
    while (ks > 1 && kdiv % (16 * ks * nw) != 0) ks /= 2;
    return ks;
  };
  if (max_m <= 32) {
    if (tiles_for(bt, 32, 64) >= 128) return {1, 2, 8, ks_for(8, 2)};
    return {1, 1, 8, ks_for(8, 4)};
  }
  const int t64 = tiles_for(bt, 64, 64);
  if (t64 >= 1024) return {4, 2, 4, 2};
  if (t64 >= 128) return {2, 2, 8, ks_for(8, 2)};
  return {1, 1, 8, ks_for(8, 4)};
}

// One workgroup range per problem, each a multiple of 8 long (so a tile's id
// mod 8 is its XCD).
template <int TM, int TN, int NW, int KS>
void launch_cfg(const FBatch& bt, int wgs, hipStream_t s) {
  bool relu_sq_frag = true, plain = true, act_frag = true, row_major = true;
  for (int i = 0; i < bt.n; ++i) {
    const FProb& P = bt.p[i];
    relu_sq_frag = relu_sq_frag && P.c_frag && P.epi == VKWR_GEMM_EPI_RELU_SQUARE;
    plain = plain && !P.c_frag && P.epi == VKWR_GEMM_EPI_NONE;
    act_frag = act_frag && (P.c_frag ? (P.epi == VKWR_GEMM_EPI_NONE || P.epi == VKWR_FRAG_EPI_TANH ||
                                        P.epi == VKWR_FRAG_EPI_SIGMOID)
                                     : P.epi == VKWR_GEMM_EPI_NONE);
    row_major = row_major && !P.c_frag &&
                (P.epi == VKWR_GEMM_EPI_NONE || P.epi == VKWR_GEMM_EPI_BIAS || P.epi == VKWR_GEMM_EPI_VALUE_RESIDUAL);
  }
  const dim3 grid(wgs), block(NW * 64);
  if (bt.n > 1 && act_frag)
    hipLaunchKernelGGL((frag_gemm_kernel<TM, TN, NW, KS, kStoreActFrag, true>), grid, block, 0, s, bt);
  else if (bt.n > 1 && row_major)
    hipLaunchKernelGGL((frag_gemm_kernel<TM, TN, NW, KS, kStoreRowMajor, true>), grid, block, 0, s, bt);
  else if (bt.n > 1)
    hipLaunchKernelGGL((frag_gemm_kernel<TM, TN, NW, KS, kStoreAny, true>), grid, block, 0, s, bt);
  else if (relu_sq_frag)
    hipLaunchKernelGGL((frag_gemm_kernel<TM, TN, NW, KS, kStoreReluSqFrag, false>), grid, block, 0, s, bt);
  else if (plain)
    hipLaunchKernelGGL((frag_gemm_kernel<TM, TN, NW, KS, kStorePlain, false>), grid, block, 0, s, bt);
  else
    hipLaunchKernelGGL((frag_gemm_kernel<TM, TN, NW, KS, kStoreAny, false>), grid, block, 0, s, bt);
}

int launch_frag(const FBatch& bt, FragConfig c, int wgs, hipStream_t s) {
#define VK_FRAG_CASE(a, b_, c_, d)                                        \
  if (c.tm == a && c.tn == b_ && c.nw == c_ && c.ks == d) {               \
    launch_cfg<a, b_, c_, d>(bt, wgs, s);                                 \
    return VKWR_OK;                                                       \
  }
  VK_FRAG_CASE(4, 2, 4, 2)
  VK_FRAG_CASE(2, 2, 8, 2)
  VK_FRAG_CASE(2, 2, 8, 1)
  VK_FRAG_CASE(1, 1, 8, 4)
  VK_FRAG_CASE(1, 1, 8, 2)
  VK_FRAG_CASE(1, 1, 8, 1)
  VK_FRAG_CASE(1, 2, 8, 2)
  VK_FRAG_CASE(1, 2, 8, 1)
#undef VK_FRAG_CASE
  set_error("vkwr_frag_gemm_f16: no kernel for tile config %dx%dx%dx%d", c.tm, c.tn, c.nw, c.ks);
  return VKWR_ERR_INVALID;
}

}  // namespace
}  // namespace vk

using namespace vk;

extern "C" int vkwr_frag_pack_f16(int64_t rows, int64_t k, const uint16_t* src, int src_layout,
                                  uint16_t* dst, void* stream) {
  clear_error();
  const char* fn = "vkwr_frag_pack_f16";
  VK_REQUIRE(rows >= 0 && k >= 0, "%s: negative size", fn);
  VK_REQUIRE(src_layout == VKWR_GEMM_B_NK || src_layout == VKWR_GEMM_B_KN, "%s: bad src_layout", fn);
  if (rows == 0 || k == 0) return VKWR_OK;
  VK_REQUIRE(src && dst, "%s: null pointer", fn);
  VK_REQUIRE(aligned16(dst), "%s: dst must be 16-byte aligned", fn);
  const int64_t kpad = frag_pad(k), rpad = frag_pad(rows);
  const int64_t nchunks = rpad * kpad / 8;
  const int vec = src_layout == VKWR_GEMM_B_NK && k % 8 == 0 && aligned16(src);
  hipLaunchKernelGGL(frag_pack_kernel, dim3(grid_blocks(nchunks)), dim3(256), 0, (hipStream_t)stream, rows, k,
                     reinterpret_cast<const _Float16*>(src), src_layout == VKWR_GEMM_B_KN, kpad, nchunks, vec,
                     reinterpret_cast<_Float16*>(dst));
  return check_launch(fn);
}

extern "C" int vkwr_frag_unpack_f16(int64_t rows, int64_t k, const uint16_t* src, uint16_t* dst,
                                    void* stream) {
  clear_error();
  const char* fn = "vkwr_frag_unpack_f16";
  VK_REQUIRE(rows >= 0 && k >= 0, "%s: negative size", fn);
  if (rows == 0 || k == 0) return VKWR_OK;
  VK_REQUIRE(src && dst, "%s: null pointer", fn);
  hipLaunchKernelGGL(frag_unpack_kernel, dim3(grid_blocks(rows * k)), dim3(256), 0, (hipStream_t)stream, rows, k,
                     reinterpret_cast<const _Float16*>(src), frag_pad(k), reinterpret_cast<_Float16*>(dst));
  return check_launch(fn);
}

namespace {

// Validates one problem and fills its kernel descriptor (sizes, pointers,
// epilogue); tiling fields are set by the caller.
int fill_problem(const char* fn, int i, const vkwr_frag_gemm_problem& q, FProb& P, bool& empty,
                 bool need_c = true) {
  VK_REQUIRE(q.m >= 0 && q.n >= 0 && q.k >= 0, "%s: negative size in problem %d", fn, i);
  VK_REQUIRE(q.m <= (1 << 20) && q.n <= (1 << 24) && q.k <= (1 << 20), "%s: problem %d too large", fn, i);
  VK_REQUIRE(q.epilogue >= VKWR_GEMM_EPI_NONE && q.epilogue <= VKWR_FRAG_EPI_SIGMOID, "%s: bad epilogue", fn);
  VK_REQUIRE(q.c_frag == 0 || q.c_frag == 1, "%s: bad c_frag", fn);
  empty = q.m == 0 || q.n == 0;
  if (empty) return VKWR_OK;
  VK_REQUIRE(q.k > 0, "%s: k == 0 in problem %d", fn, i);
  VK_REQUIRE(q.a && q.b && (q.c || !need_c), "%s: null pointer in problem %d", fn, i);
  VK_REQUIRE(aligned16(q.a) && aligned16(q.b) && aligned16(q.c), "%s: operands must be 16-byte aligned", fn);
  if (q.c_frag) {
    VK_REQUIRE(q.epilogue != VKWR_GEMM_EPI_VALUE_RESIDUAL && q.epilogue != VKWR_GEMM_EPI_BIAS,
               "%s: value-residual / bias epilogues need a row-major output", fn);
  } else {
    VK_REQUIRE(q.n % 8 == 0, "%s: row-major output needs n %% 8 == 0 (problem %d)", fn, i);
  }
  if (q.epilogue == VKWR_GEMM_EPI_VALUE_RESIDUAL) {
    VK_REQUIRE(q.v && q.v_first && q.v0, "%s: value-residual epilogue needs v, v_first, v0", fn);
    VK_REQUIRE(aligned16(q.v) && aligned16(q.v_first) && aligned16(q.v0), "%s: epilogue operands alignment", fn);
  }
  if (q.epilogue == VKWR_GEMM_EPI_BIAS) {
    VK_REQUIRE(q.v0 && aligned16(q.v0), "%s: bias epilogue needs an aligned v0", fn);
  }
  P = FProb{};
  P.a = reinterpret_cast<const _Float16*>(q.a);
  P.b = reinterpret_cast<const _Float16*>(q.b);
  P.c = reinterpret_cast<_Float16*>(q.c);
  P.v = reinterpret_cast<const _Float16*>(q.v);
  P.vf = reinterpret_cast<const _Float16*>(q.v_first);
  P.v0 = reinterpret_cast<const _Float16*>(q.v0);
  P.m = (int)q.m;
  P.n = (int)q.n;
  P.npad = (int)frag_pad(q.n);
  P.kpad = (int)frag_pad(q.k);
  P.epi = q.epilogue;
  P.c_frag = q.c_frag;
  P.ksplit = 1;
  return VKWR_OK;
}

// The K-split GEMM runs on 64 x 64 tiles, 8 waves, two 16-k steps per load.
constexpr int kSplitTile = 64, kSplitKRound = 16 * 2 * 8;

}  // namespace

extern "C" int vkwr_frag_gemm_f16(int n_problems, const vkwr_frag_gemm_problem* problems, void* stream) {
  clear_error();
  const char* fn = "vkwr_frag_gemm_f16";
  VK_REQUIRE(n_problems >= 1 && n_problems <= kMaxFragProblems, "%s: 1..%d problems per launch (got %d)", fn,
             kMaxFragProblems, n_problems);
  VK_REQUIRE(problems != nullptr, "%s: null problem list", fn);
  FBatch bt;
  bt.n = 0;
  for (int i = 0; i < n_problems; ++i) {
    bool empty = false;
    if (int e = fill_problem(fn, i, problems[i], bt.p[bt.n], empty)) return e;
    if (!empty) ++bt.n;
  }
  if (bt.n == 0) return VKWR_OK;
  const FragConfig cfg = pick_frag_config(bt);
  const int bm = 32 * cfg.tm, bn = 32 * cfg.tn;
  int wgs = 0;
  for (int i = 0; i < bt.n; ++i) {
    FProb& P = bt.p[i];
    VK_REQUIRE(P.kpad % (16 * cfg.ks * cfg.nw) == 0, "%s: internal: K split", fn);
    P.ncol = P.npad / bn;
    P.nmb = (P.m + bm - 1) / bm;
    P.xcd_map = P.nmb > 1 && P.ncol % 8 == 0;
    P.wg_begin = wgs;
    wgs += (P.ncol * P.nmb + 7) / 8 * 8;
  }
  if (int e = launch_frag(bt, cfg, wgs, (hipStream_t)stream)) return e;
  return check_launch(fn);
}

extern "C" int64_t vkwr_frag_gemm_splitk_workspace_bytes(int64_t m, int64_t n, int splits) {
  if (m <= 0 || n <= 0 || splits < 1) return 0;
  return (int64_t)splits * ((m + kSplitTile - 1) / kSplitTile * kSplitTile) * frag_pad(n) * (int64_t)sizeof(float);
}

namespace {

// Validates a K-split problem and launches its partial-tile kernel.
int splitk_partials(const char* fn, const vkwr_frag_gemm_problem* problem, int splits, void* workspace,
                    int64_t workspace_bytes, bool need_c, FBatch& bt, bool& empty, hipStream_t stream) {
  VK_REQUIRE(problem != nullptr, "%s: null problem", fn);
  VK_REQUIRE(splits >= 1 && splits <= 16, "%s: splits must be in 1..16 (got %d)", fn, splits);
  bt.n = 1;
  if (int e = fill_problem(fn, 0, *problem, bt.p[0], empty, need_c)) return e;
  if (empty) return VKWR_OK;
  FProb& P = bt.p[0];
  VK_REQUIRE(P.kpad % (kSplitKRound * splits) == 0, "%s: padded k (%d) must be a multiple of %d * splits", fn,
             P.kpad, kSplitKRound);
  const int64_t need = vkwr_frag_gemm_splitk_workspace_bytes(P.m, P.n, splits);
  VK_REQUIRE(workspace != nullptr && aligned16(workspace), "%s: workspace must be non-null and 16-byte aligned", fn);
  VK_REQUIRE(workspace_bytes >= need, "%s: workspace of %lld bytes, %lld needed", fn, (long long)workspace_bytes,
             (long long)need);
  P.ncol = P.npad / kSplitTile;
  P.nmb = (P.m + kSplitTile - 1) / kSplitTile;
  P.xcd_map = P.ncol % 8 == 0;
  P.wg_begin = 0;
  P.ws = static_cast<float*>(workspace);
  P.ksplit = splits;
  const int wgs = (P.ncol * P.nmb * splits + 7) / 8 * 8;
  hipLaunchKernelGGL((frag_gemm_kernel<2, 2, 8, 2, kStorePartial, false>), dim3(wgs), dim3(512), 0, stream, bt);
  return VKWR_OK;
}

}  // namespace

extern "C" int vkwr_frag_gemm_splitk_f16(const vkwr_frag_gemm_problem* problem, int splits, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
  clear_error();
  const char* fn = "vkwr_frag_gemm_splitk_f16";
  FBatch bt;
  bool empty = false;
  if (int e = splitk_partials(fn, problem, splits, workspace, workspace_bytes, true, bt, empty, (hipStream_t)stream))
    return e;
  if (empty) return VKWR_OK;
  const FProb& P = bt.p[0];
  const int64_t threads = (int64_t)P.m * (P.npad / 4);
  hipLaunchKernelGGL(frag_splitk_reduce_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, P, P.nmb * kSplitTile);
  return check_launch(fn);
}

extern "C" int vkwr_frag_gemm_splitk_parts_f16(const vkwr_frag_gemm_problem* problem, int splits, void* workspace,
                                               int64_t workspace_bytes, void* stream) {
  clear_error();
  const char* fn = "vkwr_frag_gemm_splitk_parts_f16";
  VK_REQUIRE(problem != nullptr, "%s: null problem", fn);
  VK_REQUIRE(problem->epilogue == VKWR_GEMM_EPI_NONE && problem->c_frag == 0,
             "%s: the parts carry no epilogue (epilogue NONE, c_frag 0)", fn);
  FBatch bt;
  bool empty = false;
  if (int e = splitk_partials(fn, problem, splits, workspace, workspace_bytes, false, bt, empty, (hipStream_t)stream))
    return e;
  return empty ? VKWR_OK : check_launch(fn);
}
