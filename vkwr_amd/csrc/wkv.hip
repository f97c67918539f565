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

#include <algorithm>

#include "vk_capi.h"
#include "vk_common.cuh"

namespace vk {
namespace {

typedef _Float16 hv8 __attribute__((ext_vector_type(8)));

struct Fp32Args {
  int T, C, H, n_slots;
  float* state;
  const int32_t* slots;
  const _Float16 *r, *w, *k, *v, *a, *b;
  _Float16* y;
};

// Kernel-argument pinning.  Left alone the compiler requested a kernel's arguments in
// dependent rounds of scalar loads around the slot lookup -- four before a decode step's
// state load, each ~0.3 us on every wave's path.  Passing every field through an empty asm
// above the first branch makes every later use wait on one round.  The asm is not volatile
// and names no memory, so the slot lookup after it still counts as unclobbered and stays a
// scalar load (a volatile asm may write memory: the lookup then became a vector load, slower
// than the rounds it saved).  A pointer that comes out of an asm has lost its address space;
// passing it through as a global-space pointer keeps its loads and stores global rather
// than flat ones.
template <class T>
__device__ __forceinline__ void pin_ptr(T*& ptr) {
  auto g = (__attribute__((address_space(1))) T*)ptr;
  asm("" : "+s"(g));
  ptr = (T*)g;
}
__device__ __forceinline__ void pin_int(int& x) { asm("" : "+s"(x)); }

__device__ __forceinline__ void pin_args(Fp32Args& p) {
  pin_int(p.T), pin_int(p.C), pin_int(p.H), pin_int(p.n_slots);
  pin_ptr(p.state), pin_ptr(p.slots), pin_ptr(p.r), pin_ptr(p.w), pin_ptr(p.k), pin_ptr(p.v);
  pin_ptr(p.a), pin_ptr(p.b), pin_ptr(p.y);
}

// ---- fp32 state staging: HBM <-> LDS (swizzled) <-> VGPRs, one column half
// per phase (see the State I/O note above).  `st` is the 8 KiB tile.  kNT: the
// state is loaded and stored with the non-temporal cache policy.
template <bool kNT = false>
__device__ __forceinline__ void load_state_fp32(const float* S, f4* st, float* s, int lane) {
  const int sub = lane & 7;
#pragma unroll
  for (int ph = 0; ph < 2; ++ph) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int row = 8 * c + (lane >> 3);
      if constexpr (kNT) dma16_nt(S + row * kHead + ph * 32 + (sub ^ (row & 7)) * 4, &st[c * 64]);
      else dma16(S + row * kHead + ph * 32 + (sub ^ (row & 7)) * 4, &st[c * 64]);
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

template <bool kNT = false>
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
      f4* const dst = reinterpret_cast<f4*>(S + row * kHead + ph * 32 + (sub ^ (row & 7)) * 4);
      if constexpr (kNT) __builtin_nontemporal_store(st[c * 64 + lane], dst);
      else *dst = st[c * 64 + lane];
    }
    __syncthreads();
  }
}

// One token of the fp32-state recurrence for row `lane` (state row in s[]),
// in two parts: token_stage writes the token's channel vectors (r, decay, k,
// a, b; one channel per lane) to vb (5*64 floats of LDS), token_run reads them
// back as broadcasts after a barrier.
__device__ __forceinline__ void token_stage(float* vb, int lane, _Float16 xr, _Float16 xw, _Float16 xk,
                                            _Float16 xa, _Float16 xb) {
  vb[lane] = (float)xr;
  vb[kHead + lane] = decay((float)xw);
  vb[2 * kHead + lane] = (float)xk;
  vb[3 * kHead + lane] = (float)xa;
  vb[4 * kHead + lane] = (float)xb;
}

__device__ __forceinline__ _Float16 token_run(float* s, const float* vb, float vi) {
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

__device__ __forceinline__ _Float16 token_fp32(float* s, float* vb, int lane, _Float16 xr,
                                               _Float16 xw, _Float16 xk, _Float16 xv,
                                               _Float16 xa, _Float16 xb) {
  token_stage(vb, lane, xr, xw, xk, xa, xb);
  __syncthreads();
  return token_run(s, vb, (float)xv);
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
// latency overlaps the state transfer.  kNT: non-temporal state loads and
// stores, for state tables larger than the memory-side cache (a step's slots
// are then unlikely to be cached when next visited, and the stores would only
// evict other lines): cold 64 MiB read-modify-write measures 26 us with them
// against 31 us without, while a cache-resident set is faster without them
// (21 us against 24 us).
template <bool kSlots, bool kNT>
__global__ __launch_bounds__(64, 4) void wkv7_fp32_step_kernel(Fp32Args p) {
  __shared__ f4 st[512];
  pin_args(p);
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
  load_state_fp32<kNT>(S, st, s, lane);
  p.y[tok] = token_fp32(s, reinterpret_cast<float*>(st), lane, xr, xw, xk, xv, xa, xb);
  store_state_fp32<kNT>(S, st, s, lane);
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

// The same recurrence and order for T > 1 when the (sequence, head) chains are few (at most
// one wave per SIMD), scheduled for a lone wave whose latency nothing else hides.  Every
// value is computed as in wkv7_fp32_seq_kernel; what moves is when:
//  - token t+1's sa chain (sum over j of s[j] * a_{t+1}[j], in j order, on the state just
//    updated by token t) runs inside token t's update loop beside the y chain, column by
//    column, instead of alone at the start of token t+1;
//  - the token vectors are read from LDS eight columns ahead of their use (the compiler
//    would otherwise issue each read just before the FMAs that consume it);
//  - the loop body has no branch (token indices past the end are clamped, the values
//    they stage are never used), the decay of token t+2 is computed among the FMAs, and
//    inputs are fetched three tokens ahead, two tokens per loop trip with two register sets.
template <bool kSlots>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 1))) void wkv7_fp32_seq_lat_kernel(
    Fp32Args p) {
  __shared__ f4 st[512];
  const int lane = threadIdx.x;
  const int bh = blockIdx.x;
  const int bi = bh / p.H;
  const int h = bh - bi * p.H;
  const int T = p.T;
  const size_t tok0 = (size_t)bi * T * p.C + (size_t)h * kHead + lane;
  float* S = state_block<kSlots>(p, bi, h);
  if (S == nullptr) {
    for (int t = 0; t < T; ++t) p.y[tok0 + (size_t)t * p.C] = (_Float16)__builtin_nanf("");
    return;
  }
  struct Tok {
    _Float16 r, w, k, v, a, b;
  };
  auto fetch = [&](int t) {
    const size_t o = tok0 + (size_t)(t < T ? t : T - 1) * p.C;
    return Tok{p.r[o], p.w[o], p.k[o], p.v[o], p.a[o], p.b[o]};
  };
  const Tok x0 = fetch(0), x1 = fetch(1);
  Tok x2 = fetch(2);
  float s[kHead];
  load_state_fp32(S, st, s, lane);
  float* vec = reinterpret_cast<float*>(st);
  auto stage = [&](int buf, const Tok& x, float d) {
    float* vb = vec + buf * (5 * kHead);
    vb[lane] = (float)x.r;
    vb[kHead + lane] = d;
    vb[2 * kHead + lane] = (float)x.k;
    vb[3 * kHead + lane] = (float)x.a;
    vb[4 * kHead + lane] = (float)x.b;
  };
  stage(0, x0, decay((float)x0.w));
  stage(1, x1, decay((float)x1.w));
  float v_cur = (float)x0.v, v_next = (float)x1.v;
  __syncthreads();
  float sa = 0.0f;
  {
    const f4* A4 = reinterpret_cast<const f4*>(vec) + 48;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const f4 a4 = A4[q];
      sa = __builtin_fmaf(s[4 * q + 0], a4.x, sa);
      sa = __builtin_fmaf(s[4 * q + 1], a4.y, sa);
      sa = __builtin_fmaf(s[4 * q + 2], a4.z, sa);
      sa = __builtin_fmaf(s[4 * q + 3], a4.w, sa);
    }
  }

  // one token: xs holds token t+2's inputs (fetched an iteration ago), xl receives t+3's
  auto token = [&](int t, const Tok& xs, Tok& xl) {
    xl = fetch(t + 3);
    const int cb = t & 1;
    const f4* V4 = reinterpret_cast<const f4*>(vec + cb * (5 * kHead));
    const f4* An4 = reinterpret_cast<const f4*>(vec + (cb ^ 1) * (5 * kHead)) + 48;
    const float vi = v_cur;
    float acc = 0.0f, sn = 0.0f, d2 = 0.0f;
    // group g: columns 8g .. 8g+7 (two f4 of each vector)
    f4 R[2][2], D[2][2], K[2][2], Bv[2][2], A[2][2];
    auto rd = [&](int g, int set) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int q = 2 * g + u;
        R[set][u] = V4[q];
        D[set][u] = V4[16 + q];
        K[set][u] = V4[32 + q];
        Bv[set][u] = V4[64 + q];
        A[set][u] = An4[q];
      }
    };
    rd(0, 0);
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const int set = g & 1;
      if (g + 1 < 8) rd(g + 1, set ^ 1);
      if (g == 2) d2 = decay((float)xs.w);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = 8 * g + 4 * u + e;
          float x = s[j] * D[set][u][e];
          x = __builtin_fmaf(sa, Bv[set][u][e], x);
          x = __builtin_fmaf(K[set][u][e], vi, x);
          s[j] = x;
          acc = __builtin_fmaf(x, R[set][u][e], acc);
          sn = __builtin_fmaf(x, A[set][u][e], sn);
        }
      __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("" : "+v"(acc));
    p.y[tok0 + (size_t)t * p.C] = (_Float16)acc;
    sa = sn;
    // every lane has read buffer cb (single-wave workgroup): token t+2 replaces token t
    __syncthreads();
    stage(cb, xs, d2);
    v_cur = v_next;
    v_next = (float)xs.v;
    __syncthreads();
  };
  Tok x3;
  int t = 0;
  for (; t + 1 < T; t += 2) {
    token(t, x2, x3);
    token(t + 1, x3, x2);
  }
  if (t < T) token(t, x2, x3);
  __syncthreads();
  store_state_fp32(S, st, s, lane);
}

// ---- row-split prefill (T > 1): one 256-lane workgroup per (sequence, head).
//
// The rows of the state are independent recurrences; only the two per-row dot
// products couple a row's 64 columns.  So the head's 4096 state values are
// spread over 256 lanes -- wave v owns rows 16v..16v+15, lane (g = lane & 7,
// q = lane >> 3) owns rows 16v+2q and 16v+2q+1 at columns 4g..4g+3 and
// 32+4g..32+4g+3 -- and each dot product is eight 8-term FMA chains (one per
// lane) combined by a DPP butterfly over the eight lanes of the row:
// ((p0+p1)+(p2+p3)) + ((p4+p5)+(p6+p7)) in every lane (IEEE addition commutes,
// so both lanes of each pair hold the same bits).  All four SIMDs of the CU
// work on the head, and a lane issues 16 FMAs per dot product pair instead of 64.
//
// Per token t a lane updates its 16 state values with (decay_t, sa_t, b_t,
// k_t, v_t), then forms y_t = S.r_t and sa_{t+1} = S.a_{t+1} together: both
// read the same updated state, so the four FMA chains (2 rows x 2 vectors)
// and the four butterflies interleave and the dependent latency of one hides
// behind the others.  The arithmetic of every value is unchanged.
//
// Token vectors: the workgroup stages chunks of kRowsTC tokens' r, decay(w),
// k, v, a, b (fp16 in HBM) as fp32 in LDS -- the decay is computed once per
// (token, channel) here instead of once per row group.  Three buffers: chunk
// c is read, chunk c+1 is ready (its first token's a is needed by chunk c's
// last token), chunk c+2 is written at the end of chunk c from registers
// loaded one chunk earlier.  Lanes read their columns as 16-byte LDS reads
// (eight distinct addresses per instruction, 128 contiguous bytes: no bank
// conflicts).  y goes through a per-wave LDS tile and leaves as 8-byte stores
// once per chunk, after the prefetch has landed, so no wait for outstanding
// loads covers freshly issued stores.
constexpr int kRowsTC = 16;    // tokens per staged chunk
constexpr int kRowsVecs = 6;   // r, decay, k, v, a, b
constexpr int kRowsBufs = 3;

// Sum over the 8 lanes 8m..8m+7 (see above); every lane gets the same value.
__device__ __forceinline__ float sum8(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x141, 0xF, 0xF, false));
  return x;
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations
// and joins the workgroup, without the wait for outstanding global loads and
// stores that __syncthreads' fence implies.  The memory clobber keeps the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ---- decode step (T == 1) in the row-split order, without LDS.
//
// One wave per (sequence, head); lane (g = lane & 7, q = lane >> 3) holds rows 8q..8q+7 of the
// state at columns 4g..4g+3 and 32+4g..32+4g+3 (64 values in VGPRs) -- the row-split kernel's
// column ownership, so each dot product is its eight 8-term FMA chains and sum8 butterfly and
// the results are the bits of the row-split order.  Each state load or store instruction covers
// 8 rows x 128 contiguous bytes (8 whole lines), so the state moves straight between HBM and
// registers with no staging tile and no barrier.  Using no LDS, the kernel fits beside the
// chunked prefill kernel (144 KiB of LDS per CU) on the same CUs: a mixed batch runs its
// decode rows on a second stream while the prefill chunks run, the HBM-bound state traffic of
// one hidden under the matrix-core work of the other.  kNT: non-temporal state accesses
// (state tables larger than the memory-side cache).
template <bool kNT>
__global__ __launch_bounds__(64) void wkv7_fp32_step_rows_kernel(Fp32Args p) {
  pin_args(p);
  const int lane = threadIdx.x, g = lane & 7, q = lane >> 3;
  const int bh = blockIdx.x;
  const int bi = bh / p.H;
  const int h = bh - bi * p.H;
  const size_t tok = (size_t)bi * p.C + (size_t)h * kHead;
  float* S = state_block<true>(p, bi, h);
  if (S == nullptr) {
    p.y[tok + lane] = (_Float16)__builtin_nanf("");
    return;
  }
  // token vectors: the lane's 8 columns (4 + 4 fp16, 8-byte loads) and its 8 rows of v
  typedef _Float16 hv4 __attribute__((ext_vector_type(4)));
  const int c0 = 4 * g, c1 = 32 + 4 * g;
  auto ld4 = [&](const _Float16* x, int c) { return *reinterpret_cast<const hv4*>(x + tok + c); };
  const hv4 r0 = ld4(p.r, c0), r1 = ld4(p.r, c1), w0 = ld4(p.w, c0), w1 = ld4(p.w, c1);
  const hv4 k0 = ld4(p.k, c0), k1 = ld4(p.k, c1), a0 = ld4(p.a, c0), a1 = ld4(p.a, c1);
  const hv4 b0 = ld4(p.b, c0), b1 = ld4(p.b, c1);
  const hv8 vv = *reinterpret_cast<const hv8*>(p.v + tok + 8 * q);
  f4 st[8][2];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const f4* src = reinterpret_cast<const f4*>(S + (8 * q + i) * kHead + (hf ? c1 : c0));
      st[i][hf] = kNT ? __builtin_nontemporal_load(src) : *src;
    }
  float rr[8], dd[8], kk[8], aa[8], bb[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    rr[e] = (float)r0[e];
    rr[4 + e] = (float)r1[e];
    dd[e] = decay((float)w0[e]);
    dd[4 + e] = decay((float)w1[e]);
    kk[e] = (float)k0[e];
    kk[4 + e] = (float)k1[e];
    aa[e] = (float)a0[e];
    aa[4 + e] = (float)a1[e];
    bb[e] = (float)b0[e];
    bb[4 + e] = (float)b1[e];
  }
  float yv = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float s[8] = {st[i][0].x, st[i][0].y, st[i][0].z, st[i][0].w,
                  st[i][1].x, st[i][1].y, st[i][1].z, st[i][1].w};
    float sa = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) sa = __builtin_fmaf(s[e], aa[e], sa);
    sa = sum8(sa);
    const float vi = (float)vv[i];
    float acc = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x = s[e] * dd[e];
      x = __builtin_fmaf(sa, bb[e], x);
      x = __builtin_fmaf(kk[e], vi, x);
      s[e] = x;
      acc = __builtin_fmaf(x, rr[e], acc);
    }
    acc = sum8(acc);
    yv = g == i ? acc : yv;  // lane g keeps row 8q + g
    st[i][0] = f4{s[0], s[1], s[2], s[3]};
    st[i][1] = f4{s[4], s[5], s[6], s[7]};
  }
  p.y[tok + 8 * q + g] = f16_of(yv);
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      f4* dst = reinterpret_cast<f4*>(S + (8 * q + i) * kHead + (hf ? c1 : c0));
      if constexpr (kNT) __builtin_nontemporal_store(st[i][hf], dst);
      else *dst = st[i][hf];
    }
}

struct RowsArgs {
  Fp32Args a;
  int vec;  // 16-byte aligned r..b and 8-byte aligned y: vector loads/stores
};

// kRPL = state rows per lane.  2: one workgroup per (sequence, head), lanes own rows
// 16 wv + 2 q, +1.  1: two workgroups per (sequence, head), each owning 32 rows
// (32 half + 8 wv + q): rows are independent (sa and y reduce within a row), so the
// halves share nothing but the staged token vectors, which each stages itself.  With
// fewer (sequence, head) pairs than twice the CUs this puts two waves on each SIMD to
// hide the dependent-chain latency of a token step.  Every row sees the same lane
// column mapping and reduction order in both forms, so the results are identical.
template <bool kSlots, int kRPL>
__global__ __launch_bounds__(256) void wkv7_fp32_rows_kernel(RowsArgs ra) {
  const Fp32Args& p = ra.a;
  __shared__ f4 vl[kRowsBufs * kRowsTC * kRowsVecs * 16];  // [buffer][token][vector][16 x f4]
  __shared__ _Float16 ybuf[4][kRowsTC][8][kRPL];            // per wave: 16 tokens x 8 kRPL rows
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int g = lane & 7, q = lane >> 3;
  const int bh = kRPL == 2 ? blockIdx.x : blockIdx.x >> 1;
  const int half = kRPL == 2 ? 0 : blockIdx.x & 1;
  const int i0 = kRPL == 2 ? 16 * wv + 2 * q : 32 * half + 8 * wv + q;
  const int bi = bh / p.H;
  const int h = bh - bi * p.H;
  const int T = p.T;
  const size_t tok0 = (size_t)bi * T * p.C + (size_t)h * kHead;
  float* S = state_block<kSlots>(p, bi, h);
  if (S == nullptr) {
    constexpr int kRows = 32 * kRPL;  // rows of this workgroup
    for (int idx = tid; idx < T * kRows; idx += 256)
      p.y[tok0 + (size_t)(idx / kRows) * p.C + 32 * half + (idx % kRows)] = (_Float16)__builtin_nanf("");
    return;
  }

  // staging: piece c = tid + 256 u (u = 0..2) is vector c >> 7, token (c >> 3) & 15,
  // channels 8 (c & 7) .. + 7; tokens past T re-read token T - 1 (never used)
  const _Float16* src[kRowsVecs] = {p.r, p.w, p.k, p.v, p.a, p.b};
  hv8 stg[3];
  auto stage_load = [&](int t0) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      const int c = tid + 256 * u;
      const int tt = (c >> 3) & 15, part = c & 7;
      const int t = min(t0 + tt, T - 1);
      const _Float16* x = (c & 128) ? src[2 * u + 1] : src[2 * u];
      const _Float16* at = x + tok0 + (size_t)t * p.C + part * 8;
      if (ra.vec) {
        stg[u] = *reinterpret_cast<const hv8*>(at);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) stg[u][e] = at[e];
      }
    }
  };
  auto stage_store = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      const int c = tid + 256 * u;
      const int vec = c >> 7, tt = (c >> 3) & 15, part = c & 7;
      float f[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = (u == 0 && vec == 1) ? decay((float)stg[u][e]) : (float)stg[u][e];
      f4* d = &vl[((buf * kRowsTC + tt) * kRowsVecs + vec) * 16 + part * 2];
      d[0] = f4{f[0], f[1], f[2], f[3]};
      d[1] = f4{f[4], f[5], f[6], f[7]};
    }
  };

  float s[kRPL][8];
#pragma unroll
  for (int rr = 0; rr < kRPL; ++rr) {
    const float* row = S + (i0 + rr) * kHead;
    const f4 lo = *reinterpret_cast<const f4*>(row + 4 * g);
    const f4 hi = *reinterpret_cast<const f4*>(row + 32 + 4 * g);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s[rr][e] = lo[e];
      s[rr][4 + e] = hi[e];
    }
  }

  struct Tok {
    f4 a[2], r[2], d[2], k[2], b[2];
    float v[kRPL];
  };
  // slot = buffer * kRowsTC + token; a is read first (it is needed first)
  auto read_tok = [&](int slot) __attribute__((always_inline)) {
    const f4* base = &vl[slot * kRowsVecs * 16];
    Tok o;
    o.a[0] = base[4 * 16 + g], o.a[1] = base[4 * 16 + 8 + g];
    o.r[0] = base[0 * 16 + g], o.r[1] = base[0 * 16 + 8 + g];
    o.d[0] = base[1 * 16 + g], o.d[1] = base[1 * 16 + 8 + g];
    o.k[0] = base[2 * 16 + g], o.k[1] = base[2 * 16 + 8 + g];
    o.b[0] = base[5 * 16 + g], o.b[1] = base[5 * 16 + 8 + g];
    const float* vv = reinterpret_cast<const float*>(base + 3 * 16) + i0;
#pragma unroll
    for (int rr = 0; rr < kRPL; ++rr) o.v[rr] = vv[rr];
    return o;
  };

  float sa[kRPL];
  // token `cur` (chunk token tt): state update, then y_t with cur.r and sa_{t+1} with nx.a
  auto token = [&](const Tok& cur, const Tok& nx, int tt) __attribute__((always_inline)) {
#pragma unroll
    for (int rr = 0; rr < kRPL; ++rr) {
      const float vi = cur.v[rr];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float x = s[rr][e] * cur.d[e >> 2][e & 3];
        x = __builtin_fmaf(sa[rr], cur.b[e >> 2][e & 3], x);
        s[rr][e] = __builtin_fmaf(cur.k[e >> 2][e & 3], vi, x);
      }
    }
    float py[kRPL], pa[kRPL];
#pragma unroll
    for (int rr = 0; rr < kRPL; ++rr) py[rr] = pa[rr] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
#pragma unroll
      for (int rr = 0; rr < kRPL; ++rr) {
        py[rr] = __builtin_fmaf(s[rr][e], cur.r[e >> 2][e & 3], py[rr]);
        pa[rr] = __builtin_fmaf(s[rr][e], nx.a[e >> 2][e & 3], pa[rr]);
      }
    }
    float y[kRPL];
#pragma unroll
    for (int rr = 0; rr < kRPL; ++rr) {
      y[rr] = sum8(py[rr]);
      sa[rr] = sum8(pa[rr]);
      // keep the sum an fp32 value before the fp16 conversion (no fused mixed-precision op)
      asm volatile("" : "+v"(y[rr]));
    }
    // the eight lanes of a row group hold the same bits: all write the same words
    if constexpr (kRPL == 2) {
      *reinterpret_cast<h2*>(&ybuf[wv][tt][q][0]) = h2{(_Float16)y[0], (_Float16)y[1]};
    } else {
      ybuf[wv][tt][q][0] = (_Float16)y[0];
    }
  };

  const int nchunk = (T + kRowsTC - 1) / kRowsTC;
  stage_load(0);
  stage_store(0);
  if (nchunk > 1) {
    stage_load(kRowsTC);
    stage_store(1);
    if (nchunk > 2) stage_load(2 * kRowsTC);
  }
  lds_barrier();
  {
    const Tok t0v = read_tok(0);
#pragma unroll
    for (int rr = 0; rr < kRPL; ++rr) {
      float acc = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(s[rr][e], t0v.a[e >> 2][e & 3], acc);
      sa[rr] = sum8(acc);
    }
  }
  int buf = 0;
  for (int c = 0; c < nchunk; ++c) {
    const int nbuf = buf == kRowsBufs - 1 ? 0 : buf + 1;
    const int t0 = c * kRowsTC;
    const int nt = min(kRowsTC, T - t0);
    // LDS slot of chunk token j, j <= kRowsTC + 2: past the chunk, the next buffer's
    // first tokens (past T they hold stale values that are never used)
    auto slot = [&](int j) { return j < kRowsTC ? buf * kRowsTC + j : nbuf * kRowsTC + (j - kRowsTC); };
    // three token register sets: token j's vectors are read while token j - 2 computes,
    // so the read has a whole token step to land before token j - 1 needs j's a
    Tok ta = read_tok(slot(0)), tb = read_tok(slot(1));
    for (int tt = 0; tt < nt; tt += 3) {
      Tok tc = read_tok(slot(tt + 2));
      token(ta, tb, tt);
      if (tt + 1 >= nt) break;
      ta = read_tok(slot(tt + 3));
      token(tb, tc, tt + 1);
      if (tt + 2 >= nt) break;
      tb = read_tok(slot(tt + 4));
      token(tc, ta, tt + 2);
    }
    // chunk c + 2 -> the buffer chunk c - 1 used (its readers passed the last barrier)
    if (c + 2 < nchunk) {
      stage_store(nbuf == kRowsBufs - 1 ? 0 : nbuf + 1);
      if (c + 3 < nchunk) stage_load((c + 3) * kRowsTC);
    }
    // this wave's y tile -> HBM: lane -> token lane >> 2 and 2 kRPL consecutive rows
    // (row groups 2 (lane & 3), +1 of this wave)
    {
      const int tt = lane >> 2, r4 = lane & 3;
      if (tt < nt) {
        const _Float16* yb = &ybuf[wv][tt][2 * r4][0];  // 2 kRPL values, row order
        const int row0 = kRPL == 2 ? 16 * wv + 4 * r4 : 32 * half + 8 * wv + 2 * r4;
        _Float16* yd = p.y + tok0 + (size_t)(t0 + tt) * p.C + row0;
        if constexpr (kRPL == 2) {
          if (ra.vec) {
            typedef _Float16 hv4 __attribute__((ext_vector_type(4)));
            *reinterpret_cast<hv4*>(yd) = hv4{yb[0], yb[1], yb[2], yb[3]};
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) yd[e] = yb[e];
          }
        } else {
          if (ra.vec) {
            *reinterpret_cast<h2*>(yd) = h2{yb[0], yb[1]};
          } else {
            yd[0] = yb[0];
            yd[1] = yb[1];
          }
        }
      }
    }
    lds_barrier();
    buf = nbuf;
  }

#pragma unroll
  for (int rr = 0; rr < kRPL; ++rr) {
    float* row = S + (i0 + rr) * kHead;
    *reinterpret_cast<f4*>(row + 4 * g) = f4{s[rr][0], s[rr][1], s[rr][2], s[rr][3]};
    *reinterpret_cast<f4*>(row + 32 + 4 * g) = f4{s[rr][4], s[rr][5], s[rr][6], s[rr][7]};
  }
}

// ---- chunked prefill (T >= kChunkMinT): WKV-7 over chunks of 16 tokens on the matrix cores.
//
// Within a chunk of L = 16 tokens (t = 1..L, entry state S0, Λ_t = d_1 ... d_t elementwise
// over the key index j) write S_t = X_t diag(Λ_t).  The recurrence
//     S_t = S_{t-1} diag(d_t) + (S_{t-1} a_t) b_t^T + v_t k_t^T,   y_t = S_t r_t
// becomes, with â_t = Λ_{t-1} a_t, b̂_t = b_t / Λ_t, k̂_t = k_t / Λ_t, r̂_t = Λ_t r_t and
// z_t = S_{t-1} a_t,
//     X_t = X_{t-1} + z_t b̂_t^T + v_t k̂_t^T,
//     z_t = X0 â_t + Σ_{m<t} (b̂_m·â_t) z_m + (k̂_m·â_t) v_m,
//     y_t = X0 r̂_t + Σ_{m≤t} (b̂_m·r̂_t) z_m + (k̂_m·r̂_t) v_m.
// In matrix form (rows t): with the L x L matrices N = T_ab = strict-lower(Â B̂^T),
// T_ak = strict-lower(Â K̂^T), T_rb = lower(R̂ B̂^T), T_rk = lower(R̂ K̂^T):
//     Z = (I - N)^{-1} (Â X0^T + T_ak V),   Y = R̂ X0^T + T_rb Z + T_rk V,
//     S_L^T = diag(Λ_L) (X0^T + B̂^T Z + K̂^T V),   X0 = S0,
// The ratios Λ_{t-1}/Λ_m and Λ_t/Λ_m that these products form are at most 1 and at least
// d_min^16 (d > 0.545 for every w, so > 6e-5): fp32 holds them without overflow, and the
// results agree with the token-by-token recurrence to fp32 rounding.
//
// One 512-lane workgroup per (sequence, head).  State wave w (0-3) owns the state rows
// (value index) i = 16w .. 16w + 15, which evolve independently, as X^T tiles (16 x 16, j x i)
// in the accumulator layout of v_mfma_f32_16x16x4_f32 (lane l, register r: row 4 (l / 16) + r,
// column l % 16; written D(M) below).  D(M) serves directly as the B operand of a product
// M' M when the k index is walked in the permuted order k = 4 (l / 16) + s over the 4 steps
// s of a 16-wide k tile (a sum over k does not depend on its order), and D(M^T) as the A
// operand of M M'; every other operand is read from LDS in the same permuted order.
//
// Pipeline (one barrier per chunk): in iteration c the state waves run chunk c against the
// state (Â X0^T, R̂ X0^T, K̂^T V, then Z = W RHS, Y and B̂^T Z: the dependent chain of a
// chunk), while matrix waves 4-7 prepare chunk c + 3's hat vectors (VALU work: Λ by a
// multiplicative DPP scan over the 16 lanes that hold one channel quad's tokens), chunk
// c + 2's four L x L matrices and chunk c + 1's W^T from its N (described at the kernel).
// Per chunk: 80 MFMAs on each state wave, 116 / 112 / 96 / 96 on the four SIMDs.  Measured
// at config 2: 0.174 ms per call (0.24 ms for the form with four waves, each running all
// three stages for its own rows: 132 MFMAs per wave, W^T computed four times).  The matrix
// core and the vector ALU of a SIMD do not overlap across its two waves on gfx950 (a loop of
// MFMAs on one wave beside a loop of FMAs on the other takes the sum of both times), so the
// split gains from moving the redundant W^T work out and from the second wave filling
// dependency stalls, not from concurrent execution.  To let it fill them the state waves
// read their next chunk's operands before the barrier (their chain then starts at once and
// runs without stalls) and the matrix waves, whose work is dependent chains, issue at a
// higher priority (0.201 -> 0.174 ms; at equal priority the state wave held the SIMD for its
// whole chain).  (W^T by forward substitution on the vector ALU measured 5 % slower; back
// substitution of Z on the state waves 25 % slower.)
constexpr int kCL = 16;          // tokens per chunk
constexpr int kChunkMinT = 16;   // shorter prefills take the row-split kernel
constexpr int kHP = kHead + 4;   // padded LDS row of a [t][j] hat vector (floats)
constexpr int kTP = kCL + 4;     // padded LDS row of a transposed [j][t] vector (floats)

typedef float fq4 __attribute__((ext_vector_type(4)));
typedef _Float16 hv4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ fq4 mfma4(float a, float b, fq4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// exp(-e^{-1/2} sigmoid(w)) from the hardware exp2 / reciprocal (about 2 ulp): the chunked
// form is not bit-matched to the token-by-token kernels anyway, and decay() with expf's
// range checks and an IEEE division is several times longer
__device__ __forceinline__ float decay_fast(float w) {
  const float e = __builtin_amdgcn_exp2f(w * -1.4426950408889634f);  // exp(-w)
  return __builtin_amdgcn_exp2f(-0.8750387749145276f * __builtin_amdgcn_rcpf(1.0f + e));  // e^{-1/2} log2(e)
}

typedef const __attribute__((address_space(1))) hv8 global_hv8;

// x * (the value of the lane `n` below in the same 16-lane row, 1 for the first n lanes)
#define VK_SCAN_MUL(x, ctrl) \
  x *= __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, 1.0f), __builtin_bit_cast(int, x), ctrl, 0xF, 0xF, false))

struct ChunkLds {
  // fp16 r, w, k, v, a, b: [vec][t][8 x 8 channels + 8 of padding].  The padding spreads the
  // 16 tokens that one row of 16 lanes reads (one channel quad each) over distinct banks:
  // with 128-byte rows they would all fall on two.
  hv8 raw[2][6 * kCL][9];
  __attribute__((aligned(16))) float lamL[4][kHead];         // Λ_L
  __attribute__((aligned(16))) float hat[4][2][kCL][kHP];    // Â, R̂ as [t][j]
  __attribute__((aligned(16))) float hatT[4][3][kHead][kTP]; // B̂^T, K̂^T as [j][t]; V^T as [i][t]
  __attribute__((aligned(16))) float gram[3][4][kCL][kTP];   // N, T_ak, T_rb, T_rk as [t][m]
  __attribute__((aligned(16))) float gramT[3][kCL][kTP];     // N as [m][t]
  __attribute__((aligned(16))) fq4 wt[2][64];                // D(W^T) of a chunk, lane by lane
  __attribute__((aligned(16))) float lamSink[256];           // Λ stores of lanes that hold no Λ_L
};

// Eight waves in two roles, two per SIMD (waves w and w + 4 share SIMD w), so that each
// SIMD interleaves two independent instruction streams.  State waves 0-3 own the state rows
// and run chunk c's state products.  Matrix waves 4-7 prepare the chunks ahead of it: all four
// the hat vectors of chunk c + 3 (and the token-vector staging), waves 5-7 the L x L matrices
// of chunk c + 2 (N and T_ak on wave 5, whose operands share Â), and wave 4 W^T of chunk c + 1
// from its N (computed one iteration earlier), which keeps W^T's dependent chain of 24
// products off the iteration that produces N and balances the matrix work over the SIMDs
// (116 / 112 / 96 / 96 products per SIMD and chunk).  One barrier per chunk.  The LDS
// pipeline (four hat buffers, three matrix buffers) takes 144 KiB: one workgroup per CU.
template <bool kSlots>
__global__ __launch_bounds__(512) void wkv7_fp32_chunk_kernel(RowsArgs ra) {
  const Fp32Args& p = ra.a;
  __shared__ ChunkLds L;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 15, g = lane >> 4;
  const bool state_wave = w < 4;
  const int mtid = tid & 255;  // thread index inside its role
  const int bh = blockIdx.x, bi = bh / p.H, h = bh - bi * p.H;
  const int T = p.T, C = p.C;
  const size_t tok0 = (size_t)bi * T * C + (size_t)h * kHead;
  float* S = state_block<kSlots>(p, bi, h);
  if (S == nullptr) {
    for (int idx = tid; idx < T * kHead; idx += 512)
      p.y[tok0 + (size_t)(idx / kHead) * C + (idx % kHead)] = (_Float16)__builtin_nanf("");
    return;
  }
  const int iw = 16 * (w & 3) + li;  // a state wave lane's state row (value index), accumulator layout
  // X^T tile q (j = 16 q .. 16 q + 15): register r holds X^T[16 q + 4 g + r][iw] = S[iw][16 q + 4 g + r]
  fq4 st[4];
  if (state_wave) {
#pragma unroll
    for (int q = 0; q < 4; ++q) st[q] = *reinterpret_cast<const fq4*>(S + iw * kHead + 16 * q + 4 * g);
    // the loads are waited for here: otherwise the loop keeps their waits, which in every
    // later iteration wait for the previous chunk's y stores before its first products
#pragma unroll
    for (int q = 0; q < 4; ++q) asm volatile("" : "+v"(st[q]));
  }

  // raw token vectors (matrix waves): piece c = mtid + 256 u is vector c >> 7, token
  // (c >> 3) & 15, channels 8 (c & 7) .. + 7; tokens past T re-read token T - 1 (masked out below)
  const _Float16* src[6] = {p.r, p.w, p.k, p.v, p.a, p.b};
  hv8 pre[3];
  auto load_raw = [&](int t0) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      const int c = mtid + 256 * u;
      const int t = min(t0 + ((c >> 3) & 15), T - 1);
      const _Float16* at = src[c >> 7] + tok0 + (size_t)t * C + (c & 7) * 8;
      // a global (not flat) load: a flat load would also count against the LDS counter,
      // and every wait for the LDS reads would wait for this prefetch
      if (ra.vec) {
        pre[u] = *(global_hv8*)at;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) pre[u][e] = *(const __attribute__((address_space(1))) _Float16*)(at + e);
      }
    }
  };
  auto store_raw = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      const int c = mtid + 256 * u;
      L.raw[buf][c >> 3][c & 7] = pre[u];  // row (vector, token) c >> 3, channels 8 (c & 7) ..
    }
  };

  // hat vectors of chunk cc (raw buffer cc & 1) into hat buffer cc % 4 (matrix waves): thread =
  // token ht, channels j0 .. j0 + 3 (16 lanes of a row hold one quad's 16 tokens: the Λ
  // scan).  A chunk past the end computes stale values nobody reads.  Split into the LDS
  // reads and the arithmetic, so the reads can be issued early.
  const int ht = lane & 15, j0 = 4 * (mtid >> 4);
  struct RawQuad {
    hv4 r, w, k, v, a, b;
  };
  auto hats_read = [&](int cc) __attribute__((always_inline)) {
    const int rb = cc & 1;
    auto rd4 = [&](int vec) __attribute__((always_inline)) {
      return *reinterpret_cast<const hv4*>(reinterpret_cast<const _Float16*>(&L.raw[rb][vec * kCL + ht][0]) + j0);
    };
    return RawQuad{rd4(0), rd4(1), rd4(2), rd4(3), rd4(4), rd4(5)};
  };
  auto hats_write = [&](int cc, const RawQuad& x) __attribute__((always_inline)) {
    const int b = cc & 3;
    const int n = min(kCL, T - cc * kCL);
    const float in = ht < n ? 1.0f : 0.0f;  // padded tokens: d = 1 and zero vectors (a select, no branch)
    float l1[4], l0[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float d = __builtin_fmaf(in, decay_fast((float)x.w[e]), 1.0f - in);
      VK_SCAN_MUL(d, 0x111);  // row_shr:1
      VK_SCAN_MUL(d, 0x112);  // row_shr:2
      VK_SCAN_MUL(d, 0x114);  // row_shr:4
      VK_SCAN_MUL(d, 0x118);  // row_shr:8
      l1[e] = d;              // Λ_t
      l0[e] = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, 1.0f),
                                                                     __builtin_bit_cast(int, d), 0x111, 0xF, 0xF, false));
    }
    float ah[4], rh[4], bh[4], kh[4], vv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float rl = __builtin_amdgcn_rcpf(l1[e]);
      ah[e] = l0[e] * ((float)x.a[e] * in);
      rh[e] = l1[e] * ((float)x.r[e] * in);
      bh[e] = ((float)x.b[e] * in) * rl;
      kh[e] = ((float)x.k[e] * in) * rl;
      vv[e] = (float)x.v[e] * in;
    }
    *reinterpret_cast<fq4*>(&L.hat[b][0][ht][j0]) = fq4{ah[0], ah[1], ah[2], ah[3]};
    *reinterpret_cast<fq4*>(&L.hat[b][1][ht][j0]) = fq4{rh[0], rh[1], rh[2], rh[3]};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      L.hatT[b][0][j0 + e][ht] = bh[e];
      L.hatT[b][1][j0 + e][ht] = kh[e];
      L.hatT[b][2][j0 + e][ht] = vv[e];
    }
    float* lamDst = ht == kCL - 1 ? &L.lamL[b][j0] : &L.lamSink[4 * (mtid >> 2) & 252];
    *reinterpret_cast<fq4*>(lamDst) = fq4{l1[0], l1[1], l1[2], l1[3]};
  };
  // L x L matrix (x, y) of chunk cc into matrix buffer cc % 3, slot m: (Â,B̂) (Â,K̂) (R̂,B̂)
  // (R̂,K̂) for m = 0..3, masked (strictly lower for the first two); N also transposed.  The x
  // operands come from hat ([t][j], one 16-byte read per k step), the y operands from hatT.
  auto gram_x = [&](int cc, int xsel, fq4 (&x)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < 4; ++q) x[q] = *reinterpret_cast<const fq4*>(&L.hat[cc & 3][xsel][li][16 * q + 4 * g]);
  };
  auto gram_y = [&](int cc, int ysel, fq4 (&y)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) y[q][s2] = L.hatT[cc & 3][ysel][16 * q + 4 * g + s2][li];
  };
  auto gram_mfma = [&](const fq4 (&x)[4], const fq4 (&y)[4]) __attribute__((always_inline)) {
    fq4 gm = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) gm = mfma4(x[q][s2], y[q][s2], gm);
    return gm;
  };
  auto gram_write = [&](int cc, int m, const fq4& gm) __attribute__((always_inline)) {
    const int b = cc % 3, mlim = m < 2 ? 1 : 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 4 * g + r;
      const float x = li <= t - mlim ? gm[r] : 0.0f;
      L.gram[b][m][t][li] = x;
      if (m == 0) L.gramT[b][li][t] = x;
    }
  };
  // wave 5: N and T_ak; wave 6: T_rb; wave 7: T_rk.  Every operand read is issued before the
  // first product (a scheduling barrier): left to itself the compiler interleaves each pair of
  // reads with two products and a wait for it, one LDS round trip per two products.
  auto grams = [&](int cc) __attribute__((always_inline)) {
    if (w == 5) {
      fq4 x[4], yb[4], yk[4];
      gram_x(cc, 0, x);
      gram_y(cc, 0, yb);
      gram_y(cc, 1, yk);
      __builtin_amdgcn_sched_barrier(0);
      const fq4 gn = gram_mfma(x, yb), gk = gram_mfma(x, yk);
      gram_write(cc, 0, gn);
      gram_write(cc, 1, gk);
    } else if (w >= 6) {
      fq4 x[4], y[4];
      gram_x(cc, 1, x);
      gram_y(cc, w == 6 ? 0 : 1, y);
      __builtin_amdgcn_sched_barrier(0);
      gram_write(cc, w == 6 ? 2 : 3, gram_mfma(x, y));
    }
  };
  // wave 4: W^T = ((I - N)^{-1})^T of chunk cc into wt buffer cc & 1.  N is nilpotent,
  // N^16 = 0, so (I - N)^{-1} = (I + N)(I + N^2)(I + N^4)(I + N^8); the powers in both
  // orientations: D(M^2) = Σ_s D(M^T)[s] x D(M)[s].
  auto w_transpose = [&](int cc) __attribute__((always_inline)) {
    const int b = cc % 3;
    fq4 pm[4], pmt[4];  // pm[k] = D(N^(2^k)), pmt[k] = D((N^(2^k))^T)
    pm[0] = *reinterpret_cast<const fq4*>(&L.gramT[b][li][4 * g]);
    pmt[0] = *reinterpret_cast<const fq4*>(&L.gram[b][0][li][4 * g]);
#pragma unroll
    for (int k = 1; k < 4; ++k) {
      fq4 x = {0.0f, 0.0f, 0.0f, 0.0f}, y = x;
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) {
        x = mfma4(pmt[k - 1][s2], pm[k - 1][s2], x);
        y = mfma4(pm[k - 1][s2], pmt[k - 1][s2], y);
      }
      pm[k] = x;
      pmt[k] = y;
    }
    // W^T = (I + N^T)(I + (N^T)^2)(I + (N^T)^4)(I + (N^T)^8): Q <- Q + (N^T)^(2^k) Q, whose A
    // operand D(((N^T)^(2^k))^T) is pm[k]
    fq4 wt;
#pragma unroll
    for (int r = 0; r < 4; ++r) wt[r] = (4 * g + r == li ? 1.0f : 0.0f) + pmt[0][r];
#pragma unroll
    for (int k = 1; k < 4; ++k) {
      fq4 x = wt;
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) x = mfma4(pm[k][s2], wt[s2], x);
      wt = x;
    }
    L.wt[cc & 1][lane] = wt;
  };

  const int nchunk = (T + kCL - 1) / kCL;
  // prologue (matrix waves): hats of chunks 0-2, matrices of chunks 0-1, W^T of chunk 0; chunk
  // 3's raw vectors staged, chunk 4's loaded.  (Chunks past the end read token T - 1 and are
  // never used.)
  if (!state_wave) {
    load_raw(0);
    store_raw(0);
    load_raw(kCL);
  }
  __syncthreads();
  if (!state_wave) {
    hats_write(0, hats_read(0));
    store_raw(1);
    load_raw(2 * kCL);
  }
  __syncthreads();
  if (!state_wave) {
    hats_write(1, hats_read(1));
    grams(0);
    store_raw(0);
    load_raw(3 * kCL);
  }
  __syncthreads();
  if (!state_wave) {
    hats_write(2, hats_read(2));
    grams(1);
    if (w == 4) w_transpose(0);
    store_raw(1);
    load_raw(4 * kCL);
  }
  __syncthreads();
  // The state waves' operands of chunk c other than W^T (hat vectors, L x L matrices, Λ_L) are
  // complete from the start of iteration c - 1 on (hats three chunks ahead, matrices two), so
  // each iteration reads the next chunk's right after its own products, while the state waves
  // wait at the barrier for the matrix waves; after the barrier only W^T is read.  (Read at
  // the start of the iteration, these reads queued up ~100 KiB of LDS traffic in front of the
  // first product and of the matrix waves' reads.)
  fq4 a4[4], r4[4], k4[4], b4[4], lamq[4], v4, tak, trb, trk;
  auto state_operands = [&](int cc) __attribute__((always_inline)) {
    const int hb = cc & 3, gb = cc % 3;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      a4[q] = *reinterpret_cast<const fq4*>(&L.hat[hb][0][li][16 * q + 4 * g]);
      r4[q] = *reinterpret_cast<const fq4*>(&L.hat[hb][1][li][16 * q + 4 * g]);
      k4[q] = *reinterpret_cast<const fq4*>(&L.hatT[hb][1][16 * q + li][4 * g]);
    }
    v4 = *reinterpret_cast<const fq4*>(&L.hatT[hb][2][iw][4 * g]);
#pragma unroll
    for (int q = 0; q < 4; ++q) b4[q] = *reinterpret_cast<const fq4*>(&L.hatT[hb][0][16 * q + li][4 * g]);
    tak = *reinterpret_cast<const fq4*>(&L.gram[gb][1][li][4 * g]);
    trb = *reinterpret_cast<const fq4*>(&L.gram[gb][2][li][4 * g]);
    trk = *reinterpret_cast<const fq4*>(&L.gram[gb][3][li][4 * g]);
#pragma unroll
    for (int q = 0; q < 4; ++q) lamq[q] = *reinterpret_cast<const fq4*>(&L.lamL[hb][16 * q + 4 * g]);
  };
  // One loop per role, each with the one barrier per chunk (the role is uniform over a wave, so
  // the two loops' barriers pair up): in a shared loop the state operands, live across the
  // back edge, also counted against the matrix branch's registers (252 VGPRs instead of 190).
  if (state_wave) {
    state_operands(0);
    for (int c = 0; c < nchunk; ++c) {
      // ---- chunk c against the state:  RHS = Â X0^T + T_ak V;  Y = R̂ X0^T + T_rk V + T_rb Z
      // with Z = W RHS;  X^T += K̂^T V + B̂^T Z;  S^T = diag(Λ_L) X^T
      const int n = min(kCL, T - c * kCL);
      const fq4 wt = L.wt[c & 1][lane];
      __builtin_amdgcn_sched_barrier(0);
      fq4 p1 = {0.0f, 0.0f, 0.0f, 0.0f}, y1 = p1;
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
          p1 = mfma4(a4[q][s2], st[q][s2], p1);
          y1 = mfma4(r4[q][s2], st[q][s2], y1);
        }
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) st[q] = mfma4(k4[q][s2], v4[s2], st[q]);
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) {
        p1 = mfma4(tak[s2], v4[s2], p1);
        y1 = mfma4(trk[s2], v4[s2], y1);
      }
      fq4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) z = mfma4(wt[s2], p1[s2], z);
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) y1 = mfma4(trb[s2], z[s2], y1);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) st[q] = mfma4(b4[q][s2], z[s2], st[q]);
#pragma unroll
        for (int r = 0; r < 4; ++r) st[q][r] *= lamq[q][r];
      }
      // y rows t = 4 g + r of this wave's 16 value columns
      _Float16 yh[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float yv = y1[r];
        asm volatile("" : "+v"(yv));  // an fp32 value before the fp16 conversion
        yh[r] = (_Float16)yv;
      }
      _Float16* yp = p.y + tok0 + (size_t)(c * kCL + 4 * g) * C + iw;
      if (n == kCL) {
#pragma unroll
        for (int r = 0; r < 4; ++r) yp[(size_t)r * C] = yh[r];
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (4 * g + r < n) yp[(size_t)r * C] = yh[r];
      }
      // chunk c + 1's operands (past the last chunk: stale buffers, in bounds, never used)
      __builtin_amdgcn_sched_barrier(0);
      state_operands(c + 1);
      __syncthreads();
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) *reinterpret_cast<fq4*>(S + iw * kHead + 16 * q + 4 * g) = st[q];
  } else {
    // The matrix waves' work is dependent chains (W^T's powers, LDS round trips, the Λ scans);
    // at a higher issue priority they go first whenever they can, and the state wave's
    // products fill their stalls (a SIMD issues one wave's matrix products and the other's
    // vector instructions in turn, not at once, and at equal priority the older state wave
    // held the SIMD for its whole chain).
    __builtin_amdgcn_s_setprio(1);
    for (int c = 0; c < nchunk; ++c) {
      // ---- chunk c + 3's hat vectors, chunk c + 2's matrices, chunk c + 1's W^T; chunk c + 4's
      // raw vectors into the buffer chunk c + 2's hats were read from (one iteration ago)
      const RawQuad rq = hats_read(c + 3);
      grams(c + 2);
      if (w == 4) w_transpose(c + 1);
      hats_write(c + 3, rq);
      store_raw(c & 1);
      load_raw((c + 5) * kCL);
      __syncthreads();
    }
  }
}

bool rows_vec_ok(const Fp32Args& p) {
  auto al = [](const void* x, uintptr_t m) { return ((uintptr_t)x & (m - 1)) == 0; };
  return al(p.r, 16) && al(p.w, 16) && al(p.k, 16) && al(p.v, 16) && al(p.a, 16) && al(p.b, 16) &&
         al(p.y, 8);
}

// rows: T > 1 uses the row-split kernel (dot products in its order); otherwise
// the row-per-lane kernels (one FMA chain per dot product).
// MI355X's memory-side cache (Infinity Cache).
constexpr int64_t kMallBytes = (int64_t)256 << 20;

template <bool kSlots>
void launch_fp32(const Fp32Args& p, int B, hipStream_t stream, bool rows) {
  if (p.T == 1) {
    const int64_t table = (int64_t)(kSlots ? p.n_slots : B) * p.H * kHead * kHead * 4;
    if (table > kMallBytes)
      hipLaunchKernelGGL((wkv7_fp32_step_kernel<kSlots, true>), dim3(B * p.H), dim3(64), 0, stream, p);
    else
      hipLaunchKernelGGL((wkv7_fp32_step_kernel<kSlots, false>), dim3(B * p.H), dim3(64), 0, stream, p);
  } else if (rows) {
    RowsArgs ra{p, rows_vec_ok(p) ? 1 : 0};
    if (p.T >= kChunkMinT)
      hipLaunchKernelGGL(wkv7_fp32_chunk_kernel<kSlots>, dim3(B * p.H), dim3(512), 0, stream, ra);
    else if (ra.vec && B * p.H < 2 * device_cus())
      hipLaunchKernelGGL((wkv7_fp32_rows_kernel<kSlots, 1>), dim3(2 * B * p.H), dim3(256), 0, stream, ra);
    else
      hipLaunchKernelGGL((wkv7_fp32_rows_kernel<kSlots, 2>), dim3(B * p.H), dim3(256), 0, stream, ra);
  } else if ((int64_t)B * p.H <= 4 * (int64_t)device_cus()) {
    // few chains: at most one wave per SIMD, the latency-scheduled form (same bits)
    hipLaunchKernelGGL(wkv7_fp32_seq_lat_kernel<kSlots>, dim3(B * p.H), dim3(64), 0, stream, p);
  } else {
    hipLaunchKernelGGL(wkv7_fp32_seq_kernel<kSlots>, dim3(B * p.H), dim3(64), 0, stream, p);
  }
}

// ---- fused decode step of the time mix: kk/a gate -> WKV-7 -> GroupNorm,
// bonus and output gate, one wave per (sequence, head).  Each stage is the
// arithmetic of its stand-alone kernel (mix.hip kk_a_gate_kernel,
// token_fp32 above, mix.hip groupnorm_bonus_gate_kernel) with the fp16
// roundings of their stored intermediates (new_k, -kk, kk*a, y), so the fused
// result is bit-identical to the three-kernel sequence; the intermediates
// never leave registers and the per-head reductions are wave reductions.
struct FusedArgs {
  int C, H, n_slots;
  int out_frag;  // (beside the other ints: one 16-byte scalar load for the four)
  float* pool;
  const int32_t* slots;
  const _Float16 *r, *w, *k, *v, *a12, *g;
  const _Float16 *k_k, *a0, *k_a, *r_k, *ln_w, *ln_b;
  _Float16* out;
};

// kIlv: the pool is in the interleaved layout (vkwr_amd.h VKWR_WKV_STATE_ILV):
// chunk q (columns 4q..4q+3) of the 64 rows is one contiguous kilobyte, so
// lane i loads its row straight into registers with 16 fully coalesced
// 16-byte loads, all in flight at once, and stores it back the same way -- no
// LDS staging, no barriers.  Otherwise the standard [64][64] row-major block
// goes through the two-phase LDS transpose.
template <bool kIlv>
__global__ __launch_bounds__(64, 4) void wkv7_decode_fused_kernel(FusedArgs p) {
  __shared__ f4 st[512];
  __shared__ float vb[5 * kHead];  // the token's channel vectors, staged before the state phase
  // every argument in one round of scalar loads, above the first branch (as pin_args)
  pin_int(p.C), pin_int(p.H), pin_int(p.n_slots), pin_int(p.out_frag);
  pin_ptr(p.pool), pin_ptr(p.slots), pin_ptr(p.r), pin_ptr(p.w), pin_ptr(p.k), pin_ptr(p.v), pin_ptr(p.a12);
  pin_ptr(p.g), pin_ptr(p.k_k), pin_ptr(p.a0), pin_ptr(p.k_a), pin_ptr(p.r_k), pin_ptr(p.ln_w), pin_ptr(p.ln_b);
  pin_ptr(p.out);
  const int lane = threadIdx.x;
  const int bh = blockIdx.x;
  const int bi = bh / p.H;
  const int h = bh - bi * p.H;
  const int c = h * kHead + lane;
  const size_t tok = (size_t)bi * p.C + c;
  auto out_index = [&]() { return p.out_frag ? frag_index(bi, c, p.C) : (int64_t)tok; };
  const int sl = p.slots[bi];
  if (sl < 0 || sl >= p.n_slots) {
    p.out[out_index()] = (_Float16)__builtin_nanf("");
    return;
  }
  float* S = p.pool + ((size_t)sl * p.H + h) * (kHead * kHead);
  // The lane's token and channel inputs are requested first and the state right after
  // them, before any arithmetic: the gate's reductions then run while the state is in
  // flight (every wave of the launch starts at once; with the loads after the gate the
  // memory would sit idle meanwhile), and waiting for an input never waits for the state.
  const _Float16 xr = p.r[tok], xw = p.w[tok], xv = p.v[tok];
  const _Float16 xk = p.k[tok], xa12 = p.a12[tok];
  const _Float16 pk_k = p.k_k[c], pa0 = p.a0[c], pk_a = p.k_a[c], pr_k = p.r_k[c];
  float s[kHead];
  if constexpr (kIlv) {
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      // non-temporal: the state is not read again before the next decode step
      const f4 x = __builtin_nontemporal_load(reinterpret_cast<const f4*>(S + (q * kHead + lane) * 4));
      s[4 * q + 0] = x.x;
      s[4 * q + 1] = x.y;
      s[4 * q + 2] = x.z;
      s[4 * q + 3] = x.w;
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  const float kv = (float)xk, a12 = (float)xa12;
  // kk / a gate
  const float u = kv * (float)pk_k;
  const float inv = 1.0f / fmaxf(sqrtf(wave_sum_prod(u, u)), kKkEps);
  const float kk = u * inv;
  const float a = sigmoidf((float)pa0 + a12);
  const float ka = (float)pk_a;
  const _Float16 new_k = f16_of(kv * __builtin_fmaf(a, ka, 1.0f - ka));
  const _Float16 neg_kk = (_Float16)(-kk);
  const _Float16 kka = f16_of(kk * a);
  // The r.k bonus does not depend on the WKV output: reduce it now (a
  // wave-uniform scalar) so r and new_k need not stay live across the state phase.
  const float rkv = wave_sum_prod((float)xr * (float)new_k, (float)pr_k);
  // WKV-7 (the channel vectors go to LDS first: only v stays in a register
  // across the state load)
  token_stage(vb, lane, xr, xw, new_k, neg_kk, kka);
  const float vi = (float)xv;
  if constexpr (kIlv) {
    __syncthreads();  // orders the vb writes before token_run's broadcast reads
  } else {
    load_state_fp32(S, st, s, lane);  // its barriers also order the vb writes
  }
  const float y = (float)token_run(s, vb, vi);
  // Recompute the store addresses instead of keeping the load's 16 per-lane
  // addresses live across the token (they would spill): launder S and lane.
  float* S2 = S;
  int lane2 = lane;
  asm volatile("" : "+s"(S2), "+v"(lane2));
  if constexpr (kIlv) {
    // Non-temporal stores: written as ordinary stores, 64 MiB of dirty state
    // per layer sit in the memory-side cache and are written back while the
    // next kernels stream their weights, which slows those reads.
#pragma unroll
    for (int q = 0; q < 16; ++q)
      __builtin_nontemporal_store(f4{s[4 * q], s[4 * q + 1], s[4 * q + 2], s[4 * q + 3]},
                                  reinterpret_cast<f4*>(S2 + (q * kHead + lane2) * 4));
  } else {
    store_state_fp32(S2, st, s, lane2);
  }
  // GroupNorm over the head + r.k bonus + gate.  The memory clobber keeps these
  // loads below the state phase (hoisted, they would hold registers across it).
  asm volatile("" ::: "memory");
  const float gv = (float)p.g[tok], lw = (float)p.ln_w[c], lb = (float)p.ln_b[c];
  const float mean = wave_sum(y) * (1.0f / 64.0f);
  const float d = y - mean;
  const float var = wave_sum_prod(d, d) * (1.0f / 64.0f);
  const float rstd = rsqrtf(var + kGroupNormEps);
  float z = __builtin_fmaf(d * rstd, lw, lb);
  z = __builtin_fmaf(rkv, vi, z);
  p.out[out_index()] = f16_of(z * gv);
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
  // every argument in one round of scalar loads, above the first branch (as pin_args)
  pin_int(p.T), pin_int(p.C), pin_int(p.H);
  pin_ptr(p.state), pin_ptr(p.r), pin_ptr(p.w), pin_ptr(p.w0), pin_ptr(p.k), pin_ptr(p.v), pin_ptr(p.a);
  pin_ptr(p.b), pin_ptr(p.y), pin_ptr(p.elapsed);
  const int lane = threadIdx.x;
  const int bh = blockIdx.x;
  const int bi = bh / p.H;
  const int h = bh - bi * p.H;
  const size_t tok0 = (size_t)bi * p.T * p.C + (size_t)h * kHead + lane;
  _Float16* S = p.state + (size_t)bh * (kHead * kHead);

  // the first token's inputs, the phase and w0 are requested before the state, so their
  // latency overlaps the state transfer instead of following it
  const uint32_t el = (uint32_t)p.elapsed[bi];
  const uint32_t chan = (uint32_t)(h * kHead + lane);
  const bool has_w0 = !kLegacy && p.w0 != nullptr;
  // loaded without a branch (p.r stands in when there is no w0), so no wait follows it here
  const _Float16 w0h = *(has_w0 ? p.w0 + chan : p.r + tok0);
  _Float16 xr = p.r[tok0], xw = p.w[tok0], xk = p.k[tok0];
  _Float16 xv = p.v[tok0], xa = p.a[tok0], xb = p.b[tok0];

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

  _Float16* vec = reinterpret_cast<_Float16*>(st);
  for (int t = 0; t < p.T; ++t) {
    _Float16* vb = vec + (t & 1) * (5 * kHead);
    float wf = (float)xw;
    uint32_t phase;
    if constexpr (kLegacy) {
      phase = el + (uint32_t)t;
    } else {
      if (has_w0) wf = wf + (float)w0h;
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

// The same recurrence for T > 1 when the (sequence, head) chains are few (at most one
// wave per SIMD; config 2's shape has 256), scheduled for a lone wave whose latency nothing
// else hides.  The arithmetic and the order of every sum are wkv7_fp16_kernel's; what moves
// is when each part runs:
//  - token t+1's sa chain (sum over columns of a[j] * s[j] with the state just updated)
//    runs inside token t's update loop, column by column, beside token t's y chain, so the
//    two dependent chains overlap instead of the sa chain running alone before the update;
//  - the loop body has no branch (token indices past the end are clamped and the values
//    they stage are never used), so the next token's decay (two exp2 and a division) is
//    scheduled among the chains' FMAs;
//  - inputs are fetched from global memory three tokens ahead and staged in LDS two ahead.
template <bool kLegacy>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 1))) void wkv7_fp16_seq_kernel(
    Fp16Args p) {
  __shared__ f4 st[512];  // one head's fp16 state (8 KiB); then two buffers of token vectors
  const int lane = threadIdx.x;
  const int bh = blockIdx.x;
  const int bi = bh / p.H;
  const int h = bh - bi * p.H;
  const int T = p.T;
  const size_t tok0 = (size_t)bi * T * p.C + (size_t)h * kHead + lane;
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
  auto wdelta = [&](_Float16 xw, int t) {
    float wf = (float)xw;
    uint32_t phase;
    if constexpr (kLegacy) {
      phase = el + (uint32_t)t;
    } else {
      if (p.w0 != nullptr) wf = wf + w0f;
      phase = el + chan + (uint32_t)t;
    }
    return w_delta(wf, phase);
  };
  struct Tok {
    _Float16 r, w, k, v, a, b;
  };
  auto fetch = [&](int t) {
    const size_t o = tok0 + (size_t)(t < T ? t : T - 1) * p.C;
    return Tok{p.r[o], p.w[o], p.k[o], p.v[o], p.a[o], p.b[o]};
  };
  _Float16* vec = reinterpret_cast<_Float16*>(st);
  auto stage = [&](int buf, const Tok& x, _Float16 wd) {
    _Float16* vb = vec + buf * (5 * kHead);
    vb[lane] = x.r;
    vb[kHead + lane] = wd;
    vb[2 * kHead + lane] = x.k;
    vb[3 * kHead + lane] = x.a;
    vb[4 * kHead + lane] = x.b;
  };

  const Tok x0 = fetch(0), x1 = fetch(1);
  Tok x2 = fetch(2);
  stage(0, x0, wdelta(x0.w, 0));
  stage(1, x1, wdelta(x1.w, 1));
  _Float16 v_cur = x0.v, v_next = x1.v;
  __syncthreads();
  // token 0's sa chain
  _Float16 sa;
  {
    const h2* A = reinterpret_cast<const h2*>(vec + 3 * kHead);
    h2 sa2 = {(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
    for (int m = 0; m < 32; ++m) {
      if constexpr (kLegacy) {
        sa2 = sa2 + A[m] * s[m];
      } else {
        sa2 = __builtin_elementwise_fma(A[m], s[m], sa2);
      }
    }
    sa = sa2.x + sa2.y;
  }

  // one token: xs holds token t+2's inputs (fetched an iteration ago), xl receives t+3's
  auto token = [&](int t, const Tok& xs, Tok& xl) {
    xl = fetch(t + 3);
    const int cb = t & 1;
    const h2* V = reinterpret_cast<const h2*>(vec + cb * (5 * kHead));
    const h2* An = reinterpret_cast<const h2*>(vec + (cb ^ 1) * (5 * kHead) + 3 * kHead);
    const _Float16 wd2 = wdelta(xs.w, t + 2);
    const h2 sav = {sa, sa};
    const h2 vv = {v_cur, v_cur};
    h2 y2 = {(_Float16)0.0f, (_Float16)0.0f};
    h2 sn2 = {(_Float16)0.0f, (_Float16)0.0f};
    // all five token vectors into registers at once (broadcast LDS reads), so that no FMA
    // of the chains waits on an LDS read issued just before it
    h2 Rv[32], Wv[32], Kv[32], Bvv[32], Av[32];
#pragma unroll
    for (int m = 0; m < 32; ++m) {
      Rv[m] = V[m];
      Wv[m] = V[32 + m];
      Kv[m] = V[64 + m];
      Bvv[m] = V[128 + m];
      Av[m] = An[m];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < 32; ++m) {
      const h2 R = Rv[m], W = Wv[m], K = Kv[m], Bv = Bvv[m];
      if constexpr (kLegacy) {
        const h2 t1 = s[m] * W;
        const h2 t2 = K * vv;
        const h2 t3 = t1 + t2;
        const h2 t4 = sav * Bv;
        const h2 t5 = t3 + t4;
        s[m] = s[m] + t5;
        y2 = y2 + s[m] * R;
        sn2 = sn2 + Av[m] * s[m];
      } else {
        const h2 in1 = __builtin_elementwise_fma(sav, Bv, s[m]);
        const h2 in2 = __builtin_elementwise_fma(K, vv, in1);
        s[m] = __builtin_elementwise_fma(s[m], W, in2);
        y2 = __builtin_elementwise_fma(s[m], R, y2);
        sn2 = __builtin_elementwise_fma(Av[m], s[m], sn2);
      }
    }
    p.y[tok0 + (size_t)t * p.C] = y2.x + y2.y;
    sa = sn2.x + sn2.y;
    __builtin_amdgcn_sched_barrier(0);  // keeps the next token's sa chain among these FMAs
    // every lane has read buffer cb (single-wave workgroup): token t+2 replaces token t
    __syncthreads();
    stage(cb, xs, wd2);
    v_cur = v_next;
    v_next = xs.v;
    __syncthreads();
  };
  // two tokens per trip, the two register sets swapping roles, so that no copy of a set
  // waits for loads issued in the same token
  Tok x3;
  int t = 0;
  for (; t + 1 < T; t += 2) {
    token(t, x2, x3);
    token(t + 1, x3, x2);
  }
  if (t < T) token(t, x2, x3);

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

// Converts n_blocks 64x64 fp32 state blocks between the standard row-major
// layout and the interleaved one (float (q*64 + i)*4 + e holds S[i][4q+e]).
__global__ __launch_bounds__(256) void wkv_state_layout_kernel(int64_t n_blocks, const float* src, float* dst,
                                                               int to_ilv) {
  const int64_t n = n_blocks * 1024;  // 16-byte chunks
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < n; t += stride) {
    const int64_t blk = t >> 10;
    const int c = (int)(t & 1023);
    const int i = c >> 4, q = c & 15;  // standard chunk c = (row i, column chunk q)
    const int64_t std_off = blk * 4096 + (int64_t)c * 4;
    const int64_t ilv_off = blk * 4096 + ((int64_t)q * kHead + i) * 4;
    if (to_ilv) *reinterpret_cast<f4*>(dst + ilv_off) = *reinterpret_cast<const f4*>(src + std_off);
    else *reinterpret_cast<f4*>(dst + std_off) = *reinterpret_cast<const f4*>(src + ilv_off);
  }
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
  launch_fp32<false>(p, B, (hipStream_t)stream, mode == 0);
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
  launch_fp32<true>(p, B, (hipStream_t)stream, true);
  return check_launch("vkwr_wkv7_fp32_forward_slots");
}

extern "C" int vkwr_wkv7_fp32_step_rows_slots(int B, int C, int H, float* pool, int n_slots,
                                              const int32_t* slots, const uint16_t* r, const uint16_t* w,
                                              const uint16_t* k, const uint16_t* v, const uint16_t* a,
                                              const uint16_t* b, uint16_t* y, void* stream) {
  clear_error();
  const char* fn = "vkwr_wkv7_fp32_step_rows_slots";
  if (int e = check_wkv_dims(fn, B, 1, C, H)) return e;
  VK_REQUIRE(n_slots >= 0, "%s: negative pool size", fn);
  if (B == 0 || H == 0) return VKWR_OK;
  VK_REQUIRE(pool && slots && r && w && k && v && a && b && y, "%s: null pointer", fn);
  VK_REQUIRE(((uintptr_t)pool | (uintptr_t)v) % 16 == 0 &&
                 ((uintptr_t)r | (uintptr_t)w | (uintptr_t)k | (uintptr_t)a | (uintptr_t)b) % 8 == 0,
             "%s: pool and v must be 16-byte aligned, r, w, k, a, b 8-byte aligned", fn);
  Fp32Args p{1, C, H, n_slots, pool, slots,
             reinterpret_cast<const _Float16*>(r), reinterpret_cast<const _Float16*>(w),
             reinterpret_cast<const _Float16*>(k), reinterpret_cast<const _Float16*>(v),
             reinterpret_cast<const _Float16*>(a), reinterpret_cast<const _Float16*>(b),
             reinterpret_cast<_Float16*>(y)};
  const int64_t table = (int64_t)n_slots * H * kHead * kHead * 4;
  if (table > kMallBytes)
    hipLaunchKernelGGL(wkv7_fp32_step_rows_kernel<true>, dim3(B * H), dim3(64), 0, (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL(wkv7_fp32_step_rows_kernel<false>, dim3(B * H), dim3(64), 0, (hipStream_t)stream, p);
  return check_launch(fn);
}

extern "C" int vkwr_wkv7_decode_fused_f16(int B, int C, int H, float* pool, int n_slots, int state_layout,
                                          const int32_t* slots, const uint16_t* r, const uint16_t* w,
                                          const uint16_t* k, const uint16_t* v, const uint16_t* a12,
                                          const uint16_t* g, const uint16_t* k_k, const uint16_t* a0,
                                          const uint16_t* k_a, const uint16_t* r_k, const uint16_t* ln_w,
                                          const uint16_t* ln_b, uint16_t* out, int out_frag,
                                          void* stream) {
  clear_error();
  const char* fn = "vkwr_wkv7_decode_fused_f16";
  if (int e = check_wkv_dims(fn, B, 1, C, H)) return e;
  VK_REQUIRE(n_slots >= 0, "%s: negative pool size", fn);
  VK_REQUIRE(out_frag == 0 || out_frag == 1, "%s: bad out_frag", fn);
  VK_REQUIRE(state_layout == VKWR_WKV_STATE_STD || state_layout == VKWR_WKV_STATE_ILV, "%s: bad state_layout", fn);
  VK_REQUIRE(!out_frag || C % kFragPad == 0, "%s: frag output needs C %% %d == 0", fn, kFragPad);
  if (B == 0 || H == 0) return VKWR_OK;
  VK_REQUIRE(pool && slots && r && w && k && v && a12 && g && k_k && a0 && k_a && r_k && ln_w && ln_b && out,
             "%s: null pointer", fn);
  auto h = [](const uint16_t* x) { return reinterpret_cast<const _Float16*>(x); };
  FusedArgs p{C, H, n_slots, out_frag, pool, slots, h(r), h(w), h(k), h(v), h(a12), h(g),
              h(k_k), h(a0), h(k_a), h(r_k), h(ln_w), h(ln_b), reinterpret_cast<_Float16*>(out)};
  if (state_layout == VKWR_WKV_STATE_ILV)
    hipLaunchKernelGGL(wkv7_decode_fused_kernel<true>, dim3(B * H), dim3(64), 0, (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL(wkv7_decode_fused_kernel<false>, dim3(B * H), dim3(64), 0, (hipStream_t)stream, p);
  return check_launch(fn);
}

extern "C" int vkwr_wkv7_state_layout_f32(int64_t n_blocks, const float* src, float* dst, int to_layout,
                                          void* stream) {
  clear_error();
  const char* fn = "vkwr_wkv7_state_layout_f32";
  VK_REQUIRE(n_blocks >= 0, "%s: negative size", fn);
  VK_REQUIRE(to_layout == VKWR_WKV_STATE_STD || to_layout == VKWR_WKV_STATE_ILV, "%s: bad layout", fn);
  if (n_blocks == 0) return VKWR_OK;
  VK_REQUIRE(src && dst && src != dst, "%s: null or aliased pointers", fn);
  VK_REQUIRE((((uintptr_t)src | (uintptr_t)dst) & 15) == 0, "%s: pointers must be 16-byte aligned", fn);
  const int64_t blocks = std::min<int64_t>((n_blocks * 1024 + 255) / 256, 16384);
  hipLaunchKernelGGL(wkv_state_layout_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, n_blocks,
                     src, dst, to_layout == VKWR_WKV_STATE_ILV);
  return check_launch(fn);
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
  // T > 1 with at most one wave per SIMD: the latency-scheduled form (same arithmetic)
  const bool seq = T > 1 && (int64_t)B * H <= 4 * (int64_t)device_cus();
  if (legacy) {
    if (seq) hipLaunchKernelGGL(wkv7_fp16_seq_kernel<true>, dim3(B * H), dim3(64), 0, (hipStream_t)stream, p);
    else hipLaunchKernelGGL(wkv7_fp16_kernel<true>, dim3(B * H), dim3(64), 0, (hipStream_t)stream, p);
  } else {
    if (seq) hipLaunchKernelGGL(wkv7_fp16_seq_kernel<false>, dim3(B * H), dim3(64), 0, (hipStream_t)stream, p);
    else hipLaunchKernelGGL(wkv7_fp16_kernel<false>, dim3(B * H), dim3(64), 0, (hipStream_t)stream, p);
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
