// Token sampling after the logits: temperature, optional presence / repetition
// penalties, top-k and top-p truncation, and one draw per batch row.
//
// Semantics (reference csrc/sampling/sampling.cu:134-359, 438-646, 648-835):
//   u_i   = sf((sf(l_i) - pen_i) * log2(e) / temperature)      (pen = 0 without penalties)
//   x_i   = 2^(u_i - max u)        (the softmax is p_i = x_i / S, S = sum x; every
//                                   test below is scale-free, so p is never formed)
//   tau   = the largest value v for which {x >= v} holds at least top_k entries or
//           at least top_p of the mass (sum >= top_p S): "not small"; top_p = 1
//           sets no mass limit
//   kept  = x_i for x_i > tau;  x_i * comp for x_i == tau, where
//           comp = clamp(min((top_p S - mass(x > tau)) / (tau * #(x == tau)),
//                                (top_k - #(x > tau)) / #(x == tau), 1), 0, 1)
//           (the first term only when top_p < 1)
//   token = inverse CDF of `kept` at a uniform draw in (0, 1], visiting the row in
//           lane order: lane 0's entries, then lane 1's, ... (the slots below);
//   with penalties, pen_i <- fma(pen_i, decay, i == token ? (pen_i == 0 ? presence
//                                                                 : repetition) : 0).
// sf() maps NaN to 0 and +-inf to +-FLT_MAX.  The reference finds tau by a 4-way
// bisection over float bit patterns and draws with its own two-level order over
// its 1024 threads; the kept weights, and so the law of the draw, are the same.
//
// Work split: one 1024-lane workgroup (16 waves) per batch row.  Lane t owns the
// float4 slots t, t + 1024, t + 2048, ... (so every load instruction of a wave is
// one contiguous 1 KiB); for V <= 65536 the lane keeps them in VGPRs for every
// pass, so the row is read from HBM once (and penalties twice).  Larger
// vocabularies (up to 2^20) keep the values in a caller scratch buffer.  Every
// reduction runs in a fixed order (DPP butterfly, then the 16 wave values in wave
// order), so results are run-to-run identical.
//
// Random numbers: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC'11), one counter block per draw: key = seed,
// counter = (draw index low, draw index high, row, 0); uniform = (x0 >> 8 + 1) / 2^24
// in (0, 1].  The reference draws with curand's Philox generator; its streams are
// not reproduced (parity of the random stream is not claimed).

#include <cfloat>

#include "vk_capi.h"
#include "vk_common.cuh"

namespace vk {
namespace {

constexpr int kSampThreads = 1024;
constexpr int kSampWaves = kSampThreads / 64;
constexpr int kCandCap = 1024;  // window entries compacted for the single-wave part of the search
constexpr int kCandPerLane = kCandCap / 64;
constexpr int kRankCap = 64;    // window size at which the search ranks the entries directly

struct PhiloxState {
  uint32_t key[2];
  uint32_t ctr[4];
  uint32_t reserved[2];
};
static_assert(sizeof(PhiloxState) == VKWR_SAMPLING_STATE_BYTES, "state size");

__host__ __device__ inline void philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
  uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
  uint32_t k0 = key_in[0], k1 = key_in[1];
  for (int r = 0; r < 10; ++r) {
    if (r > 0) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    c0 = hi1 ^ c1 ^ k0;
    c1 = lo1;
    c2 = hi0 ^ c3 ^ k1;
    c3 = lo0;
  }
  out[0] = c0;
  out[1] = c1;
  out[2] = c2;
  out[3] = c3;
}

__device__ __forceinline__ float sf(float x) {
  const float y = __builtin_isnan(x) ? 0.0f : x;
  return __builtin_isinf(y) ? __builtin_copysignf(FLT_MAX, y) : y;
}

// ---- wave-level primitives (DPP inside rows of 16 lanes, readlane across rows)
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float lane_read(float x, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}
// Butterfly over quad pairs, quads, half rows and rows (every lane of a row ends
// with the same bits: each step adds the same two partials, commuted), then the
// four row values in a fixed order.  The result is wave-uniform.
__device__ __forceinline__ float wave_sum(float x) {
  x += dpp<0xB1>(x);
  x += dpp<0x4E>(x);
  x += dpp<0x141>(x);
  x += dpp<0x140>(x);
  return (lane_read(x, 0) + lane_read(x, 16)) + (lane_read(x, 32) + lane_read(x, 48));
}
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp<0xB1>(x));
  x = fmaxf(x, dpp<0x4E>(x));
  x = fmaxf(x, dpp<0x141>(x));
  x = fmaxf(x, dpp<0x140>(x));
  return fmaxf(fmaxf(lane_read(x, 0), lane_read(x, 16)), fmaxf(lane_read(x, 32), lane_read(x, 48)));
}
__device__ __forceinline__ float wave_min(float x) {
  x = fminf(x, dpp<0xB1>(x));
  x = fminf(x, dpp<0x4E>(x));
  x = fminf(x, dpp<0x141>(x));
  x = fminf(x, dpp<0x140>(x));
  return fminf(fminf(lane_read(x, 0), lane_read(x, 16)), fminf(lane_read(x, 32), lane_read(x, 48)));
}
// Inclusive scan in lane order: Hillis-Steele inside each row (row_shr 1, 2, 4, 8
// with zero fill), then the totals of the rows before.
__device__ __forceinline__ float wave_incl_scan(float x, int lane) {
  x += dpp<0x111>(x);
  x += dpp<0x112>(x);
  x += dpp<0x114>(x);
  x += dpp<0x118>(x);
  const float r0 = lane_read(x, 15), r1 = lane_read(x, 31), r2 = lane_read(x, 47);
  const float r01 = r0 + r1;
  const int row = lane >> 4;
  return x + (row == 0 ? 0.0f : row == 1 ? r0 : row == 2 ? r01 : r01 + r2);
}
__device__ __forceinline__ int popc(uint64_t m) { return __builtin_popcountll(m); }
template <int CTRL>
__device__ __forceinline__ int dppi(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ int wave_incl_scan_i(int x, int lane) {
  x += dppi<0x111>(x);
  x += dppi<0x112>(x);
  x += dppi<0x114>(x);
  x += dppi<0x118>(x);
  const int r0 = __builtin_amdgcn_readlane(x, 15), r1 = __builtin_amdgcn_readlane(x, 31),
            r2 = __builtin_amdgcn_readlane(x, 47);
  const int row = lane >> 4;
  return x + (row == 0 ? 0 : row == 1 ? r0 : row == 2 ? r0 + r1 : r0 + r1 + r2);
}
__device__ __forceinline__ int wave_sum_i(int x) {
  x += dppi<0xB1>(x);
  x += dppi<0x4E>(x);
  x += dppi<0x141>(x);
  x += dppi<0x140>(x);
  return (__builtin_amdgcn_readlane(x, 0) + __builtin_amdgcn_readlane(x, 16)) +
         (__builtin_amdgcn_readlane(x, 32) + __builtin_amdgcn_readlane(x, 48));
}
__device__ __forceinline__ uint64_t ballot(bool b) { return __builtin_amdgcn_ballot_w64(b); }
__device__ __forceinline__ float fbits(uint32_t u) { return __builtin_bit_cast(float, u); }

// Block reductions publish one wave-uniform value set per wave and wait once; every
// lane then combines the 16 wave values in wave order, so all lanes hold the same
// totals.  Consecutive reductions alternate between two buffers: a wave can only
// overwrite a buffer after the next barrier, which every wave reaches only once it
// has finished reading that buffer.
struct SampShared {
  float fa[2][kSampWaves];
  float fb[2][kSampWaves];
  int ia[2][kSampWaves];
  int ib[2][kSampWaves];
  float u;
  int chosen;
  float tau, comp;
  float cand[kCandCap + 64];  // + one spare slot per lane for writes that are not kept
  alignas(16) float rank[kRankCap];
};

__device__ __forceinline__ void publish(SampShared& sh, int par, int wv, int lane, float a, float b, int c, int d) {
  if (lane == 0) {
    sh.fa[par][wv] = a;
    sh.fb[par][wv] = b;
    sh.ia[par][wv] = c;
    sh.ib[par][wv] = d;
  }
  __syncthreads();
}
__device__ __forceinline__ float sum_fa(const SampShared& sh, int par) {
  float s = sh.fa[par][0];
#pragma unroll
  for (int w = 1; w < kSampWaves; ++w) s += sh.fa[par][w];
  return s;
}
__device__ __forceinline__ int sum_ia(const SampShared& sh, int par) {
  int s = 0;
#pragma unroll
  for (int w = 0; w < kSampWaves; ++w) s += sh.ia[par][w];
  return s;
}

struct SampArgs {
  int T, V;
  const float* logits;  // [B, T, V]: row b uses token T-1
  float* penalties;     // [B, V] or nullptr
  PhiloxState* states;  // [B]
  int32_t* out;         // [B]
  float* scratch;       // [B, V] when J == 0
  float presence, repetition, decay;
  float log2e_inv_temp;
  int top_k;
  float top_p;
};

// Lane t of the workgroup of row b owns the float4 slots t + 1024 j of the row
// (elements 4 slot .. 4 slot + 3), j < J: in VGPRs for J > 0 (slots past the end
// of the row are padding with x = 0), in the scratch row for J == 0.
//
//   1. u = sf((sf(l) - pen) log2e / temperature); its maximum and minimum  (1 barrier)
//   2. x = 2^(u - u_max) (so x_max = 1 exactly), S = sum x                 (1 barrier)
//   3. tau by binary search over float bit patterns, from a first window [L, 1] whose
//      lower end comes from the lane maxima when top_k <= 1024 (1 barrier; below);
//      block-wide passes (count and mass of the entries >= the midpoint, 1 barrier
//      each) until the window [lo, hi] holds at most kCandCap entries; those are compacted into LDS and
//      wave 0 continues alone (no barriers) until at most kRankCap remain, which it
//      ranks directly; wave 0 publishes tau and comp                      (1 barrier)
//   4. kept weights; lane-order scan; owner lane of the draw; its pick (2 barriers)
//   5. penalties, re-read and updated with float4 accesses
//
// The slot loops are VALU-bound (64 entries per lane), so the common case skips the
// sf() clamps: every u = (l - pen) k is folded into fma(u, 0, acc), which becomes NaN
// exactly when some u is NaN or infinite.  If none is, both clamps were identities;
// a lane that meets one recomputes its slots with the clamps.
template <int J, bool PEN>
__global__ __launch_bounds__(kSampThreads) void sampling_kernel(SampArgs p) {
  __shared__ SampShared sh;
  const int b = blockIdx.x, t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int V = p.V, V4 = V >> 2;
  const int nslot = J > 0 ? J : (t < V4 ? (V4 - t + kSampThreads - 1) / kSampThreads : 0);
  const float4* lgb = reinterpret_cast<const float4*>(p.logits + ((size_t)b * p.T + (p.T - 1)) * V);
  float4* penb = PEN ? reinterpret_cast<float4*>(p.penalties + (size_t)b * V) : nullptr;
  float4* scr = J > 0 ? nullptr : reinterpret_cast<float4*>(p.scratch + (size_t)b * V) + t;
  float4 reg[J > 0 ? J : 1];
  auto get = [&](int j) -> float4 {
    if constexpr (J > 0) return reg[j];
    else return scr[(size_t)j * kSampThreads];
  };
  auto put = [&](int j, float4 v) {
    if constexpr (J > 0) reg[j] = v;
    else scr[(size_t)j * kSampThreads] = v;
  };
  auto valid = [&](int j) { return J > 0 ? t + j * kSampThreads < V4 : true; };
  // slot index clamped to the row: padding slots (J > 0) and the loads a batch issues
  // past a lane's last slot (J == 0) read the row's last slot, and are discarded
  const auto slot_of = [&](int j) -> uint32_t { return (uint32_t)min(t + j * kSampThreads, V4 - 1); };
  int par = 0;

  // This row's generator state: loaded now by wave 0, used once step 1's loads have
  // landed; only this workgroup reads or writes it.
  PhiloxState* st = p.states + b;
  uint4 ctr_in = make_uint4(0u, 0u, 0u, 0u);
  uint2 key_in = make_uint2(0u, 0u);
  if (wv == 0) {
    ctr_in = *reinterpret_cast<const uint4*>(st->ctr);
    key_in = *reinterpret_cast<const uint2*>(st->key);
  }

  // 1. u, its maximum and minimum.  Loads are issued before any result is used:
  // without penalties a lane has all its slots in flight at once, with penalties
  // (twice the registers) batches of 8.  Padding slots load the last slot: copies of
  // real values, which leave the maximum and minimum unchanged; they become -inf below.
  const float k = p.log2e_inv_temp;
  float mx = -INFINITY, mn = INFINITY;
  float nan_acc = 0.0f;  // becomes NaN once some u is NaN or infinite (u * 0 is NaN exactly then)
  const auto scale = [&](int j, float4 l, float4 q) {
    const float4 u = make_float4((l.x - q.x) * k, (l.y - q.y) * k, (l.z - q.z) * k, (l.w - q.w) * k);
    nan_acc = __builtin_fmaf(u.x, 0.0f, nan_acc);
    nan_acc = __builtin_fmaf(u.y, 0.0f, nan_acc);
    nan_acc = __builtin_fmaf(u.z, 0.0f, nan_acc);
    nan_acc = __builtin_fmaf(u.w, 0.0f, nan_acc);
    put(j, u);
    mx = fmaxf(mx, fmaxf(fmaxf(u.x, u.y), fmaxf(u.z, u.w)));
    mn = fminf(mn, fminf(fminf(u.x, u.y), fminf(u.z, u.w)));
  };
  if constexpr (!PEN && J > 0) {
#pragma unroll
    for (int j = 0; j < J; ++j) reg[j] = lgb[slot_of(j)];
#pragma unroll
    for (int j = 0; j < J; ++j) scale(j, reg[j], make_float4(0.0f, 0.0f, 0.0f, 0.0f));
  } else {
    constexpr int kPB = PEN ? (J > 4 ? 4 : (J > 0 ? J : 4)) : (J > 8 ? 8 : (J > 0 ? J : 8));
    for (int j0 = 0; j0 < nslot; j0 += kPB) {
      // the previous batch is finished (mx depends on it) before this one loads
      asm volatile("" : "+v"(mx)::"memory");
      float4 l[kPB], q[kPB];
#pragma unroll
      for (int jj = 0; jj < kPB; ++jj) {
        l[jj] = lgb[slot_of(j0 + jj)];
        q[jj] = PEN ? penb[slot_of(j0 + jj)] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
#pragma unroll
      for (int jj = 0; jj < kPB; ++jj) {
        if (J == 0 && j0 + jj >= nslot) break;
        scale(j0 + jj, l[jj], q[jj]);
      }
    }
  }
  if (__builtin_isnan(nan_acc)) {
    // NaN or infinity somewhere in this lane's slots: u = sf((sf(l) - pen) k)
    mx = -INFINITY;
    mn = INFINITY;
    int tt = t;  // opaque copy: the fast path's addresses are not kept alive for this path
    asm volatile("" : "+v"(tt));
    for (int j = 0; j < nslot; ++j) {
      const uint32_t sj = (uint32_t)min(tt + j * kSampThreads, V4 - 1);
      const float4 l = lgb[sj];
      const float4 q = PEN ? penb[sj] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      const float4 u = make_float4(sf((sf(l.x) - q.x) * k), sf((sf(l.y) - q.y) * k), sf((sf(l.z) - q.z) * k),
                                   sf((sf(l.w) - q.w) * k));
      put(j, u);
      mx = fmaxf(mx, fmaxf(fmaxf(u.x, u.y), fmaxf(u.z, u.w)));
      mn = fminf(mn, fminf(fminf(u.x, u.y), fminf(u.z, u.w)));
    }
  }
  if (J > 0 && t + (nslot - 1) * kSampThreads >= V4) {
    // this lane holds padding: u = -inf there, so x = 0
#pragma unroll
    for (int j = 0; j < nslot; ++j)
      if (!valid(j)) put(j, make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY));
  }
  mx = wave_max(mx);
  mn = wave_min(mn);
  publish(sh, par, wv, lane, mx, mn, 0, 0);
  float umax = sh.fa[par][0], umin = sh.fb[par][0];
#pragma unroll
  for (int w = 1; w < kSampWaves; ++w) {
    umax = fmaxf(umax, sh.fa[par][w]);
    umin = fminf(umin, sh.fb[par][w]);
  }
  par ^= 1;
  if (wv == 0) {
    // this call's uniform in (0, 1], and the state advanced to the next counter block
    const uint32_t key[2] = {key_in.x, key_in.y}, ctr[4] = {ctr_in.x, ctr_in.y, ctr_in.z, ctr_in.w};
    uint32_t x[4];
    philox4x32_10(ctr, key, x);
    if (lane == 0) {
      sh.u = (float)((x[0] >> 8) + 1) * (1.0f / 16777216.0f);
      const uint32_t c0 = ctr[0] + 1u;
      st->ctr[0] = c0;
      st->ctr[1] = ctr[1] + (c0 == 0u ? 1u : 0u);
    }
  }

  // 2. x = 2^(u - umax) (v_exp_f32: weights below 2^-126 of the largest count as 0;
  // padding gives 2^-inf = 0)
  float s = 0.0f, lane_xmax = 0.0f;
#pragma unroll
  for (int j = 0; j < nslot; ++j) {
    const float4 u = get(j);
    float4 x = make_float4(__builtin_amdgcn_exp2f(u.x - umax), __builtin_amdgcn_exp2f(u.y - umax),
                           __builtin_amdgcn_exp2f(u.z - umax), __builtin_amdgcn_exp2f(u.w - umax));
    put(j, x);
    s += (x.x + x.y) + (x.z + x.w);
    lane_xmax = fmaxf(lane_xmax, fmaxf(fmaxf(x.x, x.y), fmaxf(x.z, x.w)));
  }
  const float lane_sum = s;
  s = wave_sum(s);
  publish(sh, par, wv, lane, s, 0.0f, 0, 0);
  const float S = sum_fa(sh, par);
  par ^= 1;

  // 3. threshold
  const bool use_mass = p.top_p < 1.0f;  // top_p = 1: no mass limit
  const bool truncate = p.top_k < V || use_mass;
  const float goal = p.top_p * S;        // top_p of the mass, in units of x
  float tau = 0.0f, comp = 1.0f;
  if (truncate && p.top_k == 1 && !use_mass) {
    // greedy: tau is the maximum (x = 1); ties keep equal weights whatever comp is
    tau = 1.0f;
  } else if (truncate) {
    // Invariants: notsmall(lo) (or lo below every positive entry, which gives the
    // same kept weights), !notsmall(hi + 1); cnt_lo = #(x >= lo) once known,
    // cnt_hi1 = #(x > hi), m_hi1 = mass(x > hi).
    const float xmin = __builtin_amdgcn_exp2f(umin - umax);
    uint32_t lo = max(__builtin_bit_cast(uint32_t, xmin), 1u), hi = __builtin_bit_cast(uint32_t, 1.0f);
    int cnt_lo = 0x7fffffff, cnt_hi1 = 0;
    float m_hi1 = 0.0f;
    const auto decide = [&](uint32_t mid, int C, float M) {
      if (C >= p.top_k || (use_mass && M >= goal)) {
        lo = mid;
        cnt_lo = C;
      } else {
        hi = mid - 1u;
        cnt_hi1 = C;
        m_hi1 = M;
      }
    };
    // Window count: wc = this lane's entries in [lo, hi], at = the lane-order index of its
    // first one, n = the block total.  Valid while `counted` (lo and hi unchanged since).
    int wc = 0, at = 0, n = 0;
    bool counted = false;
    const auto window_count = [&]() {
      const float lof = fbits(lo), hif = fbits(hi);
      wc = 0;
#pragma unroll
      for (int j = 0; j < nslot; ++j) {
        const float4 x = get(j);
        const float e[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) wc += (e[q] >= lof && e[q] <= hif) ? 1 : 0;
      }
      const int wincl = wave_incl_scan_i(wc, lane);
      publish(sh, par, wv, lane, 0.0f, 0.0f, __builtin_amdgcn_readlane(wincl, 63), 0);
      at = wincl - wc;
      for (int w = 0; w < wv; ++w) at += sh.ia[par][w];
      n = sum_ia(sh, par);
      par ^= 1;
      counted = true;
    };
    if (J > 0 && p.top_k <= kSampThreads) {
      // A first window from the lane maxima.  In each wave, the q-th largest of its 64 lane
      // maxima (q = ceil(top_k / 16); one lane per step, so ties count once per lane) is at
      // or below q distinct entries of the wave; the smallest of the 16 such values, L, has
      // at least 16 q >= top_k entries at or above it.  So notsmall(L): tau >= L, and the
      // window [L, 1] usually holds a few hundred entries, where the bisection from the
      // smallest entry would take three block-wide passes to get below kCandCap.
      const int q = (p.top_k + kSampWaves - 1) / kSampWaves;
      float lm = lane_xmax, lw = 0.0f;
      for (int i = 0; i < q; ++i) {
        lw = wave_max(lm);
        const uint64_t hit = ballot(lm == lw);  // nonzero: lw is some lane's value
        if (lane == (int)__builtin_ctzll(hit)) lm = -1.0f;
      }
      publish(sh, par, wv, lane, lw, 0.0f, 0, 0);
      float L = sh.fa[par][0];
#pragma unroll
      for (int w = 1; w < kSampWaves; ++w) L = fminf(L, sh.fa[par][w]);
      par ^= 1;
      const uint32_t Lb = __builtin_bit_cast(uint32_t, L);
      if (L > 0.0f && Lb > lo) {
        lo = Lb;
        window_count();
        cnt_lo = n;  // #(x >= lo); cnt_hi1 = 0 (nothing exceeds 1 = the maximum)
      }
    }
    // block-wide passes over every entry
    while (lo < hi && cnt_lo - cnt_hi1 > kCandCap) {
      counted = false;
      const uint32_t mid = lo + (hi - lo + 1u) / 2u;
      const float v = fbits(mid);
      int c = 0;
      float m = 0.0f;
#pragma unroll
      for (int j = 0; j < nslot; ++j) {
        const float4 x = get(j);
        const float e[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const bool ge = e[q] >= v;
          c += ge ? 1 : 0;
          m += ge ? e[q] : 0.0f;
        }
      }
      c = wave_sum_i(c);
      m = use_mass ? wave_sum(m) : 0.0f;
      publish(sh, par, wv, lane, m, 0.0f, c, 0);
      const int C = sum_ia(sh, par);
      const float M = sum_fa(sh, par);
      par ^= 1;
      decide(mid, C, M);
    }
    if (lo < hi) {
      // compact the window [lo, hi] (at most kCandCap entries; lo > 0, so padding
      // never falls in it) into LDS in lane order
      if (!counted) window_count();
#pragma unroll
      for (int j = 0; j < nslot; ++j) {
        const float4 x = get(j);
        const float e[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          // the window test again, on the bit patterns (the same test for
          // non-negative floats), so that the compiler does not keep the first
          // sweep's results alive across the barrier.  A few hundred of the row's
          // entries are in the window, so most (slot, element) positions hold none in
          // any lane of the wave: the wave skips those (a uniform branch on the ballot).
          const bool in = __builtin_bit_cast(uint32_t, e[q]) - lo <= hi - lo;
          if (ballot(in) != 0) {
            sh.cand[in ? min(at, kCandCap) : kCandCap + lane] = e[q];
            at += in ? 1 : 0;
          }
        }
      }
      __syncthreads();
      if (wv == 0) {
        // wave 0 alone: count(v) = c0 + #(cand >= v), mass(v) = m0 + sum(cand >= v)
        const int c0 = cnt_hi1;
        const float m0 = m_hi1;
        float cd[kCandPerLane];
#pragma unroll
        for (int i = 0; i < kCandPerLane; ++i) cd[i] = lane + 64 * i < n ? sh.cand[lane + 64 * i] : -1.0f;
        while (lo < hi && cnt_lo - cnt_hi1 > kRankCap) {
          const uint32_t mid = lo + (hi - lo + 1u) / 2u;
          const float v = fbits(mid);
          int c = 0;
          float m = 0.0f;
#pragma unroll
          for (int i = 0; i < kCandPerLane; ++i) {
            const bool ge = cd[i] >= v;
            c += ge ? 1 : 0;
            m += ge ? cd[i] : 0.0f;
          }
          decide(mid, c0 + wave_sum_i(c), use_mass ? m0 + wave_sum(m) : 0.0f);
        }
        tau = fbits(lo);
        if (lo < hi) {
          // at most kRankCap entries in [lo, hi]: gather them (in lane order) and
          // test each one directly; tau is the largest that is not small
          const float lof2 = fbits(lo), hif2 = fbits(hi);
          sh.rank[lane] = -1.0f;  // unused slots never count
          int base = 0;
#pragma unroll
          for (int i = 0; i < kCandPerLane; ++i) {
            const bool in = cd[i] >= lof2 && cd[i] <= hif2;
            const uint64_t msk = ballot(in);
            const int at2 = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(msk >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)msk, 0u));
            if (in && at2 < kRankCap) sh.rank[at2] = cd[i];
            base += popc(msk);
          }
          const int nr = min(base, kRankCap);
          const float mine = lane < nr ? sh.rank[lane] : -1.0f;
          int c = 0;
          float m = 0.0f;
#pragma unroll 2
          for (int r = 0; r < kRankCap; r += 4) {
            const float4 e4 = *reinterpret_cast<const float4*>(&sh.rank[r]);
            const float e[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              c += e[q] >= mine ? 1 : 0;
              m += e[q] >= mine ? e[q] : 0.0f;
            }
          }
          const bool ok = lane < nr && (cnt_hi1 + c >= p.top_k || (use_mass && m_hi1 + m >= goal));
          const float best = wave_max(ok ? mine : -1.0f);
          tau = best >= 0.0f ? best : wave_min(lane < nr ? mine : INFINITY);
        }
        // entries above and at tau
        int ngt = 0, neq = 0;
        float mgt = 0.0f;
#pragma unroll
        for (int i = 0; i < kCandPerLane; ++i) {
          ngt += cd[i] > tau ? 1 : 0;
          neq += cd[i] == tau ? 1 : 0;
          mgt += cd[i] > tau ? cd[i] : 0.0f;
        }
        const int NGT = c0 + wave_sum_i(ngt), NEQ = wave_sum_i(neq);
        const float MGT = m0 + (use_mass ? wave_sum(mgt) : 0.0f);
        if (NEQ > 0) {
          comp = fminf((float)(p.top_k - NGT) / (float)NEQ, 1.0f);
          if (use_mass) comp = fminf(sf((goal - MGT) / (tau * (float)NEQ)), comp);
          comp = fmaxf(comp, 0.0f);
        }
        if (lane == 0) {
          sh.tau = tau;
          sh.comp = comp;
        }
      }
      __syncthreads();
      tau = sh.tau;
      comp = sh.comp;
    } else {
      // the search ended over more than kCandCap entries (ties): count them all
      tau = fbits(lo);
      int ngt = 0, neq = 0;
      float mgt = 0.0f;
#pragma unroll
      for (int j = 0; j < nslot; ++j) {
        const float4 x = get(j);
        const float e[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {  // tau > 0: padding is never counted
          ngt += e[q] > tau ? 1 : 0;
          neq += e[q] == tau ? 1 : 0;
          mgt += e[q] > tau ? e[q] : 0.0f;
        }
      }
      ngt = wave_sum_i(ngt);
      neq = wave_sum_i(neq);
      mgt = use_mass ? wave_sum(mgt) : 0.0f;
      publish(sh, par, wv, lane, mgt, 0.0f, ngt, neq);
      const int NGT = sum_ia(sh, par);
      const float MGT = sum_fa(sh, par);
      int NEQ = 0;
#pragma unroll
      for (int w = 0; w < kSampWaves; ++w) NEQ += sh.ib[par][w];
      par ^= 1;
      if (NEQ > 0) {
        comp = fminf((float)(p.top_k - NGT) / (float)NEQ, 1.0f);
        if (use_mass) comp = fminf(sf((goal - MGT) / (tau * (float)NEQ)), comp);
        comp = fmaxf(comp, 0.0f);
      }
    }
  }

  // 4. kept weights and the draw (inverse CDF in lane order)
  float wsum = lane_sum;
  if (truncate) {
    wsum = 0.0f;
#pragma unroll
    for (int j = 0; j < nslot; ++j) {
      float4 x = get(j);
      x.x = x.x > tau ? x.x : (x.x == tau ? x.x * comp : 0.0f);
      x.y = x.y > tau ? x.y : (x.y == tau ? x.y * comp : 0.0f);
      x.z = x.z > tau ? x.z : (x.z == tau ? x.z * comp : 0.0f);
      x.w = x.w > tau ? x.w : (x.w == tau ? x.w * comp : 0.0f);
      put(j, x);
      wsum += (x.x + x.y) + (x.z + x.w);
    }
  }
  const float wincl = wave_incl_scan(wsum, lane);
  publish(sh, par, wv, lane, lane_read(wincl, 63), 0.0f, 0, 0);
  float pre = 0.0f;
  for (int w = 0; w < wv; ++w) pre += sh.fa[par][w];
  const float total = sum_fa(sh, par);
  par ^= 1;
  const float incl = pre + wincl;
  const float target = total * sh.u;  // written by wave 0 before several barriers
  // owner: the first lane holding weight whose inclusive prefix reaches the target,
  // else (prefixes short of the target by rounding) the last lane holding weight
  const bool pos = wsum > 0.0f;
  const uint64_t mge = ballot(pos && incl >= target), mpos = ballot(pos);
  publish(sh, par, wv, lane, 0.0f, 0.0f, mge ? wv * 64 + __builtin_ctzll(mge) : 0x7fffffff,
          mpos ? wv * 64 + 63 - __builtin_clzll(mpos) : -1);
  int first = 0x7fffffff, last = -1;
#pragma unroll
  for (int w = 0; w < kSampWaves; ++w) {
    first = min(first, sh.ia[par][w]);
    last = max(last, sh.ib[par][w]);
  }
  par ^= 1;
  const int owner = first != 0x7fffffff ? first : last;
  if (t == owner) {
    float run = incl - wsum;
    int pick = -1, lastk = -1;
    for (int j = 0; j < nslot; ++j) {
      const float4 x = get(j);
      const float e[4] = {x.x, x.y, x.z, x.w};
      for (int q = 0; q < 4; ++q) {
        const int idx = 4 * (t + j * kSampThreads) + q;
        run += e[q];
        const bool w = e[q] > 0.0f;
        lastk = w ? idx : lastk;
        pick = (pick < 0 && w && run >= target) ? idx : pick;
      }
    }
    const int tok = pick >= 0 ? pick : lastk;
    p.out[b] = tok;
    sh.chosen = tok;
  }

  // 5. penalties (loads of a batch issued together, stores masked)
  if constexpr (PEN) {
    __syncthreads();
    const int tok = sh.chosen;
    const float d = p.decay;
    // slot indices recomputed from an opaque copy of t: otherwise the compiler keeps
    // step 1's indices alive across the whole kernel
    int tt = t;
    asm volatile("" : "+v"(tt));
    const auto pslot = [&](int j) -> uint32_t {
      return (uint32_t)((j < nslot && tt + j * kSampThreads < V4) ? tt + j * kSampThreads : 0);
    };
    constexpr int kBatch = J > 0 ? J : 8;
    for (int j0 = 0; j0 < nslot; j0 += kBatch) {
      float4 q[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) q[j] = penb[pslot(j0 + j)];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int i0 = 4 * (tt + (j0 + j) * kSampThreads);
        float e[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
        for (int c = 0; c < 4; ++c)
          e[c] = __builtin_fmaf(e[c], d, i0 + c == tok ? (e[c] == 0.0f ? p.presence : p.repetition) : 0.0f);
        if (j0 + j < nslot && tt + (j0 + j) * kSampThreads < V4)
          penb[(uint32_t)(tt + (j0 + j) * kSampThreads)] = make_float4(e[0], e[1], e[2], e[3]);
      }
    }
  }
}

__global__ void setup_rand_kernel(PhiloxState* st, uint64_t seed, int B) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  PhiloxState s;
  s.key[0] = (uint32_t)seed;
  s.key[1] = (uint32_t)(seed >> 32);
  s.ctr[0] = 0;
  s.ctr[1] = 0;
  s.ctr[2] = (uint32_t)b;
  s.ctr[3] = 0;
  s.reserved[0] = s.reserved[1] = 0;
  st[b] = s;
}

int launch_sampling(const char* fn, int B, int T, int V, const float* logits, float* penalties, void* states,
                    int32_t* out, float* scratch, float presence, float repetition, float decay,
                    double temperature, int top_k, double top_p, void* stream) {
  VK_REQUIRE(B > 0 && T > 0, "%s: B and T must be positive, got B=%d, T=%d", fn, B, T);
  VK_REQUIRE(V > 0 && V <= 1048576 && V % 4 == 0,
             "%s: vocabulary size must be a multiple of 4 and at most 1048576, got %d", fn, V);
  VK_REQUIRE(temperature >= 0.001 && temperature <= 1000, "%s: temperature %g outside [0.001, 1000]", fn,
             temperature);
  VK_REQUIRE(logits && states && out, "%s: null pointer", fn);
  VK_REQUIRE(((uintptr_t)logits | (uintptr_t)penalties) % 16 == 0, "%s: logits and penalties must be 16-byte aligned",
             fn);
  if (top_k <= 0 || top_k > V) top_k = V;
  if (top_p < 0 || top_p > 1) top_p = 1;
  if (top_p == 0) {
    top_k = 1;
    top_p = 1;
  }
  SampArgs a{};
  a.T = T;
  a.V = V;
  a.logits = logits;
  a.penalties = penalties;
  a.states = reinterpret_cast<PhiloxState*>(states);
  a.out = out;
  a.scratch = scratch;
  a.presence = presence;
  a.repetition = repetition;
  a.decay = decay;
  a.log2e_inv_temp = (float)(1.4426950408889634 / temperature);
  a.top_k = top_k;
  a.top_p = (float)top_p;
  const int slots = (V / 4 + kSampThreads - 1) / kSampThreads;  // float4 slots per lane
  VK_REQUIRE(slots <= 16 || scratch != nullptr,
             "%s: vocabularies above 65536 need a scratch buffer of B*V floats", fn);
  VK_REQUIRE((uintptr_t)scratch % 16 == 0, "%s: scratch must be 16-byte aligned", fn);
  const dim3 grid(B), block(kSampThreads);
  hipStream_t s = (hipStream_t)stream;
  if (penalties) {
    if (slots <= 1) hipLaunchKernelGGL((sampling_kernel<1, true>), grid, block, 0, s, a);
    else if (slots <= 4) hipLaunchKernelGGL((sampling_kernel<4, true>), grid, block, 0, s, a);
    else if (slots <= 16) hipLaunchKernelGGL((sampling_kernel<16, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((sampling_kernel<0, true>), grid, block, 0, s, a);
  } else {
    if (slots <= 1) hipLaunchKernelGGL((sampling_kernel<1, false>), grid, block, 0, s, a);
    else if (slots <= 4) hipLaunchKernelGGL((sampling_kernel<4, false>), grid, block, 0, s, a);
    else if (slots <= 16) hipLaunchKernelGGL((sampling_kernel<16, false>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((sampling_kernel<0, false>), grid, block, 0, s, a);
  }
  return check_launch(fn);
}

}  // namespace
}  // namespace vk

using namespace vk;

extern "C" int vkwr_sampling_setup_rand(int64_t seed, int B, void* states, void* stream) {
  clear_error();
  const char* fn = "vkwr_sampling_setup_rand";
  VK_REQUIRE(B > 0, "%s: B must be positive", fn);
  VK_REQUIRE(states != nullptr, "%s: null pointer", fn);
  hipLaunchKernelGGL(setup_rand_kernel, dim3((B + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<PhiloxState*>(states), (uint64_t)seed, B);
  return check_launch(fn);
}

extern "C" int vkwr_sampling_temperature_topk_topp(int B, int T, int V, const float* logits, void* states,
                                                   int32_t* out, float* scratch, double temperature, int top_k,
                                                   double top_p, void* stream) {
  clear_error();
  return launch_sampling("vkwr_sampling_temperature_topk_topp", B, T, V, logits, nullptr, states, out, scratch,
                         0.0f, 0.0f, 1.0f, temperature, top_k, top_p, stream);
}

extern "C" int vkwr_sampling_repetition_topk_topp(int B, int T, int V, const float* logits, float* penalties,
                                                  void* states, int32_t* out, float* scratch,
                                                  double presence_penalty, double repetition_penalty,
                                                  double penalty_decay, double temperature, int top_k,
                                                  double top_p, void* stream) {
  clear_error();
  const char* fn = "vkwr_sampling_repetition_topk_topp";
  VK_REQUIRE(penalties != nullptr, "%s: null penalties", fn);
  return launch_sampling(fn, B, T, V, logits, penalties, states, out, scratch, (float)presence_penalty,
                         (float)repetition_penalty, (float)penalty_decay, temperature, top_k, top_p, stream);
}

extern "C" void vkwr_sampling_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  philox4x32_10(ctr, key, out);
}
