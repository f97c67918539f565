// Token sampling after the logits: temperature, optional presence / repetition
// penalties, top-k and top-p truncation, and one draw per batch row.
//
// Semantics (reference csrc/sampling/sampling.cu:134-359, 438-646, 648-835):
//   u_i   = sf((sf(l_i) - pen_i) * log2(e) / temperature)      (pen = 0 without penalties)
//   p_i   = 2^(u_i - max u) / sum_j 2^(u_j - max u)
//   tau   = the largest p value v for which {p >= v} holds at least top_k entries
//           or at least top_p of the mass ("not small");
//   kept  = p_i for p_i > tau;  p_i * comp for p_i == tau, where
//           comp = clamp(min((top_p - mass(p > tau)) / (tau * #(p == tau)),
//                                (top_k - #(p > tau)) / #(p == tau), 1), 0, 1)
//   token = inverse CDF of `kept` (vocabulary order) at a uniform draw in (0, 1];
//   with penalties, pen_i <- fma(pen_i, decay, i == token ? (pen_i == 0 ? presence
//                                                                 : repetition) : 0).
// sf() maps NaN to 0 and +-inf to +-FLT_MAX.  The reference finds tau by a 4-way
// bisection over float bit patterns and draws with a two-level scheme over its
// 1024 threads; this file finds the same tau by a binary search over bit patterns
// and draws by inverse CDF in vocabulary order: the kept weights and the law of
// the draw are the same.
//
// Work split: one 1024-lane workgroup (16 waves) per batch row.  Lane t owns the
// contiguous elements [t*PER, t*PER + PER) of the row; for V <= 65536 the lane
// keeps them in VGPRs (PER <= 64) for every pass -- max, sum, the ~30 passes of
// the threshold search, the draw -- so the row is read from HBM once.  Larger
// vocabularies (up to 2^20) keep the probabilities in a caller scratch buffer.
// Every reduction runs in a fixed order (wave butterfly, then the 16 wave values
// in wave order), so results are run-to-run identical.
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

// ---- block-wide reductions over the 16 waves, fixed order
__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
__device__ __forceinline__ float wave_min_f(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fminf(v, __shfl_xor(v, m, 64));
  return v;
}

struct SampShared {
  float f[kSampWaves];
  int i[kSampWaves];
  float f2[kSampWaves];
  float bcast_f[4];
  int bcast_i[4];
};

// Sum of one float and one int per lane over the workgroup; every lane gets both.
// The wave values are added in wave order by lane 0 of wave 0 (deterministic).
__device__ __forceinline__ void block_sum2(SampShared& sh, float fv, int iv, float& fo, int& io) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  fv = wave_sum_f(fv);
  iv = wave_sum_i(iv);
  if (lane == 0) {
    sh.f[wv] = fv;
    sh.i[wv] = iv;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float fs = 0.0f;
    int is = 0;
    for (int w = 0; w < kSampWaves; ++w) {
      fs += sh.f[w];
      is += sh.i[w];
    }
    sh.bcast_f[0] = fs;
    sh.bcast_i[0] = is;
  }
  __syncthreads();
  fo = sh.bcast_f[0];
  io = sh.bcast_i[0];
  __syncthreads();
}

__device__ __forceinline__ void block_minmax(SampShared& sh, float mn, float mx, float& mno, float& mxo) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  mn = wave_min_f(mn);
  mx = wave_max_f(mx);
  if (lane == 0) {
    sh.f[wv] = mn;
    sh.f2[wv] = mx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float a = sh.f[0], b = sh.f2[0];
    for (int w = 1; w < kSampWaves; ++w) {
      a = fminf(a, sh.f[w]);
      b = fmaxf(b, sh.f2[w]);
    }
    sh.bcast_f[0] = a;
    sh.bcast_f[1] = b;
  }
  __syncthreads();
  mno = sh.bcast_f[0];
  mxo = sh.bcast_f[1];
  __syncthreads();
}

// Inclusive scan of one float per lane over the workgroup (lane order); also the total.
__device__ __forceinline__ float block_scan(SampShared& sh, float v, float& total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  float x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const float y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) sh.f[wv] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    float run = 0.0f;
    for (int w = 0; w < kSampWaves; ++w) {
      const float t = sh.f[w];
      sh.f2[w] = run;  // exclusive prefix of wave w
      run += t;
    }
    sh.bcast_f[2] = run;
  }
  __syncthreads();
  const float r = x + sh.f2[wv];
  total = sh.bcast_f[2];
  __syncthreads();
  return r;
}

struct SampArgs {
  int T, V;
  const float* logits;  // [B, T, V]: row b uses token T-1
  float* penalties;     // [B, V] or nullptr
  PhiloxState* states;  // [B]
  int32_t* out;         // [B]
  float* scratch;       // [B, V] when PER == 0
  float presence, repetition, decay;
  float log2e_inv_temp;
  int top_k;
  float top_p;
  int per;  // elements per lane (runtime; PER template bounds it for registers)
};

// PER > 0: the lane's elements live in VGPRs (PER >= p.per); PER == 0: in p.scratch.
// In register mode a lane past the end of the row holds padding entries with
// u = -inf, i.e. probability exactly 0 -- the same as a real entry whose
// probability underflowed, which changes neither tau (counts and masses at any
// v > 0 are unaffected, and at v = 0 only zeros are added) nor the kept weights.
template <int PER>
__global__ __launch_bounds__(kSampThreads) void sampling_kernel(SampArgs p) {
  __shared__ SampShared sh;
  __shared__ int chosen;
  const int b = blockIdx.x, t = threadIdx.x;
  const int V = p.V;
  const int per = PER > 0 ? PER : p.per;
  const int c0 = t * per, c1 = min(V, c0 + per);
  const float* lg = p.logits + ((size_t)b * p.T + (p.T - 1)) * V;
  float* pen = p.penalties ? p.penalties + (size_t)b * V : nullptr;
  float* scr = PER > 0 ? nullptr : p.scratch + (size_t)b * V;

  float reg[PER > 0 ? PER : 1];
  auto get = [&](int e) -> float { return PER > 0 ? reg[e] : scr[c0 + e]; };
  auto set = [&](int e, float v) {
    if constexpr (PER > 0) reg[e] = v;
    else scr[c0 + e] = v;
  };
  // entries this lane walks: all PER registers (padding included), or its valid range
  const int lim = PER > 0 ? PER : max(0, c1 - c0);

  // 1. scaled logits and their maximum
  float mx = -INFINITY;
  if constexpr (PER > 0) {
#pragma unroll
    for (int j = 0; j < PER; j += 4) {
      const bool valid = c0 + j < V;  // V and PER are multiples of 4: whole vectors
      const int i = valid ? c0 + j : 0;
      const float4 l4 = *reinterpret_cast<const float4*>(lg + i);
      float4 p4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (pen) p4 = *reinterpret_cast<const float4*>(pen + i);
      const float lv[4] = {l4.x, l4.y, l4.z, l4.w}, pv[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float u = valid ? sf((sf(lv[q]) - pv[q]) * p.log2e_inv_temp) : -INFINITY;
        reg[j + q] = u;
        mx = fmaxf(mx, u);
      }
    }
  } else {
    for (int e = 0; e < lim; ++e) {
      const float pe = pen ? pen[c0 + e] : 0.0f;
      const float u = sf((sf(lg[c0 + e]) - pe) * p.log2e_inv_temp);
      set(e, u);
      mx = fmaxf(mx, u);
    }
  }
  float gmin, gmax;
  block_minmax(sh, INFINITY, mx, gmin, gmax);
  // 2. softmax
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < lim; ++e) {
    const float x = exp2f(get(e) - gmax);
    set(e, x);
    s += x;
  }
  float denom;
  int dummy;
  block_sum2(sh, s, 0, denom, dummy);
  float pmn = INFINITY, pmx = -INFINITY;
#pragma unroll
  for (int e = 0; e < lim; ++e) {
    const float q = get(e) / denom;
    set(e, q);
    pmn = fminf(pmn, q);
    pmx = fmaxf(pmx, q);
  }
  float pmin, pmax;
  block_minmax(sh, pmn, pmx, pmin, pmax);

  // 3. threshold: largest p value v whose set {p >= v} is not small
  auto count_mass = [&](float v, int& cnt, float& mass) {
    int c = 0;
    float m = 0.0f;
#pragma unroll
    for (int e = 0; e < lim; ++e) {
      const float q = get(e);
      if (q >= v) {
        ++c;
        m += q;
      }
    }
    block_sum2(sh, m, c, mass, cnt);
  };
  const bool truncate = p.top_k < V || p.top_p < 1.0f;
  float tau = 0.0f, comp = 1.0f;
  if (truncate) {
    uint32_t lo = __builtin_bit_cast(uint32_t, pmin), hi = __builtin_bit_cast(uint32_t, pmax);
    while (lo < hi) {
      const uint32_t mid = lo + (hi - lo + 1) / 2;
      int cnt;
      float mass;
      count_mass(__builtin_bit_cast(float, mid), cnt, mass);
      if (cnt >= p.top_k || mass >= p.top_p) lo = mid;
      else hi = mid - 1;
    }
    tau = __builtin_bit_cast(float, lo);
    int neq = 0, ngt = 0;
    float mgt = 0.0f;
#pragma unroll
    for (int e = 0; e < lim; ++e) {
      const float q = get(e);
      if (q == tau) ++neq;
      if (q > tau) {
        ++ngt;
        mgt += q;
      }
    }
    int gneq, gngt;
    float gmgt, unused;
    block_sum2(sh, mgt, ngt, gmgt, gngt);
    block_sum2(sh, 0.0f, neq, unused, gneq);
    if (gneq > 0) {
      comp = fminf(sf((p.top_p - gmgt) / (tau * (float)gneq)), 1.0f);
      comp = fminf(sf((float)(p.top_k - gngt) / (float)gneq), comp);
      comp = fmaxf(comp, 0.0f);
    }
  }
  auto kept = [&](float q) -> float {
    if (!truncate) return q;
    return q > tau ? q : (q == tau ? q * comp : 0.0f);
  };

  // 4. draw: inverse CDF of the kept weights in vocabulary order (the lane's
  // entries are replaced by their kept weights)
  float wsum = 0.0f;
#pragma unroll
  for (int e = 0; e < lim; ++e) {
    const float w = kept(get(e));
    set(e, w);
    wsum += w;
  }
  float total;
  const float incl = block_scan(sh, wsum, total);
  const float excl = incl - wsum;
  PhiloxState* st = p.states + b;
  __shared__ float target_sh;
  if (t == 0) {
    uint32_t x[4];
    philox4x32_10(st->ctr, st->key, x);
    const float u = (float)((x[0] >> 8) + 1) * (1.0f / 16777216.0f);  // (0, 1]
    target_sh = total * u;
    chosen = -1;
    // next draw
    if (++st->ctr[0] == 0) ++st->ctr[1];
  }
  __syncthreads();
  const float target = target_sh;
  // the lowest lane holding weight whose inclusive prefix reaches the target (if the
  // float prefixes stop short of the target by rounding: the last lane holding weight)
  __shared__ int lane_lo, lane_hi;
  if (t == 0) {
    lane_lo = kSampThreads;
    lane_hi = -1;
  }
  __syncthreads();
  if (wsum > 0.0f) {
    if (incl >= target) atomicMin(&lane_lo, t);
    atomicMax(&lane_hi, t);
  }
  __syncthreads();
  const int owner = lane_lo < kSampThreads ? lane_lo : lane_hi;
  if (t == owner) {
    // first kept entry whose running sum reaches the target, else the lane's last kept entry
    float run = excl;
    int pick = -1, last = -1;
#pragma unroll
    for (int e = 0; e < lim; ++e) {
      const float w = get(e);
      run += w;
      const bool pos = w > 0.0f;
      last = pos ? c0 + e : last;
      pick = (pick < 0 && pos && run >= target) ? c0 + e : pick;
    }
    chosen = pick >= 0 ? pick : last;
  }
  __syncthreads();
  const int tok = chosen;
  if (t == 0) p.out[b] = tok;

  // 5. penalties
  if (pen) {
    for (int i = t; i < V; i += kSampThreads) {
      const float q = pen[i];
      pen[i] = __builtin_fmaf(q, p.decay, i == tok ? (q == 0.0f ? p.presence : p.repetition) : 0.0f);
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
  const int per = ((V + kSampThreads - 1) / kSampThreads + 3) / 4 * 4;
  a.per = per;
  hipStream_t s = (hipStream_t)stream;
  if (per <= 4) hipLaunchKernelGGL(sampling_kernel<4>, dim3(B), dim3(kSampThreads), 0, s, a);
  else if (per <= 16) hipLaunchKernelGGL(sampling_kernel<16>, dim3(B), dim3(kSampThreads), 0, s, a);
  else if (per <= 64) hipLaunchKernelGGL(sampling_kernel<64>, dim3(B), dim3(kSampThreads), 0, s, a);
  else {
    VK_REQUIRE(scratch != nullptr, "%s: vocabularies above 65536 need a scratch buffer of B*V floats", fn);
    hipLaunchKernelGGL(sampling_kernel<0>, dim3(B), dim3(kSampThreads), 0, s, a);
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
