// LayerNorm family for gfx950: plain, residual-add, last-token, bf16 embedding
// table, and the decode-step fusion of residual add + LayerNorm + token-shift
// lerp (1 or 6 mix vectors).
//
// One 256-lane workgroup (4 waves) per row.  The row (at most 8192 values) is
// read once into VGPRs -- 16-byte loads of 8 fp16 values per lane when C is a
// multiple of 8 and the tensors are 16-byte aligned, scalar loads otherwise --
// and the two statistics passes (mean, then the centred sum of squares) run on
// the registers, so HBM sees each input byte once and each output byte once.
// Reductions use a fixed order (wave butterfly + wave-ordered block sum), so
// results are run-to-run deterministic.
//
// At decode sizes (128 rows of 2048) the kernel is latency-bound, so the code is
// arranged to have as few dependent memory round trips as possible: all kernel
// arguments in one scalar round trip, then every load of the row issued back to
// back with no branch or wait between them (the slot-table lookup among them),
// the shift row as soon as its slot arrives, and the conversions behind a
// scheduling barrier.  Measured in a graph without a profiler (HIP events,
// difference of 40-launch graphs with and without the kernel): an empty launch
// costs 1.5 us, the residual + LN + 1 lerp 3.2 us, the 4-part + LN + 6 lerps
// 5.4 us, of which ~1 us is the 6 frag outputs' 16-byte scattered stores (the
// same kernel with row-major outputs: 4.5 us; spreading a row's stores over 2
// or 4 workgroups does not shorten it, so the cost is in the L2, not the CU).
//
// Roofline: HBM.  Algorithmic bytes per row of C channels: plain LN 4C (read
// x, write y); residual add 8C; decode fusion with n mix vectors
// 2C (x) + 2C (residual) + 2C (shift read) + 2C (shift write) + 2C (x_out)
// + 2nC (outputs), plus the C-length parameter vectors (cache resident).

#include "vk_capi.h"
#include "vk_common.cuh"

namespace vk {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxC = 8192;

// Sum over the 64 lanes of a wave with DPP (pairs, quads, 8, 16, then the row broadcasts
// into the last row); the total is read from lane 63.  Fixed order, deterministic.
__device__ __forceinline__ float wave_sum_dpp(float v) {
#define VK_DPP_ADD(ctrl, rows)                                                                                 \
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, rows, 0xF, false))
  VK_DPP_ADD(0xB1, 0xF);   // quad_perm [1,0,3,2]
  VK_DPP_ADD(0x4E, 0xF);   // quad_perm [2,3,0,1]
  VK_DPP_ADD(0x141, 0xF);  // row_half_mirror: 8-lane sums
  VK_DPP_ADD(0x140, 0xF);  // row_mirror: 16-lane (row) sums
  VK_DPP_ADD(0x142, 0xA);  // row_bcast15 into rows 1 and 3: 32-lane sums there
  VK_DPP_ADD(0x143, 0xC);  // row_bcast31 into rows 2 and 3: the 64-lane sum in row 3
#undef VK_DPP_ADD
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Workgroup sum: DPP wave sums, then the wave totals added in wave order.  The barrier waits
// only for LDS traffic (loads of the row's other inputs may stay in flight); each call site
// has its own `red` slots, so no barrier is needed after the read.
template <int NW>
__device__ __forceinline__ float block_sum_ln(float v, float* red) {
  v = wave_sum_dpp(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  float t = red[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) t += red[w];
  return t;
}

struct LnArgs {
  int C;
  int64_t rows;
  int64_t src_mul, src_add;  // source row = row * src_mul + src_add (last-token LN)
  const void* x;             // fp16, or bf16 bits when kBf16
  const _Float16* residual;  // may be null
  const void* weight;        // fp16, or bf16 bits when kBf16
  const void* bias;
  float eps;
  _Float16* x_out;  // may be null
  _Float16* y;      // plain mode output
  const int32_t* x_rows;       // may be null: x row = row
  const int32_t* shift_slots;  // may be null: shift row = row
  int64_t n_x, n_shift;        // rows of x / shift when x_rows / shift_slots index them
  // mix mode
  _Float16* shift;
  const _Float16* mix[6];
  _Float16* out[6];
  int out_frag;  // y / out[] in frag layout (row blocks of 32, K = C; needs VW == 8)
  // x given as the fp32 K-part planes of a split GEMM (vkwr_frag_gemm_splitk_parts_f16):
  // x[row, c] = fp16(sum over q of x_parts[q * part_stride + row * C + c]), added in q order
  const float* x_parts;
  int64_t part_stride;
  int n_parts;
};

// One int32 through a vector load whose wait the compiler places at the first use (the
// address is moved to VGPRs, so the load cannot become a scalar one).
// Global (not flat) address space, so the load counts only against vmcnt.
__device__ __forceinline__ int32_t ld_vgpr(const int32_t* q) {
  typedef const int32_t __attribute__((address_space(1)))* gptr;
  gptr g = (gptr)q;
  asm("" : "+v"(g));
  return *g;
}

template <bool kBf16>
__device__ __forceinline__ float ld_in(const void* p, int64_t i) {
  if constexpr (kBf16) {
    return bf16f(reinterpret_cast<const uint16_t*>(p)[i]);
  } else {
    return (float)reinterpret_cast<const _Float16*>(p)[i];
  }
}

// VW: elements per lane access (8 = one 16-byte load, 1 = scalar); NV: accesses
// per lane (VW * NV * 256 >= C); NMIX: 0 = plain LN output, 1 or 6 = decode
// fusion with that many token-shift mix vectors.
// NP > 0: x comes as NP fp32 K-part planes (vector path only).  kSlots: shift_slots is
// given (its lookup then issues with the row's loads instead of ahead of them).
template <int VW, int NV, int NMIX, bool kBf16, int NP = 0, bool kSlots = false>
__global__ __launch_bounds__(kThreads) void layer_norm_kernel(LnArgs p) {
  __shared__ float red[2][kWaves];
  // Every argument the row needs, into SGPRs in one scalar round trip: left to itself the
  // compiler loads them a cache line at a time as each is first used, behind branches that
  // wait for the previous load.
  if constexpr (NMIX > 0) {
    asm volatile("" ::"s"(p.C), "s"(p.rows), "s"(p.src_mul), "s"(p.src_add), "s"(p.x), "s"(p.residual),
                 "s"(p.weight), "s"(p.bias), "s"(p.eps), "s"(p.x_out), "s"(p.x_rows), "s"(p.shift_slots),
                 "s"(p.n_x), "s"(p.n_shift), "s"(p.shift), "s"(p.mix[0]), "s"(p.mix[NMIX - 1]),
                 "s"(p.out[0]), "s"(p.out[NMIX - 1]), "s"(p.out_frag), "s"(p.x_parts), "s"(p.part_stride));
  } else {
    asm volatile("" ::"s"(p.C), "s"(p.rows), "s"(p.src_mul), "s"(p.src_add), "s"(p.x), "s"(p.residual),
                 "s"(p.weight), "s"(p.bias), "s"(p.eps), "s"(p.x_out), "s"(p.y), "s"(p.out_frag));
  }
  // Frag outputs: 8 consecutive rows share each 128-byte line of the output, so those rows
  // are given to workgroups of one XCD (workgroup b runs on XCD b % 8): row block x of
  // rows / 8 rows goes to XCD x, and the partial-line stores meet in one L2.
  const int64_t row = (p.out_frag && (p.rows & 7) == 0)
                          ? (int64_t)(blockIdx.x & 7) * (p.rows >> 3) + (blockIdx.x >> 3)
                          : (int64_t)blockIdx.x;
  const int tid = threadIdx.x;
  const int C = p.C;
  const int64_t rrow = row * p.src_mul + p.src_add;  // residual row
  const int64_t rsrc = rrow * (int64_t)C;
  const int64_t dst = row * (int64_t)C;
  // Index-table lookups first, as vector loads (a scalar load would be waited for before
  // the row's loads issue), so their round trip overlaps the row's loads below and the
  // shift row can be requested as soon as its slot arrives.
  int32_t slot_raw = 0, xrow_raw = 0;
  if constexpr (NMIX > 0) {
    if constexpr (kSlots) slot_raw = ld_vgpr(p.shift_slots + row);
    if (p.x_rows) xrow_raw = ld_vgpr(p.x_rows + row);
    __builtin_amdgcn_sched_barrier(0);
  }

  // Vector path: every input of the row -- x, residual, the LN weight and bias, the
  // previous token's shift row and the mix vectors -- is requested before the two
  // reductions, so the row costs one memory round trip instead of several.  The loads sit
  // outside any branch (a lane past C reads the row's last 8 values and discards them),
  // so they all issue back to back; loads that need no index table go out first, the
  // x_rows / shift_slots lookups (a dependent round trip) overlap them, and the shift row,
  // needed only by the final lerp, is requested last.
  constexpr bool kVec = VW == 8 && !kBf16;
  constexpr int kPre = kVec ? NV : 1;
  auto col = [&](int n) {
    const int c = (tid + n * kThreads) * VW;
    return c < C ? c : C - VW;
  };
  h8 wpre[kPre], bpre[kPre], ppre[kPre], mpre[kPre][NMIX > 0 ? NMIX : 1];
  if constexpr (kVec) {
#pragma unroll
    for (int n = 0; n < NV; ++n) {
      const int cl = col(n);
      wpre[n] = ld8(reinterpret_cast<const _Float16*>(p.weight) + cl);
      bpre[n] = ld8(reinterpret_cast<const _Float16*>(p.bias) + cl);
      if constexpr (NMIX > 0) {
#pragma unroll
        for (int i = 0; i < NMIX; ++i) mpre[n][i] = ld8(p.mix[i] + cl);
      }
    }
  }

  float v[NV][VW];
  float sum = 0.0f;
  // Vector path in two halves: issue_row requests x (or its K-part planes) and the
  // residual into raw registers; finish_row, behind a scheduling barrier, converts them
  // and forms the running sum, so no load waits for an earlier one's data.
  h8 xraw[kPre], rraw[kPre];
  f4 praw[kPre][NP > 0 ? NP : 1][2];
  auto issue_row = [&](int64_t src) {
#pragma unroll
    for (int n = 0; n < kPre; ++n) {
      const int cl = col(n);
      if constexpr (NP > 0) {
        const float* xp = p.x_parts + dst + cl;
#pragma unroll
        for (int q = 0; q < NP; ++q) {
          praw[n][q][0] = *reinterpret_cast<const f4*>(xp + q * p.part_stride);
          praw[n][q][1] = *reinterpret_cast<const f4*>(xp + q * p.part_stride + 4);
        }
      } else {
        xraw[n] = ld8(reinterpret_cast<const _Float16*>(p.x) + src + cl);
      }
      if (p.residual) rraw[n] = ld8(p.residual + rsrc + cl);
    }
  };
  auto finish_row = [&]() {
#pragma unroll
    for (int n = 0; n < kPre; ++n) {
      const bool in = (tid + n * kThreads) * VW < C;
      if constexpr (NP > 0) {
        // the split GEMM's epilogue: parts added in K order, rounded to fp16
        f4 a0 = praw[n][0][0], a1 = praw[n][0][1];
#pragma unroll
        for (int q = 1; q < NP; ++q) {
          a0 += praw[n][q][0];
          a1 += praw[n][q][1];
        }
        const float xs[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) v[n][e] = (float)(_Float16)xs[e];
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[n][e] = (float)xraw[n].v[e];
      }
      if (p.residual) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[n][e] = v[n][e] + (float)rraw[n].v[e];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) sum += in ? v[n][e] : 0.0f;
    }
  };
  // Scalar path (C not a multiple of 8, unaligned rows, or the bf16 table).
  auto load_row_scalar = [&](int64_t src) {
#pragma unroll
    for (int n = 0; n < NV; ++n) {
      const int c0 = (tid + n * kThreads) * VW;
      if (c0 < C) {
#pragma unroll
        for (int e = 0; e < VW; ++e) {
          v[n][e] = ld_in<kBf16>(p.x, src + c0 + e);
          if (p.residual) v[n][e] = v[n][e] + (float)p.residual[rsrc + c0 + e];
        }
#pragma unroll
        for (int e = 0; e < VW; ++e) sum += v[n][e];
      }
    }
  };
  const bool gather = NMIX > 0 && p.x_rows;
  const int64_t src0 = (row * p.src_mul + p.src_add) * (int64_t)C;
  if constexpr (kVec) {
    if (!gather) issue_row(src0);
    __builtin_amdgcn_sched_barrier(0);
  }

  const int64_t srow = (NMIX > 0 && kSlots) ? (int64_t)__builtin_amdgcn_readfirstlane(slot_raw) : row;
  const int64_t sdst = srow * (int64_t)C;
  const int64_t xrow = __builtin_amdgcn_readfirstlane(xrow_raw);
  if constexpr (NMIX > 0) {
    // An index outside its table (x_rows past the embedding, shift_slots past the pool):
    // the row's outputs are NaN and no shift row is read or written.  Block-uniform.
    if ((p.x_rows && (xrow < 0 || xrow >= p.n_x)) || (kSlots && (srow < 0 || srow >= p.n_shift))) {
      const _Float16 nan = (_Float16)__builtin_nanf("");
      for (int c = tid; c < C; c += kThreads) {
        p.x_out[dst + c] = nan;
        const int64_t o = p.out_frag ? frag_index(row, c, C) : dst + c;
#pragma unroll
        for (int i = 0; i < NMIX; ++i) p.out[i][o] = nan;
      }
      return;
    }
    if constexpr (kVec) {
      if (gather) issue_row(xrow * (int64_t)C);
#pragma unroll
      for (int n = 0; n < NV; ++n) ppre[n] = ld8(p.shift + sdst + col(n));
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if constexpr (kVec) finish_row();
  else load_row_scalar(NMIX > 0 && p.x_rows ? xrow * (int64_t)C : src0);
  const float mean = block_sum_ln<kWaves>(sum, red[0]) / (float)C;
  float ss = 0.0f;
#pragma unroll
  for (int n = 0; n < NV; ++n) {
    const int c0 = (tid + n * kThreads) * VW;
    if (c0 < C) {
#pragma unroll
      for (int e = 0; e < VW; ++e) {
        const float d = v[n][e] - mean;
        ss = __builtin_fmaf(d, d, ss);
      }
    }
  }
  const float rstd = rsqrtf(block_sum_ln<kWaves>(ss, red[1]) / (float)C + p.eps);

#pragma unroll
  for (int n = 0; n < NV; ++n) {
    const int c0 = (tid + n * kThreads) * VW;
    if (c0 >= C) continue;
    _Float16 yh[VW], xo[VW];
#pragma unroll
    for (int e = 0; e < VW; ++e) {
      const float t = (v[n][e] - mean) * rstd;
      const float wt = kVec ? (float)wpre[n % kPre].v[e] : ld_in<kBf16>(p.weight, c0 + e);
      const float bs = kVec ? (float)bpre[n % kPre].v[e] : ld_in<kBf16>(p.bias, c0 + e);
      yh[e] = f16_of(__builtin_fmaf(t, wt, bs));
      xo[e] = (_Float16)v[n][e];
    }
    const int64_t odst = p.out_frag ? frag_index(row, c0, C) : dst + c0;  // y / out[] element offset
    if constexpr (NMIX == 0) {
      if constexpr (VW == 8) {
        st8(p.y + odst, *reinterpret_cast<const h8*>(yh));
        if (p.x_out) st8(p.x_out + dst + c0, *reinterpret_cast<const h8*>(xo));
      } else {
#pragma unroll
        for (int e = 0; e < VW; ++e) {
          p.y[dst + c0 + e] = yh[e];
          if (p.x_out) p.x_out[dst + c0 + e] = xo[e];
        }
      }
    } else {
      // Token-shift lerp of the fp16-rounded LN output with the previous token's.
      _Float16 prev[VW];
      if constexpr (VW == 8) {
        if constexpr (kVec) *reinterpret_cast<h8*>(prev) = ppre[n % kPre];
        else *reinterpret_cast<h8*>(prev) = ld8(p.shift + sdst + c0);
        st8(p.x_out + dst + c0, *reinterpret_cast<const h8*>(xo));
        st8(p.shift + sdst + c0, *reinterpret_cast<const h8*>(yh));
      } else {
#pragma unroll
        for (int e = 0; e < VW; ++e) {
          prev[e] = p.shift[sdst + c0 + e];
          p.x_out[dst + c0 + e] = xo[e];
          p.shift[sdst + c0 + e] = yh[e];
        }
      }
#pragma unroll
      for (int i = 0; i < NMIX; ++i) {
        _Float16 o[VW];
#pragma unroll
        for (int e = 0; e < VW; ++e) {
          const float yv = (float)yh[e];
          const float mv = kVec ? (float)mpre[n % kPre][i % (NMIX > 0 ? NMIX : 1)].v[e] : (float)p.mix[i][c0 + e];
          o[e] = f16_of(__builtin_fmaf((float)prev[e] - yv, mv, yv));
        }
        if constexpr (VW == 8) {
          st8(p.out[i] + odst, *reinterpret_cast<const h8*>(o));
        } else {
#pragma unroll
          for (int e = 0; e < VW; ++e) p.out[i][dst + c0 + e] = o[e];
        }
      }
    }
  }
}

__global__ __launch_bounds__(256) void add_kernel(const _Float16* x, const _Float16* y, _Float16* out,
                                                  int64_t n, int vec) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (vec) {
    if (i * 8 >= n) return;
    const h8 a = ld8(x + i * 8), b = ld8(y + i * 8);
    h8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o.v[e] = (_Float16)((float)a.v[e] + (float)b.v[e]);
    st8(out + i * 8, o);
  } else {
    if (i >= n) return;
    out[i] = (_Float16)((float)x[i] + (float)y[i]);
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <int NMIX, bool kBf16>
int launch_ln(const char* fn, const LnArgs& p, bool vec_ok, hipStream_t stream) {
  VK_REQUIRE(p.C > 0 && p.C <= kMaxC, "%s: unsupported C=%d (need 0 < C <= 8192)", fn, p.C);
  VK_REQUIRE(p.rows >= 0 && p.rows <= 0x7fffffff, "%s: too many rows", fn);
  if (p.rows == 0) return VKWR_OK;
  VK_REQUIRE(!p.out_frag || (vec_ok && p.C % kFragPad == 0),
             "%s: frag output needs C %% %d == 0 and 16-byte aligned rows", fn, kFragPad);
  const dim3 grid((unsigned)p.rows), block(kThreads);
  // launches instance K<..., kSlots> of the kernel, kSlots = (shift_slots given)
#define VK_LN_GO(...)                                                                             \
  do {                                                                                            \
    bool launched = false;                                                                        \
    if constexpr (NMIX > 0) {                                                                     \
      if (p.shift_slots) {                                                                        \
        hipLaunchKernelGGL((layer_norm_kernel<__VA_ARGS__, true>), grid, block, 0, stream, p);    \
        launched = true;                                                                          \
      }                                                                                           \
    }                                                                                             \
    if (!launched)                                                                                \
      hipLaunchKernelGGL((layer_norm_kernel<__VA_ARGS__, false>), grid, block, 0, stream, p);     \
  } while (0)
  if constexpr (NMIX > 0 && !kBf16) {
    if (p.x_parts) {
      VK_REQUIRE(vec_ok && p.C % kFragPad == 0 && p.C <= 4096,
                 "%s: K-part input needs C %% %d == 0, C <= 4096 and 16-byte aligned rows", fn, kFragPad);
      const bool one = p.C <= 8 * kThreads;
#define VK_LN_PARTS(np)                                 \
  if (p.n_parts == np) {                                \
    if (one) VK_LN_GO(8, 1, NMIX, false, np);           \
    else VK_LN_GO(8, 2, NMIX, false, np);               \
    return check_launch(fn);                            \
  }
      VK_LN_PARTS(2)
      VK_LN_PARTS(4)
      VK_LN_PARTS(8)
#undef VK_LN_PARTS
      VK_REQUIRE(false, "%s: n_parts must be 2, 4 or 8 (got %d)", fn, p.n_parts);
    }
  }
  if (vec_ok && p.C % 8 == 0) {
    const int per = (p.C / 8 + kThreads - 1) / kThreads;  // 1..4
    if (per == 1) VK_LN_GO(8, 1, NMIX, kBf16, 0);
    else if (per == 2) VK_LN_GO(8, 2, NMIX, kBf16, 0);
    else VK_LN_GO(8, 4, NMIX, kBf16, 0);
  } else {
    const int per = (p.C + kThreads - 1) / kThreads;  // 1..32
    if (per <= 8) VK_LN_GO(1, 8, NMIX, kBf16, 0);
    else VK_LN_GO(1, 32, NMIX, kBf16, 0);
  }
#undef VK_LN_GO
  return check_launch(fn);
}

// ---- mixed-batch fusion: residual add + LayerNorm + token-shift lerp over row groups.
//
// Rows are laid out group by group (a decode group: B sequences of one row; a prefill
// chunk group: B sequences of T consecutive rows).  For row t of a sequence the lerp's
// "previous token" is the LayerNorm output of row t - 1, or for t = 0 the sequence's shift
// row in the slot pool, which then receives the output of the sequence's last row.  One
// 256-lane workgroup per row computes the LayerNorm of its row and of one more: row t - 1
// (t > 0), or the sequence's last row (t = 0, T > 1; the t = 0 workgroup is the only reader
// and the only writer of the shift row, so no other workgroup races it).  The two rows'
// reductions share their barriers.  The results are the bits of vkwr_layer_norm_f16 (with
// the residual) followed by vkwr_token_shift_mix_slots_f16 per group, without the LayerNorm
// output's trip through HBM and the second launch.  Algorithmic bytes per row: 2C (x) +
// 2C (residual) + 2C (x_out) + 2nC (n lerp outputs), plus the shift row of each sequence.
// Measured at 2304 rows x 4096 (256 decode rows + 4 chunks of 512): 34 us with 6 lerps
// (5.5 TB/s of algorithmic bytes), 21 us with 1, where the launches it replaces took 13 us
// (the LayerNorm) plus 37 us (6 lerps) or 17 us (1 lerp) for the two token-shift launches.
constexpr int kMaxShiftGroups = 8;

struct LnShiftGroup {
  int64_t r0;
  int B, T;
  const int32_t* slots;
  int64_t run0;  // runs kernel: the group's first run
  int rps;       // runs kernel: runs per sequence, ceil(T / kLnRun)
};

struct LnShiftArgs {
  int C, n_groups;
  const _Float16* x;
  const _Float16* residual;  // may be null
  const _Float16* weight;
  const _Float16* bias;
  float eps;
  _Float16* x_out;
  _Float16* shift;
  int64_t n_shift;
  const _Float16* mix[6];
  _Float16* out[6];
  LnShiftGroup g[kMaxShiftGroups];
};

// Residual add + LayerNorm + token shift over runs of up to kLnRun consecutive rows of one
// sequence per workgroup (runs never cross a sequence): the LayerNorm weight, bias and mix vectors are
// loaded once per run instead of once per row, and each row's LayerNorm output is the next
// row's "previous token" straight from registers, so a run of n rows normalises n + 1 rows
// (the row before the run, or for the sequence's first run its last row, which goes to the
// shift pool) instead of 2n.  Each row's arithmetic is layer_norm_kernel's, in the same order.
// Measured at 2304 rows x 4096 (256 decode rows + 4 chunks of 512): 31.1 us with 6 lerps and
// 16.9 us with 1 (6.1 / 5.6 TB/s), against 34.1 / 20.9 us for one row per workgroup (runs of
// 8 rows: 31.1 / 18.3 us).
constexpr int kLnRun = 4;

template <int NV, int NMIX>
__global__ __launch_bounds__(kThreads) void ln_shift_runs_kernel(LnShiftArgs p) {
  __shared__ float red[2][2][kWaves];  // [row parity][statistics pass]
  const int64_t run = blockIdx.x;
  const int tid = threadIdx.x, C = p.C;
  int gi = 0;
#pragma unroll
  for (int i = 1; i < kMaxShiftGroups; ++i)
    if (i < p.n_groups && run >= p.g[i].run0) gi = i;
  const LnShiftGroup& G = p.g[gi];
  const int T = G.T;
  const int64_t local = run - G.run0;
  const int b = (int)(local / G.rps);
  const int t0 = (int)(local - (int64_t)b * G.rps) * kLnRun, t1 = min(T, t0 + kLnRun);
  const int64_t seq0 = G.r0 + (int64_t)b * T;  // the sequence's row 0
  const int64_t slot = G.slots[b];
  auto col = [&](int n) {
    const int c = (tid + n * kThreads) * 8;
    return c < C ? c : C - 8;
  };
  if (slot < 0 || slot >= p.n_shift) {
    // A slot outside the pool: the run's outputs are NaN and no shift row is touched.
    const _Float16 nan = (_Float16)__builtin_nanf("");
    for (int t = t0; t < t1; ++t)
      for (int c = tid; c < C; c += kThreads) {
        const int64_t o = (seq0 + t) * (int64_t)C + c;
        p.x_out[o] = nan;
#pragma unroll
        for (int i = 0; i < NMIX; ++i) p.out[i][o] = nan;
      }
    return;
  }
  const int64_t sdst = slot * (int64_t)C;
  h8 wp[NV], bp[NV], mp[NV][NMIX], prev[NV];
  h8 xa[NV], ra[NV];  // raw x / residual of the row being loaded
  auto load_row = [&](int64_t row) __attribute__((always_inline)) {
    const int64_t o = row * (int64_t)C;
#pragma unroll
    for (int n = 0; n < NV; ++n) {
      xa[n] = ld8(p.x + o + col(n));
      if (p.residual) ra[n] = ld8(p.residual + o + col(n));
    }
  };
  // LayerNorm of the loaded row (layer_norm_kernel's arithmetic and order): y and x + residual
  auto ln_row = [&](float* rd, h8 (&y)[NV], h8 (&xo)[NV]) __attribute__((always_inline)) {
    float v[NV][8], sum = 0.0f;
#pragma unroll
    for (int n = 0; n < NV; ++n) {
      const bool in = (tid + n * kThreads) * 8 < C;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[n][e] = (float)xa[n].v[e];
      if (p.residual) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[n][e] = v[n][e] + (float)ra[n].v[e];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) sum += in ? v[n][e] : 0.0f;
    }
    const float mean = block_sum_ln<kWaves>(sum, rd) / (float)C;
    float ss = 0.0f;
#pragma unroll
    for (int n = 0; n < NV; ++n) {
      if ((tid + n * kThreads) * 8 < C) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = v[n][e] - mean;
          ss = __builtin_fmaf(d, d, ss);
        }
      }
    }
    const float rstd = rsqrtf(block_sum_ln<kWaves>(ss, rd + kWaves) / (float)C + p.eps);
#pragma unroll
    for (int n = 0; n < NV; ++n)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        y[n].v[e] = f16_of(__builtin_fmaf((v[n][e] - mean) * rstd, (float)wp[n].v[e], (float)bp[n].v[e]));
        xo[n].v[e] = (_Float16)v[n][e];
      }
  };
  // parameters, and the first row's (or the row before the run's) inputs
  const bool first = t0 == 0;
  load_row(first ? seq0 : seq0 + t0 - 1);
#pragma unroll
  for (int n = 0; n < NV; ++n) {
    wp[n] = ld8(p.weight + col(n));
    bp[n] = ld8(p.bias + col(n));
#pragma unroll
    for (int i = 0; i < NMIX; ++i) mp[n][i] = ld8(p.mix[i] + col(n));
    if (first) prev[n] = ld8(p.shift + sdst + col(n));
  }
  h8 y[NV], xo[NV];
  int par = 0;
  if (!first) {
    ln_row(&red[par][0][0], prev, xo);  // the row before the run: only its y is used
    par ^= 1;
    load_row(seq0 + t0);
  }
#pragma unroll 1
  for (int t = t0; t < t1; ++t) {
    // keep the parameters in fp16 registers: converted once outside the loop they would
    // double their register count
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int n = 0; n < NV; ++n) {
      u4 wu = __builtin_bit_cast(u4, wp[n]), bu = __builtin_bit_cast(u4, bp[n]);
      asm volatile("" : "+v"(wu), "+v"(bu));
      wp[n] = __builtin_bit_cast(h8, wu);
      bp[n] = __builtin_bit_cast(h8, bu);
#pragma unroll
      for (int i = 0; i < NMIX; ++i) {
        u4 mu = __builtin_bit_cast(u4, mp[n][i]);
        asm volatile("" : "+v"(mu));
        mp[n][i] = __builtin_bit_cast(h8, mu);
      }
    }
    ln_row(&red[par][0][0], y, xo);
    par ^= 1;
    if (t + 1 < t1) load_row(seq0 + t + 1);  // the next row's loads go out before this row's stores
    const int64_t dst = (seq0 + t) * (int64_t)C;
#pragma unroll
    for (int n = 0; n < NV; ++n) {
      const int c0 = (tid + n * kThreads) * 8;
      if (c0 >= C) continue;
      st8(p.x_out + dst + c0, xo[n]);
#pragma unroll
      for (int i = 0; i < NMIX; ++i) {
        h8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float yv = (float)y[n].v[e];
          o.v[e] = f16_of(__builtin_fmaf((float)prev[n].v[e] - yv, (float)mp[n][i].v[e], yv));
        }
        st8(p.out[i] + dst + c0, o);
      }
      prev[n] = y[n];
    }
  }
  if (first) {
    // the sequence's last row to the shift pool (this workgroup read the old value above)
    if (t1 < T) {
      load_row(seq0 + T - 1);
      ln_row(&red[par][0][0], y, xo);
    }
#pragma unroll
    for (int n = 0; n < NV; ++n) {
      const int c0 = (tid + n * kThreads) * 8;
      if (c0 < C) st8(p.shift + sdst + c0, y[n]);
    }
  }
}

}  // namespace
}  // namespace vk

using namespace vk;

extern "C" int vkwr_layer_norm_f16(int64_t rows, int C, const uint16_t* x, const uint16_t* residual,
                                   const uint16_t* weight, const uint16_t* bias, float eps,
                                   uint16_t* x_out, uint16_t* y, void* stream) {
  clear_error();
  const char* fn = "vkwr_layer_norm_f16";
  VK_REQUIRE(rows == 0 || (x && weight && bias && y), "%s: null pointer", fn);
  LnArgs p{};
  p.C = C;
  p.rows = rows;
  p.src_mul = 1;
  p.x = x;
  p.residual = reinterpret_cast<const _Float16*>(residual);
  p.weight = weight;
  p.bias = bias;
  p.eps = eps;
  p.x_out = reinterpret_cast<_Float16*>(x_out);
  p.y = reinterpret_cast<_Float16*>(y);
  const bool vec = aligned16(x) && aligned16(y) && (!residual || aligned16(residual)) &&
                   (!x_out || aligned16(x_out));
  return launch_ln<0, false>(fn, p, vec, (hipStream_t)stream);
}

namespace {
int add_last_ln(const char* fn, int B, int T, int C, const uint16_t* x, const uint16_t* residual,
                const uint16_t* weight, const uint16_t* bias, float eps, uint16_t* y, int frag,
                void* stream) {
  VK_REQUIRE(B >= 0 && T > 0, "%s: bad B=%d T=%d", fn, B, T);
  VK_REQUIRE(B == 0 || (x && residual && weight && bias && y), "%s: null pointer", fn);
  LnArgs p{};
  p.C = C;
  p.rows = B;
  p.src_mul = T;
  p.src_add = T - 1;
  p.x = x;
  p.residual = reinterpret_cast<const _Float16*>(residual);
  p.weight = weight;
  p.bias = bias;
  p.eps = eps;
  p.y = reinterpret_cast<_Float16*>(y);
  p.out_frag = frag;
  const bool vec = aligned16(x) && aligned16(residual) && aligned16(y);
  return launch_ln<0, false>(fn, p, vec, (hipStream_t)stream);
}
}  // namespace

extern "C" int vkwr_add_last_layer_norm_f16(int B, int T, int C, const uint16_t* x,
                                            const uint16_t* residual, const uint16_t* weight,
                                            const uint16_t* bias, float eps, uint16_t* y,
                                            void* stream) {
  clear_error();
  return add_last_ln("vkwr_add_last_layer_norm_f16", B, T, C, x, residual, weight, bias, eps, y, 0, stream);
}

extern "C" int vkwr_add_last_layer_norm_frag_f16(int B, int T, int C, const uint16_t* x,
                                                 const uint16_t* residual, const uint16_t* weight,
                                                 const uint16_t* bias, float eps, uint16_t* y,
                                                 void* stream) {
  clear_error();
  return add_last_ln("vkwr_add_last_layer_norm_frag_f16", B, T, C, x, residual, weight, bias, eps, y, 1,
                     stream);
}

extern "C" int vkwr_emb_ln0_bf16_to_f16(int64_t V, int C, const uint16_t* emb,
                                        const uint16_t* weight, const uint16_t* bias, float eps,
                                        uint16_t* out, void* stream) {
  clear_error();
  const char* fn = "vkwr_emb_ln0_bf16_to_f16";
  VK_REQUIRE(V == 0 || (emb && weight && bias && out), "%s: null pointer", fn);
  LnArgs p{};
  p.C = C;
  p.rows = V;
  p.src_mul = 1;
  p.x = emb;
  p.weight = weight;
  p.bias = bias;
  p.eps = eps;
  p.y = reinterpret_cast<_Float16*>(out);
  return launch_ln<0, true>(fn, p, false, (hipStream_t)stream);
}

namespace {
int add_ln_mix(const char* fn, int64_t rows, int C, const uint16_t* x, const uint16_t* residual,
               uint16_t* shift_state, const uint16_t* weight, const uint16_t* bias, int n_mix,
               const uint16_t* const* mix, float eps, uint16_t* x_out, uint16_t* const* out,
               const int32_t* x_rows, const int32_t* shift_slots, int64_t n_x, int64_t n_shift, int frag,
               void* stream, const float* x_parts = nullptr, int n_parts = 0, int64_t part_stride = 0) {
  VK_REQUIRE(n_mix == 1 || n_mix == 6, "%s: n_mix must be 1 or 6 (got %d)", fn, n_mix);
  VK_REQUIRE(mix && out, "%s: null pointer", fn);
  LnArgs p{};
  p.C = C;
  p.rows = rows;
  p.src_mul = 1;
  p.x = x;
  p.residual = reinterpret_cast<const _Float16*>(residual);
  p.weight = weight;
  p.bias = bias;
  p.eps = eps;
  p.x_out = reinterpret_cast<_Float16*>(x_out);
  p.shift = reinterpret_cast<_Float16*>(shift_state);
  VK_REQUIRE(!x_rows || n_x >= 0, "%s: negative n_x", fn);
  VK_REQUIRE(!shift_slots || n_shift >= 0, "%s: negative n_shift", fn);
  p.x_rows = x_rows;
  p.shift_slots = shift_slots;
  p.n_x = n_x;
  p.n_shift = n_shift;
  p.out_frag = frag;
  p.x_parts = x_parts;
  p.n_parts = n_parts;
  p.part_stride = part_stride;
  bool vec = aligned16(x_parts ? (const void*)x_parts : (const void*)x) && (!residual || aligned16(residual)) &&
             aligned16(shift_state) && aligned16(x_out);
  for (int i = 0; i < n_mix; ++i) {
    VK_REQUIRE(rows == 0 || (mix[i] && out[i]), "%s: null pointer", fn);
    p.mix[i] = reinterpret_cast<const _Float16*>(mix[i]);
    p.out[i] = reinterpret_cast<_Float16*>(out[i]);
    vec = vec && aligned16(out[i]);
  }
  VK_REQUIRE(rows == 0 || ((x || x_parts) && shift_state && weight && bias && x_out), "%s: null pointer", fn);
  if (n_mix == 1) return launch_ln<1, false>(fn, p, vec, (hipStream_t)stream);
  return launch_ln<6, false>(fn, p, vec, (hipStream_t)stream);
}
}  // namespace

extern "C" int vkwr_add_layer_norm_mix_f16(int64_t rows, int C, const uint16_t* x,
                                           const uint16_t* residual, uint16_t* shift_state,
                                           const uint16_t* weight, const uint16_t* bias, int n_mix,
                                           const uint16_t* const* mix, float eps, uint16_t* x_out,
                                           uint16_t* const* out, const int32_t* x_rows,
                                           const int32_t* shift_slots, int64_t n_x, int64_t n_shift,
                                           void* stream) {
  clear_error();
  return add_ln_mix("vkwr_add_layer_norm_mix_f16", rows, C, x, residual, shift_state, weight, bias, n_mix,
                    mix, eps, x_out, out, x_rows, shift_slots, n_x, n_shift, 0, stream);
}

extern "C" int vkwr_add_layer_norm_mix_frag_f16(int64_t rows, int C, const uint16_t* x,
                                                const uint16_t* residual, uint16_t* shift_state,
                                                const uint16_t* weight, const uint16_t* bias,
                                                int n_mix, const uint16_t* const* mix, float eps,
                                                uint16_t* x_out, uint16_t* const* out,
                                                const int32_t* x_rows, const int32_t* shift_slots,
                                                int64_t n_x, int64_t n_shift, void* stream) {
  clear_error();
  return add_ln_mix("vkwr_add_layer_norm_mix_frag_f16", rows, C, x, residual, shift_state, weight, bias,
                    n_mix, mix, eps, x_out, out, x_rows, shift_slots, n_x, n_shift, 1, stream);
}

extern "C" int vkwr_add_layer_norm_mix_parts_frag_f16(int64_t rows, int C, const float* x_parts, int n_parts,
                                                      int64_t part_stride, const uint16_t* residual,
                                                      uint16_t* shift_state, const uint16_t* weight,
                                                      const uint16_t* bias, int n_mix, const uint16_t* const* mix,
                                                      float eps, uint16_t* x_out, uint16_t* const* out,
                                                      const int32_t* shift_slots, int64_t n_shift,
                                                      void* stream) {
  clear_error();
  const char* fn = "vkwr_add_layer_norm_mix_parts_frag_f16";
  VK_REQUIRE(rows == 0 || x_parts, "%s: null x_parts", fn);
  VK_REQUIRE(part_stride >= rows * (int64_t)C, "%s: part_stride below rows * C", fn);
  return add_ln_mix(fn, rows, C, nullptr, residual, shift_state, weight, bias, n_mix, mix, eps, x_out, out, nullptr,
                    shift_slots, 0, n_shift, 1, stream, x_parts, n_parts, part_stride);
}

extern "C" int vkwr_add_layer_norm_shift_rows_f16(int64_t rows, int C, const uint16_t* x,
                                                  const uint16_t* residual, const uint16_t* weight,
                                                  const uint16_t* bias, float eps, uint16_t* x_out, int n_mix,
                                                  const uint16_t* const* mix, uint16_t* const* out,
                                                  uint16_t* shift_state, int64_t n_shift, int n_groups,
                                                  const vkwr_ln_shift_group* groups, void* stream) {
  clear_error();
  const char* fn = "vkwr_add_layer_norm_shift_rows_f16";
  VK_REQUIRE(n_mix == 1 || n_mix == 6, "%s: n_mix must be 1 or 6 (got %d)", fn, n_mix);
  VK_REQUIRE(n_groups >= 1 && n_groups <= kMaxShiftGroups, "%s: 1..%d groups (got %d)", fn, kMaxShiftGroups,
             n_groups);
  VK_REQUIRE(groups && mix && out, "%s: null pointer", fn);
  VK_REQUIRE(rows >= 0 && rows <= 0x7fffffff, "%s: bad rows", fn);
  VK_REQUIRE(C > 0 && C % 8 == 0 && C <= 4096, "%s: C must be a multiple of 8 in 8..4096 (got %d)", fn, C);
  VK_REQUIRE(n_shift >= 0, "%s: negative n_shift", fn);
  LnShiftArgs p{};
  p.C = C;
  p.n_groups = n_groups;
  int64_t r = 0, runs = 0;
  for (int i = 0; i < n_groups; ++i) {
    const vkwr_ln_shift_group& g = groups[i];
    VK_REQUIRE(g.row0 == r, "%s: group %d starts at row %lld, expected %lld", fn, i, (long long)g.row0,
               (long long)r);
    VK_REQUIRE(g.B >= 1 && g.T >= 1 && g.slots, "%s: group %d needs B >= 1, T >= 1 and slots", fn, i);
    const int rps = (g.T + kLnRun - 1) / kLnRun;
    p.g[i] = LnShiftGroup{g.row0, g.B, g.T, g.slots, runs, rps};
    r += (int64_t)g.B * g.T;
    runs += (int64_t)g.B * rps;
  }
  VK_REQUIRE(r == rows, "%s: the groups cover %lld rows, not %lld", fn, (long long)r, (long long)rows);
  if (rows == 0) return VKWR_OK;
  VK_REQUIRE(x && weight && bias && x_out && shift_state, "%s: null pointer", fn);
  bool vec = aligned16(x) && (!residual || aligned16(residual)) && aligned16(weight) && aligned16(bias) &&
             aligned16(x_out) && aligned16(shift_state);
  p.x = reinterpret_cast<const _Float16*>(x);
  p.residual = reinterpret_cast<const _Float16*>(residual);
  p.weight = reinterpret_cast<const _Float16*>(weight);
  p.bias = reinterpret_cast<const _Float16*>(bias);
  p.eps = eps;
  p.x_out = reinterpret_cast<_Float16*>(x_out);
  p.shift = reinterpret_cast<_Float16*>(shift_state);
  p.n_shift = n_shift;
  for (int i = 0; i < n_mix; ++i) {
    VK_REQUIRE(mix[i] && out[i], "%s: null pointer", fn);
    p.mix[i] = reinterpret_cast<const _Float16*>(mix[i]);
    p.out[i] = reinterpret_cast<_Float16*>(out[i]);
    vec = vec && aligned16(mix[i]) && aligned16(out[i]);
  }
  VK_REQUIRE(vec, "%s: every tensor must be 16-byte aligned", fn);
  // a workgroup reads rows of x and residual that other workgroups own: no output may overlap them
  const int64_t span = rows * (int64_t)C * 2;
  auto overlap = [&](const void* o, const void* i) {
    const uintptr_t a = (uintptr_t)o, b = (uintptr_t)i;
    return i != nullptr && a < b + span && b < a + span;
  };
  bool alias = overlap(x_out, x) || overlap(x_out, residual);
  for (int i = 0; i < n_mix; ++i) alias = alias || overlap(out[i], x) || overlap(out[i], residual);
  VK_REQUIRE(!alias, "%s: x_out and out[] must not overlap x or residual (rows are read across workgroups)", fn);
  const dim3 grid((unsigned)runs), block(kThreads);
  const bool one = C <= 8 * kThreads;
  if (n_mix == 1) {
    if (one) hipLaunchKernelGGL((ln_shift_runs_kernel<1, 1>), grid, block, 0, (hipStream_t)stream, p);
    else hipLaunchKernelGGL((ln_shift_runs_kernel<2, 1>), grid, block, 0, (hipStream_t)stream, p);
  } else {
    if (one) hipLaunchKernelGGL((ln_shift_runs_kernel<1, 6>), grid, block, 0, (hipStream_t)stream, p);
    else hipLaunchKernelGGL((ln_shift_runs_kernel<2, 6>), grid, block, 0, (hipStream_t)stream, p);
  }
  return check_launch(fn);
}

extern "C" int vkwr_add_f16(int64_t n, const uint16_t* x, const uint16_t* y, uint16_t* out,
                            void* stream) {
  clear_error();
  VK_REQUIRE(n >= 0, "vkwr_add_f16: negative size");
  if (n == 0) return VKWR_OK;
  VK_REQUIRE(x && y && out, "vkwr_add_f16: null pointer");
  const int vec = (n % 8 == 0) && aligned16(x) && aligned16(y) && aligned16(out);
  const int64_t items = vec ? n / 8 : n;
  const int64_t blocks = (items + 255) / 256;
  VK_REQUIRE(blocks <= 0x7fffffff, "vkwr_add_f16: too many elements");
  hipLaunchKernelGGL(add_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<const _Float16*>(x), reinterpret_cast<const _Float16*>(y),
                     reinterpret_cast<_Float16*>(out), n, vec);
  return check_launch("vkwr_add_f16");
}
