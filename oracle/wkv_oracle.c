/*
 * CPU oracle for the RWKV-7 WKV hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, on the CPU, the arithmetic of the reference's WKV-7
 * kernels (szxysdt/VKWR).  It is the checker that the HIP kernels of this
 * repository are compared against, and the "reference CPU path" that bench.py
 * times as a baseline.  Nothing in the product (vkwr/, vkwr_amd/) links, imports or
 * calls it; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * load it.
 *
 * Every operation is an IEEE-754 correctly rounded primitive (+, -, *, /, fma,
 * rint, ldexp, int->float), evaluated in a fixed order, so a GPU kernel that
 * performs the same primitives in the same order produces identical bits.
 * Build with -ffp-contract=off (see Makefile): no implicit FMA contraction.
 *
 * Reference files restated (paths relative to the reference root):
 *   fp32-state WKV   csrc/v1/wkv/wkv_fp32_v2.cu:14-29 (constants, w_eff),
 *                    :79-124 (row-per-thread state, recurrence, fp16 store)
 *   fp16-state WKV   csrc/v1/wkv/wkv_fp16_v2.cu:13-39 (rotator1, w_delta, w0),
 *                    :259-291 and :357-389 (half2 FMA nesting and order)
 *   legacy WKV       csrc/rwkv7/state_fwd_fp16.cu:22-25, 57-83, 129-152
 *   advance_i32      csrc/v1/wkv/advance_i32_ops.cu:8-13
 *
 * Choices this restatement fixes where the reference source leaves them to
 * the CUDA compiler (documented, applied identically by the HIP kernels):
 *   - the decay d = exp2(C1 / (1 + exp2(C2*w))) uses a deterministic exp2
 *     (rint range reduction + degree-7 Taylor polynomial of 2^f in Horner/FMA
 *     form + ldexp) instead of the reference's fast-math exp2f, and an IEEE
 *     division; accuracy ~1e-7 relative, checked against float64 closed forms;
 *   - `s*w + sa*b + k*v` (wkv_fp32_v2.cu:114) is evaluated as
 *     fma(k, v, fma(sa, b, s*w)), and the sa/y dot products as sequential FMA
 *     chains over j = 0..63 (wkv_fp32_v2.cu:103-117); oracle_wkv_fp32_rows
 *     evaluates them in the row-split order of row_dot below;
 *   - the legacy half2 operators (state_fwd_fp16.cu:69,79-80) are evaluated as
 *     separately rounded fp16 multiplies and adds, left to right.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define HS 64 /* head size */

static const float C1 = -0.8750387749145276f; /* -e^{-1/2} * log2(e)  (wkv_fp32_v2.cu:14) */
static const float C2 = -1.4426950408889634f; /* -log2(e)             (wkv_fp32_v2.cu:15) */
static const float TWO_NEG_41 = 4.547473508864641e-13f; /* wkv_fp16_v2.cu:16 */

/* ---------------------------------------------------------------- fp16 bits */

float oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  uint32_t bits;
  if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (man << 13);
  } else if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: value = man * 2^-24, exact in float */
      float f = (float)man * 5.9604644775390625e-08f;
      memcpy(&bits, &f, 4);
      bits |= sign;
    }
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* Round the exact real value s + err to binary16, round-to-nearest-even.
 * err is the exact low part of a TwoSum (|err| <= ulp(s)/2) or 0; it only
 * decides ties that s alone would see. */
static uint16_t f16_round(double s, double err) {
  uint16_t sign = 0;
  if (s != s) return 0x7e00;
  if (s < 0 || (s == 0 && signbit(s))) {
    sign = 0x8000;
    s = -s;
    err = -err;
  }
  if (s == INFINITY) return sign | 0x7c00;
  double ulp;
  int e2;
  if (s < 6.103515625e-05) { /* below 2^-14: subnormal quantum 2^-24 */
    ulp = 5.9604644775390625e-08;
  } else {
    (void)frexp(s, &e2); /* s in [2^(e2-1), 2^e2) */
    ulp = ldexp(1.0, e2 - 1 - 10);
  }
  double q = s / ulp; /* exact: power-of-two scaling */
  double fl = floor(q);
  double rem = q - fl; /* exact */
  int up;
  if (rem > 0.5) up = 1;
  else if (rem < 0.5) up = 0;
  else if (err > 0) up = 1;
  else if (err < 0) up = 0;
  else up = (fmod(fl, 2.0) != 0.0);
  double v = (fl + (up ? 1.0 : 0.0)) * ulp;
  if (v >= 65536.0) return sign | 0x7c00;
  if (v < 6.103515625e-05) { /* subnormal or zero */
    return sign | (uint16_t)(v / 5.9604644775390625e-08);
  }
  int e;
  double m = frexp(v, &e); /* v = m * 2^e, m in [0.5,1) */
  uint16_t exp_bits = (uint16_t)(e - 1 + 15);
  uint16_t man = (uint16_t)((m * 2.0 - 1.0) * 1024.0);
  return sign | (uint16_t)(exp_bits << 10) | man;
}

uint16_t oracle_f32_to_f16(float f) { return f16_round((double)f, 0.0); }

/* Exactly rounded fp16 fused multiply-add / add / multiply. */
static uint16_t fma16(uint16_t a, uint16_t b, uint16_t c) {
  double p = (double)oracle_f16_to_f32(a) * (double)oracle_f16_to_f32(b); /* exact (22 bits) */
  double cc = (double)oracle_f16_to_f32(c);
  if (p != p || cc != cc || isinf(p) || isinf(cc)) return f16_round(p + cc, 0.0);
  double s = p + cc; /* TwoSum */
  double bb = s - p;
  double err = (p - (s - bb)) + (cc - bb);
  return f16_round(s, err);
}
static uint16_t add16(uint16_t a, uint16_t b) {
  return f16_round((double)oracle_f16_to_f32(a) + (double)oracle_f16_to_f32(b), 0.0); /* exact in double */
}
static uint16_t mul16(uint16_t a, uint16_t b) {
  return f16_round((double)oracle_f16_to_f32(a) * (double)oracle_f16_to_f32(b), 0.0); /* exact in double */
}

/* ---------------------------------------------------------------- decay */

/* 2^x from correctly rounded primitives only.  Results below 2^-126 return 0:
 * the decay only uses 2^x inside 1 + 2^x, where they vanish anyway. */
float oracle_exp2(float x) {
  if (x != x) return x;
  if (x >= 128.0f) return INFINITY;
  if (x < -126.0f) return 0.0f;
  float n = rintf(x);
  float f = x - n; /* exact, |f| <= 0.5 */
  /* Taylor coefficients (ln 2)^k / k! */
  float p = 1.525273380405984e-05f;
  p = fmaf(p, f, 1.5403530393381608e-04f);
  p = fmaf(p, f, 1.3333558146428443e-03f);
  p = fmaf(p, f, 9.618129107628477e-03f);
  p = fmaf(p, f, 5.550410866482158e-02f);
  p = fmaf(p, f, 2.402265069591007e-01f);
  p = fmaf(p, f, 6.931471805599453e-01f);
  p = fmaf(p, f, 1.0f);
  return ldexpf(p, (int)n);
}

/* d = exp(-e^{-1/2} * sigmoid(w)) in the reference's exp2 form
 * (wkv_fp32_v2.cu:27-29). */
float oracle_decay(float w) {
  float e = oracle_exp2(C2 * w);
  float den = 1.0f + e;
  float q = C1 / den;
  return oracle_exp2(q);
}

/* rotator1 (wkv_fp16_v2.cu:23-25): 2^-41 * float(int32(2654435769 * phase)),
 * with 32-bit wrap-around. */
float oracle_rotator(int32_t phase) {
  uint32_t m = 2654435769u * (uint32_t)phase;
  return TWO_NEG_41 * (float)(int32_t)m;
}

/* w_delta (wkv_fp16_v2.cu:27-30): fp16_rn((d - 1) + rot). */
uint16_t oracle_w_delta(float w, int32_t phase) {
  float d = oracle_decay(w) - 1.0f;
  d = d + oracle_rotator(phase);
  return oracle_f32_to_f16(d);
}

/* ---------------------------------------------------------------- threads */

void oracle_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

int oracle_get_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ---------------------------------------------------------------- fp32 WKV */

/* Dot product of one state row with a token vector in one of two orders:
 *   order 0: one FMA chain over j = 0..63 (the reference's row-per-thread
 *            kernel, wkv_fp32_v2.cu:103-117);
 *   order 1: eight FMA chains, chain g over the columns 4g..4g+3 then
 *            32+4g..32+4g+3 in that order, combined by the pairwise tree
 *            ((p0+p1)+(p2+p3)) + ((p4+p5)+(p6+p7)).  This is the row-split
 *            order of vkwr_amd's prefill kernel (eight lanes per state row).
 *            The reference's own split-row kernels (wkv_fp32_v2.cu:127-166
 *            warp-split, :169-218 block-split) likewise reduce partial sums
 *            across lanes instead of one chain; the order here is this build's. */
static float row_dot(const float* s, const float* x, int order) {
  if (order == 0) {
    float acc = 0.0f;
    for (int j = 0; j < HS; ++j) acc = fmaf(s[j], x[j], acc);
    return acc;
  }
  float p[8];
  for (int g = 0; g < 8; ++g) {
    float acc = 0.0f;
    for (int e = 0; e < 8; ++e) {
      const int j = (e < 4) ? 4 * g + e : 32 + 4 * g + (e - 4);
      acc = fmaf(s[j], x[j], acc);
    }
    p[g] = acc;
  }
  return ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
}

/* wkv_forward_fp32 family.  state [B,H,64,64] fp32 in place; r,w,k,v,a,b,y
 * [B,T,C] fp16 bits.  `order` selects the dot-product order (row_dot); the
 * per-element update fma(k, v, fma(sa, b, s*d)) is the same in both. */
static void wkv_fp32_impl(int B, int T, int C, int H, float* state,
                          const uint16_t* r, const uint16_t* w, const uint16_t* k,
                          const uint16_t* v, const uint16_t* a, const uint16_t* b,
                          uint16_t* y, int order) {
#pragma omp parallel for schedule(static)
  for (int bh = 0; bh < B * H; ++bh) {
    const int bi = bh / H, h = bh % H;
    float* S = state + (size_t)bh * HS * HS;
    float rr[HS], dd[HS], kk[HS], aa[HS], bb[HS];
    for (int t = 0; t < T; ++t) {
      const size_t base = ((size_t)bi * T + t) * C + (size_t)h * HS;
      for (int j = 0; j < HS; ++j) {
        rr[j] = oracle_f16_to_f32(r[base + j]);
        dd[j] = oracle_decay(oracle_f16_to_f32(w[base + j]));
        kk[j] = oracle_f16_to_f32(k[base + j]);
        aa[j] = oracle_f16_to_f32(a[base + j]);
        bb[j] = oracle_f16_to_f32(b[base + j]);
      }
      for (int i = 0; i < HS; ++i) {
        float* row = S + i * HS;
        const float sa = row_dot(row, aa, order);
        const float vi = oracle_f16_to_f32(v[base + i]);
        for (int j = 0; j < HS; ++j) {
          float s = row[j] * dd[j];
          s = fmaf(sa, bb[j], s);
          s = fmaf(kk[j], vi, s);
          row[j] = s;
        }
        y[base + i] = oracle_f32_to_f16(row_dot(row, rr, order));
      }
    }
  }
}

/* Row-per-thread order: the reference's wkv_fp32_v2_kernel (all four of this
 * build's fp32 dispatch modes at T == 1, and modes 1-3 at T > 1). */
void oracle_wkv_fp32(int B, int T, int C, int H, float* state,
                     const uint16_t* r, const uint16_t* w, const uint16_t* k,
                     const uint16_t* v, const uint16_t* a, const uint16_t* b,
                     uint16_t* y) {
  wkv_fp32_impl(B, T, C, H, state, r, w, k, v, a, b, y, 0);
}

/* Row-split order (row_dot order 1): this build's row-split kernels -- mode 0 and
 * the slot-pool entry point at 1 < T < 16, and the mixed step's LDS-free decode
 * kernel.  At T >= 16 mode 0 and the slot-pool entry point take the chunked
 * (16-token block) kernel, which no order here reproduces bit for bit: its
 * tests compare it with the row-per-thread order within a stated tolerance. */
void oracle_wkv_fp32_rows(int B, int T, int C, int H, float* state,
                          const uint16_t* r, const uint16_t* w, const uint16_t* k,
                          const uint16_t* v, const uint16_t* a, const uint16_t* b,
                          uint16_t* y) {
  wkv_fp32_impl(B, T, C, H, state, r, w, k, v, a, b, y, 1);
}

/* ---------------------------------------------------------------- fp16 WKV */

/* fp16-state family.  legacy == 0: vkwr_v1_wkv::wkv_{seq,one}{,_w0}_fp16
 * (wkv_fp16_v2.cu), phase = elapsed_t[b] + c + t, hfma2 nesting.
 * legacy == 1: vkwr_rwkv7::forward_{seq,one} (state_fwd_fp16.cu), phase =
 * elapsed_t[b] + t, separately rounded operators, w0 ignored.
 * w0 may be NULL (no w0); only its first C entries are read. */
void oracle_wkv_fp16(int B, int T, int C, int H, uint16_t* state,
                     const uint16_t* r, const uint16_t* w, const uint16_t* w0,
                     const uint16_t* k, const uint16_t* v, const uint16_t* a,
                     const uint16_t* b, uint16_t* y, const int32_t* elapsed_t,
                     int legacy) {
#pragma omp parallel for schedule(static)
  for (int bh = 0; bh < B * H; ++bh) {
    const int bi = bh / H, h = bh % H;
    uint16_t* S = state + (size_t)bh * HS * HS;
    uint16_t rr[HS], wd[HS], kk[HS], aa[HS], bb[HS];
    for (int t = 0; t < T; ++t) {
      const size_t base = ((size_t)bi * T + t) * C + (size_t)h * HS;
      for (int j = 0; j < HS; ++j) {
        const int c = h * HS + j;
        float wf = oracle_f16_to_f32(w[base + j]);
        int32_t phase;
        if (legacy) {
          phase = (int32_t)((uint32_t)elapsed_t[bi] + (uint32_t)t);
        } else {
          if (w0) wf = wf + oracle_f16_to_f32(w0[c]);
          phase = (int32_t)((uint32_t)elapsed_t[bi] + (uint32_t)c + (uint32_t)t);
        }
        wd[j] = oracle_w_delta(wf, phase);
        rr[j] = r[base + j];
        kk[j] = k[base + j];
        aa[j] = a[base + j];
        bb[j] = b[base + j];
      }
      for (int i = 0; i < HS; ++i) {
        uint16_t* row = S + i * HS;
        const uint16_t vi = v[base + i];
        uint16_t sa2[2] = {0, 0}, y2[2] = {0, 0};
        if (!legacy) {
          for (int j = 0; j < HS; ++j) sa2[j & 1] = fma16(aa[j], row[j], sa2[j & 1]);
          const uint16_t sa = add16(sa2[0], sa2[1]);
          for (int j = 0; j < HS; ++j) {
            const uint16_t s = row[j];
            uint16_t in1 = fma16(sa, bb[j], s);
            uint16_t in2 = fma16(kk[j], vi, in1);
            const uint16_t sn = fma16(s, wd[j], in2);
            row[j] = sn;
            y2[j & 1] = fma16(sn, rr[j], y2[j & 1]);
          }
        } else {
          for (int j = 0; j < HS; ++j) sa2[j & 1] = add16(sa2[j & 1], mul16(aa[j], row[j]));
          const uint16_t sa = add16(sa2[0], sa2[1]);
          for (int j = 0; j < HS; ++j) {
            const uint16_t s = row[j];
            uint16_t t1 = mul16(s, wd[j]);
            uint16_t t2 = mul16(kk[j], vi);
            uint16_t t3 = add16(t1, t2);
            uint16_t t4 = mul16(sa, bb[j]);
            uint16_t t5 = add16(t3, t4);
            const uint16_t sn = add16(s, t5);
            row[j] = sn;
            y2[j & 1] = add16(y2[j & 1], mul16(sn, rr[j]));
          }
        }
        y[base + i] = add16(y2[0], y2[1]);
      }
    }
  }
}

/* ---------------------------------------------------------------- advance */

/* advance_i32 (advance_i32_ops.cu:8-13): x[i] += amount, 32-bit wrap. */
void oracle_advance_i32(int32_t* x, int64_t n, int32_t amount) {
  for (int64_t i = 0; i < n; ++i) x[i] = (int32_t)((uint32_t)x[i] + (uint32_t)amount);
}

/* Exported for the oracle's own tests (exactness of the fp16 primitives). */
uint16_t oracle_fma16(uint16_t a, uint16_t b, uint16_t c) { return fma16(a, b, c); }
uint16_t oracle_add16(uint16_t a, uint16_t b) { return add16(a, b); }
uint16_t oracle_mul16(uint16_t a, uint16_t b) { return mul16(a, b); }
