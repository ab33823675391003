/*
 * moe_oracle.c -- CPU restatement of the reference's MoE-block oracle path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker and the CPU-baseline leg); the HIP
 * product never links or calls this file.  See moe_oracle.h for the scope.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, so every f32 operation
 * below rounds exactly where it is written).
 */
#include "moe_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* number formats                                                           */
/* ------------------------------------------------------------------------ */

/* Doubled e2m1 values; index 8 is -0 == 0 (hip-moe/src/main.hip:49-50). */
const int8_t mo_kvalues[16] = {0, 1, 2, 3, 4, 6, 8, 12,
                               0, -1, -2, -3, -4, -6, -8, -12};

static inline float bits_to_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint32_t f32_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* hip-moe/src/main.hip:52-57: half of the E8M0 scale, i.e. 2^(e-128); the
 * e<2 patterns are f32 denormals. */
float mo_e8m0_half(uint8_t e) {
  const uint32_t bits = e < 2 ? (0x00200000u << e) : ((uint32_t)(e - 1) << 23);
  return bits_to_f32(bits);
}

/* v >> s rounded to nearest, ties to even (s >= 1). */
static uint32_t rshift_rne(uint32_t v, int s) {
  if (s >= 32) return 0; /* v < 2^24 here, so v / 2^s < 1/2 */
  const uint32_t q = v >> s;
  const uint32_t rem = v & ((1u << s) - 1u);
  const uint32_t half = 1u << (s - 1);
  return q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u);
}

/* IEEE binary32 -> binary16, round-to-nearest-even, overflow to inf.  This
 * is what F16C's _cvtss_sh(x, 0), i.e. ggml's GGML_CPU_FP32_TO_FP16 on x86,
 * computes. */
uint16_t mo_fp32_to_fp16(float f) {
  const uint32_t x = f32_to_bits(f);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t exp = (x >> 23) & 0xffu;
  const uint32_t man = x & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0u));
  if (exp == 0u) return sign; /* f32 zero/denormal: far below fp16 range */
  const int e16 = (int)exp - 127 + 15;
  if (e16 >= 1) {
    const uint32_t h = ((uint32_t)e16 << 10) + rshift_rne(man, 13); /* carry ok */
    return (uint16_t)(sign | (h >= 0x7c00u ? 0x7c00u : h));
  }
  /* fp16 subnormal range: value = (man|2^23) * 2^(exp-150) = m * 2^-24 */
  return (uint16_t)(sign | rshift_rne(man | 0x800000u, 126 - (int)exp));
}

float mo_fp16_to_fp32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
  const uint32_t man = (uint32_t)h & 0x3ffu;
  if (exp == 0x1fu) return bits_to_f32(sign | 0x7f800000u | (man << 13));
  if (exp == 0u) {
    /* subnormal: man * 2^-24, exact in f32 */
    const float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t mo_fp32_to_bf16(float f) {
  const uint32_t x = f32_to_bits(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u); /* NaN */
  return (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

float mo_bf16_to_fp32(uint16_t b) { return bits_to_f32((uint32_t)b << 16); }

/* hip-moe/src/main.hip:82-95: element j of a block is qs[j] & 0xF, element
 * j+16 is qs[j] >> 4; value = kvalue * e8m0_half(e). */
void mo_dequant_mxfp4_row(const uint8_t *blocks, int K, float *out) {
  for (int b = 0; b < K / MO_QK; b++) {
    const uint8_t *blk = blocks + (size_t)b * MO_MXFP4_BYTES;
    const float sc = mo_e8m0_half(blk[0]);
    for (int j = 0; j < 16; j++) {
      out[b * MO_QK + j] = (float)mo_kvalues[blk[1 + j] & 0x0f] * sc;
      out[b * MO_QK + j + 16] = (float)mo_kvalues[blk[1 + j] >> 4] * sc;
    }
  }
}

/* ggml quantize_row_q8_0, x86 path (un-vendored; restated):
 *   amax = max |x| over the block; d = amax / 127 (f32) stored as fp16;
 *   id = amax != 0 ? 127 / amax : 0; q = round-half-even(x * id).
 * The scalar reference path instead uses id = 1/d and roundf; the two can
 * differ by one code on exact ties -- parity unpinned against ggml. */
void mo_quantize_q8_0(const float *x, int K, int8_t *qs, uint16_t *d) {
  for (int b = 0; b < K / MO_QK; b++) {
    const float *xb = x + (size_t)b * MO_QK;
    float amax = 0.0f;
    for (int j = 0; j < MO_QK; j++) {
      const float a = fabsf(xb[j]);
      amax = a > amax ? a : amax;
    }
    const float dd = amax / 127.0f;
    d[b] = mo_fp32_to_fp16(dd);
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    for (int j = 0; j < MO_QK; j++) {
      /* nearbyintf under the default rounding mode is half-to-even */
      qs[(size_t)b * MO_QK + j] = (int8_t)(int)nearbyintf(xb[j] * id);
    }
  }
}

int32_t mo_block_isum(const uint8_t *wblock, const int8_t *q) {
  int32_t lo = 0, hi = 0;
  for (int j = 0; j < 16; j++) {
    lo += (int32_t)q[j] * mo_kvalues[wblock[1 + j] & 0x0f];
    hi += (int32_t)q[j + 16] * mo_kvalues[wblock[1 + j] >> 4];
  }
  return lo + hi;
}

/* ggml_vec_dot_mxfp4_q8_0, generic (scalar) order: per block the exact int
 * sum, scaled by fp16(d_y) * e8m0_half(e_x), accumulated in f32 in
 * ascending block order.  ggml's AVX2 body accumulates two blocks per step
 * in 8 lanes then sums horizontally: the per-block terms are identical, only
 * the f32 summation order differs (parity unpinned at that level). */
float mo_vec_dot_mxfp4_q8_0(int K, const uint8_t *wrow, const int8_t *qs,
                            const uint16_t *d) {
  float acc = 0.0f;
  for (int b = 0; b < K / MO_QK; b++) {
    const uint8_t *blk = wrow + (size_t)b * MO_MXFP4_BYTES;
    const float s = mo_fp16_to_fp32(d[b]) * mo_e8m0_half(blk[0]);
    acc += s * (float)mo_block_isum(blk, qs + (size_t)b * MO_QK);
  }
  return acc;
}

/* Eight rows at once (row i at w + i*stride), each bit for bit
 * mo_vec_dot_mxfp4_q8_0: the per-block integer sums are exact in any order,
 * and the f32 work -- s = fp16(d) * e8m0_half(e), acc = acc + s * isum, in
 * ascending block order -- is the same IEEE multiply and add per row, done
 * in eight lanes.  AVX2 where the CPU has it: the nibbles index a vpshufb
 * table of the doubled e2m1 values, |w| x (q with w's sign) goes through
 * vpmaddubsw / vpmaddwd (|w| <= 12, |q| <= 127: no int16 saturation; q is
 * never -128 here, Q8_0 codes are within +-127), and three vphaddd levels
 * turn the rows' eight partial sums into one int32 each.  This is the
 * CPU-baseline's inner loop only; the checker keeps the scalar path. */
__attribute__((target("avx2"))) static void vec_dot8_avx2(int K, const uint8_t *w, size_t stride,
                                                           const int8_t *qs, const uint16_t *d, float *out) {
  const __m256i lut = _mm256_setr_epi8(0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12,
                                       0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12);
  const __m256i m4 = _mm256_set1_epi8(0x0f);
  const __m256i ones = _mm256_set1_epi16(1);
  const __m256i two = _mm256_set1_epi32(2), one = _mm256_set1_epi32(1);
  const __m256i den = _mm256_set1_epi32(0x00200000);
  __m256 acc = _mm256_setzero_ps();
  for (int b = 0; b < K / MO_QK; b++) {
    const __m256i qv = _mm256_loadu_si256((const __m256i *)(qs + (size_t)b * MO_QK));
    const uint8_t *b0 = w + (size_t)b * MO_MXFP4_BYTES;
    __m256i part[8];
    for (int r = 0; r < 8; r++) {
      /* the 16 nibble bytes in both halves: low nibbles index half 0, high half 1 */
      const __m256i v = _mm256_broadcastsi128_si256(_mm_loadu_si128((const __m128i *)(b0 + (size_t)r * stride + 1)));
      const __m256i idx = _mm256_blend_epi32(_mm256_and_si256(v, m4), _mm256_and_si256(_mm256_srli_epi16(v, 4), m4), 0xF0);
      const __m256i wv = _mm256_shuffle_epi8(lut, idx);
      const __m256i p16 = _mm256_maddubs_epi16(_mm256_sign_epi8(wv, wv), _mm256_sign_epi8(qv, wv));
      part[r] = _mm256_madd_epi16(p16, ones);
    }
    const __m256i t01 = _mm256_hadd_epi32(part[0], part[1]), t23 = _mm256_hadd_epi32(part[2], part[3]);
    const __m256i t45 = _mm256_hadd_epi32(part[4], part[5]), t67 = _mm256_hadd_epi32(part[6], part[7]);
    const __m256i t03 = _mm256_hadd_epi32(t01, t23), t47 = _mm256_hadd_epi32(t45, t67);
    /* t03 = [r0 r1 r2 r3 | r0 r1 r2 r3] over the two 128-bit halves of the block */
    const __m256i isum = _mm256_add_epi32(_mm256_permute2x128_si256(t03, t47, 0x20),
                                          _mm256_permute2x128_si256(t03, t47, 0x31));
    /* mo_e8m0_half of the eight rows' exponents, as bit patterns */
    const __m256i e = _mm256_setr_epi32(b0[0], b0[stride], b0[2 * stride], b0[3 * stride], b0[4 * stride],
                                        b0[5 * stride], b0[6 * stride], b0[7 * stride]);
    const __m256i big = _mm256_slli_epi32(_mm256_sub_epi32(e, one), 23);
    const __m256i small = _mm256_sllv_epi32(den, e);
    const __m256i bits = _mm256_blendv_epi8(big, small, _mm256_cmpgt_epi32(two, e));
    const __m256 sc = _mm256_mul_ps(_mm256_set1_ps(mo_fp16_to_fp32(d[b])), _mm256_castsi256_ps(bits));
    acc = _mm256_add_ps(acc, _mm256_mul_ps(sc, _mm256_cvtepi32_ps(isum)));
  }
  _mm256_storeu_ps(out, acc);
}

int mo_simd_available(void) { return __builtin_cpu_supports("avx2") ? 1 : 0; }

void mo_vec_dot8_mxfp4_q8_0(int K, const uint8_t *w, size_t stride, const int8_t *qs, const uint16_t *d,
                            float *out) {
  if (mo_simd_available()) {
    vec_dot8_avx2(K, w, stride, qs, d, out);
    return;
  }
  for (int r = 0; r < 8; r++) out[r] = mo_vec_dot_mxfp4_q8_0(K, w + (size_t)r * stride, qs, d);
}

/* ------------------------------------------------------------------------ */
/* routing                                                                  */
/* ------------------------------------------------------------------------ */

/* softplus as ggml states it: x for x > 20, else log1p(exp(x)). */
static float softplus_f32(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

void mo_route_scores(const float *logits, int T, int E, int mode, float *probs) {
  for (int t = 0; t < T; t++) {
    const float *l = logits + (size_t)t * E;
    float *p = probs + (size_t)t * E;
    if (mode == MO_ROUTE_SOFTMAX) {
      /* ggml soft_max: exp(l - max), sum in double, scale by (float)(1/sum) */
      float mx = -INFINITY;
      for (int e = 0; e < E; e++) mx = l[e] > mx ? l[e] : mx;
      double sum = 0.0;
      for (int e = 0; e < E; e++) {
        p[e] = expf(l[e] - mx);
        sum += (double)p[e];
      }
      const float inv = (float)(1.0 / sum);
      for (int e = 0; e < E; e++) p[e] *= inv;
    } else if (mode == MO_ROUTE_SIGMOID) {
      for (int e = 0; e < E; e++) p[e] = 1.0f / (1.0f + expf(-l[e]));
    } else {
      for (int e = 0; e < E; e++) p[e] = sqrtf(softplus_f32(l[e]));
    }
  }
}

void mo_route(const float *logits, const float *bias, int T, int E, int k,
              int mode, int norm, float scale, int32_t *ids, float *wts) {
  float *probs = (float *)malloc(sizeof(float) * (size_t)E);
  float *sel = (float *)malloc(sizeof(float) * (size_t)E);
  unsigned char *taken = (unsigned char *)malloc((size_t)E);
  for (int t = 0; t < T; t++) {
    mo_route_scores(logits + (size_t)t * E, 1, E, mode, probs);
    for (int e = 0; e < E; e++) sel[e] = bias ? probs[e] + bias[e] : probs[e];
    memset(taken, 0, (size_t)E);
    for (int s = 0; s < k; s++) {
      int best = -1;
      for (int e = 0; e < E; e++) {
        if (taken[e]) continue;
        if (best < 0 || sel[e] > sel[best]) best = e; /* strict: lower index wins ties */
      }
      taken[best] = 1;
      ids[(size_t)t * k + s] = best;
      wts[(size_t)t * k + s] = probs[best]; /* weights from the unbiased scores */
    }
    float *w = wts + (size_t)t * k;
    if (norm) {
      double sum = 0.0; /* ggml_sum_rows: double accumulator */
      for (int s = 0; s < k; s++) sum += (double)w[s];
      float fs = (float)sum;
      fs = fs < 6.103515625e-5f ? 6.103515625e-5f : fs; /* 2^-14 floor */
      for (int s = 0; s < k; s++) w[s] = w[s] / fs;
    }
    if (scale != 0.0f && scale != 1.0f) {
      for (int s = 0; s < k; s++) w[s] *= scale;
    }
  }
  free(probs);
  free(sel);
  free(taken);
}

/* ------------------------------------------------------------------------ */
/* grouping                                                                 */
/* ------------------------------------------------------------------------ */

/* The mul_mat_id row map: visit (t, s) token-major, slot-minor and append
 * the pair to its expert's list (nano-glm/apps/moe-server/main.cpp:413-459
 * uses the same order). */
int mo_group(const int32_t *ids, int T, int k, int E, int32_t *counts,
             int32_t *offsets, int32_t *perm, int32_t *inv) {
  const int P = T * k;
  if (E <= 0 || P < 0) return -1;
  for (int e = 0; e < E; e++) counts[e] = 0;
  for (int p = 0; p < P; p++) counts[ids[p]]++;
  int distinct = 0, run = 0;
  for (int e = 0; e < E; e++) {
    offsets[e] = run;
    run += counts[e];
    distinct += counts[e] > 0;
  }
  offsets[E] = run;
  int32_t *fill = (int32_t *)calloc((size_t)E, sizeof(int32_t));
  for (int p = 0; p < P; p++) {
    const int e = ids[p];
    const int row = offsets[e] + fill[e]++;
    perm[row] = p;
    if (inv) inv[p] = row;
  }
  free(fill);
  return distinct;
}

/* ------------------------------------------------------------------------ */
/* the block                                                                */
/* ------------------------------------------------------------------------ */

typedef struct {
  const mo_layer *L;
  int T, P, nthreads;
  const float *x;
  const int32_t *ids;
  const float *wts;
  float *out, *per_slot, *h_routed, *h_shared;
  /* scratch */
  int8_t *xq;     /* [T][H]   */
  uint16_t *xd;   /* [T][H/32] */
  float *h;       /* [P+T][F] routed pairs then shared rows */
  const float *h_in; /* if set: h is given (same layout), gate/up/SwiGLU skipped */
  int8_t *hq;     /* [P+T][F] */
  uint16_t *hd;   /* [P+T][F/32] */
  float *y;       /* [P+T][H] weighted routed rows, then shared rows */
  int rows8;      /* the dot products eight rows at a time (mo_vec_dot8_mxfp4_q8_0) */
  pthread_barrier_t bar;
} fwd_state;

typedef struct {
  fwd_state *S;
  int tid;
} fwd_arg;

static void span(size_t n, int tid, int nt, size_t *b, size_t *e) {
  *b = n * (size_t)tid / (size_t)nt;
  *e = n * (size_t)(tid + 1) / (size_t)nt;
}

static inline float clampf(float v, float lo, float hi) {
  /* ggml_clamp: MAX(MIN(v, hi), lo) */
  v = v < hi ? v : hi;
  return v > lo ? v : lo;
}

static void *fwd_worker(void *argp) {
  fwd_arg *a = (fwd_arg *)argp;
  fwd_state *S = a->S;
  const mo_layer *L = S->L;
  const int H = L->H, F = L->F, k = L->k, T = S->T, P = S->P;
  const int has_sh = L->sh_gate != NULL;
  const int R = P + (has_sh ? T : 0); /* expert rows: routed pairs, then shared */
  const size_t gu_row = (size_t)(H / MO_QK) * MO_MXFP4_BYTES;
  const size_t dn_row = (size_t)(F / MO_QK) * MO_MXFP4_BYTES;
  size_t b, e;

  /* gate / up / clamp / SwiGLU for every (expert row, ffn column) */
  span((size_t)R * F, a->tid, S->nthreads, &b, &e);
  for (size_t i = b; i < e && S->h_in; i++) S->h[i] = S->h_in[i];
  if (S->rows8 && !S->h_in) {
    /* the same per column, eight ffn columns per dot call */
    span((size_t)R * (F / 8), a->tid, S->nthreads, &b, &e);
    for (size_t i = b; i < e; i++) {
      const int r = (int)(i / (size_t)(F / 8)), c0 = (int)(i % (size_t)(F / 8)) * 8;
      const uint8_t *gw, *uw;
      int t;
      if (r < P) {
        t = r / k;
        gw = L->gate[S->ids[r]];
        uw = L->up[S->ids[r]];
      } else {
        t = r - P;
        gw = L->sh_gate;
        uw = L->sh_up;
      }
      const int8_t *q = S->xq + (size_t)t * H;
      const uint16_t *d = S->xd + (size_t)t * (H / MO_QK);
      float g8[8], u8[8];
      mo_vec_dot8_mxfp4_q8_0(H, gw + (size_t)c0 * gu_row, gu_row, q, d, g8);
      mo_vec_dot8_mxfp4_q8_0(H, uw + (size_t)c0 * gu_row, gu_row, q, d, u8);
      for (int j = 0; j < 8; j++) {
        float g = g8[j], u = u8[j];
        if (L->clamp > 1e-6f) {
          u = clampf(u, -L->clamp, L->clamp);
          g = clampf(g, -INFINITY, L->clamp);
        }
        S->h[(size_t)r * F + c0 + j] = (g / (1.0f + expf(-g))) * u;
      }
    }
    b = e = 0;  /* the per-column loop below has nothing left */
  }
  for (size_t i = b; i < e && !S->h_in; i++) {
    const int r = (int)(i / (size_t)F), c = (int)(i % (size_t)F);
    const uint8_t *gw, *uw;
    int t;
    if (r < P) {
      t = r / k;
      const int ex = S->ids[r];
      gw = L->gate[ex] + (size_t)c * gu_row;
      uw = L->up[ex] + (size_t)c * gu_row;
    } else {
      t = r - P;
      gw = L->sh_gate + (size_t)c * gu_row;
      uw = L->sh_up + (size_t)c * gu_row;
    }
    const int8_t *q = S->xq + (size_t)t * H;
    const uint16_t *d = S->xd + (size_t)t * (H / MO_QK);
    float g = mo_vec_dot_mxfp4_q8_0(H, gw, q, d);
    float u = mo_vec_dot_mxfp4_q8_0(H, uw, q, d);
    if (L->clamp > 1e-6f) {
      /* deepseek4 order: up symmetric, gate one-sided, before SiLU */
      u = clampf(u, -L->clamp, L->clamp);
      g = clampf(g, -INFINITY, L->clamp);
    }
    /* ggml_swiglu_split: silu(gate) * up, silu(x) = x / (1 + exp(-x)) */
    S->h[(size_t)r * F + c] = (g / (1.0f + expf(-g))) * u;
  }
  pthread_barrier_wait(&S->bar);

  /* Q8_0 of every h row (down's src1 conversion) */
  span((size_t)R, a->tid, S->nthreads, &b, &e);
  for (size_t r = b; r < e; r++) {
    mo_quantize_q8_0(S->h + r * F, F, S->hq + r * F, S->hd + r * (F / MO_QK));
  }
  pthread_barrier_wait(&S->bar);

  /* down, times the router weight for routed rows (the MUL node) */
  span((size_t)R * H, a->tid, S->nthreads, &b, &e);
  if (S->rows8) {
    span((size_t)R * (H / 8), a->tid, S->nthreads, &b, &e);
    for (size_t i = b; i < e; i++) {
      const int r = (int)(i / (size_t)(H / 8)), c0 = (int)(i % (size_t)(H / 8)) * 8;
      const uint8_t *dw = r < P ? L->down[S->ids[r]] : L->sh_down;
      float v8[8];
      mo_vec_dot8_mxfp4_q8_0(F, dw + (size_t)c0 * dn_row, dn_row, S->hq + (size_t)r * F,
                             S->hd + (size_t)r * (F / MO_QK), v8);
      for (int j = 0; j < 8; j++) S->y[(size_t)r * H + c0 + j] = r < P ? v8[j] * S->wts[r] : v8[j];
    }
    b = e = 0;
  }
  for (size_t i = b; i < e; i++) {
    const int r = (int)(i / (size_t)H), c = (int)(i % (size_t)H);
    const uint8_t *dw = r < P ? L->down[S->ids[r]] + (size_t)c * dn_row
                              : L->sh_down + (size_t)c * dn_row;
    float v = mo_vec_dot_mxfp4_q8_0(F, dw, S->hq + (size_t)r * F,
                                    S->hd + (size_t)r * (F / MO_QK));
    if (r < P) v = v * S->wts[r];
    S->y[(size_t)r * H + c] = v;
  }
  pthread_barrier_wait(&S->bar);

  /* pairwise combine in slot order, then + shared (trunk ADDs) */
  span((size_t)T * H, a->tid, S->nthreads, &b, &e);
  for (size_t i = b; i < e; i++) {
    const int t = (int)(i / (size_t)H), c = (int)(i % (size_t)H);
    float acc = S->y[((size_t)t * k) * H + c];
    for (int s = 1; s < k; s++) acc = acc + S->y[((size_t)t * k + s) * H + c];
    if (has_sh) acc = acc + S->y[((size_t)P + t) * H + c];
    S->out[i] = acc;
  }
  return NULL;
}

static int forward_impl(const mo_layer *L, int T, const float *x, const int32_t *ids, const float *wts,
                        const float *h_in, float *out, float *per_slot, float *h_routed, float *h_shared,
                        int n_threads, int rows8);

int mo_moe_forward_taps(const mo_layer *L, int T, const float *x,
                        const int32_t *ids, const float *wts, float *out,
                        float *per_slot, float *h_routed, float *h_shared,
                        int n_threads) {
  return forward_impl(L, T, x, ids, wts, NULL, out, per_slot, h_routed, h_shared, n_threads, 0);
}

int mo_moe_forward_from_h(const mo_layer *L, int T, const int32_t *ids, const float *wts,
                          const float *h, float *out, float *per_slot, int n_threads) {
  if (!h) return -1;
  return forward_impl(L, T, NULL, ids, wts, h, out, per_slot, NULL, NULL, n_threads, 0);
}

static int forward_impl(const mo_layer *L, int T, const float *x, const int32_t *ids, const float *wts,
                        const float *h_in, float *out, float *per_slot, float *h_routed, float *h_shared,
                        int n_threads, int rows8) {
  if (!L || T <= 0 || (!x && !h_in) || !ids || !wts || !out) return -1;
  if (L->H % MO_QK || L->F % MO_QK || L->k <= 0 || L->E <= 0) return -1;
  for (int p = 0; p < T * L->k; p++) {
    if (ids[p] < 0 || ids[p] >= L->E || !L->gate[ids[p]] || !L->up[ids[p]] ||
        !L->down[ids[p]])
      return -1;
  }
  const int H = L->H, F = L->F, P = T * L->k;
  const int R = P + (L->sh_gate ? T : 0);
  if (n_threads < 1) n_threads = 1;

  fwd_state S;
  memset(&S, 0, sizeof(S));
  S.L = L;
  S.T = T;
  S.P = P;
  S.nthreads = n_threads;
  S.x = x;
  S.h_in = h_in;
  S.ids = ids;
  S.wts = wts;
  S.out = out;
  S.rows8 = rows8 && F % 8 == 0 && H % 8 == 0;
  S.xq = (int8_t *)malloc((size_t)T * H);
  S.xd = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)T * (H / MO_QK));
  S.h = (float *)malloc(sizeof(float) * (size_t)R * F);
  S.hq = (int8_t *)malloc((size_t)R * F);
  S.hd = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)R * (F / MO_QK));
  S.y = (float *)malloc(sizeof(float) * (size_t)R * H);
  if (!S.xq || !S.xd || !S.h || !S.hq || !S.hd || !S.y) {
    free(S.xq); free(S.xd); free(S.h); free(S.hq); free(S.hd); free(S.y);
    return -1;
  }
  /* src1 -> Q8_0, once per token (mul_mat_id broadcasts x over slots) */
  for (int t = 0; t < T && x; t++) {
    mo_quantize_q8_0(x + (size_t)t * H, H, S.xq + (size_t)t * H,
                     S.xd + (size_t)t * (H / MO_QK));
  }
  pthread_barrier_init(&S.bar, NULL, (unsigned)n_threads);
  pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)n_threads);
  fwd_arg *args = (fwd_arg *)malloc(sizeof(fwd_arg) * (size_t)n_threads);
  for (int i = 0; i < n_threads; i++) {
    args[i].S = &S;
    args[i].tid = i;
    if (i) pthread_create(&th[i], NULL, fwd_worker, &args[i]);
  }
  fwd_worker(&args[0]);
  for (int i = 1; i < n_threads; i++) pthread_join(th[i], NULL);
  pthread_barrier_destroy(&S.bar);
  free(th);
  free(args);

  if (per_slot) memcpy(per_slot, S.y, sizeof(float) * (size_t)P * H);
  if (h_routed) memcpy(h_routed, S.h, sizeof(float) * (size_t)P * F);
  if (h_shared && L->sh_gate) memcpy(h_shared, S.h + (size_t)P * F, sizeof(float) * (size_t)T * F);
  free(S.xq); free(S.xd); free(S.h); free(S.hq); free(S.hd); free(S.y);
  return 0;
}

int mo_moe_forward(const mo_layer *L, int T, const float *x,
                   const int32_t *ids, const float *wts, float *out,
                   float *per_slot, int n_threads) {
  return mo_moe_forward_taps(L, T, x, ids, wts, out, per_slot, NULL, NULL, n_threads);
}

int mo_moe_forward_rows8(const mo_layer *L, int T, const float *x, const int32_t *ids, const float *wts,
                         float *out, int n_threads) {
  return forward_impl(L, T, x, ids, wts, NULL, out, NULL, NULL, NULL, n_threads, 1);
}

/* ------------------------------------------------------------------------ */
/* exact h (parity checker: the yardstick for f32 summation-order error)    */
/* ------------------------------------------------------------------------ */

typedef struct {
  const mo_layer *L;
  int T, P, R, nthreads, tid;
  const int32_t *ids;
  const int8_t *xq;
  const uint16_t *xd;
  double *h;     /* [R][F] */
  double *bound; /* [R][F] or NULL: the error bound of an f32 evaluation instead of h */
} hx_arg;

/* One row of gate or up in double: every block term isum * e8m0_half(e) *
 * fp16(d) is exact in double (|isum| < 2^17, a power of two, an 11-bit
 * mantissa), and the 2^-53 rounding of the sum is far below any f32 error. */
static double dot_exact(int K, const uint8_t *wrow, const int8_t *qs, const uint16_t *d) {
  double acc = 0.0;
  for (int b = 0; b < K / MO_QK; b++) {
    const uint8_t *blk = wrow + (size_t)b * MO_MXFP4_BYTES;
    acc += (double)mo_block_isum(blk, qs + (size_t)b * MO_QK) * (double)mo_e8m0_half(blk[0]) *
           (double)mo_fp16_to_fp32(d[b]);
  }
  return acc;
}

/* The magnitude sum behind one row's dot, for its error bound: sum over the
 * blocks of e8m0_half(e) * fp16(d) * sum_j (|q_j| + 30) * |w_j|.  The device
 * multiplies the weights by the two e4m3 digit planes of q (q = 16*hi + lo,
 * lo in [0, 15]), so its block terms are bounded by |16*hi| + |lo| <= |q| +
 * 30 times |w|; every product is exact and every block's integer sum too. */
static double dot_l1(int K, const uint8_t *wrow, const int8_t *qs, const uint16_t *d) {
  double acc = 0.0;
  for (int b = 0; b < K / MO_QK; b++) {
    const uint8_t *blk = wrow + (size_t)b * MO_MXFP4_BYTES;
    const int8_t *q = qs + (size_t)b * MO_QK;
    int32_t s = 0;
    for (int j = 0; j < 16; j++) {
      s += (abs(q[j]) + 30) * abs(mo_kvalues[blk[1 + j] & 0x0f]);
      s += (abs(q[j + 16]) + 30) * abs(mo_kvalues[blk[1 + j] >> 4]);
    }
    acc += (double)s * (double)mo_e8m0_half(blk[0]) * fabs((double)mo_fp16_to_fp32(d[b]));
  }
  return acc;
}

static void *hx_worker(void *argp) {
  hx_arg *a = (hx_arg *)argp;
  const mo_layer *L = a->L;
  const int H = L->H, F = L->F, k = L->k, P = a->P;
  const size_t gu_row = (size_t)(H / MO_QK) * MO_MXFP4_BYTES;
  size_t b, e;
  span((size_t)a->R * F, a->tid, a->nthreads, &b, &e);
  for (size_t i = b; i < e; i++) {
    const int r = (int)(i / (size_t)F), c = (int)(i % (size_t)F);
    const int t = r < P ? r / k : r - P;
    const uint8_t *gw = r < P ? L->gate[a->ids[r]] : L->sh_gate;
    const uint8_t *uw = r < P ? L->up[a->ids[r]] : L->sh_up;
    const int8_t *q = a->xq + (size_t)t * H;
    const uint16_t *d = a->xd + (size_t)t * (H / MO_QK);
    double g = dot_exact(H, gw + (size_t)c * gu_row, q, d);
    double u = dot_exact(H, uw + (size_t)c * gu_row, q, d);
    if (L->clamp > 1e-6f) {
      const double l = (double)L->clamp;
      u = u < l ? u : l;
      u = u > -l ? u : -l;
      g = g < l ? g : l;
    }
    const double h = g / (1.0 + exp(-g)) * u;
    if (!a->bound) {
      a->h[i] = h;
      continue;
    }
    /* Any f32 evaluation that sums the exact block terms in any order, with
     * at most one rounding per term and per addition: |error| <= gamma_m *
     * (sum of |terms|), m = blocks + 8 (Higham, Accuracy and Stability of
     * Numerical Algorithms, 2nd ed., eq. 4.4); the clamps are 1-Lipschitz,
     * |silu'| <= 1.1; SiLU's exp, add, divide and the product add at most 8
     * roundings of h.  Twice that, first order plus the product term. */
    const double uu = ldexp(1.0, -24), m = (double)(H / MO_QK + 8), gam = m * uu / (1.0 - m * uu);
    const double eg = gam * dot_l1(H, gw + (size_t)c * gu_row, q, d);
    const double eu = gam * dot_l1(H, uw + (size_t)c * gu_row, q, d);
    const double s = g / (1.0 + exp(-g));
    a->bound[i] = 2.0 * (1.1 * eg * fabs(u) + fabs(s) * eu + 1.1 * eg * eu + 8.0 * uu * fabs(h)) + 1e-37;
  }
  return NULL;
}

static int h_exact_impl(const mo_layer *L, int T, const float *x, const int32_t *ids, double *h_routed,
                        double *h_shared, int n_threads, int bound);

int mo_moe_h_exact(const mo_layer *L, int T, const float *x, const int32_t *ids, double *h_routed,
                   double *h_shared, int n_threads) {
  return h_exact_impl(L, T, x, ids, h_routed, h_shared, n_threads, 0);
}

int mo_moe_h_bound(const mo_layer *L, int T, const float *x, const int32_t *ids, double *b_routed,
                   double *b_shared, int n_threads) {
  return h_exact_impl(L, T, x, ids, b_routed, b_shared, n_threads, 1);
}

static int h_exact_impl(const mo_layer *L, int T, const float *x, const int32_t *ids, double *h_routed,
                        double *h_shared, int n_threads, int bound) {
  if (!L || T <= 0 || !x || !ids || !h_routed) return -1;
  if (L->H % MO_QK || L->F % MO_QK || L->k <= 0 || L->E <= 0) return -1;
  for (int p = 0; p < T * L->k; p++)
    if (ids[p] < 0 || ids[p] >= L->E || !L->gate[ids[p]] || !L->up[ids[p]]) return -1;
  const int H = L->H, F = L->F, P = T * L->k;
  const int R = P + (L->sh_gate && h_shared ? T : 0);
  if (n_threads < 1) n_threads = 1;
  int8_t *xq = (int8_t *)malloc((size_t)T * H);
  uint16_t *xd = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)T * (H / MO_QK));
  double *h = (double *)malloc(sizeof(double) * (size_t)R * F);
  pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)n_threads);
  hx_arg *args = (hx_arg *)malloc(sizeof(hx_arg) * (size_t)n_threads);
  if (!xq || !xd || !h || !th || !args) {
    free(xq); free(xd); free(h); free(th); free(args);
    return -1;
  }
  for (int t = 0; t < T; t++)
    mo_quantize_q8_0(x + (size_t)t * H, H, xq + (size_t)t * H, xd + (size_t)t * (H / MO_QK));
  for (int i = 0; i < n_threads; i++) {
    args[i] = (hx_arg){L, T, P, R, n_threads, i, ids, xq, xd, bound ? NULL : h, bound ? h : NULL};
    if (i) pthread_create(&th[i], NULL, hx_worker, &args[i]);
  }
  hx_worker(&args[0]);
  for (int i = 1; i < n_threads; i++) pthread_join(th[i], NULL);
  memcpy(h_routed, h, sizeof(double) * (size_t)P * F);
  if (R > P) memcpy(h_shared, h + (size_t)P * F, sizeof(double) * (size_t)T * F);
  free(xq); free(xd); free(h); free(th); free(args);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* synthetic weights                                                        */
/* ------------------------------------------------------------------------ */

/* SplitMix64's output function applied to state z (Steele, Lea & Flood,
 * "Fast splittable pseudorandom number generators", OOPSLA 2014). */
uint64_t mo_mix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

uint64_t mo_gen_key(uint64_t seed, int layer, int tensor, int expert) {
  const uint64_t id = ((uint64_t)(uint32_t)layer << 40) ^ ((uint64_t)(uint32_t)tensor << 32) ^
                      (uint64_t)(uint32_t)expert;
  return mo_mix64(seed ^ mo_mix64(id));
}

void mo_gen_mxfp4(uint64_t seed, int layer, int tensor, int expert, int rows,
                  int K, int e_lo, int e_span, uint8_t *out) {
  const uint64_t key = mo_gen_key(seed, layer, tensor, expert);
  const uint64_t nb = (uint64_t)rows * (uint64_t)(K / MO_QK);
  for (uint64_t i = 0; i < nb; i++) {
    uint8_t *blk = out + i * MO_MXFP4_BYTES;
    const uint64_t a = mo_mix64(key + 2 * i + 1);
    const uint64_t b = mo_mix64(key + 2 * i + 2);
    const uint64_t c = mo_mix64(key ^ ~i);
    blk[0] = (uint8_t)(e_lo + (int)(((c >> 32) * (uint64_t)e_span) >> 32));
    for (int j = 0; j < 8; j++) {
      blk[1 + j] = (uint8_t)(a >> (8 * j));
      blk[9 + j] = (uint8_t)(b >> (8 * j));
    }
  }
}
