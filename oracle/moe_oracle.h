/*
 * moe_oracle.h -- CPU restatement of the reference's MoE-block oracle path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP product
 * path and the CPU baseline leg of bench.py.  Nothing in the product links it,
 * and the product never falls back to it.
 *
 * What it restates: ggml-cpu's MUL_MAT_ID over MXFP4 expert weights with
 * Q8_0-quantized activations (the reference's CPU delegate,
 * moe-serv/src/moe_backend.cpp:457-483), plus the routing, grouping and
 * combine that surround it in the reference's block definitions
 * (nano-glm/lib/models/glm_dsa/moe_block.h:48-133,
 *  nano-glm/lib/models/deepseek4/moe_block.h:168-215,
 *  hip-moe/src/moe_ggml_bench.cpp:137-213).
 *
 * ggml itself (v0.18.1, commit 6a32c29a7) is not vendored in the reference,
 * so the parts that live only inside ggml are restated from its published
 * algorithm; each function says which, and which parts of it are pinned by a
 * test and which are "parity unpinned".
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- number formats --------------------------------------------------- */

#define MO_QK 32          /* elements per MXFP4 / Q8_0 block                 */
#define MO_MXFP4_BYTES 17 /* { uint8 e; uint8 qs[16]; }                      */

/* kvalues: doubled e2m1, bit 3 is the sign (hip-moe/src/main.hip:50). */
extern const int8_t mo_kvalues[16];

/* E8M0 exponent -> 2^(e-128) as f32, with the e<2 denormal branch
 * (hip-moe/src/main.hip:52-57; moe-serv/shaders/mxfp4_pass1.comp:51-55). */
float mo_e8m0_half(uint8_t e);

uint16_t mo_fp32_to_fp16(float f); /* IEEE binary16, round-to-nearest-even    */
float mo_fp16_to_fp32(uint16_t h);
uint16_t mo_fp32_to_bf16(float f); /* round-to-nearest-even                   */
float mo_bf16_to_fp32(uint16_t b);

/* Dequantize one MXFP4 row of K elements (hip-moe/src/main.hip:82-95). */
void mo_dequant_mxfp4_row(const uint8_t *blocks, int K, float *out);

/* Q8_0 quantization of one row of K floats (K % 32 == 0): per 32-block
 * amax, d = amax/127 stored as fp16, q = rint_even(x * (127/amax)).
 * Restates ggml's x86 quantize_row_q8_0 (un-vendored; parity unpinned
 * against ggml itself, pinned here by invariants). */
void mo_quantize_q8_0(const float *x, int K, int8_t *qs, uint16_t *d);

/* Exact int32 dot of one MXFP4 block with one Q8_0 block. */
int32_t mo_block_isum(const uint8_t *wblock, const int8_t *q);

/* mo_vec_dot_mxfp4_q8_0 of eight rows (row i at w + i*stride) against one
 * Q8_0 vector, bit for bit per row; AVX2 when mo_simd_available(), else the
 * scalar routine per row.  Codes must lie in [-127, 127] (Q8_0's range). */
void mo_vec_dot8_mxfp4_q8_0(int K, const uint8_t *w, size_t stride, const int8_t *qs, const uint16_t *d,
                            float *out);
int mo_simd_available(void);

/* ggml_vec_dot_mxfp4_q8_0, generic order: acc += (fp16(d)*e8m0_half(e))*isum
 * over blocks in ascending order, f32. */
float mo_vec_dot_mxfp4_q8_0(int K, const uint8_t *wrow, const int8_t *qs,
                            const uint16_t *d);

/* ---- routing ---------------------------------------------------------- */

enum { MO_ROUTE_SOFTMAX = 0, MO_ROUTE_SIGMOID = 1, MO_ROUTE_SQRT_SOFTPLUS = 2 };

/* Scores -> (+bias for selection) -> top-k descending (ties: lower index
 * first) -> weights from the unbiased scores -> optional renorm with the
 * 2^-14 floor -> optional scale (glm_dsa/moe_block.h:48-91,
 * deepseek4/moe_block.h:91-158).  logits [T][E], bias [E] or NULL,
 * ids [T][k], wts [T][k]. */
void mo_route(const float *logits, const float *bias, int T, int E, int k,
              int mode, int norm, float scale, int32_t *ids, float *wts);

/* Scores only (the probs tensor before selection), [T][E]. */
void mo_route_scores(const float *logits, int T, int E, int mode, float *probs);

/* ---- grouping --------------------------------------------------------- */

/* ggml mul_mat_id row grouping: pairs p = t*k + s visited token-major,
 * slot-minor; counts[e] = #pairs on e; offsets[e] = exclusive prefix sum
 * (offsets[E] = T*k); perm[offsets[e] + i] = i-th pair on e in visiting
 * order; inv[p] = grouped row of pair p.  Returns the number of distinct
 * experts touched. */
int mo_group(const int32_t *ids, int T, int k, int E, int32_t *counts,
             int32_t *offsets, int32_t *perm, int32_t *inv);

/* ---- the block -------------------------------------------------------- */

typedef struct {
  int H;            /* hidden (reduction dim of gate/up, rows of down)      */
  int F;            /* expert FFN width                                     */
  int E;            /* routed experts                                       */
  int k;            /* experts used per token                               */
  float clamp;      /* SwiGLU limit; <= 1e-6 disables (deepseek4 order)     */
  /* per-expert pointers into ggml-layout MXFP4 blocks; NULL = not resident
   * on the host (must not be touched by the given ids)                     */
  const uint8_t *const *gate; /* [E] -> [F][H/32] blocks */
  const uint8_t *const *up;   /* [E] -> [F][H/32] blocks */
  const uint8_t *const *down; /* [E] -> [H][F/32] blocks */
  const uint8_t *sh_gate;     /* shared expert or NULL   */
  const uint8_t *sh_up;
  const uint8_t *sh_down;
} mo_layer;

/* One MoE block over T tokens: x [T][H] f32, ids/wts [T][k].
 * out [T][H] = ((y_0 + y_1) + ... + y_{k-1}) + shared, y_s = w_s * down(...)
 * If per_slot is non-NULL it receives the weighted per-slot rows [T][k][H]
 * (the MUL node of the reference's split).  n_threads >= 1 splits output
 * rows; results do not depend on it. Returns 0, or -1 on bad arguments. */
int mo_moe_forward(const mo_layer *L, int T, const float *x,
                   const int32_t *ids, const float *wts, float *out,
                   float *per_slot, int n_threads);

/* mo_moe_forward with the dot products eight output rows at a time
 * (mo_vec_dot8_mxfp4_q8_0): the same result bit for bit, faster.  The
 * CPU-baseline leg of bench.py times this; the checker uses mo_moe_forward.
 * F and H must be multiples of 8 for the eight-row loops (else the
 * per-row path runs). */
int mo_moe_forward_rows8(const mo_layer *L, int T, const float *x, const int32_t *ids, const float *wts,
                         float *out, int n_threads);

/* Intermediate taps for tests: h (post-SwiGLU, pre-quantization) [T][k][F]
 * and the shared expert's h [T][F] (may be NULL). */
int mo_moe_forward_taps(const mo_layer *L, int T, const float *x,
                        const int32_t *ids, const float *wts, float *out,
                        float *per_slot, float *h_routed, float *h_shared,
                        int n_threads);

/* The same block from a given h [P+T][F] (routed pairs t*k+s, then the
 * shared expert's T rows): Q8_0 of h, down, router weight, combine.  Lets a
 * test reproduce the activation quantization of another implementation's
 * h exactly. */
int mo_moe_forward_from_h(const mo_layer *L, int T, const int32_t *ids, const float *wts,
                          const float *h, float *out, float *per_slot, int n_threads);

/* The SwiGLU output h of the same block with gate and up summed exactly (in
 * double: each block term isum * e8m0_half(e) * fp16(d) is exact there) and
 * clamp / SiLU / product in double, from the same Q8_0 of x as
 * mo_moe_forward.  h_routed [T][k][F], h_shared [T][F] (NULL: not computed).
 * No counterpart in ggml: it is the parity checker's yardstick, against
 * which the f32 error of this oracle and of the device are both measured. */
int mo_moe_h_exact(const mo_layer *L, int T, const float *x, const int32_t *ids,
                   double *h_routed, double *h_shared, int n_threads);

/* For each value of that h, a bound on the error of any f32 evaluation of
 * it that sums the block terms of gate and up in any order (one rounding
 * per term and per addition at most, the device's digit-plane split of
 * each term included) and then evaluates clamp, SiLU and the product in
 * f32: |h_f32 - h_exact| <= bound.  Same layout and arguments as
 * mo_moe_h_exact.  The parity checker's yardstick for single values whose
 * gate or up sum cancels (large terms, small result). */
int mo_moe_h_bound(const mo_layer *L, int T, const float *x, const int32_t *ids,
                   double *b_routed, double *b_shared, int n_threads);

/* ---- synthetic weights ------------------------------------------------ */

/* SplitMix64 finalizer (Steele, Lea, Flood 2014). */
uint64_t mo_mix64(uint64_t z);

/* Counter-based MXFP4 weight generator shared with the device generator:
 * block i of matrix (seed, layer, tensor, expert) has
 *   qs bytes = little-endian bytes of mix(key + 2i+1), mix(key + 2i+2)
 *   e        = e_lo + ((mix(key ^ ~i) >> 32) * e_span >> 32)
 * where key = mix(seed ^ mix(layer<<40 | tensor<<32 | expert)).
 * Writes rows*(K/32) blocks of 17 bytes. */
void mo_gen_mxfp4(uint64_t seed, int layer, int tensor, int expert, int rows,
                  int K, int e_lo, int e_span, uint8_t *out);
uint64_t mo_gen_key(uint64_t seed, int layer, int tensor, int expert);

/* tensor ids for the generator */
enum { MO_T_GATE = 0, MO_T_UP = 1, MO_T_DOWN = 2, MO_T_SH_GATE = 3,
       MO_T_SH_UP = 4, MO_T_SH_DOWN = 5 };

#ifdef __cplusplus
}
#endif
#endif
