// kernels_rows.h -- the expert kernels (decode and grouped), on gfx950's
// scaled MFMA: v_mfma_scale_f32_16x16x128_f8f6f4 with the MXFP4 weights as
// the fp4 A operand (their E8M0 exponents as the A scales) and the Q8_0
// activations as the fp8 B operand.
//
// Weight layout in HBM (written by the repack/generator kernels, see
// kernels_weights.h): rows in tiles of 16, the reduction dim in quads of
// 4 blocks (128 weights), records of 4 quads; lane l of a wave reading quad
// q of a tile gets the 16 nibble bytes of block 4q + l/16 of row l%16 (ggml's
// bytes, unchanged), and one exponent dword per 4 quads (byte q%4).  That is
// exactly the A-operand lane layout of the 16x16x128 MFMA: lane r + 16g
// holds row r, K-block g, nibble e at K offset e.  A ggml byte j holds
// element j (low nibble) and j+16 (high), so K offset e of a block carries
// element sigma(e) = e/2 + 16*(e%2); the activations are laid out to match.
//
// Activations.  ggml quantizes them to Q8_0: per 32-block an fp16 scale d
// and int8 codes q in [-127, 127].  Each code is split into two exact e4m3
// digits, hi = q >> 4 in [-8, 7] and lo = q & 15 in [0, 15] (q = 16*hi + lo),
// and the B operand is block-diagonal: column n = 8*token + 4*part + g of the
// MFMA holds part (0 = hi, 1 = lo) of block g of the quad, for two tokens.
// The B scale of a hi column is 2^4, of a lo column 2^0, so every output
// column is 2^(e_w - 127) times an exact integer block sum (all products and
// partial sums are small integers in f32), i.e. ggml's per-block integer dot
// times the weight scale.  The activation scale d of each (token, block) is
// then applied in f32 by the lane that holds that column, and the 8 columns
// of a token are added in a fixed order at the end: ggml-cpu's MXFP4 x Q8_0
// arithmetic with another (fixed) f32 summation order.
//
// B-operand lane layout (probed on the device): lane n + 16*gb holds column
// n; its bytes 0-15 are K offsets 16*gb + [0, 16), bytes 16-31 are K offsets
// 64 + 16*gb + [0, 16).  So block g's 32 bytes go to lanes gb = 2*(g%2) + h
// (h = half), in bytes 16*(g/2) + [0, 16).
//
// Staged activations ("xs" format, LDS and the h buffers): per block 16
// dwords, hi[8] then lo[8], each the 32 e4m3 digits in MFMA K order, plus
// the block's fp16 scale d widened to f32 in a separate array.
#pragma once

#include "device_common.h"
#include "kernels_weights.h"

#define MOE_TILE 16     // rows per MFMA tile
#define MOE_UNIT 32     // rows per h unit (one Q8_0 block of the SwiGLU output)
#define MOE_XSW 16      // dwords per staged block
#define MOE_GRP_WAVES 4 // waves per grouped-kernel workgroup (K split 4 ways)

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__host__ __device__ __forceinline__ int moe_nq4(int NQ) { return (NQ + 3) >> 2; }

// Split of n items over c parts: part i owns [lo, hi).
__host__ __device__ __forceinline__ void split_range(int n, int c, int i, int &lo, int &hi) {
  lo = (int)(((long)n * i) / c);
  hi = (int)(((long)n * (i + 1)) / c);
}

// ---------------------------------------------------------------------------
// e4m3 digits

// Four small integers (exact in e4m3) -> one dword of e4m3 bytes, a in byte 0.
__device__ __forceinline__ uint32_t pack_e4m3x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

__device__ __forceinline__ float q_hi(float q) { return (float)(((int)q) >> 4); }
__device__ __forceinline__ float q_lo(float q) { return (float)(((int)q) & 15); }

// ---------------------------------------------------------------------------
// Staging into LDS.  Two lanes per block: lane half h takes elements
// 8h..8h+7 and 16+8h..16+8h+7, which are exactly the MFMA K offsets
// 16h..16h+15 of the block (offset 2i -> element 8h+i, 2i+1 -> 16+8h+i).

// Q8_0 of nb blocks of one f32 row (ggml's x86 rounding: d = fp16(amax/127),
// q = rint(x * 127/amax)) into the staged format.
// tid / nthr: this thread's index among the nthr threads (a multiple of
// 64, whole waves) that share the work.
__device__ __forceinline__ void stage_quant(const float *__restrict__ x, int nb, uint32_t *xs, float *dy, int tid,
                                            int nthr) {
  const int h = tid & 1;
  for (int b = tid >> 1; b < nb; b += nthr >> 1) {
    const float4 *xb = reinterpret_cast<const float4 *>(x + (size_t)b * MOE_QK + 8 * h);
    const float4 a0 = xb[0], a1 = xb[1], c0 = xb[4], c1 = xb[5];
    const float lo[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const float hi[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) amax = fmaxf(amax, fmaxf(fabsf(lo[i]), fabsf(hi[i])));
    amax = fmaxf(amax, dpp_f<0xB1>(amax));  // partner lane (lane ^ 1) holds the other half
    uint32_t wh[4], wl[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float q0 = q8_code(lo[2 * i], amax), q1 = q8_code(hi[2 * i], amax);
      const float q2 = q8_code(lo[2 * i + 1], amax), q3 = q8_code(hi[2 * i + 1], amax);
      wh[i] = pack_e4m3x4(q_hi(q0), q_hi(q1), q_hi(q2), q_hi(q3));
      wl[i] = pack_e4m3x4(q_lo(q0), q_lo(q1), q_lo(q2), q_lo(q3));
    }
    uint4 *dst = reinterpret_cast<uint4 *>(xs + (size_t)b * MOE_XSW);
    dst[h] = make_uint4(wh[0], wh[1], wh[2], wh[3]);
    dst[2 + h] = make_uint4(wl[0], wl[1], wl[2], wl[3]);
    if (!h) dy[b] = (float)q8_scale_f16(amax);
  }
}

// stage_quant in two parts, for callers with nb <= nthr/2 (one block half
// per thread): the x loads go out first, ahead of the loads the caller
// issues next (a weight ring's first quads), and the code follows; the
// arithmetic is stage_quant's (same bits).
struct xq_half {
  float4 a0, a1, c0, c1;
};

__device__ __forceinline__ void stage_quant_issue(const float *__restrict__ x, int nb, int tid, xq_half &v) {
  const int b = tid >> 1 < nb ? tid >> 1 : nb - 1, h = tid & 1;  // every lane loads (a valid block)
  const float4 *xb = reinterpret_cast<const float4 *>(x + (size_t)b * MOE_QK + 8 * h);
  v.a0 = xb[0];
  v.a1 = xb[1];
  v.c0 = xb[4];
  v.c1 = xb[5];
}

__device__ __forceinline__ void stage_quant_finish(const xq_half &v, int nb, uint32_t *xs, float *dy, int tid) {
  const int b = tid >> 1, h = tid & 1;
  if (b < nb) {
    const float lo[8] = {v.a0.x, v.a0.y, v.a0.z, v.a0.w, v.a1.x, v.a1.y, v.a1.z, v.a1.w};
    const float hi[8] = {v.c0.x, v.c0.y, v.c0.z, v.c0.w, v.c1.x, v.c1.y, v.c1.z, v.c1.w};
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) amax = fmaxf(amax, fmaxf(fabsf(lo[i]), fabsf(hi[i])));
    amax = fmaxf(amax, dpp_f<0xB1>(amax));  // partner lane (lane ^ 1) holds the other half
    uint32_t wh[4], wl[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float q0 = q8_code(lo[2 * i], amax), q1 = q8_code(hi[2 * i], amax);
      const float q2 = q8_code(lo[2 * i + 1], amax), q3 = q8_code(hi[2 * i + 1], amax);
      wh[i] = pack_e4m3x4(q_hi(q0), q_hi(q1), q_hi(q2), q_hi(q3));
      wl[i] = pack_e4m3x4(q_lo(q0), q_lo(q1), q_lo(q2), q_lo(q3));
    }
    uint4 *dst = reinterpret_cast<uint4 *>(xs + (size_t)b * MOE_XSW);
    dst[h] = make_uint4(wh[0], wh[1], wh[2], wh[3]);
    dst[2 + h] = make_uint4(wl[0], wl[1], wl[2], wl[3]);
    if (!h) dy[b] = (float)q8_scale_f16(amax);
  }
}

// stage_copy<false> in two parts, for nb <= 16 * MOE_COPY_MAX blocks (at most
// MOE_COPY_MAX 16-byte pieces and two scales per lane): loads first, LDS
// stores after the caller's next loads are issued.
#define MOE_COPY_MAX 8
struct hcopy {
  u32x4_t v[MOE_COPY_MAX];  // a clang vector type: an array of HIP's uint4 is not kept in registers
  float d[2];
};

__device__ __forceinline__ void stage_copy_issue(const uint32_t *__restrict__ src, const float *__restrict__ sd, int nb,
                                                 int lane, hcopy &c) {
  // every lane loads (a valid piece); only the stores are guarded
#pragma unroll
  for (int j = 0; j < MOE_COPY_MAX; j++) {
    const int i = lane + 64 * j;
    c.v[j] = reinterpret_cast<const u32x4_t *>(src)[i < nb * 4 ? i : nb * 4 - 1];
  }
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int i = lane + 64 * j;
    c.d[j] = sd[i < nb ? i : nb - 1];
  }
}

__device__ __forceinline__ void stage_copy_finish(const hcopy &c, int nb, uint32_t *xs, float *dy, int lane) {
#pragma unroll
  for (int j = 0; j < MOE_COPY_MAX; j++) {
    const int i = lane + 64 * j;
    if (i < nb * 4) reinterpret_cast<u32x4_t *>(xs)[i] = c.v[j];
  }
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int i = lane + 64 * j;
    if (i < nb) dy[i] = c.d[j];
  }
}

// Copy nb staged blocks from global memory into LDS.  COHERENT: the source
// was written by another workgroup of the same launch, so the loads are
// agent-scope (they bypass the XCD's L2); otherwise plain loads.
template <bool COHERENT>
__device__ __forceinline__ void stage_copy(const uint32_t *__restrict__ src, const float *__restrict__ sd, int nb,
                                           uint32_t *xs, float *dy, int lane) {
  for (int i = lane; i < nb * 4; i += 64) {
    uint4 v;
    if (COHERENT) {
      const uint32_t *p = src + (size_t)i * 4;
      v.x = __hip_atomic_load(p + 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v.y = __hip_atomic_load(p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v.z = __hip_atomic_load(p + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v.w = __hip_atomic_load(p + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      v = reinterpret_cast<const uint4 *>(src)[i];
    }
    reinterpret_cast<uint4 *>(xs)[i] = v;
  }
  for (int i = lane; i < nb; i += 64)
    dy[i] = COHERENT ? __hip_atomic_load(sd + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : sd[i];
}

__device__ __forceinline__ void stage_zero(int nb, uint32_t *xs, float *dy, int lane) {
  for (int i = lane; i < nb * 4; i += 64) reinterpret_cast<uint4 *>(xs)[i] = make_uint4(0u, 0u, 0u, 0u);
  for (int i = lane; i < nb; i += 64) dy[i] = 0.0f;
}

// ---------------------------------------------------------------------------
// Per-lane B-operand configuration for one token pair.
struct bsel {
  int off_lo, step_lo;  // dword offset (in xs) of the B bytes 0-15 and its step per quad (0: a zero area)
  int off_hi, step_hi;  // same for bytes 16-31
  int dy_off;           // offset of this column's d (in dy) at quad 0; < 0: no token
  int sb;               // B scale: 2^4 (hi part) or 2^0 (lo part), E8M0
};

// xs_tok[t] / dy_tok[t]: staged rows of the two tokens (quad 0 of the
// lane's K range); tv[t]: token present.  zero_off: a 16-byte zero area.
__device__ __forceinline__ bsel make_bsel(int lane, int xs_tok0, int xs_tok1, int dy_tok0, int dy_tok1, bool tv0,
                                          bool tv1, int zero_off) {
  const int n = lane & 15, gb = lane >> 4;
  const int tp = n >> 3, part = (n >> 2) & 1, g = n & 3;
  const bool tv = tp ? tv1 : tv0;
  const bool holds = tv && ((gb >> 1) == (g & 1));
  const int off = (tp ? xs_tok1 : xs_tok0) + g * MOE_XSW + part * 8 + (gb & 1) * 4;
  bsel s;
  const bool upper = g >= 2;
  s.off_lo = holds && !upper ? off : zero_off;
  s.step_lo = holds && !upper ? 4 * MOE_XSW : 0;
  s.off_hi = holds && upper ? off : zero_off;
  s.step_hi = holds && upper ? 4 * MOE_XSW : 0;
  s.dy_off = tv ? (tp ? dy_tok1 : dy_tok0) + g : -1;
  s.sb = part ? 127 : 131;
  return s;
}

__device__ __forceinline__ i32x8_t load_b(const bsel &s, const uint32_t *xs, int ql) {
  const u32x4_t lo = *reinterpret_cast<const u32x4_t *>(xs + s.off_lo + ql * s.step_lo);
  const u32x4_t hi = *reinterpret_cast<const u32x4_t *>(xs + s.off_hi + ql * s.step_hi);
  i32x8_t b;
  b[0] = (int)lo.x; b[1] = (int)lo.y; b[2] = (int)lo.z; b[3] = (int)lo.w;
  b[4] = (int)hi.x; b[5] = (int)hi.y; b[6] = (int)hi.z; b[7] = (int)hi.w;
  return b;
}

__device__ __forceinline__ float load_dy(const bsel &s, const float *dy, int ql) {
  return s.dy_off >= 0 ? dy[s.dy_off + 4 * ql] : 0.0f;
}

__device__ __forceinline__ f32x4_t mfma_blk(const u32x4_t w, const i32x8_t b, int sa, int sb) {
  const i32x8_t a = {(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
  const f32x4_t z = {0.0f, 0.0f, 0.0f, 0.0f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 4, 0, 0, sa, 0, sb);
}

// Sum of the 8 columns of each token, left in the lanes of columns 0 and 8:
// ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7)).
__device__ __forceinline__ float col8_sum(float v) {
  v += dpp_f<0xB1>(v);  // lane ^ 1
  v += dpp_f<0x4E>(v);  // lane ^ 2
  v += __shfl_xor(v, 4);
  return v;
}

// ---------------------------------------------------------------------------
// A wave's K loop: NW weight streams ((matrix, tile) pairs), quads [q0, q1)
// with q0 % 4 == 0, against NP staged token pairs.  The loads run 3 quads
// ahead of the math (a ring of 4, so quad q sits in slot (q - q0) % 4, a
// compile-time index); the exponent dwords (4 quads each) are loaded once per
// group of 4 quads, one group ahead, and the MFMA's op_sel picks the quad's
// byte.  Past the end the ring re-reads the last quad (an L2 hit), so every
// wait covers only the quad about to be used.
template <int NW>
struct wquad {
  u32x4_t w[NW];
};

// One weight stream: a (matrix, tile) pair's records as a buffer resource
// (base in SGPRs, bounds-checked: a read past the tile returns 0).
struct wstream {
  __amdgpu_buffer_rsrc_t rec;
};

#define MOE_RSRC_FLAGS 0x00020000  // raw buffer, 32-bit dwords, no swizzle
#define MOE_CPOL_NT 2              // non-temporal loads: weights are read once per call

// tile: index of the 16-row tile over all experts of the tensor.
__device__ __forceinline__ wstream make_wstream(const uint8_t *w, size_t tile, int NG) {
  wstream s;
  s.rec = __builtin_amdgcn_make_buffer_rsrc((void *)(w + tile * NG * MOE_REC_BYTES), 0, NG * MOE_REC_BYTES,
                                            MOE_RSRC_FLAGS);
  return s;
}

template <int NW>
__device__ __forceinline__ void load_wquad(wquad<NW> &b, const wstream (&ws)[NW], int q, int lane) {
#pragma unroll
  for (int i = 0; i < NW; i++)
    b.w[i] = __builtin_amdgcn_raw_buffer_load_b128(ws[i].rec, lane * 16, (q >> 2) * MOE_REC_BYTES + (q & 3) * 1024,
                                                   MOE_CPOL_NT);
}

template <int NW>
__device__ __forceinline__ void load_scales(uint32_t (&sc)[NW], const wstream (&ws)[NW], int g, int lane) {
#pragma unroll
  for (int i = 0; i < NW; i++)
    sc[i] = __builtin_amdgcn_raw_buffer_load_b32(ws[i].rec, lane * 4, g * MOE_REC_BYTES + MOE_REC_SC, 0);
}

template <int SEL>
__device__ __forceinline__ f32x4_t mfma_blk(const u32x4_t w, const i32x8_t b, uint32_t sa, int sb) {
  const i32x8_t a = {(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
  const f32x4_t z = {0.0f, 0.0f, 0.0f, 0.0f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 4, 0, SEL, (int)sa, 0, sb);
}

// acc[p][i] += quad ql (local) of stream i against token pair p; SEL = q % 4.
template <int SEL, int NW, int NP>
__device__ __forceinline__ void quad_mma(const wquad<NW> &b, const uint32_t (&sc)[NW], int ql, const bsel (&bs)[NP],
                                         const uint32_t *xs, const float *dy, f32x4_t (&acc)[NP][NW]) {
#pragma unroll
  for (int p = 0; p < NP; p++) {
    const i32x8_t bv = load_b(bs[p], xs, ql);
    const float d = load_dy(bs[p], dy, ql);
#pragma unroll
    for (int i = 0; i < NW; i++) {
      const f32x4_t r = mfma_blk<SEL>(b.w[i], bv, sc[i], bs[p].sb);
      acc[p][i] = acc[p][i] + d * r;
    }
  }
  // pin this quad's math here: without it the compiler sinks the (pure)
  // MFMAs below the following quads' loads, keeping every quad's weights live
#pragma unroll
  for (int p = 0; p < NP; p++)
#pragma unroll
    for (int i = 0; i < NW; i++) asm volatile("" : "+v"(acc[p][i]));
}

// Load ring of D quads (D = 4 or 8): D - 1 quads in flight ahead of the one
// being multiplied, and the exponent dwords of the D/4 groups the current
// window of D quads spans.
template <int NW, int D>
struct kring {
  static_assert(D == 4 || D == 8, "ring of 4 or 8 quads");
  wquad<NW> q[D];
  uint32_t sc[D / 4][NW];
};

// Issue the first D - 1 quads and the first window's exponents (call before
// staging the activations, so the weight loads overlap it).
template <int NW, int D>
__device__ __forceinline__ void kloop_prime(kring<NW, D> &r, const wstream (&ws)[NW], int q0, int q1, int lane) {
  if (q1 <= q0) return;
  const int glast = (q1 - 1) >> 2;
#pragma unroll
  for (int d = 0; d < D - 1; d++) load_wquad<NW>(r.q[d], ws, q0 + d < q1 ? q0 + d : q1 - 1, lane);
#pragma unroll
  for (int g = 0; g < D / 4; g++) {
    const int gg = (q0 >> 2) + g;
    load_scales<NW>(r.sc[g], ws, gg < glast ? gg : glast, lane);
  }
}

// K loop over quads [q0, q1), q0 % 4 == 0.  The main loop covers whole
// windows of D quads with no exit inside, and each quad's loads and math are
// pinned in order (quad_mma's asm pins, the memory fence below), so the ring
// slots keep their registers across iterations: no copies at the back edge,
// which would wait for every load in flight.  The last partial window is a
// guarded tail.
template <int NW, int NP, int D>
__device__ __forceinline__ void kloop(kring<NW, D> &r, const wstream (&ws)[NW], int q0, int q1, const bsel (&bs)[NP],
                                      const uint32_t *xs, const float *dy, int lane, f32x4_t (&acc)[NP][NW]) {
#pragma unroll
  for (int p = 0; p < NP; p++)
#pragma unroll
    for (int i = 0; i < NW; i++) acc[p][i] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  if (q1 <= q0) return;
  const int glast = (q1 - 1) >> 2;
  uint32_t scn[D / 4][NW];
#define MOE_KSTEP(J)                                                              \
  {                                                                               \
    const int q = qb + (J), qn = q + D - 1;                                       \
    load_wquad<NW>(r.q[((J) + D - 1) % D], ws, qn < q1 ? qn : q1 - 1, lane);      \
    asm volatile("" ::: "memory");     /* no hoisting of later loads */           \
    __builtin_amdgcn_sched_barrier(0); /* keep the prefetch ahead */              \
    quad_mma<(J) & 3, NW, NP>(r.q[J], r.sc[(J) / 4], q - q0, bs, xs, dy, acc);     \
  }
  int qb = q0;
  for (; qb + D <= q1; qb += D) {
#pragma unroll
    for (int g = 0; g < D / 4; g++) {
      const int gn = (qb >> 2) + D / 4 + g;
      load_scales<NW>(scn[g], ws, gn < glast ? gn : glast, lane);
    }
    MOE_KSTEP(0) MOE_KSTEP(1) MOE_KSTEP(2) MOE_KSTEP(3)
    if constexpr (D == 8) { MOE_KSTEP(4) MOE_KSTEP(5) MOE_KSTEP(6) MOE_KSTEP(7) }
#pragma unroll
    for (int g = 0; g < D / 4; g++)
#pragma unroll
      for (int i = 0; i < NW; i++) r.sc[g][i] = scn[g][i];
  }
  // tail: fewer than D quads (their exponents are in r.sc)
  if (qb < q1) MOE_KSTEP(0)
  if (qb + 1 < q1) MOE_KSTEP(1)
  if (qb + 2 < q1) MOE_KSTEP(2)
  if constexpr (D == 8) {
    if (qb + 3 < q1) MOE_KSTEP(3)
    if (qb + 4 < q1) MOE_KSTEP(4)
    if (qb + 5 < q1) MOE_KSTEP(5)
    if (qb + 6 < q1) MOE_KSTEP(6)
  }
#undef MOE_KSTEP
}

// The same loop for a compile-time number of quads NQW, fully unrolled:
// straight-line code, so the compiler's wait counts are exact (in the
// rolled loop it has to be conservative at the back edge and waits for more
// of the ring than the quad about to be used).
template <int NW, int NP, int D, int NQW>
__device__ __forceinline__ void kloop_fixed(kring<NW, D> &r, const wstream (&ws)[NW], int q0, const bsel (&bs)[NP],
                                            const uint32_t *xs, const float *dy, int lane, f32x4_t (&acc)[NP][NW]) {
#pragma unroll
  for (int p = 0; p < NP; p++)
#pragma unroll
    for (int i = 0; i < NW; i++) acc[p][i] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int NG = (NQW + 3) / 4;  // exponent groups of the chunk
  uint32_t sc[NG][NW];
  // the primed window's groups are in r.sc
#pragma unroll
  for (int g = 0; g < D / 4 && g < NG; g++)
#pragma unroll
    for (int i = 0; i < NW; i++) sc[g][i] = r.sc[g][i];
#pragma unroll
  for (int ql = 0; ql < NQW; ql++) {
    const int J = ql % D;
    if (J == 0) {
      // exponents of the next window, one window ahead
#pragma unroll
      for (int g = 0; g < D / 4; g++) {
        const int gn = ql / 4 + D / 4 + g;
        if (gn < NG) load_scales<NW>(sc[gn], ws, (q0 >> 2) + gn, lane);
      }
    }
    const int qn = ql + D - 1 < NQW ? ql + D - 1 : NQW - 1;
    load_wquad<NW>(r.q[(J + D - 1) % D], ws, q0 + qn, lane);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    switch (ql & 3) {
      case 0: quad_mma<0, NW, NP>(r.q[J], sc[ql >> 2], ql, bs, xs, dy, acc); break;
      case 1: quad_mma<1, NW, NP>(r.q[J], sc[ql >> 2], ql, bs, xs, dy, acc); break;
      case 2: quad_mma<2, NW, NP>(r.q[J], sc[ql >> 2], ql, bs, xs, dy, acc); break;
      default: quad_mma<3, NW, NP>(r.q[J], sc[ql >> 2], ql, bs, xs, dy, acc); break;
    }
  }
}

// Dispatch on the wave's chunk length: the lengths the V3 and C1 shapes
// produce run the unrolled loop, anything else the rolled one.
template <int NW, int NP, int D>
__device__ __forceinline__ void kloop_any(kring<NW, D> &r, const wstream (&ws)[NW], int q0, int q1,
                                          const bsel (&bs)[NP], const uint32_t *xs, const float *dy, int lane,
                                          f32x4_t (&acc)[NP][NW]) {
  switch (q1 - q0) {
    case 56: kloop_fixed<NW, NP, D, 56>(r, ws, q0, bs, xs, dy, lane, acc); break;
    case 28: kloop_fixed<NW, NP, D, 28>(r, ws, q0, bs, xs, dy, lane, acc); break;
    case 16: kloop_fixed<NW, NP, D, 16>(r, ws, q0, bs, xs, dy, lane, acc); break;
    default: kloop<NW, NP, D>(r, ws, q0, q1, bs, xs, dy, lane, acc); break;
  }
}

// ---------------------------------------------------------------------------
// SwiGLU + Q8_0 of one 32-row h unit held by 32 consecutive lanes (lane j of
// the half = row j; `base` = the half's first lane), written in the staged
// format: 16 dwords at hs, scale at *hd.  All 64 lanes of the wave call it.
__device__ __forceinline__ float swiglu(float g, float up, float clamp) {
  if (clamp > 1e-6f) {  // deepseek4 order: up symmetric, gate one-sided, before SiLU
    up = fmaxf(fminf(up, clamp), -clamp);
    g = fminf(g, clamp);
  }
  return __fmul_rn(__fdiv_rn(g, 1.0f + expf(-g)), up);
}

// amax over each 32-lane half of the wave
__device__ __forceinline__ float half_amax(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_f<0x140>(v));  // row_mirror
  return fmaxf(v, __shfl_xor(v, 16));
}

// Returns the dword lane j (< 16 of its half) writes: dword j of the staged
// block (hi[8] then lo[8]); the codes come from lanes of the same half.
// Dword w = 4h + i of a part holds elements 8h+2i, 16+8h+2i, 8h+2i+1,
// 16+8h+2i+1 (bytes 0..3).
__device__ __forceinline__ uint32_t h_unit_dword(float q, int lane) {
  const int base = lane & 32, j = lane & 31;
  const int part = (j >> 3) & 1, w = j & 7, hh = w >> 2, i = w & 3;
  const int e0 = base + 8 * hh + 2 * i, e1 = base + 16 + 8 * hh + 2 * i;
  const int src[4] = {e0, e1, e0 + 1, e1 + 1};
  const float qh = q_hi(q), ql = q_lo(q);
  float v[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const float a = __shfl(qh, src[k]), b = __shfl(ql, src[k]);
    v[k] = part ? b : a;
  }
  return pack_e4m3x4(v[0], v[1], v[2], v[3]);
}

// Q8_0 of the 32-row h unit in each half of the wave (lane j of a half =
// row j), written to hs (16 dwords) / *hd when `store` (wave-uniform per
// half is not required: lanes store only their own dword).
__device__ __forceinline__ void h_unit_store(float h, bool store, uint32_t *hs, float *hd, int lane) {
  const float am = half_amax(fabsf(h));
  const float q = q8_code(h, am);
  const uint32_t dw = h_unit_dword(q, lane);
  const int j = lane & 31;
  if (store && j < 16) hs[j] = dw;
  if (store && j == 0) *hd = (float)q8_scale_f16(am);
}

// ---------------------------------------------------------------------------
// Which expert matrix and which h rows workgroup column y works on.
//   decode (T == 1): y = slot s; s < k -> expert ids[s], s == k -> shared
//     expert (matrix E); one token; h row s.
//   grouped: y < act[0] -> expert act[1+y], h rows offsets[e]..offsets[e+1]
//     (token of row r = perm[r] / k); last y when `shared` -> the shared
//     expert, rows P..P+T-1 (token of row P+i = i).
struct unit_t {
  int mat, row0, nrows;
  bool shared, valid;
};

__device__ __forceinline__ unit_t unit_of(int y, int ny, bool grouped, const int32_t *__restrict__ ids,
                                          const int32_t *__restrict__ offsets, const int32_t *__restrict__ act,
                                          int k, int E, int shared, int P, int T) {
  unit_t u;
  u.shared = shared && y == ny - 1;
  u.valid = true;
  if (!grouped) {
    const int e = u.shared ? E : ids[y];
    u.valid = u.shared || (unsigned)e < (unsigned)E;  // an out-of-range id reads nothing, yields 0
    u.mat = u.valid ? e : 0;
    u.row0 = y;
    u.nrows = 1;
    return u;
  }
  if (u.shared) {
    u.mat = E;
    u.row0 = P;
    u.nrows = T;
    return u;
  }
  if (y >= act[0]) {
    u.valid = false;
    u.mat = 0;
    u.row0 = 0;
    u.nrows = 0;
    return u;
  }
  u.mat = act[1 + y];
  u.row0 = offsets[u.mat];
  u.nrows = offsets[u.mat + 1] - u.row0;
  return u;
}

__device__ __forceinline__ int token_of(const unit_t &u, int hrow, const int32_t *__restrict__ perm, int k, int P) {
  return u.shared ? hrow - P : perm[hrow] / k;
}

// ---------------------------------------------------------------------------
// K split of the workgroup kernels: wave w of NW owns the 4-quad groups
// [g0, g1) of ceil(NQ/4), i.e. quads [4*g0, min(4*g1, NQ)).
__host__ __device__ __forceinline__ void wave_quads(int NQ, int NW, int w, int &q0, int &q1) {
  int g0, g1;
  split_range(moe_nq4(NQ), NW, w, g0, g1);
  q0 = 4 * g0;
  q1 = 4 * g1 < NQ ? 4 * g1 : NQ;
  if (q1 < q0) q1 = q0;
}
// Largest number of staged blocks any wave holds.
__host__ __device__ __forceinline__ int wave_blocks(int NQ, int NW) {
  return 16 * ((moe_nq4(NQ) + NW - 1) / NW);
}

// gate/up -> clamp -> SwiGLU -> Q8_0(h).  One workgroup of 4 waves per
// (32-row unit of F, expert column y): wave w streams tile w%2 of the unit
// (gate and up) over K-half w/2 (whole groups of 4 quads), against the
// activations of a batch of up to 2*NP tokens, which the two waves of each
// K-half quantize into a shared LDS region.  The K-halves meet in LDS in
// order; then one wave per 2 tokens applies clamp + SwiGLU and quantizes the
// unit's 32 h values (one Q8_0 block per token).  Decode (grouped == 0) is
// the same kernel with column y = slot and one token.
// grid (F/32, ny), 256 threads.  LDS: per K-half [zero 4][xs 2NP*NBW*16]
// [dy 2NP*NBW] dwords, reused for the partials [wave][2 streams][2NP][16].
// NP == 1 (decode and small batches) is held to 3 waves per SIMD, so a V3
// decode's 576 workgroups are resident at once (3 per CU).
#define MOE_GU_KS 2    // K parts of the gate/up workgroup (x 2 tiles = 4 waves)
#define MOE_GU_RING 4  // quads in a gate/up wave's load ring

template <int NP>
__global__ __launch_bounds__(64 * 2 * MOE_GU_KS) __attribute__((amdgpu_waves_per_eu(NP == 1 ? 3 : (NP == 2 ? 2 : 1))))
void k_gate_up(
    const uint8_t *__restrict__ w_g, const uint8_t *__restrict__ w_u, const float *__restrict__ x, int grouped,
    const int32_t *__restrict__ ids, const int32_t *__restrict__ offsets, const int32_t *__restrict__ perm,
    const int32_t *__restrict__ act, int k, int E, int shared, int T, int F, int H, float clamp,
    uint32_t *__restrict__ hs, float *__restrict__ hd, float *__restrict__ htap) {
  extern __shared__ __align__(16) uint32_t lds[];
  constexpr int NTOK = 2 * NP;
  const int NQ = H / 128, NQ4 = moe_nq4(NQ), U = F / MOE_UNIT, tiles = F / MOE_TILE;
  const int NBW = wave_blocks(NQ, MOE_GU_KS);
  const int part_words = 4 + NTOK * NBW * (MOE_XSW + 1);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ti = wave & 1, kp = wave >> 1;
  const int P = T * k;
  const unit_t un = unit_of(blockIdx.y, gridDim.y, grouped, ids, offsets, act, k, E, shared, P, T);
  if (grouped && !un.valid) return;
  const int u = blockIdx.x;
  int q0, q1;
  wave_quads(NQ, MOE_GU_KS, kp, q0, q1);
  const int nb = 4 * (q1 - q0);
  uint32_t *xs = lds + (size_t)kp * part_words;
  float *dy = reinterpret_cast<float *>(xs + 4 + (size_t)NTOK * NBW * MOE_XSW);
  float *red = reinterpret_cast<float *>(lds);  // [wave][2 streams][NTOK][16], after the K loops
  const size_t t0 = (size_t)un.mat * tiles + 2 * u + ti;
  const wstream ws[2] = {make_wstream(w_g, t0, NQ4), make_wstream(w_u, t0, NQ4)};
  for (int i0 = 0; i0 < un.nrows; i0 += NTOK) {
    const int nt = un.nrows - i0 < NTOK ? un.nrows - i0 : NTOK;
    kring<2, MOE_GU_RING> ring;
    kloop_prime<2, MOE_GU_RING>(ring, ws, q0, q1, lane);
    if (ti == 0 && lane < 4) xs[lane] = 0u;
    for (int t = 0; t < nt; t++) {
      const int tok = grouped ? token_of(un, un.row0 + i0 + t, perm, k, P) : 0;
      stage_quant(x + (size_t)tok * H + (size_t)q0 * 128, nb, xs + 4 + (size_t)t * NBW * MOE_XSW,
                  dy + (size_t)t * NBW, lane + 64 * ti, 128);
    }
    __syncthreads();
    bsel bs[NP];
#pragma unroll
    for (int p = 0; p < NP; p++)
      bs[p] = make_bsel(lane, 4 + 2 * p * NBW * MOE_XSW, 4 + (2 * p + 1) * NBW * MOE_XSW, 2 * p * NBW,
                        (2 * p + 1) * NBW, 2 * p < nt, 2 * p + 1 < nt, 0);
    f32x4_t acc[NP][2];
    kloop_any<2, NP, MOE_GU_RING>(ring, ws, q0, q1, bs, xs, dy, lane, acc);
    __syncthreads();  // every wave is done with the staged rows before red overwrites them
    const int gb = lane >> 4, tp = (lane >> 3) & 1;
#pragma unroll
    for (int p = 0; p < NP; p++)
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float v = col8_sum(acc[p][i][r]);
          if ((lane & 7) == 0) red[((wave * 2 + i) * NTOK + 2 * p + tp) * MOE_TILE + 4 * gb + r] = v;
        }
    __syncthreads();
    // epilogue: wave w takes token slots 2w, 2w+1 (lane half = token, lane j = row)
    for (int t = 2 * wave; t < nt; t += 4 * MOE_GU_KS) {
      const int ts = t + (lane >> 5);
      const int j = lane & 31, tj = j >> 4, rr = j & 15;
      const bool live = ts < nt;
      float gsum = 0.0f, usum = 0.0f;
      if (live)
        for (int q = 0; q < MOE_GU_KS; q++) {
          const int w = tj + 2 * q;  // the wave of tile tj, K part q
          gsum += red[((w * 2 + 0) * NTOK + ts) * MOE_TILE + rr];
          usum += red[((w * 2 + 1) * NTOK + ts) * MOE_TILE + rr];
        }
      const float h = live && un.valid ? swiglu(gsum, usum, clamp) : 0.0f;
      const int hrow = un.row0 + i0 + (live ? ts : 0);
      h_unit_store(h, live, hs + ((size_t)hrow * U + u) * MOE_XSW, hd + (size_t)hrow * U + u, lane);
      if (htap && live) htap[(size_t)hrow * F + (size_t)u * MOE_UNIT + j] = h;
    }
    __syncthreads();
  }
}

// Decode gate/up with equal work per CU.  The step's gate/up work is
// S*U*4 one-stream wave tasks (slot s, 32-row unit u, matrix gate/up, 16-row
// tile), each streaming its tile over all of K; MOE_BAL_WAVES of them per
// workgroup (for V3: 2304 tasks = 256 workgroups of 9 waves, one per CU, all
// waves of a CU the same age).  x is quantized once per workgroup into LDS.
// The 4 tasks of a unit may sit in different workgroups: each writes its 16
// row sums with coherent stores, then counts itself on the unit's ticket;
// the 4th applies clamp + SwiGLU, writes the unit's Q8_0 h block and resets
// the ticket (so every launch starts from zero, graph replays included).
// Nothing waits.  grid ceil(S*U*4 / MOE_BAL_WAVES), 64*MOE_BAL_WAVES threads.
#define MOE_BAL_WAVES 9

// Debug timeline (the TL instances of the decode kernels; production runs
// TL = false, the same code as without it): per wave, three stamps of the
// device's constant 100 MHz clock -- entry, end of its K loop, exit -- at
// record rec: tl[3 * rec + 0 .. 2].  Lane 0 stores them with vector stores.
__device__ __forceinline__ void tl_mark(unsigned long long *tl, int rec, unsigned long long t_in,
                                        unsigned long long t_loop) {
  const unsigned long long t_out = wall_clock64();
  if ((threadIdx.x & 63) == 0) {
    tl[3 * (size_t)rec + 0] = t_in;
    tl[3 * (size_t)rec + 1] = t_loop;
    tl[3 * (size_t)rec + 2] = t_out;
  }
}
#define MOE_BAL_RING 4  // quads in a wave's load ring (8 measured slower)

__global__ __launch_bounds__(64 * MOE_BAL_WAVES) void k_gate_up_bal(
    const uint8_t *__restrict__ w_g, const uint8_t *__restrict__ w_u, const float *__restrict__ x,
    const int32_t *__restrict__ ids, int k, int E, int S, int F, int H, float clamp, float *__restrict__ part,
    int *__restrict__ tick, uint32_t *__restrict__ hs, float *__restrict__ hd, float *__restrict__ htap) {
  extern __shared__ __align__(16) uint32_t lds[];
  const int NQ = H / 128, NQ4 = moe_nq4(NQ), KB = H / MOE_QK, U = F / MOE_UNIT, tiles = F / MOE_TILE;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int task = blockIdx.x * MOE_BAL_WAVES + wave, n_tasks = S * U * 4;
  const bool active = task < n_tasks;
  const int tt = active ? task : 0;
  const int ti = tt & 1, mi = (tt >> 1) & 1, unit = tt >> 2;  // unit = s*U + u
  const int s = unit / U, u = unit % U;
  uint32_t *xs = lds;
  float *dy = reinterpret_cast<float *>(lds + 4 + (size_t)KB * MOE_XSW);
  int e = s < k ? ids[s] : E;
  const bool valid = s >= k || (unsigned)e < (unsigned)E;  // an out-of-range id reads nothing, yields 0
  e = valid ? e : 0;
  const wstream ws[1] = {make_wstream(mi ? w_u : w_g, (size_t)e * tiles + 2 * u + ti, NQ4)};
  kring<1, MOE_BAL_RING> ring;
  if (active) kloop_prime<1, MOE_BAL_RING>(ring, ws, 0, NQ, lane);
  if (threadIdx.x < 4) xs[threadIdx.x] = 0u;
  stage_quant(x, KB, xs + 4, dy, threadIdx.x, 64 * MOE_BAL_WAVES);
  __syncthreads();
  if (!active) return;
  const bsel bs[1] = {make_bsel(lane, 4, 4, 0, 0, true, false, 0)};
  f32x4_t acc[1][1];
  kloop_any<1, 1, MOE_BAL_RING>(ring, ws, 0, NQ, bs, xs, dy, lane, acc);
  const int gb = lane >> 4, tp = (lane >> 3) & 1;
  float *pu = part + (size_t)unit * 4 * MOE_TILE;  // [matrix][tile][16 rows]
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const float v = col8_sum(acc[0][0][r]);
    if ((lane & 7) == 0 && tp == 0)
      __hip_atomic_store(reinterpret_cast<uint32_t *>(pu + (mi * 2 + ti) * MOE_TILE + 4 * gb + r),
                         __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);  // the row sums are complete before they are counted
  int old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(tick + unit, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __builtin_amdgcn_readfirstlane(old);
  if (old != 3) return;
  // the unit's 4th task: lanes 0-31 = rows of the unit (tile j/16)
  const int j = lane & 31, tj = j >> 4, rr = j & 15;
  const bool live = lane < 32;
  const float g = __builtin_bit_cast(float, __hip_atomic_load(reinterpret_cast<const uint32_t *>(pu + tj * MOE_TILE + rr),
                                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  const float up = __builtin_bit_cast(float, __hip_atomic_load(
                                                 reinterpret_cast<const uint32_t *>(pu + (2 + tj) * MOE_TILE + rr),
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  const float h = live && valid ? swiglu(g, up, clamp) : 0.0f;
  h_unit_store(h, live, hs + ((size_t)s * U + u) * MOE_XSW, hd + (size_t)s * U + u, lane);
  if (htap && live) htap[(size_t)s * F + (size_t)u * MOE_UNIT + j] = h;
  if (lane == 0) __hip_atomic_store(tick + unit, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

static inline size_t gate_up_bal_lds_bytes(int H) {
  return ((size_t)4 + (size_t)(H / MOE_QK) * (MOE_XSW + 1)) * 4;
}

// The same work split with most units meeting in LDS, for shapes where the
// S*U*4 tasks are exactly 9 per workgroup and G % 4 == 0 (V3: G = 256):
// waves 0-7 of workgroup b run the 8 tasks of units 2b and 2b+1, whose row
// sums meet in LDS (no ticket); wave 8 runs one task of the last G/4 units
// (task b % 4 of unit 2G + b/4), which meet through coherent stores and the
// ticket as in k_gate_up_bal.  Wave 8 streams with a ring of 8 quads (7 in
// flight instead of 3), so it takes a larger share of the CU's bandwidth,
// finishes first, and its ticket chain runs while the other waves stream.
// grid G, 64*MOE_BAL_WAVES threads, LDS gate_up_bal2_lds_bytes(H).
#define MOE_BAL2_RING 8

template <bool TL>
__global__ __launch_bounds__(64 * MOE_BAL_WAVES) void k_gate_up_bal2(
    const uint8_t *__restrict__ w_g, const uint8_t *__restrict__ w_u, const float *__restrict__ x,
    const int32_t *__restrict__ ids, int k, int E, int S, int F, int H, float clamp, float *__restrict__ part,
    int *__restrict__ tick, uint32_t *__restrict__ hs, float *__restrict__ hd, float *__restrict__ htap,
    unsigned long long *__restrict__ tl) {
  const unsigned long long t_in = TL ? wall_clock64() : 0ull;
  extern __shared__ __align__(16) uint32_t lds[];
  const int NQ = H / 128, NQ4 = moe_nq4(NQ), KB = H / MOE_QK, U = F / MOE_UNIT, tiles = F / MOE_TILE;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = gridDim.x;
  const bool local = wave < 8;
  const int unit = local ? 2 * blockIdx.x + (wave >> 2) : 2 * G + (blockIdx.x >> 2);  // unit = s*U + u
  const int tq = local ? (wave & 3) : (blockIdx.x & 3);                                  // matrix*2 + tile
  const int ti = tq & 1, mi = tq >> 1;
  const int s = unit / U, u = unit % U;
  uint32_t *xs = lds;
  float *dy = reinterpret_cast<float *>(lds + 4 + (size_t)KB * MOE_XSW);
  float *red = dy + KB;  // [8 waves][16 rows]
  int e = s < k ? ids[s] : E;
  const bool valid = s >= k || (unsigned)e < (unsigned)E;  // an out-of-range id reads nothing, yields 0
  e = valid ? e : 0;
  const wstream ws[1] = {make_wstream(mi ? w_u : w_g, (size_t)e * tiles + 2 * u + ti, NQ4)};
  kring<1, MOE_BAL_RING> ring;
  kring<1, MOE_BAL2_RING> ring8;
  // x's loads first, then the weight rings' first quads, then x's code
  const bool x1 = 2 * KB <= 64 * MOE_BAL_WAVES;
  xq_half xv;
  if (x1) stage_quant_issue(x, KB, threadIdx.x, xv);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  if (local) kloop_prime<1, MOE_BAL_RING>(ring, ws, 0, NQ, lane);
  else kloop_prime<1, MOE_BAL2_RING>(ring8, ws, 0, NQ, lane);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  if (threadIdx.x < 4) xs[threadIdx.x] = 0u;
  if (x1) stage_quant_finish(xv, KB, xs + 4, dy, threadIdx.x);
  else stage_quant(x, KB, xs + 4, dy, threadIdx.x, 64 * MOE_BAL_WAVES);
  __syncthreads();
  const bsel bs[1] = {make_bsel(lane, 4, 4, 0, 0, true, false, 0)};
  f32x4_t acc[1][1];
  if (local) kloop_any<1, 1, MOE_BAL_RING>(ring, ws, 0, NQ, bs, xs, dy, lane, acc);
  else kloop_any<1, 1, MOE_BAL2_RING>(ring8, ws, 0, NQ, bs, xs, dy, lane, acc);
  const unsigned long long t_loop = TL ? wall_clock64() : 0ull;
  const int gb = lane >> 4, tp = (lane >> 3) & 1;
  if (local) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float v = col8_sum(acc[0][0][r]);
      if ((lane & 7) == 0 && tp == 0) red[wave * MOE_TILE + 4 * gb + r] = v;
    }
  } else {
    float *pu = part + (size_t)unit * 4 * MOE_TILE;  // [matrix][tile][16 rows]
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float v = col8_sum(acc[0][0][r]);
      if ((lane & 7) == 0 && tp == 0)
        __hip_atomic_store(reinterpret_cast<uint32_t *>(pu + tq * MOE_TILE + 4 * gb + r), __builtin_bit_cast(uint32_t, v),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);  // the row sums are complete before they are counted
    int old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(tick + unit, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __builtin_amdgcn_readfirstlane(old);
    if (old == 3) {
      // the unit's 4th task: lanes 0-31 = rows of the unit (tile j/16)
      const int j = lane & 31, tj = j >> 4, rr = j & 15;
      const bool live = lane < 32;
      const float g = __builtin_bit_cast(float, __hip_atomic_load(reinterpret_cast<const uint32_t *>(pu + tj * MOE_TILE + rr),
                                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      const float up = __builtin_bit_cast(float, __hip_atomic_load(
                                                     reinterpret_cast<const uint32_t *>(pu + (2 + tj) * MOE_TILE + rr),
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      const float h = live && valid ? swiglu(g, up, clamp) : 0.0f;
      h_unit_store(h, live, hs + ((size_t)s * U + u) * MOE_XSW, hd + (size_t)s * U + u, lane);
      if (htap && live) htap[(size_t)s * F + (size_t)u * MOE_UNIT + j] = h;
      if (lane == 0) __hip_atomic_store(tick + unit, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  if (wave == 0) {
    // half hu of the wave: unit 2b + hu, lane j of the half = row j (tile j/16)
    const int hu = lane >> 5, j = lane & 31, tj = j >> 4, rr = j & 15;
    const int un = 2 * blockIdx.x + hu, s2 = un / U, u2 = un % U;
    const float g = red[(4 * hu + tj) * MOE_TILE + rr];
    const float up = red[(4 * hu + 2 + tj) * MOE_TILE + rr];
    int e2 = s2 < k ? ids[s2] : E;
    const bool v2 = s2 >= k || (unsigned)e2 < (unsigned)E;
    const float h = v2 ? swiglu(g, up, clamp) : 0.0f;
    h_unit_store(h, true, hs + ((size_t)s2 * U + u2) * MOE_XSW, hd + (size_t)s2 * U + u2, lane);
    if (htap) htap[(size_t)s2 * F + (size_t)u2 * MOE_UNIT + j] = h;
  }
  if (TL) tl_mark(tl, blockIdx.x * MOE_BAL_WAVES + wave, t_in, t_loop);
}

static inline size_t gate_up_bal2_lds_bytes(int H) {
  return gate_up_bal_lds_bytes(H) + (size_t)8 * MOE_TILE * 4;
}

// Decode down with the top-k combine (T == 1).  One workgroup per 16-row tile
// of H with one wave per slot (S <= 16): wave s streams the tile of its
// expert's down matrix over all of F against its slot's staged h and scales
// the rows by the router weight; the slot rows meet in LDS and are added in
// slot order, ((y0 + y1) + ...) + shared (the reference's trunk ADD chain,
// nano-glm/lib/models/glm_dsa/moe_block.h:120-131).  per_slot: out[s][H] =
// y_s (the MUL node of the reference's split) instead.
// grid H/16, 64*S threads.  LDS: per wave [zero 4][xs F/32*16][dy F/32]
// dwords, then ys[S][16].
template <bool TL>
__global__ __launch_bounds__(1024) void k_down_dec(
    const uint8_t *__restrict__ w_d, const uint32_t *__restrict__ hs, const float *__restrict__ hd,
    const int32_t *__restrict__ ids, const float *__restrict__ wts, int k, int E,
    int S, int F, int H, int per_slot, float *__restrict__ out, unsigned long long *__restrict__ tl) {
  const unsigned long long t_in = TL ? wall_clock64() : 0ull;
  extern __shared__ __align__(16) uint32_t lds[];
  const int NQ = F / 128, NQ4 = moe_nq4(NQ), tiles = H / MOE_TILE, U = F / MOE_UNIT;
  const int nb = F / MOE_QK, wave_words = 4 + nb * (MOE_XSW + 1);
  const int lane = threadIdx.x & 63, s = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = blockIdx.x;
  int e = s < k ? ids[s] : E;
  const bool valid = s >= k || (unsigned)e < (unsigned)E;  // an out-of-range id reads nothing, yields 0
  e = valid ? e : 0;
  const wstream ws[1] = {make_wstream(w_d, (size_t)e * tiles + tile, NQ4)};
  kring<1, 4> ring;
  uint32_t *xs = lds + (size_t)s * wave_words;
  float *dy = reinterpret_cast<float *>(xs + 4 + (size_t)nb * MOE_XSW);
  float *ys = reinterpret_cast<float *>(lds + (size_t)S * wave_words);  // [S][16]
  if (lane < 4) xs[lane] = 0u;
  if (nb <= 16 * MOE_COPY_MAX) {  // uniform: each path straight-line (a copy held across a branch goes to scratch)
    // the slot's h loads first, then the ring's first quads, then h into LDS
    hcopy hv;
    stage_copy_issue(hs + (size_t)s * U * MOE_XSW, hd + (size_t)s * U, nb, lane, hv);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    kloop_prime<1, 4>(ring, ws, 0, NQ, lane);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    stage_copy_finish(hv, nb, xs + 4, dy, lane);
  } else {
    kloop_prime<1, 4>(ring, ws, 0, NQ, lane);
    stage_copy<false>(hs + (size_t)s * U * MOE_XSW, hd + (size_t)s * U, nb, xs + 4, dy, lane);
  }
  __syncthreads();
  const bsel bs[1] = {make_bsel(lane, 4, 4, 0, 0, true, false, 0)};
  f32x4_t acc[1][1];
  kloop_any<1, 1, 4>(ring, ws, 0, NQ, bs, xs, dy, lane, acc);
  const unsigned long long t_loop = TL ? wall_clock64() : 0ull;
  const int gb = lane >> 4;
  const float wt = s < k ? wts[s] : 1.0f;
  float v[4];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    v[r] = col8_sum(acc[0][0][r]);
    if (s < k) v[r] = __fmul_rn(v[r], wt);
    if (!valid) v[r] = 0.0f;
  }
  const int row0 = tile * MOE_TILE + 4 * gb;
  if (per_slot) {
    if ((lane & 15) == 0)
#pragma unroll
      for (int r = 0; r < 4; r++) out[(size_t)s * H + row0 + r] = v[r];
    if (TL) tl_mark(tl, blockIdx.x * S + s, t_in, t_loop);
    return;
  }
  if ((lane & 15) == 0)
#pragma unroll
    for (int r = 0; r < 4; r++) ys[s * MOE_TILE + 4 * gb + r] = v[r];
  __syncthreads();
  if (threadIdx.x < MOE_TILE) {
    float o = ys[threadIdx.x];
    for (int q = 1; q < S; q++) o = __fadd_rn(o, ys[q * MOE_TILE + threadIdx.x]);
    out[(size_t)tile * MOE_TILE + threadIdx.x] = o;
  }
  if (TL) tl_mark(tl, blockIdx.x * S + s, t_in, t_loop);
}

// LDS bytes of the kernels.
static inline size_t gate_up_lds_bytes(int H, int NP) {
  const int NBW = wave_blocks(H / 128, MOE_GU_KS);
  const size_t stage = ((size_t)4 + (size_t)2 * NP * NBW * (MOE_XSW + 1)) * 4 * MOE_GU_KS;
  const size_t red = (size_t)4 * 2 * 2 * NP * MOE_TILE * 4;
  return stage > red ? stage : red;
}
static inline size_t down_dec_lds_bytes(int F, int S) {
  const int nb = F / MOE_QK;
  return ((size_t)S * (4 + (size_t)nb * (MOE_XSW + 1)) + (size_t)S * MOE_TILE) * 4;
}

// ---------------------------------------------------------------------------
// test hook: the product quantizer (stage_quant) over n_blocks blocks of a
// flat f32 array, 32 blocks per single-wave workgroup, decoded back to
// ggml's block_q8_0 bytes (q = 16*hi + lo).
__global__ __launch_bounds__(64) void k_debug_quantize(const float *__restrict__ x, int n_blocks,
                                                       int8_t *__restrict__ qs, uint16_t *__restrict__ d) {
  __shared__ __align__(16) uint32_t xs[32 * MOE_XSW];
  __shared__ float dy[32];
  const int lane = threadIdx.x;
  const int b0 = blockIdx.x * 32;
  const int nb = n_blocks - b0 < 32 ? n_blocks - b0 : 32;
  stage_quant(x + (size_t)b0 * MOE_QK, nb, xs, dy, lane, 64);
  __syncthreads();
  for (int i = lane; i < nb * 32; i += 64) {
    const int b = i >> 5, e = i & 31;  // MFMA K offset e of block b
    const uint32_t wh = xs[b * MOE_XSW + (e >> 2)], wl = xs[b * MOE_XSW + 8 + (e >> 2)];
    const int sel = e & 3;
    const float hv = __builtin_amdgcn_cvt_f32_fp8((int)(wh >> (8 * sel)), 0);
    const float lv = __builtin_amdgcn_cvt_f32_fp8((int)(wl >> (8 * sel)), 0);
    const int elem = (e >> 1) + 16 * (e & 1);
    qs[(size_t)(b0 + b) * MOE_QK + elem] = (int8_t)(int)(16.0f * hv + lv);
  }
  if (lane < nb) d[(size_t)b0 + lane] = __builtin_bit_cast(uint16_t, (_Float16)dy[lane]);
}
