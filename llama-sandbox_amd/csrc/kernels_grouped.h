// kernels_grouped.h -- the grouped expert kernels for T > 1 (small-batch
// decode and prefill): gate/up + SwiGLU + Q8_0(h), and down x router weight,
// on the scaled MFMA of kernels_rows.h.
//
// Work items.  k_group (kernels_group.h) cuts every expert's grouped rows
// into items of at most BT rows (BT = 2 * NPMAX tokens) and appends the
// shared expert's T rows the same way; one workgroup column of the grid
// takes one item.  A hot expert therefore spreads over many workgroups
// instead of running its tokens through one workgroup in turn, and the
// items of one expert are adjacent in the grid, so their re-reads of the
// same weight tiles are issued at about the same time (and by the same XCD:
// a row of the grid is a multiple of 8 workgroups wide) and hit L2.
//
// B operand straight from global memory.  The activations (x: quantized
// once per call by k_group's extra workgroups; h: written by the gate/up
// kernel) are in the staged format of kernels_rows.h (per block hi[8] lo[8]
// dwords of e4m3 digits, and d as f32), and every lane loads its own part of
// the block-diagonal B operand and its column's d with buffer loads: 16
// bytes and 4 bytes per (quad, token pair).  A lane that holds no data (the
// block of its column lives in another lane group, or the token is absent)
// gets an out-of-range offset and reads 0.  No LDS staging, so the token
// batch per workgroup is not bounded by LDS, and no barrier precedes the K
// loop.  The loads run in two rings: B data 2 quads ahead of the MFMAs and
// weights 3 quads ahead, B issued first in each step, so that waiting for a
// quad's B data never waits for younger weight loads.
#pragma once

#include "kernels_rows.h"

#define MOE_OOB 0x80000000u  // a buffer offset past any staged buffer: the load returns 0

// Item record written by k_group: {matrix, first grouped row, rows, shared}.
// items[0] = number of items; record i is int4 number 1 + i.
__device__ __forceinline__ int4 item_of(const int32_t *__restrict__ items, int i) {
  return reinterpret_cast<const int4 *>(items)[1 + i];
}

// Buffer resources over the staged rows (digits) and their block scales.
struct gsrc {
  __amdgpu_buffer_rsrc_t x, d;
};

__device__ __forceinline__ gsrc make_gsrc(const uint32_t *xq, const float *xd, int rows, int KB) {
  gsrc s;
  s.x = __builtin_amdgcn_make_buffer_rsrc((void *)xq, 0, rows * KB * MOE_XSW * 4, MOE_RSRC_FLAGS);
  s.d = __builtin_amdgcn_make_buffer_rsrc((void *)xd, 0, rows * KB * 4, MOE_RSRC_FLAGS);
  return s;
}

// Per-lane B source for one token pair: byte offsets, at quad 0, of the 16
// digit bytes this lane feeds to the MFMA and of its column's d.  Lane
// n + 16*gb is column n = 8*tp + 4*part + g (token tp of the pair, part 0 =
// hi digits, 1 = lo digits, block g of the quad); block g's K offsets
// [16*gb', 16*gb' + 16) sit in lane group gb' = 2*(g%2) + {0,1} at bytes
// 16*(g/2) of the operand.  row: the staged row of this lane's token, < 0 if
// absent.
struct gsel {
  uint32_t voff, doff;
};

__device__ __forceinline__ gsel make_gsel(int lane, int row, int KB) {
  const int n = lane & 15, gb = lane >> 4;
  const int part = (n >> 2) & 1, g = n & 3;
  const bool holds = row >= 0 && ((gb >> 1) == (g & 1));
  gsel s;
  s.voff = holds ? (uint32_t)((row * KB + g) * (MOE_XSW * 4) + part * 32 + (gb & 1) * 16) : MOE_OOB;
  s.doff = row >= 0 ? (uint32_t)((row * KB + g) * 4) : MOE_OOB;
  return s;
}

template <int NP>
struct bquad {
  u32x4_t v[NP];
  float d[NP];
};

// quad q (absolute) of every pair: 4 blocks = 256 digit bytes and 16 bytes of d per row
template <int NP>
__device__ __forceinline__ void load_bquad(bquad<NP> &b, const gsrc &src, const gsel (&gs)[NP], int q) {
#pragma unroll
  for (int p = 0; p < NP; p++) {
    b.v[p] = __builtin_amdgcn_raw_buffer_load_b128(src.x, gs[p].voff, q * 4 * MOE_XSW * 4, 0);
    b.d[p] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(src.d, gs[p].doff, q * 16, 0));
  }
}

// Weight quad with a cache policy (0: normal, so that the items of a hot
// expert re-read its tiles from L2).
template <int NW, int CPOL>
__device__ __forceinline__ void load_wquad_p(wquad<NW> &b, const wstream (&ws)[NW], int q, int lane) {
#pragma unroll
  for (int i = 0; i < NW; i++)
    b.w[i] = __builtin_amdgcn_raw_buffer_load_b128(ws[i].rec, lane * 16, (q >> 2) * MOE_REC_BYTES + (q & 3) * 1024,
                                                   CPOL);
}

// acc[p][i] += quad (SEL = q % 4) of stream i against pair p.  upper: this
// lane's 16 bytes are operand bytes 16-31; sb: its B scale (2^4 hi, 2^0 lo).
template <int SEL, int NW, int NP>
__device__ __forceinline__ void gquad_mma(const wquad<NW> &w, const uint32_t (&sc)[NW], const bquad<NP> &b,
                                          bool upper, int sb, f32x4_t (&acc)[NP][NW]) {
#pragma unroll
  for (int p = 0; p < NP; p++) {
    const u32x4_t v = b.v[p];
    i32x8_t bv;
    bv[0] = upper ? 0 : (int)v.x; bv[1] = upper ? 0 : (int)v.y; bv[2] = upper ? 0 : (int)v.z; bv[3] = upper ? 0 : (int)v.w;
    bv[4] = upper ? (int)v.x : 0; bv[5] = upper ? (int)v.y : 0; bv[6] = upper ? (int)v.z : 0; bv[7] = upper ? (int)v.w : 0;
#pragma unroll
    for (int i = 0; i < NW; i++) {
      const f32x4_t r = mfma_blk<SEL>(w.w[i], bv, sc[i], sb);
      acc[p][i] = acc[p][i] + b.d[p] * r;
    }
  }
#pragma unroll
  for (int p = 0; p < NP; p++)
#pragma unroll
    for (int i = 0; i < NW; i++) asm volatile("" : "+v"(acc[p][i]));
}

__device__ __forceinline__ bool lane_upper(int lane) { return (lane & 2) != 0; }     // block g >= 2
__device__ __forceinline__ int lane_bscale(int lane) { return (lane & 4) ? 127 : 131; }  // lo : hi digits

#define MOE_GSTEP(QL, SLOT, QB, QW, WANT_B, WANT_W)                                     \
  {                                                                                     \
    if (WANT_B) load_bquad<NP>(b[((SLOT) + 2) & 3], src, gs, (QB));                     \
    if (WANT_W) load_wquad_p<NW, CPOL>(w[((SLOT) + 3) & 3], ws, (QW), lane);            \
    asm volatile("" ::: "memory");                                                      \
    __builtin_amdgcn_sched_barrier(0);                                                  \
    switch ((QL) & 3) {                                                                 \
      case 0: gquad_mma<0, NW, NP>(w[SLOT], scs, b[SLOT], upper, sb, acc); break;       \
      case 1: gquad_mma<1, NW, NP>(w[SLOT], scs, b[SLOT], upper, sb, acc); break;       \
      case 2: gquad_mma<2, NW, NP>(w[SLOT], scs, b[SLOT], upper, sb, acc); break;       \
      default: gquad_mma<3, NW, NP>(w[SLOT], scs, b[SLOT], upper, sb, acc); break;      \
    }                                                                                   \
  }

// K loop over NQW quads from q0 (q0 % 4 == 0), fully unrolled: loads past
// the end are simply not issued and every wait is exact.
template <int NW, int NP, int CPOL, int NQW>
__device__ __forceinline__ void gloop_fixed(const wstream (&ws)[NW], int q0, const gsrc &src, const gsel (&gs)[NP],
                                            int lane, f32x4_t (&acc)[NP][NW]) {
#pragma unroll
  for (int p = 0; p < NP; p++)
#pragma unroll
    for (int i = 0; i < NW; i++) acc[p][i] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int NG = (NQW + 3) / 4;
  const bool upper = lane_upper(lane);
  const int sb = lane_bscale(lane);
  wquad<NW> w[4];
  bquad<NP> b[4];
  uint32_t sc[NG][NW];
  load_scales<NW>(sc[0], ws, q0 >> 2, lane);
  load_bquad<NP>(b[0], src, gs, q0);
  load_wquad_p<NW, CPOL>(w[0], ws, q0, lane);
  if (NQW > 1) {
    load_bquad<NP>(b[1], src, gs, q0 + 1);
    load_wquad_p<NW, CPOL>(w[1], ws, q0 + 1, lane);
  }
  if (NQW > 2) load_wquad_p<NW, CPOL>(w[2], ws, q0 + 2, lane);
#pragma unroll
  for (int ql = 0; ql < NQW; ql++) {
    if ((ql & 3) == 0 && (ql >> 2) + 1 < NG) load_scales<NW>(sc[(ql >> 2) + 1], ws, (q0 >> 2) + (ql >> 2) + 1, lane);
    const uint32_t(&scs)[NW] = sc[ql >> 2];
    MOE_GSTEP(ql, ql & 3, q0 + ql + 2, q0 + ql + 3, ql + 2 < NQW, ql + 3 < NQW)
  }
}

// The same for a run-time number of quads [q0, q1): windows of 4 quads with
// compile-time ring slots; loads past the end re-read the last quad, so the
// waits are uniform; the last partial window is a guarded tail.
template <int NW, int NP, int CPOL>
__device__ __forceinline__ void gloop_rolled(const wstream (&ws)[NW], int q0, int q1, const gsrc &src,
                                             const gsel (&gs)[NP], int lane, f32x4_t (&acc)[NP][NW]) {
#pragma unroll
  for (int p = 0; p < NP; p++)
#pragma unroll
    for (int i = 0; i < NW; i++) acc[p][i] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  if (q1 <= q0) return;
  const bool upper = lane_upper(lane);
  const int sb = lane_bscale(lane);
  const int last = q1 - 1, glast = last >> 2;
  wquad<NW> w[4];
  bquad<NP> b[4];
  uint32_t scs[NW], scn[NW];
  load_scales<NW>(scs, ws, q0 >> 2, lane);
  load_bquad<NP>(b[0], src, gs, q0);
  load_wquad_p<NW, CPOL>(w[0], ws, q0, lane);
  load_bquad<NP>(b[1], src, gs, q0 + 1 < q1 ? q0 + 1 : last);
  load_wquad_p<NW, CPOL>(w[1], ws, q0 + 1 < q1 ? q0 + 1 : last, lane);
  load_wquad_p<NW, CPOL>(w[2], ws, q0 + 2 < q1 ? q0 + 2 : last, lane);
  int qb = q0;
  for (; qb + 4 <= q1; qb += 4) {
    const int gn = (qb >> 2) + 1;
    load_scales<NW>(scn, ws, gn < glast ? gn : glast, lane);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int qB = qb + j + 2 < q1 ? qb + j + 2 : last, qW = qb + j + 3 < q1 ? qb + j + 3 : last;
      MOE_GSTEP(j, j, qB, qW, true, true)
    }
#pragma unroll
    for (int i = 0; i < NW; i++) scs[i] = scn[i];
  }
#pragma unroll
  for (int j = 0; j < 3; j++) {
    if (qb + j < q1) {
      const int qB = qb + j + 2 < q1 ? qb + j + 2 : last, qW = qb + j + 3 < q1 ? qb + j + 3 : last;
      MOE_GSTEP(j, j, qB, qW, true, true)
    }
  }
}
#undef MOE_GSTEP

// Unrolled loops for the chunk lengths of the V3 and C1 shapes, rolled otherwise.
template <int NW, int NP, int CPOL>
__device__ __forceinline__ void gloop_any(const wstream (&ws)[NW], int q0, int q1, const gsrc &src,
                                          const gsel (&gs)[NP], int lane, f32x4_t (&acc)[NP][NW]) {
  switch (q1 - q0) {
    case 28: gloop_fixed<NW, NP, CPOL, 28>(ws, q0, src, gs, lane, acc); break;
    case 16: gloop_fixed<NW, NP, CPOL, 16>(ws, q0, src, gs, lane, acc); break;
    case 8: gloop_fixed<NW, NP, CPOL, 8>(ws, q0, src, gs, lane, acc); break;
    case 6: gloop_fixed<NW, NP, CPOL, 6>(ws, q0, src, gs, lane, acc); break;
    default: gloop_rolled<NW, NP, CPOL>(ws, q0, q1, src, gs, lane, acc); break;
  }
}

// ---------------------------------------------------------------------------
// Grouped gate/up: one workgroup of 4 waves per (32-row unit u of F, item):
// wave w streams tile w%2 of the unit (gate and up) over K-half w/2 against
// the item's tokens (x rows perm[r] / k, or r - P for the shared expert);
// the K-halves meet in LDS and one wave per 2 tokens applies clamp + SwiGLU
// and writes the unit's Q8_0 h block of each token (row r of hs / hd).
// grid (F/32, item capacity), 256 threads.
template <int NP>
__device__ __forceinline__ void gu_item(const uint8_t *__restrict__ w_g, const uint8_t *__restrict__ w_u,
                                        const gsrc &src, const int4 &it, const int32_t *__restrict__ perm, int k,
                                        int T, int F, int H, float clamp, uint32_t *__restrict__ hs,
                                        float *__restrict__ hd, float *__restrict__ htap, float *red) {
  constexpr int NTOK = 2 * NP;
  const int NQ = H / 128, NQ4 = moe_nq4(NQ), U = F / MOE_UNIT, tiles = F / MOE_TILE, KB = H / MOE_QK;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ti = wave & 1, kp = wave >> 1, P = T * k, u = blockIdx.x;
  const int row0 = it.y, nt = it.z;
  const bool shared = it.w != 0;
  int q0, q1;
  wave_quads(NQ, 2, kp, q0, q1);
  const size_t t0 = (size_t)it.x * tiles + 2 * u + ti;
  const wstream ws[2] = {make_wstream(w_g, t0, NQ4), make_wstream(w_u, t0, NQ4)};
  gsel gs[NP];
#pragma unroll
  for (int p = 0; p < NP; p++) {
    const int i = 2 * p + ((lane >> 3) & 1);
    int xr = -1;
    if (i < nt) xr = shared ? row0 + i - P : perm[row0 + i] / k;
    gs[p] = make_gsel(lane, xr, KB);
  }
  f32x4_t acc[NP][2];
  gloop_any<2, NP, 0>(ws, q0, q1, src, gs, lane, acc);
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
  // wave w takes token slots 2w, 2w+1 (lane half = token, lane j = row of the unit)
  for (int t = 2 * wave; t < nt; t += 8) {
    const int ts = t + (lane >> 5);
    const int j = lane & 31, tj = j >> 4, rr = j & 15;
    const bool live = ts < nt;
    float gsum = 0.0f, usum = 0.0f;
    if (live)
      for (int q = 0; q < 2; q++) {
        const int w = tj + 2 * q;  // the wave of tile tj, K half q
        gsum += red[((w * 2 + 0) * NTOK + ts) * MOE_TILE + rr];
        usum += red[((w * 2 + 1) * NTOK + ts) * MOE_TILE + rr];
      }
    const float h = live ? swiglu(gsum, usum, clamp) : 0.0f;
    const int hrow = row0 + (live ? ts : 0);
    h_unit_store(h, live, hs + ((size_t)hrow * U + u) * MOE_XSW, hd + (size_t)hrow * U + u, lane);
    if (htap && live) htap[(size_t)hrow * F + (size_t)u * MOE_UNIT + j] = h;
  }
}

// NPMAX: token pairs of the largest item (BT = 2 * NPMAX); each item runs
// the smallest instance that holds its rows.
template <int NPMAX>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NPMAX <= 2 ? 3 : (NPMAX == 4 ? 2 : 1))))
void k_gate_up_g(const uint8_t *__restrict__ w_g, const uint8_t *__restrict__ w_u, const uint32_t *__restrict__ xq,
                 const float *__restrict__ xd, const int32_t *__restrict__ items, const int32_t *__restrict__ perm,
                 int k, int T, int F, int H, float clamp, uint32_t *__restrict__ hs, float *__restrict__ hd,
                 float *__restrict__ htap) {
  __shared__ __align__(16) float red[4 * 2 * 2 * NPMAX * MOE_TILE];
  if ((int)blockIdx.y >= items[0]) return;
  const int4 it = item_of(items, blockIdx.y);
  const gsrc src = make_gsrc(xq, xd, T, H / MOE_QK);
  const int nt = it.z;
  if (NPMAX >= 8 && nt > 8) gu_item<(NPMAX >= 8 ? 8 : 1)>(w_g, w_u, src, it, perm, k, T, F, H, clamp, hs, hd, htap, red);
  else if (NPMAX >= 4 && nt > 4) gu_item<(NPMAX >= 4 ? 4 : 1)>(w_g, w_u, src, it, perm, k, T, F, H, clamp, hs, hd, htap, red);
  else if (NPMAX >= 2 && nt > 2) gu_item<(NPMAX >= 2 ? 2 : 1)>(w_g, w_u, src, it, perm, k, T, F, H, clamp, hs, hd, htap, red);
  else gu_item<1>(w_g, w_u, src, it, perm, k, T, F, H, clamp, hs, hd, htap, red);
}

// ---------------------------------------------------------------------------
// Grouped down x router weight: each wave streams 2 tiles (32 rows of H) of
// the item's down matrix over all of F against the item's h rows and writes
// y[r][H] = (row . h[r]) * wts[perm[r]] (routed) or * 1 (shared).  No LDS,
// no barrier.  grid (ceil(H/32 / MOE_DG_WAVES), item capacity).
#define MOE_DG_WAVES 4

template <int NP>
__device__ __forceinline__ void dn_item(const uint8_t *__restrict__ w_d, const gsrc &src, const int4 &it,
                                        const int32_t *__restrict__ perm, const float *__restrict__ wts, int F,
                                        int H, float *__restrict__ y) {
  const int NQ = F / 128, NQ4 = moe_nq4(NQ), tiles = H / MOE_TILE, KB = F / MOE_QK;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int pair = blockIdx.x * MOE_DG_WAVES + wave;  // tiles 2*pair, 2*pair + 1
  if (2 * pair >= tiles) return;
  const int row0 = it.y, nt = it.z;
  const bool shared = it.w != 0;
  const size_t t0 = (size_t)it.x * tiles + 2 * pair;
  const wstream ws[2] = {make_wstream(w_d, t0, NQ4), make_wstream(w_d, t0 + 1, NQ4)};
  gsel gs[NP];
#pragma unroll
  for (int p = 0; p < NP; p++) {
    const int i = 2 * p + ((lane >> 3) & 1);
    gs[p] = make_gsel(lane, i < nt ? row0 + i : -1, KB);
  }
  f32x4_t acc[NP][2];
  gloop_any<2, NP, 0>(ws, 0, NQ, src, gs, lane, acc);
  const int gb = lane >> 4, tp = (lane >> 3) & 1;
#pragma unroll
  for (int p = 0; p < NP; p++) {
    const int t = 2 * p + tp;
    const bool live = t < nt;
    const int r = row0 + (live ? t : 0);
    const float wt = (live && !shared) ? wts[perm[r]] : 1.0f;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        float v = col8_sum(acc[p][i][q]);
        if (!shared) v = __fmul_rn(v, wt);
        if ((lane & 7) == 0 && live) y[(size_t)r * H + (size_t)(2 * pair + i) * MOE_TILE + 4 * gb + q] = v;
      }
  }
}

template <int NPMAX>
__global__ __launch_bounds__(64 * MOE_DG_WAVES) __attribute__((amdgpu_waves_per_eu(NPMAX <= 2 ? 3 : (NPMAX == 4 ? 2 : 1))))
void k_down_g(const uint8_t *__restrict__ w_d, const uint32_t *__restrict__ hs, const float *__restrict__ hd,
              int n_rows, const int32_t *__restrict__ items, const int32_t *__restrict__ perm,
              const float *__restrict__ wts, int F, int H, float *__restrict__ y) {
  if ((int)blockIdx.y >= items[0]) return;
  const int4 it = item_of(items, blockIdx.y);
  const gsrc src = make_gsrc(hs, hd, n_rows, F / MOE_QK);
  const int nt = it.z;
  if (NPMAX >= 8 && nt > 8) dn_item<(NPMAX >= 8 ? 8 : 1)>(w_d, src, it, perm, wts, F, H, y);
  else if (NPMAX >= 4 && nt > 4) dn_item<(NPMAX >= 4 ? 4 : 1)>(w_d, src, it, perm, wts, F, H, y);
  else if (NPMAX >= 2 && nt > 2) dn_item<(NPMAX >= 2 ? 2 : 1)>(w_d, src, it, perm, wts, F, H, y);
  else dn_item<1>(w_d, src, it, perm, wts, F, H, y);
}
