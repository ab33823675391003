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
// a row of the grid is a multiple of 8 workgroups wide) and hit L2.  Only
// those items (MOE_ITEM_SPLIT) load their weights with the default cache
// policy; an expert of one item is read once per call, so its tiles stream
// non-temporal, as in decode, and leave the caches to data read again.
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

// Item record written by k_group: {matrix, first grouped row, rows, flags
// (MOE_ITEM_SHARED, MOE_ITEM_SPLIT)}.  items[0] = number of items; record i
// is int4 number 1 + i.
__device__ __forceinline__ int4 item_of(const int32_t *__restrict__ items, int i) {
  return reinterpret_cast<const int4 *>(items)[1 + i];
}

// LDS writes of this wave done, then the workgroup barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding: vmcnt
// in bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
__host__ __device__ constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x70 | 0xF00; }

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
  const bool shared = (it.w & MOE_ITEM_SHARED) != 0;
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
  // the pairs path runs for T <= 4: an expert has at most T rows, so one item
  // and every weight tile is read once per call (non-temporal, as in decode)
  gloop_any<2, NP, MOE_CPOL_NT>(ws, q0, q1, src, gs, lane, acc);
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
  const bool shared = (it.w & MOE_ITEM_SHARED) != 0;
  const size_t t0 = (size_t)it.x * tiles + 2 * pair;
  const wstream ws[2] = {make_wstream(w_d, t0, NQ4), make_wstream(w_d, t0 + 1, NQ4)};
  gsel gs[NP];
#pragma unroll
  for (int p = 0; p < NP; p++) {
    const int i = 2 * p + ((lane >> 3) & 1);
    gs[p] = make_gsel(lane, i < nt ? row0 + i : -1, KB);
  }
  f32x4_t acc[NP][2];
  gloop_any<2, NP, MOE_CPOL_NT>(ws, 0, NQ, src, gs, lane, acc);  // one item per expert (T <= 4): read once
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

// ---------------------------------------------------------------------------
// Down x router weight with the slot combine, for calls of a few tokens (the
// pairs path, T <= MOE_DF_TMAX): one workgroup of MOE_DF_WAVES waves per
// 32 rows of H (two 16-row tiles).  Wave w takes items w, w + MOE_DF_WAVES,
// ... (one expert's two tiles over all of F against the item's h rows, B
// read from the grouped h rows as in k_down_g); each (token, slot) row goes
// to LDS and the rows of a token are added in slot order, ((y0 + y1) + ...)
// + shared, straight into out -- k_combine's sum, with no y buffer and no
// launch of its own.  A pair whose expert id is out of range belongs to no
// item: its row stays 0.  per_slot: out [T][k][H] = the weighted rows.
// grid H/32, 64*MOE_DF_WAVES threads.
#define MOE_DF_WAVES 16
#define MOE_DF_TMAX 4
#define MOE_DF_SMAX 17  // slots per token: k <= 16, plus the shared expert
#define MOE_DF_ROWS (2 * MOE_TILE)

template <int NP>
__device__ __forceinline__ void df_item(const uint8_t *__restrict__ w_d, const gsrc &src, const int4 &it,
                                        const int32_t *__restrict__ perm, const float *__restrict__ wts, int k,
                                        int P, int F, int H, int pair, float *ys) {
  const int NQ = F / 128, NQ4 = moe_nq4(NQ), tiles = H / MOE_TILE, KB = F / MOE_QK;
  const int lane = threadIdx.x & 63;
  const int row0 = it.y, nt = it.z;
  const bool shared = (it.w & MOE_ITEM_SHARED) != 0;
  const size_t t0 = (size_t)it.x * tiles + 2 * pair;
  const wstream ws[2] = {make_wstream(w_d, t0, NQ4), make_wstream(w_d, t0 + 1, NQ4)};
  gsel gs[NP];
#pragma unroll
  for (int p = 0; p < NP; p++) {
    const int i = 2 * p + ((lane >> 3) & 1);
    gs[p] = make_gsel(lane, i < nt ? row0 + i : -1, KB);
  }
  f32x4_t acc[NP][2];
  gloop_any<2, NP, MOE_CPOL_NT>(ws, 0, NQ, src, gs, lane, acc);  // one item per expert (T <= 4): read once
  const int gb = lane >> 4, tp = (lane >> 3) & 1;
#pragma unroll
  for (int p = 0; p < NP; p++) {
    const int t = 2 * p + tp;
    const bool live = t < nt;
    const int r = row0 + (live ? t : 0);
    const int pr = live && !shared ? perm[r] : 0;
    const float wt = (live && !shared) ? wts[pr] : 1.0f;
    const int tok = shared ? r - P : pr / k, slot = shared ? k : pr % k;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        float v = col8_sum(acc[p][i][q]);
        if (!shared) v = __fmul_rn(v, wt);
        if ((lane & 7) == 0 && live) ys[(tok * MOE_DF_SMAX + slot) * MOE_DF_ROWS + i * MOE_TILE + 4 * gb + q] = v;
      }
  }
}

template <int NPMAX>
__global__ __launch_bounds__(64 * MOE_DF_WAVES) void k_down_few(
    const uint8_t *__restrict__ w_d, const uint32_t *__restrict__ hs, const float *__restrict__ hd, int n_rows,
    const int32_t *__restrict__ items, const int32_t *__restrict__ perm, const float *__restrict__ wts, int T, int k,
    int F, int H, int shared, int per_slot, float *__restrict__ out) {
  __shared__ float ys[MOE_DF_TMAX * MOE_DF_SMAX * MOE_DF_ROWS];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), pair = blockIdx.x, P = T * k;
  for (int i = threadIdx.x; i < T * MOE_DF_SMAX * MOE_DF_ROWS; i += blockDim.x) ys[i] = 0.0f;
  __syncthreads();
  const gsrc src = make_gsrc(hs, hd, n_rows, F / MOE_QK);
  const int n_items = items[0];
  for (int y = wave; y < n_items; y += MOE_DF_WAVES) {
    const int4 it = item_of(items, y);
    if (NPMAX >= 2 && it.z > 2) df_item<(NPMAX >= 2 ? 2 : 1)>(w_d, src, it, perm, wts, k, P, F, H, pair, ys);
    else df_item<1>(w_d, src, it, perm, wts, k, P, F, H, pair, ys);
  }
  __syncthreads();
  if ((int)threadIdx.x >= T * MOE_DF_ROWS) return;
  const int t = threadIdx.x / MOE_DF_ROWS, r = threadIdx.x % MOE_DF_ROWS;
  const float *yt = ys + t * MOE_DF_SMAX * MOE_DF_ROWS + r;
  const size_t col = (size_t)pair * MOE_DF_ROWS + r;
  if (per_slot) {
    for (int s = 0; s < k; s++) out[((size_t)t * k + s) * H + col] = yt[s * MOE_DF_ROWS];
    return;
  }
  float o = yt[0];
  for (int s = 1; s < k; s++) o = __fadd_rn(o, yt[s * MOE_DF_ROWS]);
  if (shared) o = __fadd_rn(o, yt[k * MOE_DF_ROWS]);
  out[(size_t)t * H + col] = o;
}

// ===========================================================================
// Token octets on v_mfma_scale_f32_32x32x64_f8f6f4 (items of up to 8 rows).
//
// Lane layout (probed on the device): A lane r + 32*ga holds row r of a
// 32-row tile and one whole MXFP4 block (its 16 ggml nibble bytes, nibble e
// at K offset e of the block) with that block's E8M0 exponent as its scale;
// ga picks the first or second block of the step's block pair.  B lane
// n + 32*gb holds column n: bytes 0-15 are K offsets 16*gb + [0, 16) of the
// first block, bytes 16-31 the same offsets of the second block.  D lane
// n + 32*gb holds column n, rows 8*i + 4*gb + j at element 4*i + j.
// Block-diagonal B: column n = 4*t + 2*part + g carries part (hi / lo
// digits) of block g of the pair for token t of the octet, so one MFMA
// multiplies 32 rows x 2 blocks against 8 tokens, and the 4 columns of a
// token are added at the end (lanes 4t .. 4t+3).
//
// The A operand comes from the 16-row record layout unchanged: rows r < 16
// of the 32-row tile from tile 2T, r >= 16 from tile 2T+1 (the next
// record run); block 2j + ga of quad q is lane (r % 16) + 16*(2j + ga) of
// that tile's quad, and its exponent byte q % 4 of the same lane's exponent
// dword.

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// A 32-row tile: 16-row tiles tile16 and tile16 + 1 of the tensor.
__device__ __forceinline__ wstream make_wstream32(const uint8_t *w, size_t tile16, int NG) {
  wstream s;
  s.rec = __builtin_amdgcn_make_buffer_rsrc((void *)(w + tile16 * NG * MOE_REC_BYTES), 0, 2 * NG * MOE_REC_BYTES,
                                            MOE_RSRC_FLAGS);
  return s;
}

// This lane's A byte offsets (step 0 of a quad): data, exponent dword.
struct aoff32 {
  uint32_t v, s;
};

__device__ __forceinline__ aoff32 make_aoff32(int lane, int NG) {
  const int r = lane & 31, ga = lane >> 5;
  const uint32_t tb = (uint32_t)(r >> 4) * NG * MOE_REC_BYTES;
  const uint32_t l16 = (uint32_t)((r & 15) + 16 * ga);
  aoff32 a;
  a.v = tb + l16 * 16;
  a.s = tb + MOE_REC_SC + l16 * 4;
  return a;
}

template <int NW>
struct wq32 {
  u32x4_t w[NW][2];  // [stream][step]
};

template <int NW, int CPOL>
__device__ __forceinline__ void load_wq32(wq32<NW> &b, const wstream (&ws)[NW], const aoff32 &ao, int q) {
#pragma unroll
  for (int i = 0; i < NW; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
      b.w[i][j] = __builtin_amdgcn_raw_buffer_load_b128(ws[i].rec, ao.v + j * 512,
                                                        (q >> 2) * MOE_REC_BYTES + (q & 3) * 1024, CPOL);
}

template <int NW>
__device__ __forceinline__ void load_sc32(uint32_t (&sc)[NW][2], const wstream (&ws)[NW], const aoff32 &ao, int g4) {
#pragma unroll
  for (int i = 0; i < NW; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
      sc[i][j] = __builtin_amdgcn_raw_buffer_load_b32(ws[i].rec, ao.s + j * 128, g4 * MOE_REC_BYTES, 0);
}

// B source of this lane for one octet: row = the staged row of token
// t = n / 4 of the octet (< 0: absent).
__device__ __forceinline__ gsel make_gsel32(int lane, int row, int KB) {
  const int n = lane & 31, gb = lane >> 5;
  const int part = (n >> 1) & 1, g = n & 1;
  gsel s;
  s.voff = row >= 0 ? (uint32_t)((row * KB + g) * (MOE_XSW * 4) + part * 32 + gb * 16) : MOE_OOB;
  s.doff = row >= 0 ? (uint32_t)((row * KB + g) * 4) : MOE_OOB;
  return s;
}

template <int NO>
struct bq32 {
  u32x4_t v[NO][2];
  float d[NO][2];
};

template <int NO>
__device__ __forceinline__ void load_bq32(bq32<NO> &b, const gsrc &src, const gsel (&gs)[NO], int q) {
#pragma unroll
  for (int o = 0; o < NO; o++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      b.v[o][j] = __builtin_amdgcn_raw_buffer_load_b128(src.x, gs[o].voff, (4 * q + 2 * j) * MOE_XSW * 4, 0);
      b.d[o][j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(src.d, gs[o].doff,
                                                                                 (4 * q + 2 * j) * 4, 0));
    }
}

template <int SEL, int NW, int NO>
__device__ __forceinline__ void quad_mma32(const wq32<NW> &w, const uint32_t (&sc)[NW][2], const bq32<NO> &b,
                                           bool upper, int sb, f32x16_t (&acc)[NO][NW]) {
#pragma unroll
  for (int o = 0; o < NO; o++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const u32x4_t v = b.v[o][j];
      i32x8_t bv;
      bv[0] = upper ? 0 : (int)v.x; bv[1] = upper ? 0 : (int)v.y; bv[2] = upper ? 0 : (int)v.z; bv[3] = upper ? 0 : (int)v.w;
      bv[4] = upper ? (int)v.x : 0; bv[5] = upper ? (int)v.y : 0; bv[6] = upper ? (int)v.z : 0; bv[7] = upper ? (int)v.w : 0;
#pragma unroll
      for (int i = 0; i < NW; i++) {
        const u32x4_t a4 = w.w[i][j];
        const i32x8_t a = {(int)a4.x, (int)a4.y, (int)a4.z, (int)a4.w, 0, 0, 0, 0};
        f32x16_t z;
#pragma unroll
        for (int e = 0; e < 16; e++) z[e] = 0.0f;
        const f32x16_t r = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, bv, z, 4, 0, SEL, (int)sc[i][j], 0, sb);
        acc[o][i] = acc[o][i] + b.d[o][j] * r;
      }
    }
#pragma unroll
  for (int o = 0; o < NO; o++)
#pragma unroll
    for (int i = 0; i < NW; i++) asm volatile("" : "+v"(acc[o][i]));
}

__device__ __forceinline__ bool lane_upper32(int lane) { return (lane & 1) != 0; }      // second block of the pair
__device__ __forceinline__ int lane_bscale32(int lane) { return (lane & 2) ? 127 : 131; }  // lo : hi digits

// Ring state of an octet K loop: weights of 4 quads, B data of 4 quads,
// exponent dwords of NG groups.  Every index into it is a template
// constant (the steps below are instantiated per quad), so the arrays stay
// in registers.
template <int NW, int NO, int NG>
struct oring {
  wq32<NW> w[4];
  bq32<NO> b[4];
  uint32_t sc[NG][NW][2];
};

// One quad of the loop: issue B for quad qB into slot SLOT+2 and weights
// for quad qW into slot SLOT+3 (if wanted), then multiply slot SLOT with
// exponent group G (op_sel SEL = quad % 4).
template <int SEL, int SLOT, int G, bool WB, bool WW, int NW, int NO, int NG, int CPOL>
__device__ __forceinline__ void ostep(oring<NW, NO, NG> &r, const wstream (&ws)[NW], const aoff32 &ao,
                                      const gsrc &src, const gsel (&gs)[NO], int qB, int qW, bool upper, int sb,
                                      f32x16_t (&acc)[NO][NW]) {
  if constexpr (WB) load_bq32<NO>(r.b[(SLOT + 2) & 3], src, gs, qB);
  if constexpr (WW) load_wq32<NW, CPOL>(r.w[(SLOT + 3) & 3], ws, ao, qW);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  quad_mma32<SEL, NW, NO>(r.w[SLOT], r.sc[G], r.b[SLOT], upper, sb, acc);
}

// Quads QL .. NQW-1 of a fully unrolled loop from q0 (q0 % 4 == 0).
template <int QL, int NQW, int NW, int NO, int NG, int CPOL>
__device__ __forceinline__ void ofixed_from(oring<NW, NO, NG> &r, const wstream (&ws)[NW], const aoff32 &ao,
                                            int q0, const gsrc &src, const gsel (&gs)[NO], bool upper, int sb,
                                            f32x16_t (&acc)[NO][NW]) {
  if constexpr (QL < NQW) {
    if constexpr ((QL & 3) == 0 && (QL >> 2) + 1 < NG) load_sc32<NW>(r.sc[(QL >> 2) + 1], ws, ao, (q0 >> 2) + (QL >> 2) + 1);
    ostep<QL & 3, QL & 3, QL / 4, (QL + 2 < NQW), (QL + 3 < NQW), NW, NO, NG, CPOL>(
        r, ws, ao, src, gs, q0 + QL + 2, q0 + QL + 3, upper, sb, acc);
    ofixed_from<QL + 1, NQW, NW, NO, NG, CPOL>(r, ws, ao, q0, src, gs, upper, sb, acc);
  }
}

// K loop over NQW quads from q0 (q0 % 4 == 0), fully unrolled; the rings
// as in gloop_fixed (B 2 quads ahead, weights 3 quads ahead).
template <int NW, int NO, int CPOL, int NQW>
__device__ __forceinline__ void oloop_fixed(const wstream (&ws)[NW], const aoff32 &ao, int q0, const gsrc &src,
                                            const gsel (&gs)[NO], int lane, f32x16_t (&acc)[NO][NW]) {
#pragma unroll
  for (int o = 0; o < NO; o++)
#pragma unroll
    for (int i = 0; i < NW; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[o][i][e] = 0.0f;
  constexpr int NG = (NQW + 3) / 4;
  const bool upper = lane_upper32(lane);
  const int sb = lane_bscale32(lane);
  oring<NW, NO, NG> r;
  load_sc32<NW>(r.sc[0], ws, ao, q0 >> 2);
  load_bq32<NO>(r.b[0], src, gs, q0);
  load_wq32<NW, CPOL>(r.w[0], ws, ao, q0);
  if constexpr (NQW > 1) {
    load_bq32<NO>(r.b[1], src, gs, q0 + 1);
    load_wq32<NW, CPOL>(r.w[1], ws, ao, q0 + 1);
  }
  if constexpr (NQW > 2) load_wq32<NW, CPOL>(r.w[2], ws, ao, q0 + 2);
  ofixed_from<0, NQW, NW, NO, NG, CPOL>(r, ws, ao, q0, src, gs, upper, sb, acc);
}

// Run-time number of quads [q0, q1): windows of 4 quads, loads past the
// end re-read the last quad, guarded tail.
template <int NW, int NO, int CPOL>
__device__ __forceinline__ void oloop_rolled(const wstream (&ws)[NW], const aoff32 &ao, int q0, int q1,
                                             const gsrc &src, const gsel (&gs)[NO], int lane,
                                             f32x16_t (&acc)[NO][NW]) {
#pragma unroll
  for (int o = 0; o < NO; o++)
#pragma unroll
    for (int i = 0; i < NW; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[o][i][e] = 0.0f;
  if (q1 <= q0) return;
  const bool upper = lane_upper32(lane);
  const int sb = lane_bscale32(lane);
  const int last = q1 - 1, glast = last >> 2;
  oring<NW, NO, 1> r;
  uint32_t scn[NW][2];
  load_sc32<NW>(r.sc[0], ws, ao, q0 >> 2);
  load_bq32<NO>(r.b[0], src, gs, q0);
  load_wq32<NW, CPOL>(r.w[0], ws, ao, q0);
  load_bq32<NO>(r.b[1], src, gs, q0 + 1 < q1 ? q0 + 1 : last);
  load_wq32<NW, CPOL>(r.w[1], ws, ao, q0 + 1 < q1 ? q0 + 1 : last);
  load_wq32<NW, CPOL>(r.w[2], ws, ao, q0 + 2 < q1 ? q0 + 2 : last);
  auto qc = [&](int q) { return q < q1 ? q : last; };
  int qb = q0;
  for (; qb + 4 <= q1; qb += 4) {
    const int gn = (qb >> 2) + 1;
    load_sc32<NW>(scn, ws, ao, gn < glast ? gn : glast);
    ostep<0, 0, 0, true, true, NW, NO, 1, CPOL>(r, ws, ao, src, gs, qc(qb + 2), qc(qb + 3), upper, sb, acc);
    ostep<1, 1, 0, true, true, NW, NO, 1, CPOL>(r, ws, ao, src, gs, qc(qb + 3), qc(qb + 4), upper, sb, acc);
    ostep<2, 2, 0, true, true, NW, NO, 1, CPOL>(r, ws, ao, src, gs, qc(qb + 4), qc(qb + 5), upper, sb, acc);
    ostep<3, 3, 0, true, true, NW, NO, 1, CPOL>(r, ws, ao, src, gs, qc(qb + 5), qc(qb + 6), upper, sb, acc);
#pragma unroll
    for (int i = 0; i < NW; i++)
#pragma unroll
      for (int j = 0; j < 2; j++) r.sc[0][i][j] = scn[i][j];
  }
  if (qb < q1) ostep<0, 0, 0, true, true, NW, NO, 1, CPOL>(r, ws, ao, src, gs, qc(qb + 2), qc(qb + 3), upper, sb, acc);
  if (qb + 1 < q1) ostep<1, 1, 0, true, true, NW, NO, 1, CPOL>(r, ws, ao, src, gs, qc(qb + 3), qc(qb + 4), upper, sb, acc);
  if (qb + 2 < q1) ostep<2, 2, 0, true, true, NW, NO, 1, CPOL>(r, ws, ao, src, gs, qc(qb + 4), qc(qb + 5), upper, sb, acc);
}

template <int NW, int NO, int CPOL>
__device__ __forceinline__ void oloop_any(const wstream (&ws)[NW], const aoff32 &ao, int q0, int q1,
                                          const gsrc &src, const gsel (&gs)[NO], int lane,
                                          f32x16_t (&acc)[NO][NW]) {
  switch (q1 - q0) {
    case 28: oloop_fixed<NW, NO, CPOL, 28>(ws, ao, q0, src, gs, lane, acc); break;
    case 16: oloop_fixed<NW, NO, CPOL, 16>(ws, ao, q0, src, gs, lane, acc); break;
    case 8: oloop_fixed<NW, NO, CPOL, 8>(ws, ao, q0, src, gs, lane, acc); break;
    case 6: oloop_fixed<NW, NO, CPOL, 6>(ws, ao, q0, src, gs, lane, acc); break;
    default: oloop_rolled<NW, NO, CPOL>(ws, ao, q0, q1, src, gs, lane, acc); break;
  }
}

// Sum of the 4 columns of each token (lanes 4t .. 4t+3), left in lane 4t:
// (c0 + c1) + (c2 + c3), with c = 2*part + g.
__device__ __forceinline__ float col4_sum(float v) {
  v += dpp_f<0xB1>(v);  // lane ^ 1
  v += dpp_f<0x4E>(v);  // lane ^ 2
  return v;
}

// Grouped gate/up on octets: one workgroup of 4 waves per (2 units of F,
// item of <= 8 rows): wave w streams unit 2*blockIdx.x + w%2 (gate and up,
// 32 rows each) over K-half w/2; the K-halves meet in LDS; then each
// 32-lane half of a wave takes one (unit, token), applies clamp + SwiGLU and
// writes the unit's Q8_0 h block of that token.  grid (F/64, item capacity).
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void k_gate_up_o(const uint8_t *__restrict__ w_g, const uint8_t *__restrict__ w_u, const uint32_t *__restrict__ xq,
                 const float *__restrict__ xd, const int32_t *__restrict__ items, const int32_t *__restrict__ perm,
                 int k, int T, int F, int H, float clamp, uint32_t *__restrict__ hs, float *__restrict__ hd,
                 float *__restrict__ htap) {
  __shared__ __align__(16) float red[4][2][8][MOE_UNIT];  // [wave][gate/up][token][row]
  if ((int)blockIdx.y >= items[0]) return;
  const int4 it = item_of(items, blockIdx.y);
  const int NQ = H / 128, NQ4 = moe_nq4(NQ), U = F / MOE_UNIT, tiles = F / MOE_TILE, KB = H / MOE_QK;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ul = wave & 1, kp = wave >> 1, P = T * k;
  const int u = 2 * blockIdx.x + ul;
  const int row0 = it.y, nt = it.z;
  const bool shared = (it.w & MOE_ITEM_SHARED) != 0;
  int q0, q1;
  wave_quads(NQ, 2, kp, q0, q1);
  const size_t t0 = (size_t)it.x * tiles + 2 * u;
  const wstream ws[2] = {make_wstream32(w_g, t0, NQ4), make_wstream32(w_u, t0, NQ4)};
  const aoff32 ao = make_aoff32(lane, NQ4);
  const gsrc src = make_gsrc(xq, xd, T, KB);
  gsel gs[1];
  {
    const int i = (lane & 31) >> 2;
    int xr = -1;
    if (i < nt) xr = shared ? row0 + i - P : perm[row0 + i] / k;
    gs[0] = make_gsel32(lane, xr, KB);
  }
  f32x16_t acc[1][2];
  // non-temporal weights where no other item of the expert reads them
  if (it.w & MOE_ITEM_SPLIT) oloop_any<2, 1, 0>(ws, ao, q0, q1, src, gs, lane, acc);
  else oloop_any<2, 1, MOE_CPOL_NT>(ws, ao, q0, q1, src, gs, lane, acc);
  const int n = lane & 31, gb = lane >> 5;
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const float v = col4_sum(acc[0][i][e]);
      if ((n & 3) == 0) red[wave][i][n >> 2][8 * (e >> 2) + 4 * gb + (e & 3)] = v;
    }
  __syncthreads();
  // (unit, token) c = 8*round + 2*wave + half: unit ul2 = c / 8, token c % 8
#pragma unroll
  for (int round = 0; round < 2; round++) {
    const int c = 8 * round + 2 * wave + (lane >> 5);
    const int ul2 = c >> 3, t = c & 7, j = lane & 31;
    const bool live = t < nt;
    // waves ul2 (K-half 0) and ul2 + 2 (K-half 1) hold this unit
    const float gsum = red[ul2][0][t][j] + red[ul2 + 2][0][t][j];
    const float usum = red[ul2][1][t][j] + red[ul2 + 2][1][t][j];
    const float h = live ? swiglu(gsum, usum, clamp) : 0.0f;
    const int hrow = row0 + (live ? t : 0), uu = 2 * blockIdx.x + ul2;
    h_unit_store(h, live, hs + ((size_t)hrow * U + uu) * MOE_XSW, hd + (size_t)hrow * U + uu, lane);
    if (htap && live) htap[(size_t)hrow * F + (size_t)uu * MOE_UNIT + j] = h;
  }
}

// Grouped down on octets: each wave streams one 32-row tile of H of the
// item's down matrix over all of F against the item's (<= 8) h rows;
// y[r][H] = (row . h[r]) * wts[perm[r]] (routed) or * 1 (shared).
// grid (H/128, item capacity), 4 waves.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void k_down_o(const uint8_t *__restrict__ w_d, const uint32_t *__restrict__ hs, const float *__restrict__ hd,
              int n_rows, const int32_t *__restrict__ items, const int32_t *__restrict__ perm,
              const float *__restrict__ wts, int F, int H, float *__restrict__ y) {
  if ((int)blockIdx.y >= items[0]) return;
  const int4 it = item_of(items, blockIdx.y);
  const int NQ = F / 128, NQ4 = moe_nq4(NQ), tiles = H / MOE_TILE, KB = F / MOE_QK;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t32 = blockIdx.x * 4 + wave;  // 32-row tile of H
  const int row0 = it.y, nt = it.z;
  const bool shared = (it.w & MOE_ITEM_SHARED) != 0;
  const wstream ws[1] = {make_wstream32(w_d, (size_t)it.x * tiles + 2 * t32, NQ4)};
  const aoff32 ao = make_aoff32(lane, NQ4);
  const gsrc src = make_gsrc(hs, hd, n_rows, KB);
  const int n = lane & 31, gb = lane >> 5, t = n >> 2;
  gsel gs[1] = {make_gsel32(lane, t < nt ? row0 + t : -1, KB)};
  f32x16_t acc[1][1];
  oloop_any<1, 1, 0>(ws, ao, 0, NQ, src, gs, lane, acc);
  const bool live = t < nt;
  const int r = row0 + (live ? t : 0);
  const float wt = (live && !shared) ? wts[perm[r]] : 1.0f;
  float v[16];
#pragma unroll
  for (int e = 0; e < 16; e++) {
    v[e] = col4_sum(acc[0][0][e]);
    if (!shared) v[e] = __fmul_rn(v[e], wt);
  }
  if ((n & 3) == 0 && live) {
    float *dst = y + (size_t)r * H + (size_t)t32 * 32 + 4 * gb;
#pragma unroll
    for (int i = 0; i < 4; i++)
      *reinterpret_cast<float4 *>(dst + 8 * i) = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
  }
}

// ===========================================================================
// Octet B operand staged in LDS (the grouped down kernel).  Every wave of a
// down workgroup multiplies the same item's h rows, so the workgroup copies
// them into LDS once, already in MFMA lane order: step s (blocks 2s, 2s+1)
// is 64 lanes x 16 bytes, lane n + 32*gb = column n (token n/4, part
// (n/2)%2, block 2s + n%2), bytes 16*gb .. 16*gb+15 of that block's part;
// scales d[s][token][n%2].  A lane's B read is one ds_read_b128 of 16
// consecutive bytes per step (the 64 lanes cover 1 KiB without bank
// conflicts), and the vector-memory unit only carries the weights.

// LDS bytes for KB blocks per row (KB even): digits, then scales.
__host__ __device__ constexpr size_t octet_lds_bytes(int KB) {
  return (size_t)(KB / 2) * 64 * 16 + (size_t)(KB / 2) * 16 * 4;
}

// Copy the nt (<= 8) staged rows row0 .. of KB blocks into that layout;
// columns of absent tokens get zeros.  tid / nthr: this thread among nthr.
__device__ __forceinline__ void stage_octet_lds(const uint32_t *__restrict__ hs, const float *__restrict__ hd,
                                                int row0, int nt, int KB, u32x4_t *bl, float *dl, int tid,
                                                int nthr) {
  const u32x4_t *src = reinterpret_cast<const u32x4_t *>(hs + (size_t)row0 * KB * MOE_XSW);
  const int n16 = 8 * KB * 4;  // 16-byte chunks of 8 rows
#pragma unroll 4
  for (int c = tid; c < n16; c += nthr) {
    const int t = c / (4 * KB), w = c - t * 4 * KB, b = w >> 2, sub = w & 3;
    const int L = 32 * (sub & 1) + 4 * t + 2 * (sub >> 1) + (b & 1);
    bl[(b >> 1) * 64 + L] = t < nt ? src[c] : u32x4_t{0u, 0u, 0u, 0u};
  }
  for (int c = tid; c < 8 * KB; c += nthr) {
    const int t = c / KB, b = c - t * KB;
    dl[((b >> 1) * 8 + t) * 2 + (b & 1)] = t < nt ? hd[(size_t)(row0 + t) * KB + b] : 0.0f;
  }
}

// The same layout with a 16-byte zero slot after each step's 64 lanes
// (stride 65), read by the operand half without data (bs32z).
__host__ __device__ constexpr size_t octet_lds_bytes_z(int KB) {
  return (size_t)(KB / 2) * 65 * 16 + (size_t)(KB / 2) * 16 * 4;
}

__device__ __forceinline__ void stage_octet_lds_z(const uint32_t *__restrict__ hs, const float *__restrict__ hd,
                                                  int row0, int nt, int KB, u32x4_t *bl, float *dl, int tid,
                                                  int nthr) {
  const u32x4_t *src = reinterpret_cast<const u32x4_t *>(hs + (size_t)row0 * KB * MOE_XSW);
  const int n16 = 8 * KB * 4;  // 16-byte chunks of 8 rows
#pragma unroll 4
  for (int c = tid; c < n16; c += nthr) {
    const int t = c / (4 * KB), w = c - t * 4 * KB, b = w >> 2, sub = w & 3;
    const int L = 32 * (sub & 1) + 4 * t + 2 * (sub >> 1) + (b & 1);
    bl[(b >> 1) * 65 + L] = t < nt ? src[c] : u32x4_t{0u, 0u, 0u, 0u};
  }
  for (int c = tid; c < KB / 2; c += nthr) bl[c * 65 + 64] = u32x4_t{0u, 0u, 0u, 0u};
  for (int c = tid; c < 8 * KB; c += nthr) {
    const int t = c / KB, b = c - t * KB;
    dl[((b >> 1) * 8 + t) * 2 + (b & 1)] = t < nt ? hd[(size_t)(row0 + t) * KB + b] : 0.0f;
  }
}

// Ring of the LDS-B octet loop: weights of 4 quads (3 ahead), B of 2 quads
// (1 ahead, from LDS) for NO octets, exponent dwords of NG groups.
template <int NW, int NO, int NG>
struct oring_l {
  wq32<NW> w[4];
  bq32<NO> b[2];
  uint32_t sc[NG][NW][2];
};

// B of quad q for NO octets; octet o's digits start OB 16-byte units after
// octet 0's, its scales OD floats after.
template <int NO, int OB, int OD>
__device__ __forceinline__ void load_bq32_lds(bq32<NO> &b, const u32x4_t *bl, const float *dl, int lane, int dlo,
                                              int q) {
#pragma unroll
  for (int o = 0; o < NO; o++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      b.v[o][j] = bl[o * OB + (2 * q + j) * 64 + lane];
      b.d[o][j] = dl[o * OD + (2 * q + j) * 16 + dlo];
    }
}

// Weights and exponents of the first quads, issued before the B staging.
template <int NW, int NO, int NG, int CPOL>
__device__ __forceinline__ void oprime_l(oring_l<NW, NO, NG> &r, const wstream (&ws)[NW], const aoff32 &ao, int NQW) {
  load_sc32<NW>(r.sc[0], ws, ao, 0);
  load_wq32<NW, CPOL>(r.w[0], ws, ao, 0);
  if (NQW > 1) load_wq32<NW, CPOL>(r.w[1], ws, ao, 1);
  if (NQW > 2) load_wq32<NW, CPOL>(r.w[2], ws, ao, 2);
}

template <int QL, int NQW, int NW, int NO, int NG, int CPOL, int OB, int OD>
__device__ __forceinline__ void olfixed_from(oring_l<NW, NO, NG> &r, const wstream (&ws)[NW], const aoff32 &ao,
                                             const u32x4_t *bl, const float *dl, int lane, int dlo, bool upper,
                                             int sb, f32x16_t (&acc)[NO][NW]) {
  if constexpr (QL < NQW) {
    if constexpr ((QL & 3) == 0 && (QL >> 2) + 1 < NG) load_sc32<NW>(r.sc[(QL >> 2) + 1], ws, ao, (QL >> 2) + 1);
    if constexpr (QL + 1 < NQW) load_bq32_lds<NO, OB, OD>(r.b[(QL + 1) & 1], bl, dl, lane, dlo, QL + 1);
    if constexpr (QL + 3 < NQW) load_wq32<NW, CPOL>(r.w[(QL + 3) & 3], ws, ao, QL + 3);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    quad_mma32<QL & 3, NW, NO>(r.w[QL & 3], r.sc[QL >> 2], r.b[QL & 1], upper, sb, acc);
    olfixed_from<QL + 1, NQW, NW, NO, NG, CPOL, OB, OD>(r, ws, ao, bl, dl, lane, dlo, upper, sb, acc);
  }
}

// Grouped down on octets with B in LDS: k_down_o's work split (each wave one
// 32-row tile of H over all of F, y = (row . h) * router weight), NQ = F/128
// in {6, 8, 16, 28}.  grid (H/128, item capacity), 4 waves, LDS
// octet_lds_bytes(F/32).
template <int NQ>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void k_down_ol(const uint8_t *__restrict__ w_d, const uint32_t *__restrict__ hs, const float *__restrict__ hd,
               int n_rows, const int32_t *__restrict__ items, const int32_t *__restrict__ perm,
               const float *__restrict__ wts, int F, int H, float *__restrict__ y) {
  extern __shared__ __align__(16) uint32_t lds[];
  if ((int)blockIdx.y >= items[0]) return;
  const int4 it = item_of(items, blockIdx.y);
  constexpr int NQ4 = (NQ + 3) / 4, NG = NQ4, KB = NQ * 4;
  const int tiles = H / MOE_TILE;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t32 = blockIdx.x * 4 + wave;  // 32-row tile of H
  const int row0 = it.y, nt = it.z;
  const bool shared = (it.w & MOE_ITEM_SHARED) != 0;
  const wstream ws[1] = {make_wstream32(w_d, (size_t)it.x * tiles + 2 * t32, NQ4)};
  const aoff32 ao = make_aoff32(lane, NQ4);
  oring_l<1, 1, NG> r;
  const bool split = (it.w & MOE_ITEM_SPLIT) != 0;  // else non-temporal weights: no other item reads them
  if (split) oprime_l<1, 1, NG, 0>(r, ws, ao, NQ);
  else oprime_l<1, 1, NG, MOE_CPOL_NT>(r, ws, ao, NQ);
  u32x4_t *bl = reinterpret_cast<u32x4_t *>(lds);
  float *dl = reinterpret_cast<float *>(lds + (KB / 2) * 64 * 4);
  stage_octet_lds(hs, hd, row0, nt, KB, bl, dl, threadIdx.x, 256);
  __syncthreads();
  const int n = lane & 31, gb = lane >> 5, t = n >> 2;
  const int dlo = t * 2 + (n & 1);
  f32x16_t acc[1][1];
#pragma unroll
  for (int e = 0; e < 16; e++) acc[0][0][e] = 0.0f;
  load_bq32_lds<1, 0, 0>(r.b[0], bl, dl, lane, dlo, 0);
  if (split)
    olfixed_from<0, NQ, 1, 1, NG, 0, 0, 0>(r, ws, ao, bl, dl, lane, dlo, lane_upper32(lane), lane_bscale32(lane), acc);
  else
    olfixed_from<0, NQ, 1, 1, NG, MOE_CPOL_NT, 0, 0>(r, ws, ao, bl, dl, lane, dlo, lane_upper32(lane),
                                                     lane_bscale32(lane), acc);
  const bool live = t < nt;
  const int rr = row0 + (live ? t : 0);
  const float wt = (live && !shared) ? wts[perm[rr]] : 1.0f;
  float v[16];
#pragma unroll
  for (int e = 0; e < 16; e++) {
    v[e] = col4_sum(acc[0][0][e]);
    if (!shared) v[e] = __fmul_rn(v[e], wt);
  }
  if ((n & 3) == 0 && live) {
    float *dst = y + (size_t)rr * H + (size_t)t32 * 32 + 4 * gb;
#pragma unroll
    for (int i = 0; i < 4; i++)
      *reinterpret_cast<float4 *>(dst + 8 * i) = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
  }
}

// B of one step as both 16-byte halves of each octet's MFMA operand, read
// from LDS where each step's 64 lanes are followed by a 16-byte zero slot
// (stride 65): the half that carries no data reads the zero slot, so the
// block-diagonal operand needs no selects.
template <int NO>
struct bs32z {
  u32x4_t lo[NO], hi[NO];
  float d[NO];
};

// Per-lane offsets (16-byte units within a step) of the two operand halves:
// a lane of an odd column (block 2s+1) carries its data in the upper half.
struct zoff {
  int lo, hi;
};

__device__ __forceinline__ zoff make_zoff(int lane) {
  const bool upper = lane_upper32(lane);
  return zoff{upper ? 64 : lane, upper ? lane : 64};
}

template <int NO, int OB, int OD>
__device__ __forceinline__ void load_bs32z_lds(bs32z<NO> &b, const u32x4_t *bl, const float *dl, const zoff &z,
                                               int dlo, int step) {
#pragma unroll
  for (int o = 0; o < NO; o++) {
    b.lo[o] = bl[o * OB + step * 65 + z.lo];
    b.hi[o] = bl[o * OB + step * 65 + z.hi];
    b.d[o] = dl[o * OD + step * 16 + dlo];
  }
}

template <int NO, int OB>
__device__ __forceinline__ void load_bs32z_lds_v(bs32z<NO> &b, const u32x4_t *bl, const zoff &z, int step) {
#pragma unroll
  for (int o = 0; o < NO; o++) {
    b.lo[o] = bl[o * OB + step * 65 + z.lo];
    b.hi[o] = bl[o * OB + step * 65 + z.hi];
  }
}

template <int NO, int OD>
__device__ __forceinline__ void load_bs32z_lds_d(bs32z<NO> &b, const float *dl, int dlo, int step) {
#pragma unroll
  for (int o = 0; o < NO; o++) b.d[o] = dl[o * OD + step * 16 + dlo];
}

// Step J of a quad (op_sel SEL = quad % 4): acc[o] += d[o] * (A . B[o]) for
// one weight stream; the per-octet sequence is that of quad_mma32 (same bits).
template <int SEL, int J, int NO>
__device__ __forceinline__ void step_mma32z(const wq32<1> &w, const uint32_t (&sc)[1][2], const bs32z<NO> &b, int sb,
                                            f32x16_t (&acc)[NO][1]) {
  const u32x4_t a4 = w.w[0][J];
  const i32x8_t a = {(int)a4.x, (int)a4.y, (int)a4.z, (int)a4.w, 0, 0, 0, 0};
#pragma unroll
  for (int o = 0; o < NO; o++) {
    const u32x4_t l = b.lo[o], h = b.hi[o];
    const i32x8_t bv = {(int)l.x, (int)l.y, (int)l.z, (int)l.w, (int)h.x, (int)h.y, (int)h.z, (int)h.w};
    f32x16_t z;
#pragma unroll
    for (int e = 0; e < 16; e++) z[e] = 0.0f;
    const f32x16_t r = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, bv, z, 4, 0, SEL, (int)sc[0][J], 0, sb);
    acc[o][0] = acc[o][0] + b.d[o] * r;
  }
#pragma unroll
  for (int o = 0; o < NO; o++) asm volatile("" : "+v"(acc[o][0]));
}

// step_mma32z in two parts: the NO MFMAs of the step (results and scales
// kept), then the scaling into acc (same operations per octet, same bits),
// so the next step's B can be read from LDS between the two.
template <int NO>
struct stepres {
  f32x16_t r[NO];
};

template <int SEL, int J, int NO>
__device__ __forceinline__ void step_mma32z_issue(const u32x4_t &a4, const uint32_t (&sc)[1][2], const bs32z<NO> &b,
                                                  int sb, stepres<NO> &res) {
  const i32x8_t a = {(int)a4.x, (int)a4.y, (int)a4.z, (int)a4.w, 0, 0, 0, 0};
#pragma unroll
  for (int o = 0; o < NO; o++) {
    const u32x4_t l = b.lo[o], h = b.hi[o];
    const i32x8_t bv = {(int)l.x, (int)l.y, (int)l.z, (int)l.w, (int)h.x, (int)h.y, (int)h.z, (int)h.w};
    f32x16_t z;
#pragma unroll
    for (int e = 0; e < 16; e++) z[e] = 0.0f;
    res.r[o] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, bv, z, 4, 0, SEL, (int)sc[0][J], 0, sb);
  }
}

template <int NO>
__device__ __forceinline__ void step_scale(const stepres<NO> &res, const float (&d)[NO], f32x16_t (&acc)[NO][1]) {
#pragma unroll
  for (int o = 0; o < NO; o++) acc[o][0] = acc[o][0] + d[o] * res.r[o];
#pragma unroll
  for (int o = 0; o < NO; o++) asm volatile("" : "+v"(acc[o][0]));
}

// One step's weights (step S = 2 * quad + j of the stream), cache policy CPOL.
template <int CPOL = 0>
__device__ __forceinline__ void load_w32step(u32x4_t &w, const wstream (&ws)[1], const aoff32 &ao, int S) {
  const int q = S >> 1, j = S & 1;
  w = __builtin_amdgcn_raw_buffer_load_b128(ws[0].rec, ao.v + j * 512, (q >> 2) * MOE_REC_BYTES + (q & 3) * 1024,
                                            CPOL);
}

#define MOE_DRS 4  // weight ring of the down step loop, in steps

// Ring of the step-B loop: weights of MOE_DRS steps (3 ahead) of one
// stream, exponent dwords of NG groups, B of the next step (a zero-slot
// operand, read from LDS between the step's MFMAs and its scaling, so the
// LDS latency overlaps them; a deeper B ring does not fit 128 registers).
template <int NO, int NG>
struct sring {
  u32x4_t w[MOE_DRS];  // weights of steps S .. S + MOE_DRS - 1 (slot S % MOE_DRS)
  uint32_t sc[NG][1][2];
  bs32z<NO> b[1];
};

// Quads QL .. NQW-1 with B from LDS one step ahead.
template <int QL, int NQW, int NO, int NG, int OB, int OD>
__device__ __forceinline__ void slfixed_from(sring<NO, NG> &r, const wstream (&ws)[1], const aoff32 &ao,
                                             const u32x4_t *bl, const float *dl, const zoff &z, int dlo, int sb,
                                             f32x16_t (&acc)[NO][1]) {
  if constexpr (QL < NQW) {
    if constexpr ((QL & 3) == 0 && (QL >> 2) + 1 < NG) load_sc32<1>(r.sc[(QL >> 2) + 1], ws, ao, (QL >> 2) + 1);
    constexpr int S0 = 2 * QL, RS = MOE_DRS;
    if constexpr (S0 + RS - 1 < 2 * NQW) load_w32step(r.w[(S0 + RS - 1) % RS], ws, ao, S0 + RS - 1);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    {
      stepres<NO> res;
      step_mma32z_issue<QL & 3, 0, NO>(r.w[S0 % RS], r.sc[QL >> 2], r.b[0], sb, res);
      __builtin_amdgcn_sched_barrier(0);
      load_bs32z_lds_v<NO, OB>(r.b[0], bl, z, 2 * QL + 1);
      __builtin_amdgcn_sched_barrier(0);
      step_scale<NO>(res, r.b[0].d, acc);
      __builtin_amdgcn_sched_barrier(0);
      load_bs32z_lds_d<NO, OD>(r.b[0], dl, dlo, 2 * QL + 1);
    }
    if constexpr (S0 + RS < 2 * NQW) load_w32step(r.w[(S0 + RS) % RS], ws, ao, S0 + RS);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    {
      stepres<NO> res;
      step_mma32z_issue<QL & 3, 1, NO>(r.w[(S0 + 1) % RS], r.sc[QL >> 2], r.b[0], sb, res);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (QL + 1 < NQW) load_bs32z_lds_v<NO, OB>(r.b[0], bl, z, 2 * QL + 2);
      __builtin_amdgcn_sched_barrier(0);
      step_scale<NO>(res, r.b[0].d, acc);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (QL + 1 < NQW) load_bs32z_lds_d<NO, OD>(r.b[0], dl, dlo, 2 * QL + 2);
    }
    slfixed_from<QL + 1, NQW, NO, NG, OB, OD>(r, ws, ao, bl, dl, z, dlo, sb, acc);
  }
}

#define MOE_DOL2_WAVES 8

// The item's NO octets of h staged as stage_octet_lds_z lays them out, by
// direct global-to-LDS loads (buffer_load ... lds): unit u of a step holds
// row (u>>2)&7 of the octet, block 2*step + (u&1) and 16-byte piece
// (u>>5) | ((u>>1)&1)<<1; scale f holds row (f>>1)&7 of block
// 2*(f>>4) + (f&1).  Of the 32*NO (octet, step) loads wave w issues
// w*4*NO .. w*4*NO + 4*NO - 1 (all of one octet), and of the 8*NO loads of
// 64 scales w*NO .. w*NO + NO - 1.  Rows past the item read nothing (their
// columns are never stored).  For 8 waves and KB == 64.
template <int NO, int KB>
__device__ __forceinline__ void stage_octets_dma(const gsrc &src, int row0, int nt, uint32_t *lds, int lane,
                                                 int wave) {
  static_assert(KB == 64, "32 steps per octet: 4 per wave and octet");
  typedef __attribute__((address_space(3))) void *lds_t;
  constexpr int OW = (int)(octet_lds_bytes_z(KB) / 4);  // dwords per staged octet
  const int o = (wave * NO) >> 3;
  const int td = (lane >> 2) & 7, ts = (lane >> 1) & 7;
  const int sub = (lane >> 5) | (((lane >> 1) & 1) << 1);
  const uint32_t xo = 8 * o + td < nt ? (uint32_t)(((row0 + 8 * o + td) * KB + (lane & 1)) * (MOE_XSW * 4) + sub * 16)
                                      : MOE_OOB;
  const uint32_t so = 8 * o + ts < nt ? (uint32_t)(((row0 + 8 * o + ts) * KB + 2 * (lane >> 4) + (lane & 1)) * 4)
                                      : MOE_OOB;
  uint32_t *ol = lds + o * OW;
#pragma unroll
  for (int j = 0; j < 4 * NO; j++) {
    const int st = (wave * 4 * NO + j) & 31;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(src.x, (lds_t)(ol + st * 65 * 4), 16, xo, 2 * st * (MOE_XSW * 4), 0, 0);
  }
#pragma unroll
  for (int j = 0; j < NO; j++) {
    const int hh = (wave * NO + j) & 7;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(src.d, (lds_t)(ol + (KB / 2) * 65 * 4 + hh * 64), 4, so, 8 * hh * 4, 0,
                                             0);
  }
}

// The down work of one wave against NO octets staged at lds (octet o at
// dword o * octet_lds_bytes(KB) / 4): y of token 8*o + t of the item.
template <int NQ, int NO>
__device__ __forceinline__ void dn_ol_octets(const wstream (&ws)[1], const aoff32 &ao, uint32_t *lds,
                                             const uint32_t *__restrict__ hs, const float *__restrict__ hd,
                                             int n_rows, const int4 &it, const int32_t *__restrict__ perm,
                                             const float *__restrict__ wts, int H, int t32, int lane,
                                             float *__restrict__ y) {
  constexpr int NQ4 = (NQ + 3) / 4, NG = NQ4, KB = NQ * 4;
  constexpr int OW = (int)(octet_lds_bytes_z(KB) / 4);  // dwords per staged octet
  const int row0 = it.y, nt = it.z;
  const bool shared = (it.w & MOE_ITEM_SHARED) != 0;
  sring<NO, NG> r;
  if constexpr (KB == 64) {
    // the h loads straight into LDS first, then the first weights, then the
    // zero slots; the h loads are waited for (vmcnt) right before the barrier
    stage_octets_dma<NO, KB>(make_gsrc(hs, hd, n_rows, KB), row0, nt, lds, threadIdx.x & 63,
                             __builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    load_sc32<1>(r.sc[0], ws, ao, 0);
#pragma unroll
    for (int i = 0; i + 1 < MOE_DRS; i++)
      if (i < 2 * NQ) load_w32step(r.w[i], ws, ao, i);
#pragma unroll
    for (int o = 0; o < NO; o++)
      for (int c = threadIdx.x; c < KB / 2; c += 64 * MOE_DOL2_WAVES)
        reinterpret_cast<u32x4_t *>(lds + o * OW)[c * 65 + 64] = u32x4_t{0u, 0u, 0u, 0u};
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 + (MOE_DRS - 1 < 2 * NQ ? MOE_DRS - 1 : 2 * NQ)));
    lds_barrier();
  } else {
    // first weights in flight during the staging
    load_sc32<1>(r.sc[0], ws, ao, 0);
#pragma unroll
    for (int i = 0; i + 1 < MOE_DRS; i++)
      if (i < 2 * NQ) load_w32step(r.w[i], ws, ao, i);
#pragma unroll
    for (int o = 0; o < NO; o++) {
      uint32_t *ol = lds + o * OW;
      stage_octet_lds_z(hs, hd, row0 + 8 * o, nt - 8 * o, KB, reinterpret_cast<u32x4_t *>(ol),
                        reinterpret_cast<float *>(ol + (KB / 2) * 65 * 4), threadIdx.x, 64 * MOE_DOL2_WAVES);
    }
    __syncthreads();
  }
  const u32x4_t *bl = reinterpret_cast<const u32x4_t *>(lds);
  const float *dl = reinterpret_cast<const float *>(lds + (KB / 2) * 65 * 4);
  const int n = lane & 31, gb = lane >> 5, t = n >> 2;
  const int dlo = t * 2 + (n & 1);
  f32x16_t acc[NO][1];
#pragma unroll
  for (int o = 0; o < NO; o++)
#pragma unroll
    for (int e = 0; e < 16; e++) acc[o][0][e] = 0.0f;
  const zoff z = make_zoff(lane);
  load_bs32z_lds<NO, OW / 4, OW>(r.b[0], bl, dl, z, dlo, 0);
  slfixed_from<0, NQ, NO, NG, OW / 4, OW>(r, ws, ao, bl, dl, z, dlo, lane_bscale32(lane), acc);
#pragma unroll
  for (int o = 0; o < NO; o++) {
    const int tt = 8 * o + t;
    const bool live = tt < nt;
    const int rr = row0 + (live ? tt : 0);
    const float wt = (live && !shared) ? wts[perm[rr]] : 1.0f;
    float v[16];
#pragma unroll
    for (int e = 0; e < 16; e++) {
      v[e] = col4_sum(acc[o][0][e]);
      if (!shared) v[e] = __fmul_rn(v[e], wt);
    }
    if ((n & 3) == 0 && live) {
      float *dst = y + (size_t)rr * H + (size_t)t32 * 32 + 4 * gb;
#pragma unroll
      for (int i = 0; i < 4; i++)
        *reinterpret_cast<float4 *>(dst + 8 * i) = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    }
  }
}

// k_down_ol on items of up to 16 rows: a workgroup of 8 waves stages the
// item's two octets of h in LDS (octet 1 only when the item holds more than
// 8 rows) and each wave multiplies its 32-row tile of H against both from
// the same weight registers, so one pass over the item's down weights
// serves 16 tokens.  Both halves of each block-diagonal B operand come from
// LDS (the half without data from the step's zero slot: no selects), one
// step ahead, which keeps the wave within 128 VGPRs (4 waves per SIMD with
// two workgroups per CU).  Per token the MFMA and scaling sequence is
// k_down_ol's (same bits).  grid (H/256, item capacity), 512 threads, LDS
// 2 * octet_lds_bytes_z(F/32).
template <int NQ>
__global__ __launch_bounds__(64 * MOE_DOL2_WAVES) __attribute__((amdgpu_waves_per_eu(4)))
void k_down_ol2(const uint8_t *__restrict__ w_d, const uint32_t *__restrict__ hs, const float *__restrict__ hd,
                int n_rows, const int32_t *__restrict__ items, const int32_t *__restrict__ perm,
                const float *__restrict__ wts, int F, int H, float *__restrict__ y) {
  extern __shared__ __align__(16) uint32_t lds[];
  if ((int)blockIdx.y >= items[0]) return;
  const int4 it = item_of(items, blockIdx.y);
  constexpr int NQ4 = (NQ + 3) / 4;
  const int tiles = H / MOE_TILE;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t32 = blockIdx.x * MOE_DOL2_WAVES + wave;  // 32-row tile of H
  const int nt = it.z;
  const wstream ws[1] = {make_wstream32(w_d, (size_t)it.x * tiles + 2 * t32, NQ4)};
  const aoff32 ao = make_aoff32(lane, NQ4);
  if (nt > 8) dn_ol_octets<NQ, 2>(ws, ao, lds, hs, hd, n_rows, it, perm, wts, H, t32, lane, y);  // uniform branch
  else dn_ol_octets<NQ, 1>(ws, ao, lds, hs, hd, n_rows, it, perm, wts, H, t32, lane, y);
}

// ===========================================================================
// Grouped gate/up with the item's B staged in LDS, chunk by chunk of K.
//
// One workgroup of 2*NU waves per (NU units of F, item of <= 16 rows): wave
// w streams the gate (w < NU) or up tile of unit NU*blockIdx.x + w%NU over
// all of K against the item's one or two octets.  The workgroup copies
// B (the octets' x rows) into LDS in chunks of MOE_GCH quads, already in
// MFMA lane order (the layout of stage_octet_lds, per chunk, each step's 64
// lanes followed by a 16-byte zero slot), double buffered: chunk c+1 goes
// out at chunk c's first quad as direct global-to-LDS loads and is waited
// for only at the chunk's end barrier.  Every B byte thus crosses the
// vector-memory unit once per workgroup and never occupies a VGPR; a wave
// reads both halves of each MFMA operand from LDS (the half without data
// from the zero slot, so no selects) and holds one weight stream with a
// ring of MOE_GU_RS steps: 128 VGPRs, 4 waves per SIMD, which beat deeper
// rings at 3 waves.  Each step issues its MFMAs (one result register set
// per octet), then the next step's B reads, then the scaling FMAs, so the
// LDS round trip overlaps the MFMAs and the FMAs instead of following them.
// After the K loop gate and up meet in LDS for clamp + SwiGLU + Q8_0(h) as
// in k_gate_up_o.
#define MOE_GCH 4                                  // quads per staged chunk
#define MOE_GCH_STEPS (2 * MOE_GCH)                // MFMA steps per chunk
#define MOE_GCH_OCT_U4 (MOE_GCH_STEPS * 65)        // 16-byte units per octet per chunk (digits, zero slots)
#define MOE_GCH_OCT_D (MOE_GCH_STEPS * 16)         // scales per octet per chunk
#define MOE_GCH_BUF_DW (2 * MOE_GCH_OCT_U4 * 4 + 2 * MOE_GCH_OCT_D)  // dwords per chunk buffer (two octets)


// The staging of a chunk by direct global-to-LDS loads (buffer_load ... lds):
// a wave's loads write 64 consecutive 16-byte units (one octet's step, lane
// u = unit u) or 64 consecutive scales, so the data never passes through
// VGPRs.  Unit u of a step holds token (u>>2)&7, block 2*step + (u&1) of the
// chunk and 16-byte piece (u>>5) | ((u>>1)&1)<<1 of that block; scale f of
// an octet's 128 holds token (f>>1)&7 of block 2*(f>>4) + (f&1).  Of the
// 8*NO (octet, step) loads of a chunk wave w issues w*NO .. w*NO+NO-1 (all
// of one octet), and waves 0 .. 2*NO-1 one half of an octet's scales each.
// The loads of chunk c+1 go out at chunk c's first quad; the wave waits for
// them (vmcnt) only right before the chunk's end barrier.
struct gdma {
  uint32_t xo;  // this lane's digit bytes at chunk 0 (MOE_OOB: absent token)
  uint32_t so;  // this lane's scale at chunk 0 (MOE_OOB: absent, or no scale load for this wave)
};

template <int NO>
__device__ __forceinline__ gdma make_gdma(int lane, int wave, int xr_dig, int xr_sc, int KB) {
  gdma g;
  const int sub = (lane >> 5) | (((lane >> 1) & 1) << 1);
  g.xo = xr_dig >= 0 ? (uint32_t)((xr_dig * KB + (lane & 1)) * (MOE_XSW * 4) + sub * 16) : MOE_OOB;
  g.so = (wave < 2 * NO && xr_sc >= 0) ? (uint32_t)((xr_sc * KB + 2 * (lane >> 4) + (lane & 1)) * 4) : MOE_OOB;
  return g;
}

template <int NO, int NX, int C>
__device__ __forceinline__ void gdma_issue(const gdma &g, const gsrc &src, uint32_t *buf, int wave) {
  typedef __attribute__((address_space(3))) void *lds_t;
#pragma unroll
  for (int j = 0; j < NO; j++) {
    const int i = wave * NO + j, o = i >> 3, st = i & 7;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(src.x, (lds_t)(buf + (o * MOE_GCH_OCT_U4 + st * 65) * 4), 16, g.xo,
                                             (16 * C + 2 * st) * (MOE_XSW * 4), 0, 0);
  }
  if (wave < 2 * NO) {
    const int o = wave >> 1, hh = wave & 1;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(src.d, (lds_t)(buf + NX * MOE_GCH_OCT_U4 * 4 + o * MOE_GCH_OCT_D + hh * 64),
                                             4, g.so, (16 * C + 8 * hh) * 4, 0, 0);
  }
}

// The digits (lo, hi) and the scales of one step's B, read apart.
template <int NO>
__device__ __forceinline__ void load_bs32_chunk_v(bs32z<NO> &b, const uint32_t *buf, const zoff &z, int ls) {
  const u32x4_t *bl = reinterpret_cast<const u32x4_t *>(buf);
#pragma unroll
  for (int o = 0; o < NO; o++) {
    b.lo[o] = bl[o * MOE_GCH_OCT_U4 + ls * 65 + z.lo];
    b.hi[o] = bl[o * MOE_GCH_OCT_U4 + ls * 65 + z.hi];
  }
}

template <int NO>
__device__ __forceinline__ void load_bs32_chunk_d(bs32z<NO> &b, const uint32_t *buf, int dlo, int ls) {
  const float *dl = reinterpret_cast<const float *>(buf) + 2 * MOE_GCH_OCT_U4 * 4;
#pragma unroll
  for (int o = 0; o < NO; o++) b.d[o] = dl[o * MOE_GCH_OCT_D + ls * 16 + dlo];
}

template <int NO>
__device__ __forceinline__ void load_bs32_chunk(bs32z<NO> &b, const uint32_t *buf, const zoff &z, int dlo, int ls) {
  load_bs32z_lds<NO, MOE_GCH_OCT_U4, MOE_GCH_OCT_D>(b, reinterpret_cast<const u32x4_t *>(buf),
                                                    reinterpret_cast<const float *>(buf) + 2 * MOE_GCH_OCT_U4 * 4, z,
                                                    dlo, ls);
}

#define MOE_GU_RS 4  // weight ring of the gate/up step loop, in steps (3 ahead)

template <int NO, int NG>
struct gring {
  u32x4_t w[MOE_GU_RS];  // weights of steps S .. S + MOE_GU_RS - 1 (slot S % MOE_GU_RS)
  uint32_t sc[NG][1][2];
  bs32z<NO> b[1];
};

// VMEM loads a wave issues after its chunk-C staging loads, up to the end of
// the chunk (the exponent dwords of the next group, two weight steps a quad).
template <int C, int NQ, int NG>
__host__ __device__ constexpr int gdma_after() {
  int n = 0;
  if (C + 1 < NG) n += 2;
  for (int qc = 0; qc < MOE_GCH; qc++) {
    const int S0 = 2 * (MOE_GCH * C + qc);
    if (S0 + MOE_GU_RS - 1 < 2 * NQ) n++;
    if (S0 + MOE_GU_RS < 2 * NQ) n++;
  }
  return n;
}

// Quads QL .. NQ-1 of the chunked K loop.
template <int QL, int NQ, int NO, int NG>
__device__ __forceinline__ void gl_from(gring<NO, NG> &r, const wstream (&ws)[1], const aoff32 &ao,
                                        const gsrc &src, const gdma &g, uint32_t *lds, int wave, const zoff &z,
                                        int dlo, int sb, f32x16_t (&acc)[NO][1]) {
  if constexpr (QL < NQ) {
    constexpr int C = QL / MOE_GCH, QC = QL % MOE_GCH, NC = NQ / MOE_GCH, RS = MOE_GU_RS;
    const uint32_t *buf = lds + (C & 1) * MOE_GCH_BUF_DW;
    if constexpr (C + 1 < NC && QC == 0) {  // the next chunk's staging, straight into the other buffer
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      gdma_issue<NO, 2, C + 1>(g, src, lds + ((C + 1) & 1) * MOE_GCH_BUF_DW, wave);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr ((QL & 3) == 0 && (QL >> 2) + 1 < NG) load_sc32<1>(r.sc[(QL >> 2) + 1], ws, ao, (QL >> 2) + 1);
    constexpr int S0 = 2 * QL;
    if constexpr (S0 + RS - 1 < 2 * NQ) load_w32step(r.w[(S0 + RS - 1) % RS], ws, ao, S0 + RS - 1);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    {
      stepres<NO> res;
      step_mma32z_issue<QL & 3, 0, NO>(r.w[S0 % RS], r.sc[QL >> 2], r.b[0], sb, res);
      __builtin_amdgcn_sched_barrier(0);
      load_bs32_chunk_v<NO>(r.b[0], buf, z, 2 * QC + 1);
      __builtin_amdgcn_sched_barrier(0);
      step_scale<NO>(res, r.b[0].d, acc);
      __builtin_amdgcn_sched_barrier(0);
      load_bs32_chunk_d<NO>(r.b[0], buf, dlo, 2 * QC + 1);
    }
    if constexpr (S0 + RS < 2 * NQ) load_w32step(r.w[(S0 + RS) % RS], ws, ao, S0 + RS);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    {
      stepres<NO> res;
      step_mma32z_issue<QL & 3, 1, NO>(r.w[(S0 + 1) % RS], r.sc[QL >> 2], r.b[0], sb, res);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (QC + 1 < MOE_GCH) load_bs32_chunk_v<NO>(r.b[0], buf, z, 2 * QC + 2);
      __builtin_amdgcn_sched_barrier(0);
      step_scale<NO>(res, r.b[0].d, acc);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (QC + 1 < MOE_GCH) load_bs32_chunk_d<NO>(r.b[0], buf, dlo, 2 * QC + 2);
    }
    if constexpr (QC + 1 == MOE_GCH && C + 1 < NC) {
      // the next chunk has landed in LDS (this wave's loads, then everyone's)
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(gdma_after<C, NQ, NG>()));
      uint32_t *nb = lds + ((C + 1) & 1) * MOE_GCH_BUF_DW;
      lds_barrier();
      load_bs32_chunk<NO>(r.b[0], nb, z, dlo, 0);
    }
    gl_from<QL + 1, NQ, NO, NG>(r, ws, ao, src, g, lds, wave, z, dlo, sb, acc);
  }
}

// The K loop of one wave (of 8: NU = 4) against NO octets; xrow(i) = the
// staged x row of the item's token i (< 0: absent).  Leaves this wave's sums
// (the 4 columns of a token added) in red[w%NU][w/NU][token][row].
template <int NQ, int NO, int NU, class XR>
__device__ __forceinline__ void gu_ol_octets(const wstream (&ws)[1], const aoff32 &ao, const gsrc &src,
                                             const XR &xrow, int KB, uint32_t *lds, int tid, int wave, int lane) {
  static_assert(NU == 4, "the staging loads are laid out for 8 waves");
  constexpr int NQ4 = (NQ + 3) / 4, NG = NQ4, RS = MOE_GU_RS;
  const int xr_dig = xrow(8 * ((wave * NO) >> 3) + ((lane >> 2) & 7));
  const int xr_sc = wave < 2 * NO ? xrow(8 * (wave >> 1) + ((lane >> 1) & 7)) : -1;
  const gdma g = make_gdma<NO>(lane, wave, xr_dig, xr_sc, KB);
  gring<NO, NG> r;
  // chunk 0 straight into LDS, then the first weights
  gdma_issue<NO, 2, 0>(g, src, lds, wave);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  load_sc32<1>(r.sc[0], ws, ao, 0);
#pragma unroll
  for (int i = 0; i + 1 < RS; i++)
    if (i < 2 * NQ) load_w32step(r.w[i], ws, ao, i);
  if (tid < 2 * 2 * MOE_GCH_STEPS) {  // the zero slots of both chunk buffers, never written by the staging
    const int bf = tid / (2 * MOE_GCH_STEPS), o = (tid / MOE_GCH_STEPS) & 1, st = tid % MOE_GCH_STEPS;
    reinterpret_cast<u32x4_t *>(lds + bf * MOE_GCH_BUF_DW)[o * MOE_GCH_OCT_U4 + st * 65 + 64] =
        u32x4_t{0u, 0u, 0u, 0u};
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  // the chunk-0 loads have landed (2 exponent dwords and RS-1 weight steps went out after them)
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 + (RS - 1 < 2 * NQ ? RS - 1 : 2 * NQ)));
  lds_barrier();
  const int n = lane & 31, gb = lane >> 5, t = n >> 2;
  const int dlo = t * 2 + (n & 1);
  f32x16_t acc[NO][1];
#pragma unroll
  for (int o = 0; o < NO; o++)
#pragma unroll
    for (int e = 0; e < 16; e++) acc[o][0][e] = 0.0f;
  const zoff z = make_zoff(lane);
  load_bs32_chunk<NO>(r.b[0], lds, z, dlo, 0);
  gl_from<0, NQ, NO, NG>(r, ws, ao, src, g, lds, wave, z, dlo, lane_bscale32(lane), acc);
  lds_barrier();  // every wave is done with the chunk buffers, which now hold the sums
  float *red = reinterpret_cast<float *>(lds);  // [unit][gate/up][token][row]
#pragma unroll
  for (int o = 0; o < NO; o++)
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const float v = col4_sum(acc[o][0][e]);
      if ((n & 3) == 0)
        red[(((wave % NU) * 2 + wave / NU) * 16 + 8 * o + (n >> 2)) * MOE_UNIT + 8 * (e >> 2) + 4 * gb + (e & 3)] = v;
    }
}

// grid (F/(32 NU), item capacity), 128*NU threads (NU units of F: wave w
// streams the gate (w < NU) or up tile of unit NU*blockIdx.x + w%NU), LDS
// 2 * MOE_GCH_BUF_DW dwords.  With NU = 4 the item's staged x serves twice
// the weight rows of NU = 2, so the x rows are a fifth of the bytes a
// workgroup moves instead of a third.  Requires H == 128 * NQ,
// NQ % MOE_GCH == 0, (F/32) % NU == 0.
template <int NQ, int NU>
__global__ __launch_bounds__(128 * NU) __attribute__((amdgpu_waves_per_eu(4)))
void k_gate_up_ol(const uint8_t *__restrict__ w_g, const uint8_t *__restrict__ w_u, const uint32_t *__restrict__ xq,
                  const float *__restrict__ xd, const int32_t *__restrict__ items, const int32_t *__restrict__ perm,
                  int k, int T, int F, int H, float clamp, uint32_t *__restrict__ hs, float *__restrict__ hd,
                  float *__restrict__ htap) {
  __shared__ __align__(16) uint32_t lds[2 * MOE_GCH_BUF_DW];
  if ((int)blockIdx.y >= items[0]) return;
  const int4 it = item_of(items, blockIdx.y);
  constexpr int NQ4 = (NQ + 3) / 4, KB = NQ * 4;
  const int U = F / MOE_UNIT, tiles = F / MOE_TILE;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int P = T * k, row0 = it.y, nt = it.z;
  const bool shared = (it.w & MOE_ITEM_SHARED) != 0;
  const int u = NU * blockIdx.x + wave % NU;
  const wstream ws[1] = {make_wstream32(wave >= NU ? w_u : w_g, (size_t)it.x * tiles + 2 * u, NQ4)};
  const aoff32 ao = make_aoff32(lane, NQ4);
  const gsrc src = make_gsrc(xq, xd, T, KB);
  auto xrow = [&](int i) { return i < nt ? (shared ? row0 + i - P : perm[row0 + i] / k) : -1; };
  if (nt > 8) gu_ol_octets<NQ, 2, NU>(ws, ao, src, xrow, KB, lds, tid, wave, lane);  // uniform branch
  else gu_ol_octets<NQ, 1, NU>(ws, ao, src, xrow, KB, lds, tid, wave, lane);
  __syncthreads();
  const float *red = reinterpret_cast<const float *>(lds);
  // (unit, token) c = 4*NU*round + 2*wave + half-wave: unit c / 16, token c % 16
#pragma unroll
  for (int round = 0; round < 4; round++) {
    const int c = 4 * NU * round + 2 * wave + (lane >> 5);
    const int ul2 = c >> 4, t = c & 15, j = lane & 31;
    if (((4 * NU * round) & 15) >= nt && NU == 2) continue;  // no token of this round (uniform over the workgroup)
    const bool live = t < nt;
    const float gsum = red[((ul2 * 2 + 0) * 16 + t) * MOE_UNIT + j];
    const float usum = red[((ul2 * 2 + 1) * 16 + t) * MOE_UNIT + j];
    const float h = live ? swiglu(gsum, usum, clamp) : 0.0f;
    const int hrow = row0 + (live ? t : 0), uu = NU * blockIdx.x + ul2;
    h_unit_store(h, live, hs + ((size_t)hrow * U + uu) * MOE_XSW, hd + (size_t)hrow * U + uu, lane);
    if (htap && live) htap[(size_t)hrow * F + (size_t)uu * MOE_UNIT + j] = h;
  }
}
