// kernels_group.h -- token-to-expert grouping and the grouped (T > 1) chain.
//
// Grouping is ggml mul_mat_id's row map: pairs p = t*k + s are visited
// token-major, slot-minor and appended to their expert's list, so within an
// expert the rows are in ascending pair order (nano-glm/apps/moe-server/
// main.cpp:413-459 restates the same order).  The kernel reproduces it
// exactly: a histogram, an exclusive prefix sum over experts, then a stable
// placement where each expert's thread walks the pair list in order.
//
// Grouped chain (T > 1):
//   k_quantize_q8      x [T][H] -> Q8_0 activation blocks
//   k_group            ids -> counts, offsets, perm, inv, active-expert list
//   k_gu_grouped       per (active expert | shared, 32 ffn rows): gate/up
//                      rows against each of the expert's tokens, SwiGLU,
//                      Q8_0 -> h rows in grouped order (shared rows after)
//   k_down_grouped     per (active expert | shared, RD hidden rows): down
//                      rows against each h row, times the router weight ->
//                      y [grouped row][H]
//   k_combine          out[t] = ((y[inv(t,0)] + y[inv(t,1)]) + ...) + shared
#pragma once

#include "device_common.h"
#include "kernels_decode.h"

#define MOE_GROUP_MAX_E 1024
#define MOE_GROUP_MAX_PAIRS 16384

// Workspace words for the grouped chain: counts[E] offsets[E+1] perm[P]
// inv[P] act[E+2] (act[0] = number of active experts, act[1..] their ids in
// ascending order).
static inline size_t group_ws_words(int T, int k, int E) {
  const size_t P = (size_t)T * k;
  return (size_t)E + (E + 1) + 2 * P + (E + 2);
}

__global__ __launch_bounds__(1024) void k_group(const int32_t *__restrict__ ids, int P, int E,
                                                int32_t *__restrict__ counts,
                                                int32_t *__restrict__ offsets,
                                                int32_t *__restrict__ perm, int32_t *__restrict__ inv,
                                                int32_t *__restrict__ act) {
  __shared__ int32_t sid[MOE_GROUP_MAX_PAIRS];
  __shared__ int32_t cnt[MOE_GROUP_MAX_E];
  __shared__ int32_t wsum[16], wflag[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e < E; e += 1024) cnt[e] = 0;
  __syncthreads();
  for (int p = tid; p < P; p += 1024) {
    const int e = ids[p];
    // out-of-range ids are dropped (the host validates the ids it owns)
    const bool ok = e >= 0 && e < E;
    sid[p] = ok ? e : -1;
    if (ok) atomicAdd(&cnt[e], 1);
    else if (inv) inv[p] = -1;  // dropped pair: no grouped row
  }
  __syncthreads();
  // exclusive scans over experts of the counts and of the "active" flags
  const int c = tid < E ? cnt[tid] : 0;
  const int f = c > 0 ? 1 : 0;
  int v = c, vf = f;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(v, off), uf = __shfl_up(vf, off);
    if (lane >= off) {
      v += u;
      vf += uf;
    }
  }
  if (lane == 63) {
    wsum[wave] = v;
    wflag[wave] = vf;
  }
  __syncthreads();
  int base = 0, basef = 0;
  for (int w = 0; w < wave; w++) {
    base += wsum[w];
    basef += wflag[w];
  }
  const int excl = base + v - c, exclf = basef + vf - f;
  if (tid < E) {
    counts[tid] = c;
    offsets[tid] = excl;
    if (f && act) act[1 + exclf] = tid;
  }
  if (tid == 1023) {  // thread 1023's inclusive sums are the totals
    offsets[E] = base + v;
    if (act) act[0] = basef + vf;
  }
  // stable placement: expert e's thread appends its pairs in pair order
  if (tid < E && c > 0) {
    int r = excl;
    for (int p = 0; p < P; p++) {
      if (sid[p] == tid) {
        perm[r] = p;
        if (inv) inv[p] = r;
        r++;
      }
    }
  }
}

// Which expert matrix and which h rows workgroup row `y` of a grouped launch
// owns.  y < act[0]: routed expert act[1+y], rows offsets[e]..offsets[e+1];
// the last y when `shared`: the shared expert (matrix index shared_mat),
// rows P..P+T-1.  Returns false for idle workgroups.
__device__ __forceinline__ bool grouped_slot(int y, int ny, const int32_t *__restrict__ offsets,
                                             const int32_t *__restrict__ act, int shared,
                                             int shared_mat, int P, int T, int &mat, int &row0,
                                             int &nrows, bool &is_shared) {
  is_shared = shared && y == ny - 1;
  if (is_shared) {
    mat = shared_mat;
    row0 = P;
    nrows = T;
    return true;
  }
  if (y >= act[0]) return false;
  mat = act[1 + y];
  row0 = offsets[mat];
  nrows = offsets[mat + 1] - row0;
  return true;
}

// ---------------------------------------------------------------------------
// Gate/up/SwiGLU/Q8_0 over grouped rows.  grid = (F/32, ny), 256 threads.
template <int NB>
__global__ __launch_bounds__(256) void k_gu_grouped(
    const uint4 *__restrict__ nib_g, const uint4 *__restrict__ nib_u,
    const uint8_t *__restrict__ sc_g, const uint8_t *__restrict__ sc_u,
    const uint32_t *__restrict__ xq, const float *__restrict__ xd,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ perm,
    const int32_t *__restrict__ act, int k, int T, int shared, int shared_mat, int F, int KB,
    float clamp, uint32_t *__restrict__ hq, float *__restrict__ hd, float *__restrict__ htap) {
  int mat, row0, nrows;
  bool is_shared;
  if (!grouped_slot(blockIdx.y, gridDim.y, offsets, act, shared, shared_mat, T * k, T, mat, row0, nrows,
                    is_shared))
    return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r0 = blockIdx.x * 32 + wave * GU_ROWS_PER_WAVE;
  const size_t base = (size_t)mat * (size_t)F * (size_t)KB;
  __shared__ float hs[32];
  for (int i = 0; i < nrows; i++) {
    const int hrow = row0 + i;
    const int tok = is_shared ? i : perm[hrow] / k;
    uint32_t xr[NB][16];
    float xs[NB];
    load_act_blocks<NB>(xq + (size_t)tok * KB * 16, xd + (size_t)tok * KB, KB, lane, xr, xs);
    float pg[GU_ROWS_PER_WAVE], pu[GU_ROWS_PER_WAVE];
#pragma unroll
    for (int rr = 0; rr < GU_ROWS_PER_WAVE; rr++) {
      const size_t rb = base + (size_t)(r0 + rr) * (size_t)KB;
      float ag = 0.0f, au = 0.0f;
#pragma unroll
      for (int j = 0; j < NB; j++) {
        const int b = lane + 64 * j;
        if (b < KB) {
          ag = fmaf(scale_e8m0(xs[j], sc_g[rb + b]), block_dot(nib_g[rb + b], xr[j]), ag);
          au = fmaf(scale_e8m0(xs[j], sc_u[rb + b]), block_dot(nib_u[rb + b], xr[j]), au);
        }
      }
      pg[rr] = ag;
      pu[rr] = au;
    }
#pragma unroll
    for (int rr = 0; rr < GU_ROWS_PER_WAVE; rr++) {
      float g = wave_sum(pg[rr]);
      float u = wave_sum(pu[rr]);
      if (clamp > 1e-6f) {
        u = fmaxf(fminf(u, clamp), -clamp);
        g = fminf(g, clamp);
      }
      const float h = __fmul_rn(__fdiv_rn(g, 1.0f + expf(-g)), u);
      if (lane == 0) hs[wave * GU_ROWS_PER_WAVE + rr] = h;
    }
    __syncthreads();
    if (wave == 0) {
      const float h = lane < 32 ? hs[lane] : 0.0f;
      const float amax = wave_max(fabsf(h));
      const float q = q8_code(h, amax);
      const float qhi = __shfl_down(q, 16);
      const size_t blk = (size_t)hrow * (size_t)(F / MOE_QK) + blockIdx.x;
      if (lane < 16) hq[blk * 16 + lane] = pack_f16x2(q, qhi);
      if (lane == 0) hd[blk] = (float)q8_scale_f16(amax);
      if (htap && lane < 32) htap[(size_t)hrow * F + blockIdx.x * 32 + lane] = h;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// down over grouped rows.  grid = (H/RD, ny), 256 threads; wave w takes the
// expert's h rows w, w+4, ...  y[hrow][r] = down_row(r) . h[hrow] * weight
// (weight = wts[pair] for routed rows, none for shared rows).
template <int NB, int RD>
__global__ __launch_bounds__(256) void k_down_grouped(
    const uint4 *__restrict__ nib_d, const uint8_t *__restrict__ sc_d,
    const uint32_t *__restrict__ hq, const float *__restrict__ hd,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ perm,
    const int32_t *__restrict__ act, const float *__restrict__ wts, int k, int T, int shared,
    int shared_mat, int H, int KB, float *__restrict__ y) {
  int mat, row0, nrows;
  bool is_shared;
  if (!grouped_slot(blockIdx.y, gridDim.y, offsets, act, shared, shared_mat, T * k, T, mat, row0, nrows,
                    is_shared))
    return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r0 = blockIdx.x * RD;
  const size_t base = (size_t)mat * (size_t)H * (size_t)KB;
  for (int i = wave; i < nrows; i += 4) {
    const int hrow = row0 + i;
    uint32_t hr[NB][16];
    float hsc[NB];
    load_act_blocks<NB>(hq + (size_t)hrow * KB * 16, hd + (size_t)hrow * KB, KB, lane, hr, hsc);
    float part[RD];
#pragma unroll
    for (int rr = 0; rr < RD; rr++) {
      const size_t rb = base + (size_t)(r0 + rr) * (size_t)KB;
      float a = 0.0f;
#pragma unroll
      for (int j = 0; j < NB; j++) {
        const int b = lane + 64 * j;
        if (b < KB) a = fmaf(scale_e8m0(hsc[j], sc_d[rb + b]), block_dot(nib_d[rb + b], hr[j]), a);
      }
      part[rr] = a;
    }
    const float w = is_shared ? 1.0f : wts[perm[hrow]];
#pragma unroll
    for (int rr = 0; rr < RD; rr++) {
      const float v = wave_sum(part[rr]);
      if (lane == rr) y[(size_t)hrow * H + r0 + rr] = is_shared ? v : __fmul_rn(v, w);
    }
  }
}

// ---------------------------------------------------------------------------
// out[t][c] = ((y[inv[t*k]] + y[inv[t*k+1]]) + ...) + y[P+t]   (or per slot)
__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ y,
                                                 const int32_t *__restrict__ inv, int T, int k,
                                                 int H, int shared, int per_slot,
                                                 float *__restrict__ out) {
  const size_t i = (size_t)blockIdx.x * 256u + threadIdx.x;
  if (i >= (size_t)T * H) return;
  const int t = (int)(i / H), c = (int)(i % H);
  const int P = T * k;
  // inv < 0 marks a pair whose expert id was out of range: it contributes 0.
  if (per_slot) {
    for (int s = 0; s < k; s++) {
      const int r = inv[t * k + s];
      out[((size_t)t * k + s) * H + c] = r >= 0 ? y[(size_t)r * H + c] : 0.0f;
    }
    return;
  }
  const int r0 = inv[t * k];
  float acc = r0 >= 0 ? y[(size_t)r0 * H + c] : 0.0f;
  for (int s = 1; s < k; s++) {
    const int r = inv[t * k + s];
    acc = __fadd_rn(acc, r >= 0 ? y[(size_t)r * H + c] : 0.0f);
  }
  if (shared) acc = __fadd_rn(acc, y[((size_t)P + t) * H + c]);
  out[i] = acc;
}
