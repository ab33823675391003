// kernels_group.h -- token-to-expert grouping and the grouped (T > 1) chain.
//
// Grouping is ggml mul_mat_id's row map: pairs p = t*k + s are visited
// token-major, slot-minor and appended to their expert's list, so within an
// expert the rows are in ascending pair order (nano-glm/apps/moe-server/
// main.cpp:413-459 restates the same order).  The kernel reproduces it
// exactly: a histogram, an exclusive prefix sum over experts, then a stable
// placement where each expert's thread walks the pair list in order.
//
// The grouped chain that uses it (T > 1) is k_group -> k_gate_up ->
// k_down (kernels_rows.h) -> k_combine.
#pragma once

#include "device_common.h"

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

// ---------------------------------------------------------------------------
// out[t][c] = ((y[r(t,0)] + y[r(t,1)]) + ...) + y[P+t]   (or per slot), with
// r(t,s) = inv[t*k+s] (grouped rows) or t*k+s when inv is NULL (decode: the
// y row of slot s is s).  The slot order is the reference's pairwise ADD
// chain (nano-glm/lib/models/glm_dsa/moe_block.h:120-131).
__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ y,
                                                 const int32_t *__restrict__ inv, int T, int k,
                                                 int H, int shared, int per_slot,
                                                 float *__restrict__ out) {
  const size_t i = (size_t)blockIdx.x * 256u + threadIdx.x;
  if (i >= (size_t)T * H) return;
  const int t = (int)(i / H), c = (int)(i % H);
  const int P = T * k;
  // a negative row marks a pair whose expert id was out of range: it contributes 0
  if (per_slot) {
    for (int s = 0; s < k; s++) {
      const int r = inv ? inv[t * k + s] : t * k + s;
      out[((size_t)t * k + s) * H + c] = r >= 0 ? y[(size_t)r * H + c] : 0.0f;
    }
    return;
  }
  const int r0 = inv ? inv[t * k] : t * k;
  float acc = r0 >= 0 ? y[(size_t)r0 * H + c] : 0.0f;
  for (int s = 1; s < k; s++) {
    const int r = inv ? inv[t * k + s] : t * k + s;
    acc = __fadd_rn(acc, r >= 0 ? y[(size_t)r * H + c] : 0.0f);
  }
  if (shared) acc = __fadd_rn(acc, y[((size_t)P + t) * H + c]);
  out[i] = acc;
}
