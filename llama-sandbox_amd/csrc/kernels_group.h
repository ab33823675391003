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
#include "kernels_rows.h"  // stage_quant

#define MOE_GROUP_MAX_E 1024
#define MOE_GROUP_MAX_PAIRS 65535  // grouped rows are kept in 16 bits in k_group
#define MOE_GROUP_QBLOCKS 512  // x blocks quantized per extra workgroup of k_group
#define MOE_GROUP_IT 8         // 64-pair steps per wave whose ids k_group keeps in registers

// Item capacity of a call with T tokens, top-k, E experts and items of at
// most BT rows: ceil(c_e / BT) per expert sums to at most P/BT + min(P, E),
// plus ceil(T / BT) items of the shared expert.
static inline int group_item_cap(int T, int k, int E, int BT) {
  const int P = T * k;
  return (P + BT - 1) / BT + (P < E ? P : E) + (T + BT - 1) / BT;
}

// Workspace words for the grouped chain: counts[E] offsets[E+1] perm[P]
// inv[P], then two item lists (4-word header, 4 words per item), each sized
// for BT = 1 (group_list_words).
static inline size_t group_list_words(int T, int k, int E) { return 4 + 4 * (size_t)group_item_cap(T, k, E, 1); }
static inline size_t group_ws_words(int T, int k, int E) {
  const size_t P = (size_t)T * k;
  return (size_t)E + (E + 1) + 2 * P + 2 * group_list_words(T, k, E);
}

// Lanes of the wave holding the same expert id as this lane (e >= 0, ids
// below 2^10), from one ballot per id bit.
__device__ __forceinline__ uint64_t same_id_lanes(int e, bool valid) {
  uint64_t m = __ballot(valid);
#pragma unroll
  for (int b = 0; b < 10; b++) {
    const uint64_t B = __ballot(valid && ((e >> b) & 1));
    m &= ((e >> b) & 1) ? B : ~B;
  }
  return m;
}

// Workgroup 0: the grouping.  Wave w owns the pairs [w*PW, (w+1)*PW) and
// walks them 64 at a time in pair order; lanes with the same expert are
// found by ballots over the id bits (rank = same-expert lanes below).
//   pass 1: per-wave counts wc[w][e] (one writer per expert per step);
//   then the histogram (sum over waves), exclusive scans over experts of
//   the counts and of the item counts ceil(c_e / BT), the item list
//   (items != NULL: {expert, first row, rows, flags} per item in expert
//   order, then the shared expert's {E, P + j*BT, rows, flags} when
//   `shared`; flags: MOE_ITEM_SHARED, MOE_ITEM_SPLIT), and
//   wc[w][e] turned into wave w's first row of expert e;
//   pass 2: row of a pair = wc[w][e] + rank, so rows ascend in pair order
//   within each expert (ggml mul_mat_id's order).
// items2 != NULL: a second item list of at most BT2 rows per item, the same
// way (the gate/up and down kernels of a call may take different item sizes).
// Workgroups 1..: Q8_0 of x (T rows of H, flat n_xblocks blocks) into the
// staged format of the grouped kernels (xq, xd), MOE_GROUP_QBLOCKS blocks
// each; none when xq is NULL.
__global__ __launch_bounds__(1024) void k_group(const int32_t *__restrict__ ids, int P, int E, int T, int shared,
                                                int BT, int32_t *__restrict__ counts,
                                                int32_t *__restrict__ offsets,
                                                int32_t *__restrict__ perm, int32_t *__restrict__ inv,
                                                int32_t *__restrict__ items, const float *__restrict__ x,
                                                int n_xblocks, uint32_t *__restrict__ xq, float *__restrict__ xd,
                                                int BT2, int32_t *__restrict__ items2) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (blockIdx.x > 0) {
    const int b0 = (blockIdx.x - 1) * MOE_GROUP_QBLOCKS;
    const int nb = n_xblocks - b0 < MOE_GROUP_QBLOCKS ? n_xblocks - b0 : MOE_GROUP_QBLOCKS;
    if (nb > 0) stage_quant(x + (size_t)b0 * MOE_QK, nb, xq + (size_t)b0 * MOE_XSW, xd + b0, tid, 1024);
    return;
  }
  __shared__ uint16_t wc[16][MOE_GROUP_MAX_E];  // per-wave counts, then per-wave first rows (< 2^16)
  __shared__ int32_t wsum[16], wsumi[16], wsumi2[16], tot[2];
  const int PW = ((P + 15) / 16 + 63) & ~63;    // pairs per wave, whole steps of 64
  const int p_lo = wave * PW, p_hi = p_lo + PW < P ? p_lo + PW : P;
  // up to MOE_GROUP_IT steps of 64 pairs per wave (P <= 16 * 64 * MOE_GROUP_IT):
  // the wave's ids are loaded at once and kept, with each lane's rank among
  // the lanes of its step with the same id, for pass 2
  const bool cached = p_hi - p_lo <= 64 * MOE_GROUP_IT;
  int ev[MOE_GROUP_IT];
  uint32_t rl[MOE_GROUP_IT];  // rank | (last lane of its id in the step) << 16
  if (cached) {
#pragma unroll
    for (int it = 0; it < MOE_GROUP_IT; it++) {
      const int p = p_lo + 64 * it + lane;
      ev[it] = p < p_hi ? ids[p] : -1;
    }
  }
  for (int i = tid; i < 16 * MOE_GROUP_MAX_E; i += 1024) (&wc[0][0])[i] = 0;
  __syncthreads();
  const uint64_t below = (1ull << lane) - 1ull, upto = (2ull << lane) - 1ull;
  if (cached) {
#pragma unroll
    for (int it = 0; it < MOE_GROUP_IT; it++) {
      if (p_lo + 64 * it >= p_hi) break;  // uniform over the wave
      const int e = ev[it];
      const bool ok = e >= 0 && e < E;  // out-of-range ids are dropped (the host validates the ids it owns)
      const uint64_t m = same_id_lanes(e, ok);
      const int rank = __popcll(m & below);
      const bool last = !(m & ~upto);
      rl[it] = (uint32_t)rank | (last ? 1u << 16 : 0u);
      if (ok && last) wc[wave][e] += (uint16_t)rank + 1;  // last lane of its expert
    }
  } else {
    for (int pb = p_lo; pb < p_hi; pb += 64) {
      const int p = pb + lane;
      const int e = p < p_hi ? ids[p] : -1;
      const bool ok = e >= 0 && e < E;
      const uint64_t m = same_id_lanes(e, ok);
      if (ok && !(m & ~upto)) wc[wave][e] += (uint16_t)__popcll(m & below) + 1;
    }
  }
  __syncthreads();
  // histogram and exclusive scans over experts of the counts and the item counts
  int c = 0;
  if (tid < E)
    for (int w = 0; w < 16; w++) c += wc[w][tid];
  const int ni = items ? (c + BT - 1) / BT : 0;
  const int ni2 = items2 ? (c + BT2 - 1) / BT2 : 0;
  int v = c, vi = ni, vi2 = ni2;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(v, off), ui = __shfl_up(vi, off), ui2 = __shfl_up(vi2, off);
    if (lane >= off) {
      v += u;
      vi += ui;
      vi2 += ui2;
    }
  }
  if (lane == 63) {
    wsum[wave] = v;
    wsumi[wave] = vi;
    wsumi2[wave] = vi2;
  }
  __syncthreads();
  int base = 0, basei = 0, basei2 = 0;
  for (int w = 0; w < wave; w++) {
    base += wsum[w];
    basei += wsumi[w];
    basei2 += wsumi2[w];
  }
  const int excl = base + v - c, excli = basei + vi - ni, excli2 = basei2 + vi2 - ni2;
  if (tid < E) {
    counts[tid] = c;
    offsets[tid] = excl;
    int run = excl;
    for (int w = 0; w < 16; w++) {
      const int n = wc[w][tid];
      wc[w][tid] = (uint16_t)run;
      run += n;
    }
    int4 *rec = items ? reinterpret_cast<int4 *>(items) + 1 + excli : nullptr;
    for (int j = 0; j < ni; j++) {
      const int r = j * BT;
      rec[j] = make_int4(tid, excl + r, c - r < BT ? c - r : BT, ni > 1 ? MOE_ITEM_SPLIT : 0);
    }
    int4 *rec2 = items2 ? reinterpret_cast<int4 *>(items2) + 1 + excli2 : nullptr;
    for (int j = 0; j < ni2; j++) {
      const int r = j * BT2;
      rec2[j] = make_int4(tid, excl + r, c - r < BT2 ? c - r : BT2, ni2 > 1 ? MOE_ITEM_SPLIT : 0);
    }
  }
  if (tid == 1023) {  // thread 1023's inclusive sums are the totals
    offsets[E] = base + v;
    tot[0] = basei + vi;
    tot[1] = basei2 + vi2;
  }
  __syncthreads();
  if (items) {
    const int ns = shared ? (T + BT - 1) / BT : 0;
    for (int j = tid; j < ns; j += 1024) {
      const int r = j * BT;
      reinterpret_cast<int4 *>(items)[1 + tot[0] + j] =
          make_int4(E, P + r, T - r < BT ? T - r : BT, MOE_ITEM_SHARED | (ns > 1 ? MOE_ITEM_SPLIT : 0));
    }
    if (tid == 0) items[0] = tot[0] + ns;
  }
  if (items2) {
    const int ns = shared ? (T + BT2 - 1) / BT2 : 0;
    for (int j = tid; j < ns; j += 1024) {
      const int r = j * BT2;
      reinterpret_cast<int4 *>(items2)[1 + tot[1] + j] =
          make_int4(E, P + r, T - r < BT2 ? T - r : BT2, MOE_ITEM_SHARED | (ns > 1 ? MOE_ITEM_SPLIT : 0));
    }
    if (tid == 0) items2[0] = tot[1] + ns;
  }
  // pass 2: row of a pair = wc[w][e] + rank (the lanes of one id read wc
  // before the last of them advances it)
  auto place = [&](int p, int e, int rank, bool last) {
    const bool ok = e >= 0 && e < E;
    if (ok) {
      const int pos = wc[wave][e] + rank;
      perm[pos] = p;
      if (inv) inv[p] = pos;
    } else if (p < p_hi && inv) {
      inv[p] = -1;  // dropped pair: no grouped row
    }
    if (ok && last) wc[wave][e] += (uint16_t)(rank + 1);
  };
  if (cached) {
#pragma unroll
    for (int it = 0; it < MOE_GROUP_IT; it++) {
      if (p_lo + 64 * it >= p_hi) break;
      place(p_lo + 64 * it + lane, ev[it], (int)(rl[it] & 0xffffu), (rl[it] >> 16) != 0);
    }
  } else {
    for (int pb = p_lo; pb < p_hi; pb += 64) {
      const int p = pb + lane;
      const int e = p < p_hi ? ids[p] : -1;
      const uint64_t m = same_id_lanes(e, e >= 0 && e < E);
      place(p, e, __popcll(m & below), !(m & ~upto));
    }
  }
}

// ---------------------------------------------------------------------------
// k_group for calls of at most MOE_GF_PAIRS pairs, on one wave: the same
// outputs (counts and offsets only when counts != NULL).  The pairs are
// NPL = ceil(P / 64) chunks of 64 (at most 2), lane l holding pair 64*i + l
// of each chunk i.
//   1. ballots of each chunk's valid lanes and of each id bit;
//   2. a pair walks each chunk's ballots from the top id bit down, which
//      gives the chunk's lanes with its id (eq) and with a smaller id (lt);
//      row = (valid pairs with a smaller id) + (pairs with its id before it)
//      is k_group's grouped row: experts ascending, pairs ascending within
//      an expert;
//   3. the first pair of an expert holds the expert's item count ceil(c/BT);
//      ballots of the bits of those counts give every first pair the items
//      of all smaller experts, i.e. the index of its first item.
// All in registers: no LDS, no barrier, no table over the experts and no
// scan, and short executed code (a launch this small is bound by latency,
// instruction fetch included).  Workgroups 1..: Q8_0 of x as in k_group,
// MOE_GF_QBLOCKS blocks each.
// grid 1 + ceil(n_xblocks / MOE_GF_QBLOCKS), 256 threads (wave 0 of
// workgroup 0 groups).
#define MOE_GF_NPL 2
#define MOE_GF_PAIRS (64 * MOE_GF_NPL)
#define MOE_GF_QBLOCKS 128

// Bits needed for values in [0, n] (n >= 0).
__device__ __forceinline__ int gf_bits(int n) { return n > 0 ? 32 - __clz(n) : 1; }

// Ballots of one chunk: bb[b] = lanes whose valid id has bit b set, v =
// lanes with a valid id (ids below 2^10).
__device__ __forceinline__ void chunk_ballots(int e, bool ok, uint64_t (&bb)[10], uint64_t &v) {
  v = __ballot(ok);
#pragma unroll
  for (int b = 0; b < 10; b++) bb[b] = __ballot(ok && ((e >> b) & 1));
}

// The lanes of a chunk with id e (eq) and with a valid smaller id (lt), from
// the chunk's ballots (0 <= e < 2^10).  Straight-line code: bits above the
// largest id only cost their 9 instructions, less than a branch around them.
__device__ __forceinline__ void chunk_rank(const uint64_t (&bb)[10], uint64_t v, int e, uint64_t &eq, uint64_t &lt) {
  eq = v;
  lt = 0ull;
#pragma unroll
  for (int b = 9; b >= 0; b--) {
    const uint64_t B = bb[b];
    const bool one = (e >> b) & 1;
    lt |= one ? (eq & ~B) : 0ull;
    eq &= one ? B : ~B;
  }
}

template <int NPL>
__device__ __forceinline__ void group_one_wave(const int32_t *__restrict__ ids, int P, int E, int T, int shared,
                                               int BT, int32_t *__restrict__ counts, int32_t *__restrict__ offsets,
                                               int32_t *__restrict__ perm, int32_t *__restrict__ inv,
                                               int32_t *__restrict__ items, int BT2, int32_t *__restrict__ items2) {
  const int lane = threadIdx.x;
  int e[NPL];
  bool ok[NPL];
#pragma unroll
  for (int i = 0; i < NPL; i++) {
    e[i] = 64 * i + lane < P ? ids[64 * i + lane] : -1;
    ok[i] = e[i] >= 0 && e[i] < E;
  }
  const uint64_t below = (1ull << lane) - 1ull;
  uint64_t ltm[NPL][NPL];  // [own pair][chunk]
  int less[NPL], before[NPL], cnt[NPL];
#pragma unroll
  for (int i = 0; i < NPL; i++) less[i] = before[i] = cnt[i] = 0;
#pragma unroll
  for (int c = 0; c < NPL; c++) {  // one chunk's ballots alive at a time
    uint64_t bb[10], v;
    chunk_ballots(e[c], ok[c], bb, v);
#pragma unroll
    for (int i = 0; i < NPL; i++) {
      uint64_t eq, lt;
      chunk_rank(bb, v, ok[i] ? e[i] : 0, eq, lt);
      ltm[i][c] = lt;
      less[i] += __popcll(lt);
      cnt[i] += __popcll(eq);
      before[i] += c < i ? __popcll(eq) : (c == i ? __popcll(eq & below) : 0);
    }
  }
#pragma unroll
  for (int i = 0; i < NPL; i++) {
    const int p = 64 * i + lane;
    if (ok[i]) {
      perm[less[i] + before[i]] = p;
      if (inv) inv[p] = less[i] + before[i];
    } else if (inv && p < P) {
      inv[p] = -1;  // dropped pair: no grouped row
    }
  }
  if (counts) {  // per expert: pairs with its id, valid pairs with a smaller id
    uint64_t cb[NPL][10], cv[NPL];  // the ballots are taken with every lane active, before the loop
#pragma unroll
    for (int c = 0; c < NPL; c++) chunk_ballots(e[c], ok[c], cb[c], cv[c]);
    for (int ex = lane; ex < E; ex += 64) {
      int ce = 0, le = 0;
#pragma unroll
      for (int c = 0; c < NPL; c++) {
        uint64_t q, l;
        chunk_rank(cb[c], cv[c], ex, q, l);
        ce += __popcll(q);
        le += __popcll(l);
      }
      counts[ex] = ce;
      offsets[ex] = le;
    }
    int n = 0;
#pragma unroll
    for (int c = 0; c < NPL; c++) n += __popcll(__ballot(ok[c]));
    if (lane == 0) offsets[E] = n;
  }
  for (int li = 0; li < 2; li++) {
    int32_t *list = li ? items2 : items;
    if (!list) continue;
    const int bt = li ? BT2 : BT;
    int n[NPL], base[NPL], tot = 0;
#pragma unroll
    for (int i = 0; i < NPL; i++) {
      n[i] = ok[i] && before[i] == 0 ? (cnt[i] + bt - 1) / bt : 0;  // first pair of its expert
      base[i] = 0;
    }
    bool big = false;  // an expert of more than one item on this lane
#pragma unroll
    for (int i = 0; i < NPL; i++) big |= n[i] > 1;
    // counts of 0 or 1 everywhere (the common case): one bit; else every bit a count can have
    const int nbits = __ballot(big) ? gf_bits((P + bt - 1) / bt) : 1;
    for (int b = 0; b < nbits; b++) {
#pragma unroll
      for (int c = 0; c < NPL; c++) {
        const uint64_t m = __ballot((n[c] >> b) & 1);
        tot += __popcll(m) << b;
#pragma unroll
        for (int i = 0; i < NPL; i++) base[i] += __popcll(ltm[i][c] & m) << b;
      }
    }
    int4 *rec = reinterpret_cast<int4 *>(list) + 1;
#pragma unroll
    for (int i = 0; i < NPL; i++)
      for (int j = 0; j < n[i]; j++) {
        const int r = j * bt;
        rec[base[i] + j] = make_int4(e[i], less[i] + r, cnt[i] - r < bt ? cnt[i] - r : bt, n[i] > 1 ? MOE_ITEM_SPLIT : 0);
      }
    const int ns = shared ? (T + bt - 1) / bt : 0;  // the shared expert's items follow the routed ones
    for (int j = lane; j < ns; j += 64) {
      const int r = j * bt;
      rec[tot + j] = make_int4(E, P + r, T - r < bt ? T - r : bt, MOE_ITEM_SHARED | (ns > 1 ? MOE_ITEM_SPLIT : 0));
    }
    if (lane == 0) list[0] = tot + ns;
  }
}

__global__ __launch_bounds__(256) void k_group_few(const int32_t *__restrict__ ids, int P, int E, int T, int shared,
                                                   int BT, int32_t *__restrict__ counts,
                                                   int32_t *__restrict__ offsets, int32_t *__restrict__ perm,
                                                   int32_t *__restrict__ inv, int32_t *__restrict__ items,
                                                   const float *__restrict__ x, int n_xblocks,
                                                   uint32_t *__restrict__ xq, float *__restrict__ xd, int BT2,
                                                   int32_t *__restrict__ items2) {
  if (blockIdx.x > 0) {
    const int b0 = (blockIdx.x - 1) * MOE_GF_QBLOCKS;
    const int nb = n_xblocks - b0 < MOE_GF_QBLOCKS ? n_xblocks - b0 : MOE_GF_QBLOCKS;
    if (nb > 0) stage_quant(x + (size_t)b0 * MOE_QK, nb, xq + (size_t)b0 * MOE_XSW, xd + b0, threadIdx.x, 256);
    return;
  }
  if (threadIdx.x >= 64) return;
  if (P <= 64)
    group_one_wave<1>(ids, P, E, T, shared, BT, counts, offsets, perm, inv, items, BT2, items2);
  else
    group_one_wave<2>(ids, P, E, T, shared, BT, counts, offsets, perm, inv, items, BT2, items2);
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

__device__ __forceinline__ float4 add4_rn(float4 a, float4 b) {
  return make_float4(__fadd_rn(a.x, b.x), __fadd_rn(a.y, b.y), __fadd_rn(a.z, b.z), __fadd_rn(a.w, b.w));
}

// k_combine with one thread per 4 consecutive columns (H % 4 == 0, out
// 16-byte aligned); grid ceil(T*H/4 / 256).
__global__ __launch_bounds__(256) void k_combine4(const float *__restrict__ y,
                                                 const int32_t *__restrict__ inv, int T, int k,
                                                 int H, int shared, int per_slot,
                                                 float *__restrict__ out) {
  const int H4 = H / 4;
  const size_t i = (size_t)blockIdx.x * 256u + threadIdx.x;
  if (i >= (size_t)T * H4) return;
  const int t = (int)(i / H4), c = (int)(i % H4);
  const int P = T * k;
  const float4 *y4 = reinterpret_cast<const float4 *>(y);
  float4 *o4 = reinterpret_cast<float4 *>(out);
  const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  // a negative row marks a pair whose expert id was out of range: it contributes 0
  if (per_slot) {
    for (int s = 0; s < k; s++) {
      const int r = inv ? inv[t * k + s] : t * k + s;
      o4[((size_t)t * k + s) * H4 + c] = r >= 0 ? y4[(size_t)r * H4 + c] : z;
    }
    return;
  }
  if (H4 % 256 == 0 && k <= 16 && inv) {
    // one token per workgroup: its k grouped rows read first (uniform) and
    // every row's float4 loaded before the sum (same order, same bits)
    const int tu = __builtin_amdgcn_readfirstlane(t);
    int r[16];
#pragma unroll
    for (int s = 0; s < 16; s++)
      if (s < k) r[s] = __builtin_amdgcn_readfirstlane(inv[tu * k + s]);
    float4 v[16];
#pragma unroll
    for (int s = 0; s < 16; s++)
      if (s < k) v[s] = r[s] >= 0 ? y4[(size_t)r[s] * H4 + c] : z;
    const float4 vs = shared ? y4[((size_t)P + tu) * H4 + c] : z;
    float4 acc = v[0];
#pragma unroll
    for (int s = 1; s < 16; s++)
      if (s < k) acc = add4_rn(acc, v[s]);
    if (shared) acc = add4_rn(acc, vs);
    o4[i] = acc;
    return;
  }
  const int r0 = inv ? inv[t * k] : t * k;
  float4 acc = r0 >= 0 ? y4[(size_t)r0 * H4 + c] : z;
#pragma unroll 8
  for (int s = 1; s < k; s++) {
    const int r = inv ? inv[t * k + s] : t * k + s;
    acc = add4_rn(acc, r >= 0 ? y4[(size_t)r * H4 + c] : z);
  }
  if (shared) acc = add4_rn(acc, y4[((size_t)P + t) * H4 + c]);
  o4[i] = acc;
}
