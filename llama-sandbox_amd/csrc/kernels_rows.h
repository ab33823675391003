// kernels_rows.h -- the expert vecmat kernels (decode and small-batch grouped).
//
// Weight layout in HBM (built by the repack/generator kernels): the rows of a
// matrix are taken in groups of 64 (one row per lane), and within a group the
// 16-byte nibble payloads are stored block-major:
//   nib[grp][b][l]        uint4   block b (32 weights) of row 64*grp + l
//   sc [grp][b/4][l][b%4] uint8   its E8M0 exponent (4 blocks per dword)
// where grp = matrix * (R/64) + row/64 over all experts of a tensor.  A wave
// reading block b of a row group loads 64 x 16 B = 1 KiB contiguous, and one
// dword per lane carries the exponents of 4 blocks.  The nibble bytes keep
// ggml's order (byte j = element j | element j+16 << 4), so activations are
// stored as fp16 pairs (q_j, q_{j+16}) to meet them.
//
// Work mapping: lane <-> row, so a row's dot product never crosses lanes.
// The reduction dimension K (in blocks) is split over the waves of a
// workgroup; each wave streams its K-chunk of 64 rows with the next 4 blocks'
// loads in flight while it computes the current 4, against activations
// staged in LDS (read by all lanes at one address: a broadcast).  Partials
// are summed over waves in wave order through LDS, so results do not depend
// on timing.
//
// Arithmetic (ggml-cpu's MXFP4 x Q8_0): per block, isum = sum of e2m1 code
// values x int8 activations, exact (v_cvt_scalef32_pk_f16_fp4 -> fp16 pairs,
// v_dot2_f32_f16 -> f32, all terms small integers / halves); the block adds
// fp16(d_x) * 2^(e-127) * isum/2 to an f32 accumulator.
#pragma once

#include "device_common.h"

#define MOE_RG 64         // rows per row group (= lanes per wave)
#define MOE_GU_WAVES 8    // waves per gate/up workgroup (K split 8 ways)
#define MOE_DN_WAVES 4    // waves per down workgroup (K split 4 ways)

// ---------------------------------------------------------------------------
// Split of KQ = KB/4 block groups over NW waves: wave w owns [q0, q1).
__device__ __forceinline__ void wave_groups(int KQ, int NW, int w, int &q0, int &q1) {
  q0 = (int)(((long)KQ * w) / NW);
  q1 = (int)(((long)KQ * (w + 1)) / NW);
}

// Largest number of blocks any wave owns (host and device agree on it).
__host__ __device__ __forceinline__ int max_wave_blocks(int KB, int NW) {
  const int KQ = KB / 4;
  return 4 * ((KQ + NW - 1) / NW);
}

// ---------------------------------------------------------------------------
// Q8_0 of nb blocks of one f32 row into LDS, ggml's x86 rounding:
// amax per block, d = fp16(amax / 127), q = rint(x * (127 / amax)).
// Two lanes per block: lane half 0 takes elements 0-7 and 16-23, half 1
// takes 8-15 and 24-31, so each lane forms its 8 (q_j, q_{j+16}) pairs.
// q_s: [nb][16] packed fp16 pairs; d_s: [nb] fp16(d) as f32.
__device__ __forceinline__ void stage_quantize(const float *__restrict__ xrow, int nb, uint32_t *q_s,
                                               float *d_s, int lane) {
  const int half = lane & 1;
  for (int bb = lane >> 1; bb < nb; bb += 32) {
    const float4 *xb = reinterpret_cast<const float4 *>(xrow + (size_t)bb * MOE_QK + 8 * half);
    const float4 a0 = xb[0], a1 = xb[1], c0 = xb[4], c1 = xb[5];
    const float lo[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const float hi[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) amax = fmaxf(amax, fmaxf(fabsf(lo[i]), fabsf(hi[i])));
    amax = fmaxf(amax, dpp_f<0xB1>(amax));  // partner lane (lane ^ 1) holds the other half
    uint32_t pk[8];
#pragma unroll
    for (int i = 0; i < 8; i++) pk[i] = pack_f16x2(q8_code(lo[i], amax), q8_code(hi[i], amax));
    uint4 *dst = reinterpret_cast<uint4 *>(q_s + (size_t)bb * 16 + 8 * half);
    dst[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    dst[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
    if (!half) d_s[bb] = (float)q8_scale_f16(amax);
  }
}

// Copy nb pre-quantized blocks (global [nb][16] pairs + [nb] scales) into LDS.
__device__ __forceinline__ void stage_copy(const uint32_t *__restrict__ q, const float *__restrict__ d, int nb,
                                           uint32_t *q_s, float *d_s, int lane) {
  for (int i = lane; i < nb * 4; i += 64)
    reinterpret_cast<uint4 *>(q_s)[i] = reinterpret_cast<const uint4 *>(q)[i];
  for (int i = lane; i < nb; i += 64) d_s[i] = d[i];
}

// Zero nb staged blocks (token slots of a partial batch).
__device__ __forceinline__ void stage_zero(int nb, uint32_t *q_s, float *d_s, int lane) {
  for (int i = lane; i < nb * 4; i += 64) reinterpret_cast<uint4 *>(q_s)[i] = make_uint4(0u, 0u, 0u, 0u);
  for (int i = lane; i < nb; i += 64) d_s[i] = 0.0f;
}

// ---------------------------------------------------------------------------
// Loads of one group of 4 blocks for NM matrices (16 B payload per block per
// lane, one exponent dword per lane).  Weights are read once per call, so the
// loads are nontemporal (they bypass the caches' normal allocation).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <int NM>
struct wgroup {
  u32x4_t w[NM][4];
  uint32_t e[NM];
};

template <int NM>
__device__ __forceinline__ void load_group(wgroup<NM> &g, const uint4 *const (&nib)[NM],
                                           const uint32_t *const (&sc)[NM], int q, int lane) {
#pragma unroll
  for (int m = 0; m < NM; m++) {
#pragma unroll
    for (int i = 0; i < 4; i++)
      g.w[m][i] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4_t *>(nib[m] + (size_t)(4 * q + i) * MOE_RG + lane));
    g.e[m] = __builtin_nontemporal_load(sc[m] + (size_t)q * MOE_RG + lane);
  }
}

// acc[m][t] += the 4 blocks of group g (local group index lq) against the
// NT staged tokens.
template <int NM, int NT>
__device__ __forceinline__ void dot_group(const wgroup<NM> &g, int lq, const uint32_t *q_s, const float *d_s,
                                          int NBW, float (&acc)[NM][NT]) {
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int lb = 4 * lq + i;
    float dot[NM][NT];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int t = 0; t < NT; t++) dot[m][t] = 0.0f;
#pragma unroll
    for (int dw = 0; dw < 4; dw++) {
      f16x2_t w[NM][4];
#pragma unroll
      for (int m = 0; m < NM; m++) {
        const uint32_t v = g.w[m][i][dw];
        w[m][0] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, 1.0f, 0);
        w[m][1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, 1.0f, 1);
        w[m][2] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, 1.0f, 2);
        w[m][3] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, 1.0f, 3);
      }
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const uint4 a = reinterpret_cast<const uint4 *>(q_s + (size_t)(t * NBW + lb) * 16)[dw];
#pragma unroll
        for (int m = 0; m < NM; m++) {
          float s = dot[m][t];
          s = __builtin_amdgcn_fdot2(w[m][0], __builtin_bit_cast(f16x2_t, a.x), s, false);
          s = __builtin_amdgcn_fdot2(w[m][1], __builtin_bit_cast(f16x2_t, a.y), s, false);
          s = __builtin_amdgcn_fdot2(w[m][2], __builtin_bit_cast(f16x2_t, a.z), s, false);
          s = __builtin_amdgcn_fdot2(w[m][3], __builtin_bit_cast(f16x2_t, a.w), s, false);
          dot[m][t] = s;
        }
      }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const float xd = d_s[t * NBW + lb];
#pragma unroll
      for (int m = 0; m < NM; m++) {
        const uint32_t e = (g.e[m] >> (8 * i)) & 0xFFu;
        acc[m][t] = fmaf(scale_e8m0(xd, e), dot[m][t], acc[m][t]);
      }
    }
  }
}

// One wave: NM matrices (same row group, same K) x NT staged tokens over nq
// groups of 4 blocks.  nib[m] / sc[m] point at the wave's first block of the
// row group; activation block lb of token t is at q_s + (t*NBW + lb)*16 and
// d_s + t*NBW + lb.  A ring of D load buffers keeps D-1 groups in flight
// while one is computed; the loads are always issued (past the end they
// re-read the last group, an L2 hit), so the wait before each group's math
// covers only that group's own loads.  ring_prime() issues groups 0..D-2 and
// is called by the kernel before it stages the activations, so the first
// weight loads overlap the staging.
template <int NM, int D>
__device__ __forceinline__ void ring_prime(wgroup<NM> (&buf)[D], const uint4 *const (&nib)[NM],
                                           const uint32_t *const (&sc)[NM], int nq, int lane) {
  if (nq <= 0) return;
#pragma unroll
  for (int d = 0; d < D - 1; d++) load_group<NM>(buf[d], nib, sc, d < nq ? d : nq - 1, lane);
}

template <int NM, int NT, int D>
__device__ __forceinline__ void rows_dot(wgroup<NM> (&buf)[D], const uint4 *const (&nib)[NM],
                                         const uint32_t *const (&sc)[NM], int nq, const uint32_t *q_s,
                                         const float *d_s, int NBW, int lane, float (&acc)[NM][NT]) {
#pragma unroll
  for (int m = 0; m < NM; m++)
#pragma unroll
    for (int t = 0; t < NT; t++) acc[m][t] = 0.0f;
  if (nq <= 0) return;
  for (int q0 = 0;; q0 += D) {
#pragma unroll
    for (int d = 0; d < D; d++) {
      const int q = q0 + d, qn = q + D - 1;
      load_group<NM>(buf[(d + D - 1) % D], nib, sc, qn < nq ? qn : nq - 1, lane);
      __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the math
      dot_group<NM, NT>(buf[d], q, q_s, d_s, NBW, acc);
      if (q + 1 >= nq) return;
    }
  }
}

// ---------------------------------------------------------------------------
// Which expert matrix and which rows workgroup column y works on.
//   decode (T == 1): y = slot s; s < k -> expert ids[s], s == k -> shared
//     expert (matrix E); one token; h/y row index = s.
//   grouped: y < act[0] -> expert act[1+y], h/y rows offsets[e]..offsets[e+1]
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

__device__ __forceinline__ int token_of(bool grouped, const unit_t &u, int hrow, const int32_t *__restrict__ perm,
                                        int k, int P) {
  if (!grouped) return 0;
  return u.shared ? hrow - P : perm[hrow] / k;
}

// ---------------------------------------------------------------------------
// gate/up -> clamp -> SwiGLU -> Q8_0(h).  grid (F/64, ny), MOE_GU_WAVES waves.
// Dynamic LDS: MOE_GU_WAVES * NT * NBW * 68 B (activations) + the partials.
template <int NT>
__global__ __launch_bounds__(64 * MOE_GU_WAVES) __attribute__((amdgpu_waves_per_eu(NT == 1 ? 4 : 2))) void k_gate_up(
    const uint4 *__restrict__ nib_g, const uint4 *__restrict__ nib_u, const uint32_t *__restrict__ sc_g,
    const uint32_t *__restrict__ sc_u, const float *__restrict__ x, int grouped,
    const int32_t *__restrict__ ids, const int32_t *__restrict__ offsets, const int32_t *__restrict__ perm,
    const int32_t *__restrict__ act, int k, int E, int shared, int T, int F, int H, float clamp,
    uint32_t *__restrict__ hq, float *__restrict__ hd, float *__restrict__ htap) {
  extern __shared__ __align__(16) uint32_t lds[];
  const int KB = H / MOE_QK, KQ = KB / 4, NBW = max_wave_blocks(KB, MOE_GU_WAVES);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int P = T * k;
  const unit_t u = unit_of(blockIdx.y, gridDim.y, grouped, ids, offsets, act, k, E, shared, P, T);
  if (!u.valid && grouped) return;
  int q0, q1;
  wave_groups(KQ, MOE_GU_WAVES, wave, q0, q1);
  const int nbw = 4 * (q1 - q0);
  uint32_t *q_s = lds + (size_t)wave * NT * NBW * 16;
  float *d_s = reinterpret_cast<float *>(lds + (size_t)MOE_GU_WAVES * NT * NBW * 16) + (size_t)wave * NT * NBW;
  float *red = reinterpret_cast<float *>(lds + (size_t)MOE_GU_WAVES * NT * NBW * 17);  // [waves][2][NT][64]

  const int G = F / MOE_RG;
  const size_t grp = (size_t)u.mat * G + blockIdx.x;
  const uint4 *const nibs[2] = {nib_g + grp * KB * MOE_RG + (size_t)4 * q0 * MOE_RG,
                                nib_u + grp * KB * MOE_RG + (size_t)4 * q0 * MOE_RG};
  const uint32_t *const scs[2] = {sc_g + grp * KQ * MOE_RG + (size_t)q0 * MOE_RG,
                                  sc_u + grp * KQ * MOE_RG + (size_t)q0 * MOE_RG};

  const int nq = q1 - q0;
  for (int i0 = 0; i0 < u.nrows; i0 += NT) {
    const int nt = u.nrows - i0 < NT ? u.nrows - i0 : NT;
    wgroup<2> ring[2];
    ring_prime<2, 2>(ring, nibs, scs, nq, lane);
    // stage this wave's K-chunk of the batch's activations
#pragma unroll
    for (int t = 0; t < NT; t++) {
      if (t < nt && u.valid) {
        const int tok = token_of(grouped, u, u.row0 + i0 + t, perm, k, P);
        stage_quantize(x + (size_t)tok * H + (size_t)4 * q0 * MOE_QK, nbw, q_s + (size_t)t * NBW * 16,
                       d_s + (size_t)t * NBW, lane);
      } else {
        stage_zero(nbw, q_s + (size_t)t * NBW * 16, d_s + (size_t)t * NBW, lane);
      }
    }
    float acc[2][NT];
    rows_dot<2, NT, 2>(ring, nibs, scs, nq, q_s, d_s, NBW, lane, acc);
#pragma unroll
    for (int m = 0; m < 2; m++)
#pragma unroll
      for (int t = 0; t < NT; t++) red[((wave * 2 + m) * NT + t) * MOE_RG + lane] = acc[m][t];
    __syncthreads();
    // epilogue: wave t finishes token t of the batch
    if (wave < nt) {
      const int t = wave;
      float g = 0.0f, up = 0.0f;
      for (int w = 0; w < MOE_GU_WAVES; w++) {
        g += red[((w * 2 + 0) * NT + t) * MOE_RG + lane];
        up += red[((w * 2 + 1) * NT + t) * MOE_RG + lane];
      }
      if (clamp > 1e-6f) {  // deepseek4 order: up symmetric, gate one-sided, before SiLU
        up = fmaxf(fminf(up, clamp), -clamp);
        g = fminf(g, clamp);
      }
      const float h = u.valid ? __fmul_rn(__fdiv_rn(g, 1.0f + expf(-g)), up) : 0.0f;
      const int hrow = u.row0 + i0 + t;
      // Q8_0 over each 32-lane half (two h blocks per row group)
      float amax = fabsf(h);
      amax = fmaxf(amax, dpp_f<0xB1>(amax));
      amax = fmaxf(amax, dpp_f<0x4E>(amax));
      amax = fmaxf(amax, dpp_f<0x141>(amax));
      amax = fmaxf(amax, dpp_f<0x140>(amax));
      const float am_lo = fmaxf(readlane_f(amax, 0), readlane_f(amax, 16));
      const float am_hi = fmaxf(readlane_f(amax, 32), readlane_f(amax, 48));
      const float am = lane < 32 ? am_lo : am_hi;
      const float qv = q8_code(h, am);
      const float qhi = __shfl_down(qv, 16);
      const size_t blk = (size_t)hrow * (size_t)(F / MOE_QK) + 2 * blockIdx.x + (lane >> 5);
      if ((lane & 31) < 16) hq[blk * 16 + (lane & 15)] = pack_f16x2(qv, qhi);
      if ((lane & 31) == 0) hd[blk] = (float)q8_scale_f16(am);
      if (htap) htap[(size_t)hrow * F + blockIdx.x * MOE_RG + lane] = h;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// down (x router weight).  grid (H/64, ny), MOE_DN_WAVES waves.
// y[hrow][H] = (down_row . h[hrow]) * w   (w = wts[pair] for routed rows in
// grouped mode, wts[s] in decode mode, none for the shared expert).
template <int NT>
__global__ __launch_bounds__(64 * MOE_DN_WAVES) void k_down(
    const uint4 *__restrict__ nib_d, const uint32_t *__restrict__ sc_d, const uint32_t *__restrict__ hq,
    const float *__restrict__ hd, int grouped, const int32_t *__restrict__ ids,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ perm, const int32_t *__restrict__ act,
    const float *__restrict__ wts, int k, int E, int shared, int T, int F, int H, float *__restrict__ y) {
  extern __shared__ __align__(16) uint32_t lds[];
  const int KB = F / MOE_QK, KQ = KB / 4, NBW = max_wave_blocks(KB, MOE_DN_WAVES);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int P = T * k;
  const unit_t u = unit_of(blockIdx.y, gridDim.y, grouped, ids, offsets, act, k, E, shared, P, T);
  if (!u.valid && grouped) return;
  int q0, q1;
  wave_groups(KQ, MOE_DN_WAVES, wave, q0, q1);
  const int nbw = 4 * (q1 - q0);
  uint32_t *q_s = lds + (size_t)wave * NT * NBW * 16;
  float *d_s = reinterpret_cast<float *>(lds + (size_t)MOE_DN_WAVES * NT * NBW * 16) + (size_t)wave * NT * NBW;
  float *red = reinterpret_cast<float *>(lds + (size_t)MOE_DN_WAVES * NT * NBW * 17);  // [waves][NT][64]

  const int G = H / MOE_RG;
  const size_t grp = (size_t)u.mat * G + blockIdx.x;
  const uint4 *const nibs[1] = {nib_d + grp * KB * MOE_RG + (size_t)4 * q0 * MOE_RG};
  const uint32_t *const scs[1] = {sc_d + grp * KQ * MOE_RG + (size_t)q0 * MOE_RG};

  const int nq = q1 - q0;
  for (int i0 = 0; i0 < u.nrows; i0 += NT) {
    const int nt = u.nrows - i0 < NT ? u.nrows - i0 : NT;
    wgroup<1> ring[2];
    ring_prime<1, 2>(ring, nibs, scs, nq, lane);
#pragma unroll
    for (int t = 0; t < NT; t++) {
      if (t < nt && u.valid) {
        const size_t hrow = (size_t)(u.row0 + i0 + t);
        stage_copy(hq + (hrow * KB + 4 * q0) * 16, hd + hrow * KB + 4 * q0, nbw, q_s + (size_t)t * NBW * 16,
                   d_s + (size_t)t * NBW, lane);
      } else {
        stage_zero(nbw, q_s + (size_t)t * NBW * 16, d_s + (size_t)t * NBW, lane);
      }
    }
    float acc[1][NT];
    rows_dot<1, NT, 2>(ring, nibs, scs, nq, q_s, d_s, NBW, lane, acc);
#pragma unroll
    for (int t = 0; t < NT; t++) red[(wave * NT + t) * MOE_RG + lane] = acc[0][t];
    __syncthreads();
    if (wave < nt) {
      const int t = wave;
      float v = 0.0f;
      for (int w = 0; w < MOE_DN_WAVES; w++) v += red[(w * NT + t) * MOE_RG + lane];
      const int hrow = u.row0 + i0 + t;
      if (!u.shared) {
        const float wt = grouped ? wts[perm[hrow]] : wts[hrow];
        v = __fmul_rn(v, wt);
      }
      if (!u.valid) v = 0.0f;
      y[(size_t)hrow * H + (size_t)blockIdx.x * MOE_RG + lane] = v;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Decode gate/up (T == 1) as split-K one-wave workgroups.
//
// A decode call is small (the 9 touched experts of a V3 layer) and HBM-bound
// only if every CU streams the same share: a workgroup per (slot, row group)
// leaves the chip unevenly loaded (288 units on 256 CUs).  So the reduction
// K of every (slot, row group) unit is cut into C chunks, one single-wave
// workgroup each (2304 equal workgroups for V3 gate/up).
// Each writes its 64 partial sums; the last workgroup of a unit to finish
// adds the chunks in chunk order and finishes the unit, then resets the
// ticket for the next call.  No workgroup ever waits on another, and the
// sums do not depend on arrival order.
//
// Visibility without cache write-backs: every access to the shared partials
// and tickets is an agent-scope atomic (stores and loads carry sc1, so they
// are coherent across the XCDs' L2s on their own).  A chunk's stores have
// completed (s_waitcnt vmcnt(0)) before its ticket increment is issued, and
// the last chunk's loads are issued after its increment has returned, so the
// last chunk reads every other chunk's partials.  (An acq_rel ticket would
// also be correct, but its release writes back the whole L2 of the XCD --
// buffer_wbl2 -- once per workgroup, which measured 4x slower.)
#define MOE_DEC_DEPTH 3  // groups of 4 blocks in the load ring

__device__ __forceinline__ void store_shared(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// All of this wave's stores complete, then lane 0 takes a ticket; the
// ticket's previous value is returned wave-uniform (an SGPR via readfirstlane,
// read while every lane is active), so branches on it are scalar branches.
__device__ __forceinline__ int ticket_take(int32_t *ctr, int lane) {
  __builtin_amdgcn_s_waitcnt(0);
  int t = 0;
  if (lane == 0) t = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return __builtin_amdgcn_readfirstlane(t);
}

__device__ __forceinline__ float load_acquired(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// gate/up -> SwiGLU -> Q8_0(h).  grid S*G*C (G = F/64), 64 threads;
// block id = (s*G + g)*C + c.  part: [S*G][C][2][64] f32, ctr: [S*G].
__global__ __launch_bounds__(64) void k_gate_up_dec(
    const uint4 *__restrict__ nib_g, const uint4 *__restrict__ nib_u, const uint32_t *__restrict__ sc_g,
    const uint32_t *__restrict__ sc_u, const float *__restrict__ x, const int32_t *__restrict__ ids, int k, int E,
    int F, int H, int C, float clamp, float *__restrict__ part, int32_t *__restrict__ ctr,
    uint32_t *__restrict__ hq, float *__restrict__ hd, float *__restrict__ htap) {
  extern __shared__ __align__(16) uint32_t lds[];
  const int KB = H / MOE_QK, KQ = KB / 4, G = F / MOE_RG;
  const int lane = threadIdx.x;
  const int unit = blockIdx.x / C, c = blockIdx.x - unit * C;
  const int s = unit / G, g = unit - s * G;
  int e = s < k ? ids[s] : E;
  const bool valid = s >= k || (unsigned)e < (unsigned)E;  // an out-of-range id reads nothing, yields 0
  e = valid ? e : 0;
  int q0, q1;
  wave_groups(KQ, C, c, q0, q1);
  const int nq = q1 - q0;
  const size_t grp = (size_t)e * G + g;
  const uint4 *const nibs[2] = {nib_g + (grp * KB + 4 * q0) * MOE_RG, nib_u + (grp * KB + 4 * q0) * MOE_RG};
  const uint32_t *const scs[2] = {sc_g + (grp * KQ + q0) * MOE_RG, sc_u + (grp * KQ + q0) * MOE_RG};
  wgroup<2> ring[MOE_DEC_DEPTH];
  ring_prime<2, MOE_DEC_DEPTH>(ring, nibs, scs, nq, lane);
  uint32_t *q_s = lds;
  float *d_s = reinterpret_cast<float *>(lds + (size_t)4 * nq * 16);
  stage_quantize(x + (size_t)4 * q0 * MOE_QK, 4 * nq, q_s, d_s, lane);
  __syncthreads();
  float acc[2][1];
  rows_dot<2, 1, MOE_DEC_DEPTH>(ring, nibs, scs, nq, q_s, d_s, 0, lane, acc);
  float *pp = part + ((size_t)unit * C + c) * 2 * MOE_RG;
  store_shared(pp + lane, valid ? acc[0][0] : 0.0f);
  store_shared(pp + MOE_RG + lane, valid ? acc[1][0] : 0.0f);
  if (ticket_take(ctr + unit, lane) != C - 1) return;
  // last chunk of this unit: sum the chunks in order, clamp, SwiGLU, Q8_0
  float gs = 0.0f, us = 0.0f;
  const float *pu = part + (size_t)unit * C * 2 * MOE_RG;
  for (int cc = 0; cc < C; cc++) {
    gs += load_acquired(pu + (size_t)cc * 2 * MOE_RG + lane);
    us += load_acquired(pu + (size_t)cc * 2 * MOE_RG + MOE_RG + lane);
  }
  if (lane == 0) __hip_atomic_store(ctr + unit, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (clamp > 1e-6f) {  // deepseek4 order: up symmetric, gate one-sided, before SiLU
    us = fmaxf(fminf(us, clamp), -clamp);
    gs = fminf(gs, clamp);
  }
  const float h = valid ? __fmul_rn(__fdiv_rn(gs, 1.0f + expf(-gs)), us) : 0.0f;
  float amax = fabsf(h);
  amax = fmaxf(amax, dpp_f<0xB1>(amax));
  amax = fmaxf(amax, dpp_f<0x4E>(amax));
  amax = fmaxf(amax, dpp_f<0x141>(amax));
  amax = fmaxf(amax, dpp_f<0x140>(amax));
  const float am = lane < 32 ? fmaxf(readlane_f(amax, 0), readlane_f(amax, 16))
                             : fmaxf(readlane_f(amax, 32), readlane_f(amax, 48));
  const float qv = q8_code(h, am);
  const float qhi = __shfl_down(qv, 16);
  const size_t blk = (size_t)s * (size_t)(F / MOE_QK) + 2 * g + (lane >> 5);
  if ((lane & 31) < 16) hq[blk * 16 + (lane & 15)] = pack_f16x2(qv, qhi);
  if ((lane & 31) == 0) hd[blk] = (float)q8_scale_f16(am);
  if (htap) htap[(size_t)s * F + (size_t)g * MOE_RG + lane] = h;
}

// Decode down with the top-k combine fused (T == 1).  grid H/16, 64*S
// threads: wave s computes slot s (s == k: the shared expert) for 16 output
// rows; lane = (row r16 = lane & 15, K-quarter kq = lane >> 4), quarter kq
// takes the 4-block groups g = 4j + kq.  The quarters are summed with two
// lane swaps, each slot's rows are scaled by its router weight, and the
// slots are added in slot order, ((y0 + y1) + ...) + shared (the
// reference's trunk ADD chain, nano-glm/lib/models/glm_dsa/moe_block.h:120-131).
// per_slot: out[s][H] = y_s (the MUL node of the reference's split) instead.
// A 16-row workgroup reads 256 B runs of every 1 KiB block row (the layout's
// 64-row groups); all slots of a row live in one workgroup, so nothing
// crosses workgroups.  LDS: per slot KQ groups of 272 B (4 h blocks + 16 B so
// the four quarters' reads fall in different banks) + KB scales, then the
// [S][16] slot rows.
#define MOE_DN_GROUP_BYTES 272

__device__ __forceinline__ void dq_load(wgroup<1> &g, const uint4 *__restrict__ nib, const uint32_t *__restrict__ sc,
                                        int grp, int lane64) {
#pragma unroll
  for (int i = 0; i < 4; i++)
    g.w[0][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(nib + (size_t)(4 * grp + i) * MOE_RG + lane64));
  g.e[0] = __builtin_nontemporal_load(sc + (size_t)grp * MOE_RG + lane64);
}

__global__ __launch_bounds__(1024) void k_down_decode(
    const uint4 *__restrict__ nib_d, const uint32_t *__restrict__ sc_d, const uint32_t *__restrict__ hq,
    const float *__restrict__ hd, const int32_t *__restrict__ ids, const float *__restrict__ wts, int k, int E,
    int S, int F, int H, int per_slot, float *__restrict__ out) {
  extern __shared__ __align__(16) uint32_t lds[];
  const int KB = F / MOE_QK, KQ = KB / 4;
  const int lane = threadIdx.x & 63, s = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, kq = lane >> 4;
  const size_t slot_bytes = (size_t)KQ * MOE_DN_GROUP_BYTES + (size_t)KB * 4;
  uint8_t *base = reinterpret_cast<uint8_t *>(lds) + (size_t)s * slot_bytes;
  float *d_s = reinterpret_cast<float *>(base + (size_t)KQ * MOE_DN_GROUP_BYTES);
  float *ys = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(lds) + (size_t)S * slot_bytes);  // [S][16]

  int e = s < k ? ids[s] : E;
  const bool valid = s >= k || (unsigned)e < (unsigned)E;  // an out-of-range id reads nothing, yields 0
  e = valid ? e : 0;
  const int G = H / MOE_RG;
  const int grp64 = blockIdx.x >> 2, lane64 = (blockIdx.x & 3) * 16 + r16;
  const size_t mg = (size_t)e * G + grp64;
  const uint4 *nib = nib_d + mg * KB * MOE_RG;
  const uint32_t *sc = sc_d + mg * KQ * MOE_RG;
  const int nj = (KQ + 3) / 4;

  // first weight group in flight before the h staging
  wgroup<1> ga, gb;
  dq_load(ga, nib, sc, kq < KQ ? kq : KQ - 1, lane64);
  // stage h of this slot: block b -> group b/4 at 272 B, offset (b%4)*64
  const uint4 *hsrc = reinterpret_cast<const uint4 *>(hq + (size_t)s * KB * 16);
  const int n16 = KB * 4;  // 16-byte pieces of this slot's h
  for (int i0 = 0; i0 < n16; i0 += 256) {
    uint32_t off[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {  // a piece past the end lands in group 0's (unread) pad
      const int i = i0 + 64 * r + lane;
      const int b = i >> 2, part = i & 3;
      off[r] = i < n16 ? (uint32_t)((b >> 2) * MOE_DN_GROUP_BYTES + (b & 3) * 64 + part * 16) : 256u;
    }
    uint4 v[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {  // all four loads in flight, clamped in range
      const int i = i0 + 64 * r + lane;
      v[r] = hsrc[i < n16 ? i : n16 - 1];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < 4; r++) *reinterpret_cast<uint4 *>(base + off[r]) = v[r];
  }
  for (int b = lane; b < KB; b += 64) d_s[b] = hd[(size_t)s * KB + b];
  __syncthreads();

  float acc = 0.0f;
  for (int j = 0;; j += 2) {
    const int g0 = 4 * j + kq, g1 = 4 * j + 4 + kq, g2 = 4 * j + 8 + kq;
    dq_load(gb, nib, sc, g1 < KQ ? g1 : KQ - 1, lane64);
    __builtin_amdgcn_sched_barrier(0);
    {
      float a[1][1];
      a[0][0] = 0.0f;
      dot_group<1, 1>(ga, 0, reinterpret_cast<const uint32_t *>(base + (size_t)(g0 < KQ ? g0 : 0) * MOE_DN_GROUP_BYTES),
                      d_s + 4 * (g0 < KQ ? g0 : 0), 0, a);
      acc += g0 < KQ ? a[0][0] : 0.0f;
    }
    if (j + 1 >= nj) break;
    dq_load(ga, nib, sc, g2 < KQ ? g2 : KQ - 1, lane64);
    __builtin_amdgcn_sched_barrier(0);
    {
      float a[1][1];
      a[0][0] = 0.0f;
      dot_group<1, 1>(gb, 0, reinterpret_cast<const uint32_t *>(base + (size_t)(g1 < KQ ? g1 : 0) * MOE_DN_GROUP_BYTES),
                      d_s + 4 * (g1 < KQ ? g1 : 0), 0, a);
      acc += g1 < KQ ? a[0][0] : 0.0f;
    }
    if (j + 2 >= nj) break;
  }
  // sum the four K-quarters: (q0 + q1) + (q2 + q3) in every quarter's lanes
  acc += __shfl_xor(acc, 16);
  acc += __shfl_xor(acc, 32);
  float v = valid ? acc : 0.0f;
  if (s < k) v = __fmul_rn(v, wts[s]);
  const int row = blockIdx.x * 16 + r16;
  if (per_slot) {
    if (lane < 16) out[(size_t)s * H + row] = v;
    return;
  }
  if (lane < 16) ys[s * 16 + lane] = v;
  __syncthreads();
  if (threadIdx.x < 16) {
    float o = ys[threadIdx.x];
    for (int q = 1; q < S; q++) o = __fadd_rn(o, ys[q * 16 + threadIdx.x]);
    out[blockIdx.x * 16 + threadIdx.x] = o;
  }
}

static inline size_t down_decode_lds_bytes(int F, int S) {
  const int KB = F / MOE_QK, KQ = KB / 4;
  return (size_t)S * ((size_t)KQ * MOE_DN_GROUP_BYTES + (size_t)KB * 4) + (size_t)S * 16 * 4;
}

// Chunks per unit for the split-K decode kernels: about 9 single-wave
// workgroups per CU in all, each chunk at least one group of 4 blocks.
static inline int decode_chunks(int units, int KQ, int n_cu) {
  int c = (9 * n_cu + units / 2) / units;
  c = c < 1 ? 1 : c;
  return c > KQ ? KQ : c;
}

// LDS bytes of the two kernels (activations + partials).
static inline size_t gate_up_lds_bytes(int H, int NT) {
  const int NBW = max_wave_blocks(H / MOE_QK, MOE_GU_WAVES);
  return (size_t)MOE_GU_WAVES * NT * NBW * 68 + (size_t)MOE_GU_WAVES * 2 * NT * MOE_RG * 4;
}
static inline size_t down_lds_bytes(int F, int NT) {
  const int NBW = max_wave_blocks(F / MOE_QK, MOE_DN_WAVES);
  return (size_t)MOE_DN_WAVES * NT * NBW * 68 + (size_t)MOE_DN_WAVES * NT * MOE_RG * 4;
}

// ---------------------------------------------------------------------------
// test hook: the product quantizer (stage_quantize) over n_blocks blocks of
// a flat f32 array, 64 blocks per workgroup of one wave; ggml's byte layout.
__global__ __launch_bounds__(64) void k_debug_quantize(const float *__restrict__ x, int n_blocks,
                                                       int8_t *__restrict__ qs, uint16_t *__restrict__ d) {
  __shared__ __align__(16) uint32_t q_s[64 * 16];
  __shared__ float d_s[64];
  const int lane = threadIdx.x;
  const int b0 = blockIdx.x * 64;
  const int nb = n_blocks - b0 < 64 ? n_blocks - b0 : 64;
  stage_quantize(x + (size_t)b0 * MOE_QK, nb, q_s, d_s, lane);
  __syncthreads();
  for (int i = lane; i < nb * 16; i += 64) {
    const f16x2_t p = __builtin_bit_cast(f16x2_t, q_s[i]);
    const size_t b = (size_t)b0 + (i >> 4);
    const int j = i & 15;
    qs[b * MOE_QK + j] = (int8_t)(int)(float)p.x;
    qs[b * MOE_QK + j + 16] = (int8_t)(int)(float)p.y;
  }
  if (lane < nb) d[(size_t)b0 + lane] = __builtin_bit_cast(uint16_t, (_Float16)d_s[lane]);
}
