// kernels_decode.h -- single-token decode chain and the small per-call kernels.
//
// Decode (T = 1) is three launches:
//   k_quantize_q8   x [H] f32 -> Q8_0 activation blocks (packed fp16 pairs)
//   k_gu_decode     per slot (k routed + shared): gate and up rows of the
//                   slot's expert against x, clamp, SwiGLU, then Q8_0 of the
//                   32 h values a workgroup owns -> h blocks for down
//   k_down_decode   per group of output rows: every slot's down row against
//                   its h, times the router weight, summed in slot order
//                   (+ shared) -> out [H]  (the reference's trunk ADDs,
//                   nano-glm/lib/models/glm_dsa/moe_block.h:120-131, fused)
//
// Work mapping for the vecmats: lane <-> weight block along the reduction
// dimension (a wave reads 64 consecutive 16-byte blocks = 1 KiB of one row
// per load instruction), wave <-> rows, f32 partial per lane, one 64-lane
// DPP/permlane reduction per row.  The activation blocks a lane needs are
// the same for every row, so they stay in registers for the whole kernel.
#pragma once

#include "device_common.h"

// ---------------------------------------------------------------------------
// Q8_0 quantization of n_rows rows of K floats (one thread per 32-block).
// xq[row][b][16] packed (q_j, q_{j+16}) fp16 pairs, xd[row][b] = fp16(d) as
// f32.  qs_dbg / d_dbg (nullable): ggml's byte layout, for tests.
__global__ __launch_bounds__(256) void k_quantize_q8(const float *__restrict__ x, uint32_t n_blocks,
                                                     uint32_t *__restrict__ xq,
                                                     float *__restrict__ xd,
                                                     int8_t *__restrict__ qs_dbg,
                                                     uint16_t *__restrict__ d_dbg) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= n_blocks) return;
  const float4 *xb = reinterpret_cast<const float4 *>(x + (size_t)i * MOE_QK);
  float v[MOE_QK];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const float4 f = xb[j];
    v[4 * j + 0] = f.x;
    v[4 * j + 1] = f.y;
    v[4 * j + 2] = f.z;
    v[4 * j + 3] = f.w;
  }
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < MOE_QK; j++) amax = fmaxf(amax, fabsf(v[j]));
  const _Float16 d16 = q8_scale_f16(amax);
  float q[MOE_QK];
#pragma unroll
  for (int j = 0; j < MOE_QK; j++) q[j] = q8_code(v[j], amax);
  uint4 *dst = reinterpret_cast<uint4 *>(xq + (size_t)i * 16);
#pragma unroll
  for (int j = 0; j < 4; j++) {
    dst[j] = make_uint4(pack_f16x2(q[4 * j + 0], q[4 * j + 16]), pack_f16x2(q[4 * j + 1], q[4 * j + 17]),
                        pack_f16x2(q[4 * j + 2], q[4 * j + 18]), pack_f16x2(q[4 * j + 3], q[4 * j + 19]));
  }
  xd[i] = (float)d16;
  if (qs_dbg) {
#pragma unroll
    for (int j = 0; j < MOE_QK; j++) qs_dbg[(size_t)i * MOE_QK + j] = (int8_t)(int)q[j];
    d_dbg[i] = __builtin_bit_cast(uint16_t, d16);
  }
}

// ---------------------------------------------------------------------------
// Router, one workgroup per token (E <= 1024).  Scores, selection bias,
// top-k (ties -> lower id), weights from the unbiased scores, renorm with
// the 2^-14 floor, scale (glm_dsa/moe_block.h:48-91).
#define MOE_ROUTE_MAX_E 1024

__device__ __forceinline__ void argmax_merge(float &v, int &i, float v2, int i2) {
  if (i2 >= 0 && (i < 0 || v2 > v || (v2 == v && i2 < i))) {
    v = v2;
    i = i2;
  }
}

__global__ __launch_bounds__(256) void k_route(const float *__restrict__ logits,
                                               const float *__restrict__ bias, int E, int k,
                                               int mode, int norm, float scale,
                                               int32_t *__restrict__ ids, float *__restrict__ wts) {
  __shared__ float probs[MOE_ROUTE_MAX_E];
  __shared__ float sel[MOE_ROUTE_MAX_E];
  __shared__ float red_f[4];
  __shared__ double red_d[4];
  __shared__ int red_i[4];
  __shared__ int picked[64];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float *l = logits + (size_t)t * E;

  if (mode == 0) { // softmax: exp(l - max), sum in double, scale by (float)(1/sum)
    float mx = -INFINITY;
    for (int e = tid; e < E; e += 256) mx = fmaxf(mx, l[e]);
    mx = wave_max(mx);
    if (lane == 0) red_f[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red_f[0], red_f[1]), fmaxf(red_f[2], red_f[3]));
    double s = 0.0;
    for (int e = tid; e < E; e += 256) {
      const float pe = expf(l[e] - mx);
      probs[e] = pe;
      s += (double)pe;
    }
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
    if (lane == 0) red_d[wave] = s;
    __syncthreads();
    const float inv = (float)(1.0 / (((red_d[0] + red_d[1]) + red_d[2]) + red_d[3]));
    for (int e = tid; e < E; e += 256) probs[e] = probs[e] * inv;
  } else if (mode == 1) {
    for (int e = tid; e < E; e += 256) probs[e] = __fdiv_rn(1.0f, 1.0f + expf(-l[e]));
  } else {
    for (int e = tid; e < E; e += 256) {
      const float v = l[e];
      probs[e] = sqrtf(v > 20.0f ? v : log1pf(expf(v)));
    }
  }
  __syncthreads();
  for (int e = tid; e < E; e += 256) sel[e] = bias ? probs[e] + bias[e] : probs[e];
  __syncthreads();

  for (int s = 0; s < k; s++) {
    float bv = 0.0f;
    int bi = -1;
    for (int e = tid; e < E; e += 256) {
      bool taken = false;
      for (int q = 0; q < s; q++) taken |= picked[q] == e;
      if (!taken) argmax_merge(bv, bi, sel[e], e);
    }
    for (int off = 32; off >= 1; off >>= 1) {
      const float v2 = __shfl_xor(bv, off);
      const int i2 = __shfl_xor(bi, off);
      argmax_merge(bv, bi, v2, i2);
    }
    if (lane == 0) {
      red_f[wave] = bv;
      red_i[wave] = bi;
    }
    __syncthreads();
    if (tid == 0) {
      float v = red_f[0];
      int i = red_i[0];
      for (int w = 1; w < 4; w++) argmax_merge(v, i, red_f[w], red_i[w]);
      picked[s] = i >= 0 ? i : 0;  // only NaN scores leave nothing selectable
    }
    __syncthreads();
  }
  if (tid == 0) {
    float w[64];
    for (int s = 0; s < k; s++) w[s] = probs[picked[s]];
    if (norm) {
      double sum = 0.0;
      for (int s = 0; s < k; s++) sum += (double)w[s];
      float fs = (float)sum;
      fs = fs < 6.103515625e-5f ? 6.103515625e-5f : fs;
      for (int s = 0; s < k; s++) w[s] = __fdiv_rn(w[s], fs);
    }
    if (scale != 0.0f && scale != 1.0f) {
      for (int s = 0; s < k; s++) w[s] = __fmul_rn(w[s], scale);
    }
    for (int s = 0; s < k; s++) {
      ids[(size_t)t * k + s] = picked[s];
      wts[(size_t)t * k + s] = w[s];
    }
  }
}

// ---------------------------------------------------------------------------
// Load the NB activation blocks lane `lane` owns (blocks lane, lane+64, ...).
template <int NB>
__device__ __forceinline__ void load_act_blocks(const uint32_t *__restrict__ q,
                                                const float *__restrict__ d, int KB, int lane,
                                                uint32_t (&xr)[NB][16], float (&xs)[NB]) {
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const int b = lane + 64 * j;
    if (b < KB) {
      const uint4 *p = reinterpret_cast<const uint4 *>(q + (size_t)b * 16);
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const uint4 v = p[c];
        xr[j][4 * c + 0] = v.x;
        xr[j][4 * c + 1] = v.y;
        xr[j][4 * c + 2] = v.z;
        xr[j][4 * c + 3] = v.w;
      }
      xs[j] = d[b];
    } else {
#pragma unroll
      for (int c = 0; c < 16; c++) xr[j][c] = 0u;
      xs[j] = 0.0f;
    }
  }
}

// ---------------------------------------------------------------------------
// Fused gate/up/SwiGLU/Q8_0(h) for one token.  grid = (F/32, S), 256 threads;
// wave w owns rows [32*bx + 8w, +8) of gate and of up.
#define GU_ROWS_PER_WAVE 8

template <int NB>
__global__ __launch_bounds__(256) void k_gu_decode(
    const uint4 *__restrict__ nib_g, const uint4 *__restrict__ nib_u,
    const uint8_t *__restrict__ sc_g, const uint8_t *__restrict__ sc_u,
    const uint32_t *__restrict__ xq, const float *__restrict__ xd,
    const int32_t *__restrict__ ids, int k, int shared_expert, int F, int KB, float clamp,
    uint32_t *__restrict__ hq, float *__restrict__ hd, float *__restrict__ htap) {
  const int s = blockIdx.y;
  int e = s < k ? ids[s] : shared_expert;
  // An id outside [0, E) reads no weights and yields h = 0 for its slot.
  const bool valid = s >= k || (unsigned)e < (unsigned)shared_expert;
  e = valid ? e : 0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r0 = blockIdx.x * 32 + wave * GU_ROWS_PER_WAVE;

  uint32_t xr[NB][16];
  float xs[NB];
  load_act_blocks<NB>(xq, xd, KB, lane, xr, xs);

  const size_t ebase = (size_t)e * (size_t)F * (size_t)KB;
  float pg[GU_ROWS_PER_WAVE], pu[GU_ROWS_PER_WAVE];
#pragma unroll
  for (int rr = 0; rr < GU_ROWS_PER_WAVE; rr++) {
    const size_t rb = ebase + (size_t)(r0 + rr) * (size_t)KB;
    float ag = 0.0f, au = 0.0f;
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const int b = lane + 64 * j;
      if (valid && b < KB) {
        const uint4 wg = nib_g[rb + b];
        const uint4 wu = nib_u[rb + b];
        const uint32_t eg = sc_g[rb + b], eu = sc_u[rb + b];
        ag = fmaf(scale_e8m0(xs[j], eg), block_dot(wg, xr[j]), ag);
        au = fmaf(scale_e8m0(xs[j], eu), block_dot(wu, xr[j]), au);
      }
    }
    pg[rr] = ag;
    pu[rr] = au;
  }

  __shared__ float hs[32];
#pragma unroll
  for (int rr = 0; rr < GU_ROWS_PER_WAVE; rr++) {
    float g = wave_sum(pg[rr]);
    float u = wave_sum(pu[rr]);
    if (clamp > 1e-6f) { // deepseek4 order: up symmetric, gate one-sided, before SiLU
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
    const size_t blk = (size_t)s * (size_t)(F / MOE_QK) + blockIdx.x;
    if (lane < 16) hq[blk * 16 + lane] = pack_f16x2(q, qhi);
    if (lane == 0) hd[blk] = (float)q8_scale_f16(amax);
    if (htap && lane < 32) htap[(size_t)s * F + blockIdx.x * 32 + lane] = h;
  }
}

// ---------------------------------------------------------------------------
// down for one token with the top-k weighted combine fused.  grid = H/RD,
// 64*S threads: wave s owns slot s (s == k is the shared expert) for RD
// output rows; the slot rows are summed in slot order in LDS.
template <int NB, int RD>
__global__ __launch_bounds__(1024) void k_down_decode(
    const uint4 *__restrict__ nib_d, const uint8_t *__restrict__ sc_d,
    const uint32_t *__restrict__ hq, const float *__restrict__ hd,
    const int32_t *__restrict__ ids, const float *__restrict__ wts, int k, int shared_expert,
    int S, int H, int KB, float *__restrict__ out, int per_slot) {
  const int s = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int e = s < k ? ids[s] : shared_expert;
  // An id outside [0, E) reads no weights and contributes 0.
  const bool valid = s >= k || (unsigned)e < (unsigned)shared_expert;
  e = valid ? e : 0;
  const int r0 = blockIdx.x * RD;

  uint32_t hr[NB][16];
  float hsc[NB];
  load_act_blocks<NB>(hq + (size_t)s * KB * 16, hd + (size_t)s * KB, KB, lane, hr, hsc);

  __shared__ float ys[16][RD];
  const size_t ebase = (size_t)e * (size_t)H * (size_t)KB;
  float part[RD];
#pragma unroll
  for (int rr = 0; rr < RD; rr++) {
    const size_t rb = ebase + (size_t)(r0 + rr) * (size_t)KB;
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const int b = lane + 64 * j;
      if (valid && b < KB) a = fmaf(scale_e8m0(hsc[j], sc_d[rb + b]), block_dot(nib_d[rb + b], hr[j]), a);
    }
    part[rr] = a;
  }
#pragma unroll
  for (int rr = 0; rr < RD; rr++) {
    const float v = wave_sum(part[rr]);
    if (lane == 0) ys[s][rr] = v;
  }
  __syncthreads();
  if (threadIdx.x < RD) {
    const int t = threadIdx.x, r = r0 + t;
    if (per_slot) {
      for (int q = 0; q < k; q++) out[(size_t)q * H + r] = __fmul_rn(ys[q][t], wts[q]);
    } else {
      float acc = __fmul_rn(ys[0][t], wts[0]);
      for (int q = 1; q < k; q++) acc = __fadd_rn(acc, __fmul_rn(ys[q][t], wts[q]));
      if (S > k) acc = __fadd_rn(acc, ys[k][t]);
      out[r] = acc;
    }
  }
}

// ---------------------------------------------------------------------------
// test hook: one wave_sum per 64 inputs
__global__ __launch_bounds__(64) void k_debug_wave_sum(const float *__restrict__ x,
                                                       float *__restrict__ out) {
  const float v = wave_sum(x[blockIdx.x * 64 + threadIdx.x]);
  out[blockIdx.x * 64 + threadIdx.x] = v;
}
