// kernels_decode.h -- small per-call kernels: the router and the test hook of
// the wave reduction.  The expert vecmats are in kernels_rows.h.
#pragma once

#include "device_common.h"

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

// Score of one logit for the element-wise score functions (mode 1: sigmoid,
// 2: sqrt(softplus)); softmax (mode 0) needs the whole row and stays in k_route.
__device__ __forceinline__ float route_score(float v, int mode) {
  return mode == 1 ? __fdiv_rn(1.0f, 1.0f + expf(-v)) : sqrtf(v > 20.0f ? v : log1pf(expf(v)));
}

// Top-k of sel[0..E) by one wave (called by all 64 lanes of it), with no
// barrier between rounds: lane l holds experts l, l + 64, ...; each round
// every lane offers its best expert not yet taken, the wave keeps the largest
// (ties: the lower id), and the lane holding it marks it taken.  picked[s] is
// written by lane 0.
__device__ __forceinline__ void route_topk_wave(const float *sel, int E, int k, int *picked, int lane) {
  uint32_t taken = 0;  // bit j: expert lane + 64 j (E <= 1024)
  const int nj = (E + 63) / 64;
  for (int s = 0; s < k; s++) {
    float bv = 0.0f;
    int bi = -1;
    for (int j = 0; j < nj; j++) {
      const int e = lane + 64 * j;
      if (e < E && !((taken >> j) & 1u)) argmax_merge(bv, bi, sel[e], e);
    }
    for (int off = 32; off >= 1; off >>= 1) {
      const float v2 = __shfl_xor(bv, off);
      const int i2 = __shfl_xor(bi, off);
      argmax_merge(bv, bi, v2, i2);
    }
    if (bi >= 0 && (bi & 63) == lane) taken |= 1u << (bi >> 6);
    if (lane == 0) picked[s] = bi >= 0 ? bi : 0;  // only NaN scores leave nothing selectable
  }
}

// Weights of the picked experts from the unbiased scores: renorm by
// max(sum, 2^-14) when norm, then the scale when it is not 0 or 1 (one thread).
__device__ __forceinline__ void route_weights(const float *probs, const int *picked, int k, int norm, float scale,
                                              float *w) {
  for (int s = 0; s < k; s++) w[s] = probs[picked[s]];
  if (norm) {
    double sum = 0.0;
    for (int s = 0; s < k; s++) sum += (double)w[s];
    float fs = (float)sum;
    fs = fs < 6.103515625e-5f ? 6.103515625e-5f : fs;
    for (int s = 0; s < k; s++) w[s] = __fdiv_rn(w[s], fs);
  }
  if (scale != 0.0f && scale != 1.0f)
    for (int s = 0; s < k; s++) w[s] = __fmul_rn(w[s], scale);
}

__global__ __launch_bounds__(256) void k_route(const float *__restrict__ logits,
                                               const float *__restrict__ bias, int E, int k,
                                               int mode, int norm, float scale,
                                               int32_t *__restrict__ ids, float *__restrict__ wts) {
  __shared__ float probs[MOE_ROUTE_MAX_E];
  __shared__ float sel[MOE_ROUTE_MAX_E];
  __shared__ float red_f[4];
  __shared__ double red_d[4];
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
  } else {
    for (int e = tid; e < E; e += 256) probs[e] = route_score(l[e], mode);
  }
  __syncthreads();
  for (int e = tid; e < E; e += 256) sel[e] = bias ? probs[e] + bias[e] : probs[e];
  __syncthreads();

  if (wave == 0) route_topk_wave(sel, E, k, picked, lane);
  __syncthreads();
  if (tid == 0) {
    float w[64];
    route_weights(probs, picked, k, norm, scale, w);
    for (int s = 0; s < k; s++) {
      ids[(size_t)t * k + s] = picked[s];
      wts[(size_t)t * k + s] = w[s];
    }
  }
}

// ---------------------------------------------------------------------------
// Router logits for the moe-server protocol: logits[t][e] = sum_h W[e][h] *
// x[t][h] in f32 (ggml_mul_mat of ffn_gate_inp [H, E] with x [H, T],
// nano-glm/lib/models/glm_dsa/moe_block.h:52).  One wave per expert and 4
// tokens: each lane accumulates a strided quarter-row slice with FMAs, then
// wave_sum.  grid (ceil(E/4), ceil(T/4)), 256 threads; H % 4 == 0, rows
// 16-byte aligned.
// x rounded to the router weight's type before the products (XR: 0 f32 = as
// is, 1 f16, 2 bf16, each round to nearest even): ggml-cpu's mul_mat converts
// src1 to src0's vec_dot_type (f16 -> f16, bf16 -> bf16) and accumulates the
// products in f32.  A product of two f16 (or two bf16) values is exact in
// f32, so only the order of the f32 sum differs from ggml's.
template <int XR>
__device__ __forceinline__ float router_x(float v) {
  if (XR == 1) return (float)(_Float16)v;
  if (XR == 2) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return v;  // NaN stays NaN
    return __builtin_bit_cast(float, (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u);
  }
  return v;
}

template <int XR>
__global__ __launch_bounds__(256) void k_router_logits(const float *__restrict__ W, const float *__restrict__ x,
                                                       int T, int E, int H, float *__restrict__ logits) {
  const int lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6), t0 = blockIdx.y * 4;
  if (e >= E) return;  // whole waves
  const float4 *w4 = reinterpret_cast<const float4 *>(W + (size_t)e * H);
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int i = lane; i < H / 4; i += 64) {
    const float4 w = w4[i];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      if (t0 + j >= T) break;
      const float4 v = reinterpret_cast<const float4 *>(x + (size_t)(t0 + j) * H)[i];
      acc[j] = fmaf(w.x, router_x<XR>(v.x),
                    fmaf(w.y, router_x<XR>(v.y), fmaf(w.z, router_x<XR>(v.z), fmaf(w.w, router_x<XR>(v.w), acc[j]))));
    }
  }
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const float v = wave_sum(acc[j]);
    if (lane == 0 && t0 + j < T) logits[(size_t)(t0 + j) * E + e] = v;
  }
}

// ---------------------------------------------------------------------------
// test hook: one wave_sum per 64 inputs
__global__ __launch_bounds__(64) void k_debug_wave_sum(const float *__restrict__ x,
                                                       float *__restrict__ out) {
  const float v = wave_sum(x[blockIdx.x * 64 + threadIdx.x]);
  out[blockIdx.x * 64 + threadIdx.x] = v;
}
