// device_common.h -- gfx950 device helpers shared by the MoE-block kernels.
//
// Number formats (ggml's, restated; hip-moe/src/main.hip:44-57):
//   MXFP4 block  = 32 weights along the reduction dim: one E8M0 exponent e
//                  and 16 bytes where byte j holds element j (low nibble)
//                  and element j+16 (high nibble); the nibble is an OCP
//                  e2m1 code, value = e2m1(code) * 2^(e-127)
//                  (== ggml's kvalue(code) * 2^(e-128)).
//   Q8_0 block   = 32 activations: int8 q in [-127, 127] and an fp16 d.
//
// Activation blocks are kept on the device as 16 packed fp16 pairs
// (q_j, q_{j+16}) plus d as f32, so that one weight byte converts to one
// fp16 pair (v_cvt_scalef32_pk_f16_fp4) that meets its activation pair in
// one v_dot2_f32_f16.  All of those values are small integers or halves:
// every per-block sum below is exact in f32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

#define MOE_QK 32

// Flags of a work item (k_group's item records, word 3).
#define MOE_ITEM_SHARED 1  // the shared expert's rows
#define MOE_ITEM_SPLIT 2   // the expert's rows span more than one item (its tiles are read again)

// 2^(e-127) * d, exact whenever the result is a normal f32.
__device__ __forceinline__ float scale_e8m0(float d, uint32_t e) {
  return __builtin_amdgcn_ldexpf(d, (int)e - 127);
}

// Sum over one MXFP4 block of e2m1(w) * q with w the block's 16 nibble bytes
// and xq its 16 packed activation pairs.  Exact (the result is isum / 2).
__device__ __forceinline__ float block_dot(const uint4 w, const uint32_t *xq) {
  float acc = 0.0f;
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int d = 0; d < 4; d++) {
    const f16x2_t w0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wd[d], 1.0f, 0);
    const f16x2_t w1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wd[d], 1.0f, 1);
    const f16x2_t w2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wd[d], 1.0f, 2);
    const f16x2_t w3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wd[d], 1.0f, 3);
    acc = __builtin_amdgcn_fdot2(w0, __builtin_bit_cast(f16x2_t, xq[4 * d + 0]), acc, false);
    acc = __builtin_amdgcn_fdot2(w1, __builtin_bit_cast(f16x2_t, xq[4 * d + 1]), acc, false);
    acc = __builtin_amdgcn_fdot2(w2, __builtin_bit_cast(f16x2_t, xq[4 * d + 2]), acc, false);
    acc = __builtin_amdgcn_fdot2(w3, __builtin_bit_cast(f16x2_t, xq[4 * d + 3]), acc, false);
  }
  return acc;
}

// ---- cross-lane reductions (wave64) ----------------------------------------

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over 16-lane rows, every lane of a row gets its row's sum.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);  // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);  // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v); // row_half_mirror
  v += dpp_f<0x140>(v); // row_mirror
  return v;
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over all 64 lanes; every lane gets the same total.  After row16_sum
// every lane of a 16-lane row holds that row's sum; the four row sums are
// read as scalars (lanes 0, 16, 32, 48) and added in a fixed order.
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

// ---- Q8_0 ------------------------------------------------------------------

// ggml's x86 quantize_row_q8_0 for one value of a 32-block, given the
// block's amax: d = amax / 127 (f32, then fp16 RNE), id = 127 / amax,
// q = round-half-even(x * id).
__device__ __forceinline__ float q8_code(float x, float amax) {
  const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
  return __builtin_rintf(__fmul_rn(x, id));
}
__device__ __forceinline__ _Float16 q8_scale_f16(float amax) {
  return (_Float16)__fdiv_rn(amax, 127.0f); // v_cvt_f16_f32: round to nearest even
}

// Pack two int-valued floats as an fp16 pair (exact for |v| <= 2048).
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  f16x2_t p;
  p.x = (_Float16)lo;
  p.y = (_Float16)hi;
  return __builtin_bit_cast(uint32_t, p);
}

// ---- synthetic weights -----------------------------------------------------

// SplitMix64's output function (Steele, Lea & Flood, OOPSLA 2014); the
// host-side test generator uses the same function.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
