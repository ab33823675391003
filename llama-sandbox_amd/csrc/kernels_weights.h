// kernels_weights.h -- expert-weight residency kernels (device repack).
//
// Device layout of one expert matrix of R rows x K reduction (KB = K/32
// blocks per row), for all experts of a layer back to back:
//   nib[e][r][b] : uint4  -- the block's 16 nibble bytes, unchanged order
//   sc [e][r][b] : uint8  -- the block's E8M0 exponent
// i.e. ggml's 17-byte block split into a 16-byte-aligned nibble stream and a
// separate exponent stream, so every weight load is one 128-bit coalesced
// load (the reference splits the same two planes for the same reason,
// moe-serv/src/moe_tp.h:235-278, in a column-interleaved order built for its
// 4-column threads; here rows stay contiguous because a wave reads 64
// consecutive blocks of one row).
#pragma once

#include "device_common.h"

// 17-byte blocks -> (nib, sc).  One thread per block.
__global__ __launch_bounds__(256) void k_repack_blocks(const uint8_t *__restrict__ src,
                                                       uint64_t n_blocks,
                                                       uint4 *__restrict__ nib,
                                                       uint8_t *__restrict__ sc) {
  const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (i >= n_blocks) return;
  const uint8_t *b = src + i * 17u;
  uint32_t w[4];
#pragma unroll
  for (int d = 0; d < 4; d++) {
    w[d] = (uint32_t)b[1 + 4 * d] | ((uint32_t)b[2 + 4 * d] << 8) |
           ((uint32_t)b[3 + 4 * d] << 16) | ((uint32_t)b[4 + 4 * d] << 24);
  }
  nib[i] = make_uint4(w[0], w[1], w[2], w[3]);
  sc[i] = b[0];
}

// Inverse: (nib, sc) -> 17-byte blocks.
__global__ __launch_bounds__(256) void k_unpack_blocks(const uint4 *__restrict__ nib,
                                                       const uint8_t *__restrict__ sc,
                                                       uint64_t n_blocks,
                                                       uint8_t *__restrict__ dst) {
  const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (i >= n_blocks) return;
  uint8_t *b = dst + i * 17u;
  const uint4 v = nib[i];
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  b[0] = sc[i];
#pragma unroll
  for (int d = 0; d < 4; d++) {
#pragma unroll
    for (int j = 0; j < 4; j++) b[1 + 4 * d + j] = (uint8_t)(w[d] >> (8 * j));
  }
}

// Counter-based synthetic MXFP4: block i of a matrix with key `key` has
// nibble bytes = little-endian bytes of mix(key+2i+1), mix(key+2i+2) and
// exponent e_lo + floor((mix(key ^ ~i) >> 32) * e_span / 2^32).
__global__ __launch_bounds__(256) void k_generate_blocks(uint64_t key, uint64_t n_blocks,
                                                         uint32_t e_lo, uint32_t e_span,
                                                         uint4 *__restrict__ nib,
                                                         uint8_t *__restrict__ sc) {
  const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (i >= n_blocks) return;
  const uint64_t a = mix64(key + 2u * i + 1u);
  const uint64_t b = mix64(key + 2u * i + 2u);
  const uint64_t c = mix64(key ^ ~i);
  nib[i] = make_uint4((uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32));
  sc[i] = (uint8_t)(e_lo + (uint32_t)(((c >> 32) * (uint64_t)e_span) >> 32));
}
