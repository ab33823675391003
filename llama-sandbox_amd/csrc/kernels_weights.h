// kernels_weights.h -- expert-weight residency kernels (device repack).
//
// ggml stores an expert matrix of R rows x K reduction as R*KB 17-byte
// blocks {uint8 e; uint8 qs[16]} (KB = K/32), row-major.  On the device the
// two parts are split into the tiled layout the MFMA kernels stream
// (kernels_rows.h), with NQ = KB/4 quads of 4 blocks and NQ4 = ceil(NQ/4):
//   nib[tile][q][l]        uint4  qs of block 4q + l/16 of row 16*tile + l%16
//   sc [tile][q/4][l][q%4] uint8  e  of the same block
// for every 16-row tile of every expert, experts back to back (an expert's
// exponent plane is R/16 * NQ4 * 256 bytes; the bytes of quads past NQ in
// the last dword group are padding).  The reference splits the same two
// planes for the same reason (moe-serv/src/moe_tp.h:235-278: nibble plane +
// scale plane, interleaved for its kernel's access pattern); here one wave
// reads a (tile, quad) as one contiguous KiB, which is the A-operand lane
// layout of the 16x16x128 scaled MFMA.
//
// Every kernel below runs one thread per block of one expert matrix, indexed
// by its position o in the device layout (so the device-side accesses are
// coalesced), and maps it back to ggml's block index i = r*KB + b.
#pragma once

#include "device_common.h"

// Exponent-plane bytes of one expert matrix of R rows and KB blocks per row.
__host__ __device__ __forceinline__ uint64_t sc_plane_bytes(int R, int KB) {
  const int NQ = KB / 4;
  return (uint64_t)(R / 16) * (uint64_t)((NQ + 3) / 4) * 256u;
}

__device__ __forceinline__ void layout_of(uint64_t o, int KB, uint64_t &i, uint64_t &sc_byte) {
  const int NQ = KB >> 2, NQ4 = (NQ + 3) >> 2;
  const uint32_t l = (uint32_t)(o & 63u);
  const uint64_t tq = o >> 6;  // tile*NQ + q
  const uint64_t tile = tq / (uint64_t)NQ;
  const uint32_t q = (uint32_t)(tq - tile * (uint64_t)NQ);
  const uint64_t r = tile * 16u + (l & 15u);
  const uint32_t b = 4u * q + (l >> 4);
  i = r * (uint64_t)KB + b;
  sc_byte = ((tile * (uint64_t)NQ4 + (q >> 2)) * 64u + l) * 4u + (q & 3u);
}

// ggml 17-byte blocks of consecutive expert matrices (per_exp = R*KB blocks
// each, n_blocks in all) -> (nib, sc) of the same experts.
// sc points at the first expert's exponent plane (sc_per_exp bytes each).
__global__ __launch_bounds__(256) void k_repack_blocks(const uint8_t *__restrict__ src, uint64_t n_blocks,
                                                       uint64_t per_exp, uint64_t sc_per_exp, int KB,
                                                       uint4 *__restrict__ nib, uint8_t *__restrict__ sc) {
  const uint64_t o = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (o >= n_blocks) return;
  const uint64_t e = o / per_exp, base = e * per_exp;
  uint64_t i, sb;
  layout_of(o - base, KB, i, sb);
  i += base;
  sb += e * sc_per_exp;
  const uint8_t *b = src + i * 17u;
  uint32_t w[4];
#pragma unroll
  for (int d = 0; d < 4; d++) {
    w[d] = (uint32_t)b[1 + 4 * d] | ((uint32_t)b[2 + 4 * d] << 8) | ((uint32_t)b[3 + 4 * d] << 16) |
           ((uint32_t)b[4 + 4 * d] << 24);
  }
  nib[o] = make_uint4(w[0], w[1], w[2], w[3]);
  sc[sb] = b[0];
}

// Inverse: (nib, sc) of one matrix -> ggml 17-byte blocks.
__global__ __launch_bounds__(256) void k_unpack_blocks(const uint4 *__restrict__ nib,
                                                       const uint8_t *__restrict__ sc, uint64_t n_blocks,
                                                       int KB, uint8_t *__restrict__ dst) {
  const uint64_t o = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (o >= n_blocks) return;
  uint64_t i, sb;
  layout_of(o, KB, i, sb);
  uint8_t *b = dst + i * 17u;
  const uint4 v = nib[o];
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  b[0] = sc[sb];
#pragma unroll
  for (int d = 0; d < 4; d++) {
#pragma unroll
    for (int j = 0; j < 4; j++) b[1 + 4 * d + j] = (uint8_t)(w[d] >> (8 * j));
  }
}

// Counter-based synthetic MXFP4: ggml block i of a matrix with key `key` has
// nibble bytes = little-endian bytes of mix(key+2i+1), mix(key+2i+2) and
// exponent e_lo + floor((mix(key ^ ~i) >> 32) * e_span / 2^32).
__global__ __launch_bounds__(256) void k_generate_blocks(uint64_t key, uint64_t n_blocks, int KB, uint32_t e_lo,
                                                         uint32_t e_span, uint4 *__restrict__ nib,
                                                         uint8_t *__restrict__ sc) {
  const uint64_t o = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (o >= n_blocks) return;
  uint64_t i, sb;
  layout_of(o, KB, i, sb);
  const uint64_t a = mix64(key + 2u * i + 1u);
  const uint64_t b = mix64(key + 2u * i + 2u);
  const uint64_t c = mix64(key ^ ~i);
  nib[o] = make_uint4((uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32));
  sc[sb] = (uint8_t)(e_lo + (uint32_t)(((c >> 32) * (uint64_t)e_span) >> 32));
}
