// kernels_weights.h -- expert-weight residency kernels (device repack).
//
// ggml stores an expert matrix of R rows x K reduction as R*KB 17-byte
// blocks {uint8 e; uint8 qs[16]} (KB = K/32), row-major.  On the device each
// matrix is a sequence of records, one per (16-row tile, group of 4 quads),
// where a quad is 4 consecutive blocks (128 weights) of the tile's rows:
//   record (tile, g) = 4352 bytes:
//     [j*1024 + l*16, +16)  quad 4g+j: the 16 nibble bytes (ggml's qs,
//                           unchanged) of block 4(4g+j) + l/16 of row
//                           16*tile + l%16, for lanes l = 0..63
//     [4096 + l*4 + j]      the E8M0 exponent e of that same block
// records in (tile, g) order; NQ = KB/4 quads per row, NG = ceil(NQ/4)
// groups (the quads past NQ of a last partial group are padding).  One wave
// reads a quad as one contiguous KiB -- the A-operand lane layout of the
// 16x16x128 scaled MFMA -- and the exponents of 4 quads as one dword per
// lane from the same 4352-byte run, so the two streams share DRAM pages.
// When NQ % 4 == 0 a matrix is exactly as large as ggml's (4352 = 256 * 17).
// The reference splits nibbles and exponents the same way for the same
// reason (moe-serv/src/moe_tp.h:235-278: nibble plane + scale plane,
// interleaved for its kernel's access pattern).
//
// Every kernel below runs one thread per block of one expert matrix, indexed
// by its position o = ((tile*NQ + q)*64 + l) in the device order (so the
// device-side accesses are coalesced), and maps it back to ggml's block
// index i = r*KB + b.
#pragma once

#include "device_common.h"

#define MOE_REC_BYTES 4352u  // one (tile, 4-quad group) record
#define MOE_REC_SC 4096u     // offset of the exponent dwords in a record

// Device bytes of one expert matrix of R rows and KB blocks per row.
__host__ __device__ __forceinline__ uint64_t mat_bytes(int R, int KB) {
  const int NQ = KB / 4;
  return (uint64_t)(R / 16) * (uint64_t)((NQ + 3) / 4) * MOE_REC_BYTES;
}

// Position o -> ggml block index i, byte offset of the nibbles and of the
// exponent within the matrix.
__device__ __forceinline__ void layout_of(uint64_t o, int KB, uint64_t &i, uint64_t &nib_byte, uint64_t &sc_byte) {
  const int NQ = KB >> 2, NG = (NQ + 3) >> 2;
  const uint32_t l = (uint32_t)(o & 63u);
  const uint64_t tq = o >> 6;  // tile*NQ + q
  const uint64_t tile = tq / (uint64_t)NQ;
  const uint32_t q = (uint32_t)(tq - tile * (uint64_t)NQ);
  const uint64_t r = tile * 16u + (l & 15u);
  const uint32_t b = 4u * q + (l >> 4);
  i = r * (uint64_t)KB + b;
  const uint64_t rec = (tile * (uint64_t)NG + (q >> 2)) * MOE_REC_BYTES;
  nib_byte = rec + (uint64_t)(q & 3u) * 1024u + (uint64_t)l * 16u;
  sc_byte = rec + MOE_REC_SC + (uint64_t)l * 4u + (q & 3u);
}

// ggml 17-byte blocks of consecutive expert matrices (per_exp = R*KB blocks
// each, n_blocks in all) -> the device records of the same experts, whose
// matrices are mat_stride bytes apart from w on.
__global__ __launch_bounds__(256) void k_repack_blocks(const uint8_t *__restrict__ src, uint64_t n_blocks,
                                                       uint64_t per_exp, uint64_t mat_stride, int KB,
                                                       uint8_t *__restrict__ w) {
  const uint64_t o = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (o >= n_blocks) return;
  const uint64_t e = o / per_exp, base = e * per_exp;
  uint64_t i, nb, sb;
  layout_of(o - base, KB, i, nb, sb);
  i += base;
  uint8_t *m = w + e * mat_stride;
  const uint8_t *b = src + i * 17u;
  uint32_t v[4];
#pragma unroll
  for (int d = 0; d < 4; d++) {
    v[d] = (uint32_t)b[1 + 4 * d] | ((uint32_t)b[2 + 4 * d] << 8) | ((uint32_t)b[3 + 4 * d] << 16) |
           ((uint32_t)b[4 + 4 * d] << 24);
  }
  *reinterpret_cast<uint4 *>(m + nb) = make_uint4(v[0], v[1], v[2], v[3]);
  m[sb] = b[0];
}

// Inverse: the device records of one matrix -> ggml 17-byte blocks.
__global__ __launch_bounds__(256) void k_unpack_blocks(const uint8_t *__restrict__ m, uint64_t n_blocks, int KB,
                                                       uint8_t *__restrict__ dst) {
  const uint64_t o = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (o >= n_blocks) return;
  uint64_t i, nb, sb;
  layout_of(o, KB, i, nb, sb);
  uint8_t *b = dst + i * 17u;
  const uint4 v = *reinterpret_cast<const uint4 *>(m + nb);
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  b[0] = m[sb];
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
                                                         uint32_t e_span, uint8_t *__restrict__ m) {
  const uint64_t o = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (o >= n_blocks) return;
  uint64_t i, nb, sb;
  layout_of(o, KB, i, nb, sb);
  const uint64_t a = mix64(key + 2u * i + 1u);
  const uint64_t b = mix64(key + 2u * i + 2u);
  const uint64_t c = mix64(key ^ ~i);
  *reinterpret_cast<uint4 *>(m + nb) = make_uint4((uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32));
  m[sb] = (uint8_t)(e_lo + (uint32_t)(((c >> 32) * (uint64_t)e_span) >> 32));
}
