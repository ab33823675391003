// kernels_stacked.h -- grouped gate/up and down on items of up to 32 rows,
// the two Q8_0 digit planes stacked along K of one MFMA.
//
// v_mfma_scale_f32_32x32x64_f8f6f4 reduces 64 K per output column.  Here a
// column is one token and its 64 K are one MXFP4 block twice: K 0-31 carry
// the block's hi digits (B scale 2^4), K 32-63 its lo digits (B scale 2^0),
// and both A lane halves (lane r + 32*ga, ga = 0, 1) hold the same weight
// block of row r with its exponent.  Column n of the result is then
// 2^(e_w - 127) times token n's exact integer block dot (16*hi + lo = q):
// one MFMA is 32 rows x 32 tokens x one block with no zero half in B, and
// each result value is scaled by its token's d once (16 FMAs per 32x32
// block product; the octet kernels spend 16 per 32 rows x 8 tokens x 2
// blocks).  Against an item of up to 32 rows one pass over the expert's
// weights serves every row of the item, so an expert with 17-32 rows is
// streamed once, not twice.
//
// Operand lanes (the layouts the octet kernels use): A lane r + 32*ga holds
// row r and K [32*ga, 32*ga + 32); the record layout gives lane (r, ga) block
// 2j + ga of a quad in one load (step j), and v_permlane32_swap turns that
// pair into [block 2j | block 2j] and [block 2j+1 | block 2j+1].  B lane
// n + 32*gb holds column n: bytes 0-15 = K [16*gb, +16) (hi digits 16*gb ..
// 16*gb + 15), bytes 16-31 = K [32 + 16*gb, +16) (lo digits, same offsets).
// The B scale of lane n + 32*gb is that of K block gb (hi: 2^4, lo: 2^0).
// D lane n + 32*gb holds column n, rows 8*i + 4*gb + j at element 4*i + j.
//
// B is staged in LDS by chunks of MOE_SK_CH quads (8 blocks), double
// buffered, with direct global-to-LDS loads: per block, two 1 KiB runs (the
// 64 lanes' bytes 0-15, then bytes 16-31, each lane 16 consecutive bytes,
// so the operand reads are conflict-free), then the chunk's scales
// [block][32 tokens].  An absent token reads zeros (out-of-range offset).
// The x rows are read from the grouped chain's staged x; the h rows that
// k_gate_up_sk writes for k_down_sk are block-major, so the 32 rows of an
// item are adjacent for each block.
#pragma once

#include "kernels_grouped.h"

#define MOE_SK_CH 2                            // quads per staged chunk (4: 16 blocks, 100 VGPRs, measured 2% slower)
#define MOE_SK_STEPS (4 * MOE_SK_CH)           // blocks (MFMA steps) per chunk
#define MOE_SK_STEP_U4 128                     // 16-byte units per block: [2 halves][64 lanes]
#define MOE_SK_SC_DW (MOE_SK_STEPS * MOE_SK_STEP_U4 * 4)  // dword offset of the scales in a chunk buffer
#define MOE_SK_BUF_DW (MOE_SK_SC_DW + MOE_SK_STEPS * 32)  // dwords per chunk buffer (17 KiB)
#define MOE_SK_LDS_BYTES (2 * MOE_SK_BUF_DW * 4)          // two chunk buffers (34 KiB)
#define MOE_SK_WAVES 8                          // waves per workgroup (one 32-row weight tile each)
#define MOE_SK_RP 4  // weight ring, in block pairs (3 ahead: 3 KiB in flight per wave; 2 and 5 ahead measured the same)

// This lane's staging offsets at block 0 of the staged rows (MOE_OOB: absent
// token): digits of token lane&31, K half lane>>5; scale of token lane&31,
// block lane>>5.  The staged rows are row-major ([row][block], x) or
// block-major ([block][row], the h rows these kernels write): bs / bs4 =
// bytes from one block to the next of a row, digits / scales.
struct sdma {
  uint32_t xo, so, bs, bs4;
};

__device__ __forceinline__ sdma make_sdma(int lane, int xr, int KB, bool block_major, int n_rows) {
  sdma s;
  const uint32_t rs = block_major ? MOE_XSW * 4 : (uint32_t)KB * MOE_XSW * 4, rs4 = block_major ? 4 : (uint32_t)KB * 4;
  s.bs = block_major ? (uint32_t)n_rows * MOE_XSW * 4 : MOE_XSW * 4;
  s.bs4 = block_major ? (uint32_t)n_rows * 4 : 4;
  s.xo = xr >= 0 ? (uint32_t)xr * rs + (uint32_t)(lane >> 5) * 16 : MOE_OOB;
  s.so = xr >= 0 ? (uint32_t)xr * rs4 + (uint32_t)(lane >> 5) * s.bs4 : MOE_OOB;
  return s;
}

// Chunk C of the staged rows into buf: wave w loads the blocks w*SW ..
// w*SW + SW - 1 of the chunk (both halves; SW = blocks per wave) and the
// scales of two blocks (waves below MOE_SK_STEPS/2): 2*SW + 1 loads or 2*SW.
#define MOE_SK_SW (MOE_SK_STEPS / MOE_SK_WAVES)
template <int C>
__device__ __forceinline__ void sdma_issue(const sdma &g, const gsrc &src, uint32_t *buf, int wave) {
  typedef __attribute__((address_space(3))) void *lds_t;
#pragma unroll
  for (int i = 0; i < MOE_SK_SW; i++) {
    const int st = MOE_SK_SW * wave + i;
#pragma unroll
    for (int h = 0; h < 2; h++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(src.x, (lds_t)(buf + (st * 2 + h) * 64 * 4), 16, g.xo,
                                               (MOE_SK_STEPS * C + st) * g.bs + h * 32, 0, 0);
  }
  if (wave < MOE_SK_STEPS / 2)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(src.d, (lds_t)(buf + MOE_SK_SC_DW + 2 * wave * 32), 4, g.so,
                                             (MOE_SK_STEPS * C + 2 * wave) * g.bs4, 0, 0);
}

// One block's B operand and d of this lane, from a chunk buffer.
struct skb {
  u32x4_t lo, hi;
  float d;
};

__device__ __forceinline__ void load_skb_v(skb &b, const uint32_t *buf, int lane, int st) {
  const u32x4_t *bl = reinterpret_cast<const u32x4_t *>(buf);
  b.lo = bl[(st * 2 + 0) * 64 + lane];
  b.hi = bl[(st * 2 + 1) * 64 + lane];
}

__device__ __forceinline__ void load_skb_d(skb &b, const uint32_t *buf, int lane, int st) {
  b.d = reinterpret_cast<const float *>(buf + MOE_SK_SC_DW)[st * 32 + (lane & 31)];
}

// [x | x] and [y | y] from a register holding x in lanes 0-31, y in 32-63.
__device__ __forceinline__ void dup_halves(const u32x4_t &w, u32x4_t &a0, u32x4_t &a1) {
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const auto p = __builtin_amdgcn_permlane32_swap(w[c], w[c], false, false);
    a0[c] = p[0];
    a1[c] = p[1];
  }
}

__device__ __forceinline__ void dup_halves1(uint32_t w, uint32_t &a0, uint32_t &a1) {
  const auto p = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  a0 = p[0];
  a1 = p[1];
}

template <int NG>
struct skring {
  u32x4_t w[MOE_SK_RP];  // block pair P in slot P % MOE_SK_RP (pair P = blocks 2P, 2P+1 of the stream)
  uint32_t sc[NG][1][2];  // exponent dwords of each 4-quad group: lane (r, ga) holds block position 2j + ga
  skb b;                 // the next step's B
};

// VMEM loads a wave issues after its chunk-C staging loads up to the end of
// chunk C: the next group's 2 exponent dwords, and the weight pairs issued
// during the chunk's 8 pairs (3 ahead).
template <int C, int NQ>
__host__ __device__ constexpr int sdma_after() {
  int n = 0;
  for (int q = MOE_SK_CH * C; q < MOE_SK_CH * (C + 1); q++) {
    if ((q & 3) == 0 && q / 4 + 1 < NQ / 4) n += 2;  // the next group's exponent dwords
    for (int j = 0; j < 2; j++)
      if (2 * q + j + MOE_SK_RP - 1 < 2 * NQ) n++;  // weight pairs
  }
  return n;
}

// One MFMA step (block position POS of quad QL, block st of the chunk),
// software-pipelined by one step: the MFMA goes out into its own result
// registers, then the next step's digits are read from LDS, then the
// previous step's result is scaled by its d into acc (PREV) while this MFMA
// runs, then the next d.  The scaled sums reach acc in block order, as
// without the pipelining; sk_loop adds the last step's after the loop.
template <int SEL, bool PREV>
__device__ __forceinline__ void sk_step(const u32x4_t &a4, uint32_t sa, skb &b, const uint32_t *nbuf, int nst,
                                        bool next, int lane, int sb, f32x16_t &acc, f32x16_t &rp, float &dp) {
  const i32x8_t a = {(int)a4.x, (int)a4.y, (int)a4.z, (int)a4.w, 0, 0, 0, 0};
  const i32x8_t bv = {(int)b.lo.x, (int)b.lo.y, (int)b.lo.z, (int)b.lo.w,
                      (int)b.hi.x, (int)b.hi.y, (int)b.hi.z, (int)b.hi.w};
  f32x16_t z;
#pragma unroll
  for (int e = 0; e < 16; e++) z[e] = 0.0f;
  const f32x16_t r = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, bv, z, 4, 0, SEL, (int)sa, 0, sb);
  const float d = b.d;
  __builtin_amdgcn_sched_barrier(0);
  if (next) load_skb_v(b, nbuf, lane, nst);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (PREV) {
    acc = acc + dp * rp;
    asm volatile("" : "+v"(acc));
  }
  __builtin_amdgcn_sched_barrier(0);
  rp = r;
  dp = d;
  if (next) load_skb_d(b, nbuf, lane, nst);
}

// Quads QL .. NQ-1 of the K loop (weights loaded with cache policy CPOL).
template <int QL, int NQ, int CPOL>
__device__ __forceinline__ void sk_from(skring<NQ / 4> &r, const wstream (&ws)[1], const aoff32 &ao,
                                        const gsrc &src, const sdma &g, uint32_t *lds, int wave, int lane, int sb,
                                        f32x16_t &acc, f32x16_t &rp, float &dp) {
  if constexpr (QL < NQ) {
    constexpr int NG = NQ / 4, C = QL / MOE_SK_CH, QC = QL % MOE_SK_CH, NC = NQ / MOE_SK_CH, RP = MOE_SK_RP;
    const uint32_t *buf = lds + (C & 1) * MOE_SK_BUF_DW;
    if constexpr (QC == 0 && C + 1 < NC) {  // the next chunk's staging, straight into the other buffer
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      sdma_issue<C + 1>(g, src, lds + ((C + 1) & 1) * MOE_SK_BUF_DW, wave);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr ((QL & 3) == 0 && QL / 4 + 1 < NG) load_sc32<1>(r.sc[QL / 4 + 1], ws, ao, QL / 4 + 1);
    uint32_t e[4];  // this quad's group exponents, every lane block position 0..3
    dup_halves1(r.sc[QL / 4][0][0], e[0], e[1]);
    dup_halves1(r.sc[QL / 4][0][1], e[2], e[3]);
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int P = 2 * QL + j;
      if (P + RP - 1 < 2 * NQ) load_w32step<CPOL>(r.w[(P + RP - 1) % RP], ws, ao, P + RP - 1);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      u32x4_t a0, a1;
      dup_halves(r.w[P % RP], a0, a1);
      const int st = 4 * QC + 2 * j;  // block of the chunk
      if (QL == 0 && j == 0) sk_step<QL & 3, false>(a0, e[2 * j], r.b, buf, st + 1, true, lane, sb, acc, rp, dp);
      else sk_step<QL & 3, true>(a0, e[2 * j], r.b, buf, st + 1, true, lane, sb, acc, rp, dp);
      const bool last_of_chunk = QC + 1 == MOE_SK_CH && j == 1;
      sk_step<QL & 3, true>(a1, e[2 * j + 1], r.b, buf, st + 2, !last_of_chunk, lane, sb, acc, rp, dp);
    }
    if constexpr (QC + 1 == MOE_SK_CH && C + 1 < NC) {
      // the next chunk has landed in LDS (this wave's loads, then everyone's)
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(sdma_after<C, NQ>()));
      const uint32_t *nb = lds + ((C + 1) & 1) * MOE_SK_BUF_DW;
      lds_barrier();
      load_skb_v(r.b, nb, lane, 0);
      load_skb_d(r.b, nb, lane, 0);
    }
    sk_from<QL + 1, NQ, CPOL>(r, ws, ao, src, g, lds, wave, lane, sb, acc, rp, dp);
  }
}

// The K loop of one wave: its 32-row weight tile over NQ quads against the
// 32 staged tokens (xr: the staged row of token lane&31, < 0 absent).
// acc: lane n + 32*gb, element 4i + j = token n, row 8i + 4gb + j.  CPOL:
// the weights' cache policy (non-temporal where no other item reads them).
template <int NQ, int CPOL>
__device__ __forceinline__ void sk_loop(const wstream (&ws)[1], const aoff32 &ao, const gsrc &src, int xr, int KB,
                                        bool block_major, int n_rows, uint32_t *lds, int wave, int lane,
                                        f32x16_t &acc) {
  static_assert(NQ % MOE_SK_CH == 0, "whole chunks");
  const sdma g = make_sdma(lane, xr, KB, block_major, n_rows);
  skring<NQ / 4> r;
  sdma_issue<0>(g, src, lds, wave);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  load_sc32<1>(r.sc[0], ws, ao, 0);
#pragma unroll
  for (int i = 0; i + 1 < MOE_SK_RP; i++)
    if (i < 2 * NQ) load_w32step<CPOL>(r.w[i], ws, ao, i);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  // chunk 0 has landed (2 exponent dwords and the first weight pairs went out after it)
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 + (MOE_SK_RP - 1 < 2 * NQ ? MOE_SK_RP - 1 : 2 * NQ)));
  lds_barrier();
#pragma unroll
  for (int e = 0; e < 16; e++) acc[e] = 0.0f;
  load_skb_v(r.b, lds, lane, 0);
  load_skb_d(r.b, lds, lane, 0);
  f32x16_t rp;
  float dp = 0.0f;
  sk_from<0, NQ, CPOL>(r, ws, ao, src, g, lds, wave, lane, (lane >> 5) ? 127 : 131, acc, rp, dp);
  acc = acc + dp * rp;  // the last step's scaled sum
}

// gate/up -> clamp -> SwiGLU -> Q8_0(h) on items of up to 32 rows.  One
// workgroup of 8 waves per (4 units of F, item): wave w streams the gate
// (w < 4) or up tile of unit 4*blockIdx.x + w%4 over all of K against the
// item's tokens; gate and up meet in LDS.  grid (F/128, item capacity), 512
// threads, LDS MOE_SK_LDS_BYTES.  Requires H == 128 * NQ, NQ % 4 == 0,
// (F/32) % 4 == 0.
template <int NQ>
__global__ __launch_bounds__(64 * MOE_SK_WAVES) __attribute__((amdgpu_waves_per_eu(4)))
void k_gate_up_sk(const uint8_t *__restrict__ w_g, const uint8_t *__restrict__ w_u, const uint32_t *__restrict__ xq,
                  const float *__restrict__ xd, const int32_t *__restrict__ items, const int32_t *__restrict__ perm,
                  int k, int T, int F, int H, float clamp, uint32_t *__restrict__ hs, float *__restrict__ hd,
                  float *__restrict__ htap) {
  extern __shared__ __align__(16) uint32_t lds[];
  if ((int)blockIdx.y >= items[0]) return;
  const int4 it = item_of(items, blockIdx.y);
  constexpr int NQ4 = NQ / 4, KB = NQ * 4;
  const int tiles = F / MOE_TILE;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int P = T * k, NR = P + T, row0 = it.y, nt = it.z;
  const bool shared = (it.w & MOE_ITEM_SHARED) != 0;
  const int u = 4 * blockIdx.x + (wave & 3);
  const wstream ws[1] = {make_wstream32(wave >= 4 ? w_u : w_g, (size_t)it.x * tiles + 2 * u, NQ4)};
  const aoff32 ao = make_aoff32(lane, NQ4);
  const gsrc src = make_gsrc(xq, xd, T, KB);
  const int n = lane & 31, gb = lane >> 5;
  const int xr = n < nt ? (shared ? row0 + n - P : perm[row0 + n] / k) : -1;
  f32x16_t acc;
  // an expert of one item reads its tiles once: non-temporal, as in decode;
  // the items of a larger expert share them through L2
  if (it.w & MOE_ITEM_SPLIT) sk_loop<NQ, 0>(ws, ao, src, xr, KB, false, T, lds, wave, lane, acc);
  else sk_loop<NQ, MOE_CPOL_NT>(ws, ao, src, xr, KB, false, T, lds, wave, lane, acc);
  lds_barrier();  // every wave is done with the chunk buffers
  float *red = reinterpret_cast<float *>(lds);  // [unit][gate/up][token][row]
#pragma unroll
  for (int e = 0; e < 16; e++)
    red[(((wave & 3) * 2 + (wave >> 2)) * 32 + n) * MOE_UNIT + 8 * (e >> 2) + 4 * gb + (e & 3)] = acc[e];
  __syncthreads();
  // (unit, token) c = 16*round + 2*wave + half-wave: unit c / 32, token c % 32
#pragma unroll
  for (int round = 0; round < 8; round++) {
    if ((round & 1) && nt <= 16) continue;  // odd rounds hold tokens 16..31 (uniform over the workgroup)
    const int c = 16 * round + 2 * wave + (lane >> 5);
    const int ul = c >> 5, t = c & 31, j = lane & 31;
    const bool live = t < nt;
    const float gsum = red[((ul * 2 + 0) * 32 + t) * MOE_UNIT + j];
    const float usum = red[((ul * 2 + 1) * 32 + t) * MOE_UNIT + j];
    const float h = live ? swiglu(gsum, usum, clamp) : 0.0f;
    const int hrow = row0 + (live ? t : 0), uu = 4 * blockIdx.x + ul;
    // h block-major ([unit of F][grouped row]): an item's rows of one unit are adjacent
    h_unit_store(h, live, hs + ((size_t)uu * NR + hrow) * MOE_XSW, hd + (size_t)uu * NR + hrow, lane);
    if (htap && live) htap[(size_t)hrow * F + (size_t)uu * MOE_UNIT + j] = h;
  }
}

// down x router weight on items of up to 32 rows: one workgroup of 8 waves
// per (256 rows of H, item), wave = one 32-row tile of H over all of F
// against the item's h rows; y[row] = the tile's rows x the pair's router
// weight (the shared expert's rows unweighted).  grid (H/256, item
// capacity), 512 threads, LDS MOE_SK_LDS_BYTES.  Requires F == 128 * NQ,
// NQ % 4 == 0, H % 256 == 0.
template <int NQ>
__global__ __launch_bounds__(64 * MOE_SK_WAVES) __attribute__((amdgpu_waves_per_eu(4)))
void k_down_sk(const uint8_t *__restrict__ w_d, const uint32_t *__restrict__ hs, const float *__restrict__ hd,
               int n_rows, const int32_t *__restrict__ items, const int32_t *__restrict__ perm,
               const float *__restrict__ wts, int F, int H, float *__restrict__ y) {
  extern __shared__ __align__(16) uint32_t lds[];
  if ((int)blockIdx.y >= items[0]) return;
  const int4 it = item_of(items, blockIdx.y);
  constexpr int NQ4 = NQ / 4, KB = NQ * 4;
  const int tiles = H / MOE_TILE;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = it.y, nt = it.z;
  const bool shared = (it.w & MOE_ITEM_SHARED) != 0;
  const int t32 = blockIdx.x * MOE_SK_WAVES + wave;  // 32-row tile of H
  const wstream ws[1] = {make_wstream32(w_d, (size_t)it.x * tiles + 2 * t32, NQ4)};
  const aoff32 ao = make_aoff32(lane, NQ4);
  const gsrc src = make_gsrc(hs, hd, n_rows, KB);
  const int n = lane & 31, gb = lane >> 5;
  const bool live = n < nt;
  f32x16_t acc;
  if (it.w & MOE_ITEM_SPLIT) sk_loop<NQ, 0>(ws, ao, src, live ? row0 + n : -1, KB, true, n_rows, lds, wave, lane, acc);
  else sk_loop<NQ, MOE_CPOL_NT>(ws, ao, src, live ? row0 + n : -1, KB, true, n_rows, lds, wave, lane, acc);
  const int rr = row0 + (live ? n : 0);
  const float wt = (live && !shared) ? wts[perm[rr]] : 1.0f;
  float v[16];
#pragma unroll
  for (int e = 0; e < 16; e++) v[e] = shared ? acc[e] : __fmul_rn(acc[e], wt);
  if (live) {
    float *dst = y + (size_t)rr * H + (size_t)t32 * 32 + 4 * gb;
#pragma unroll
    for (int i = 0; i < 4; i++)
      *reinterpret_cast<float4 *>(dst + 8 * i) = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
  }
}
