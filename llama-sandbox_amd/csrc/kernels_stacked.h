// kernels_stacked.h -- grouped gate/up and down on items of up to 32 rows,
// the two Q8_0 digit planes stacked along K of one MFMA.
//
// v_mfma_scale_f32_32x32x64_f8f6f4 reduces 64 K per output value.  Here A
// is the item's tokens (A row t = token t) and B the weight tile (B column
// r = weight row r), and the 64 K are one MXFP4 block twice: K 0-31 carry
// the block's hi digits (A scale 2^4), K 32-63 its lo digits (A scale 2^0),
// and both B lane halves (lane r + 32*gb, gb = 0, 1) hold the same weight
// block of row r with its exponent.  D[t][r] is then 2^(e_w - 127) times
// the exact integer block dot of token t and row r (16*hi + lo = q): one
// MFMA is 32 tokens x 32 rows x one block with no zero half, and each
// result value is scaled by its token's d once.  Against an item of up to
// 32 rows one pass over the expert's weights serves every row of the item,
// so an expert with 17-32 rows is streamed once, not twice.
//
// Tokens are A's rows so that a lane's 16 result values are 16 tokens of one
// weight row (D lane r + 32*gb holds column r, tokens 8*i + 4*gb + j at
// element 4*i + j): the d scaling of the tokens an item lacks is skipped
// whole, 4 FMAs per 8 tokens (an item of 9-16 rows pays 8 FMAs per MFMA, not
// 16), at the price of each lane reading its tokens' d as float4s.
//
// Operand lanes (the layouts the octet kernels use): B lane r + 32*gb holds
// weight row r and K [32*gb, 32*gb + 32); the record layout gives lane (r, gb)
// block 2j + gb of a quad in one load (step j), and v_permlane32_swap turns
// that pair into [block 2j | block 2j] and [block 2j+1 | block 2j+1].  A lane
// t + 32*ga holds token t: bytes 0-15 = K [16*ga, +16) (hi digits 16*ga ..
// 16*ga + 15), bytes 16-31 = K [32 + 16*ga, +16) (lo digits, same offsets).
// The A scale of lane t + 32*ga is that of K block ga (hi: 2^4, lo: 2^0).
//
// A is staged in LDS by chunks of MOE_SK_CH quads (8 blocks), double
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
#define MOE_SK_DN_LDS_BYTES (MOE_SK_LDS_BYTES + MOE_SK_WAVES * 32 * 4)  // k_down_sk: + 32 router weights per wave
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
__device__ __forceinline__ void sdma_issue(const sdma &g, const gsrc &src, uint32_t *buf, int wave, int C) {
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

// One block's A operand (the tokens' digits) of this lane, from a chunk buffer.
struct skb {
  u32x4_t lo, hi;
};

__device__ __forceinline__ void load_skb_v(skb &b, const uint32_t *buf, int lane, int st) {
  const u32x4_t *bl = reinterpret_cast<const u32x4_t *>(buf);
  b.lo = bl[(st * 2 + 0) * 64 + lane];
  b.hi = bl[(st * 2 + 1) * 64 + lane];
}

// The d of this lane's result tokens 8*i + 4*gb + (0..3), i < NK, of block
// st of a chunk buffer (NK = the groups of 8 tokens that the item holds).
template <int NK>
__device__ __forceinline__ void load_skd(f32x4_t (&dq)[NK], const uint32_t *buf, int lane, int st) {
  const f32x4_t *s = reinterpret_cast<const f32x4_t *>(buf + MOE_SK_SC_DW + st * 32 + 4 * (lane >> 5));
#pragma unroll
  for (int i = 0; i < NK; i++) dq[i] = s[2 * i];
}

// acc[4i + j] += dq[i][j] * r[4i + j] for the token groups i < NK.
template <int NK>
__device__ __forceinline__ void sk_scale(f32x16_t &acc, const f32x16_t &r, const f32x4_t (&dq)[NK]) {
#pragma unroll
  for (int i = 0; i < NK; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[4 * i + j] = __builtin_fmaf(dq[i][j], r[4 * i + j], acc[4 * i + j]);
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

struct skring {
  u32x4_t w[MOE_SK_RP];  // block pair P in slot P % MOE_SK_RP (pair P = blocks 2P, 2P+1 of the stream)
  uint32_t sc[1][2], scn[1][2];  // exponent dwords of this 4-quad group and the next: lane (r, gb) holds
                                 // block position 2j + gb
  skb b;                         // the next step's A
};

// Weight pair 8*G + SL of the stream (SL may reach into the next group).
template <int CPOL>
__device__ __forceinline__ void load_w32g(u32x4_t &w, const wstream (&ws)[1], const aoff32 &ao, int G, int SL) {
  const int q = SL >> 1, j = SL & 1;
  w = __builtin_amdgcn_raw_buffer_load_b128(ws[0].rec, ao.v + j * 512, (G + (q >> 2)) * MOE_REC_BYTES + (q & 3) * 1024,
                                            CPOL);
}

// VMEM loads a wave issues after its chunk-C staging loads up to the end of
// chunk C: the next group's 2 exponent dwords, and the weight pairs issued
// during the chunk's 4 pairs (3 ahead).
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

// One MFMA step (block st of the chunk buffer cbuf), software-pipelined by
// one step: the MFMA goes out into its own result registers, then the next
// step's digits are read from LDS (nbuf, block nst), then the previous
// step's result is scaled by its tokens' d into acc while this MFMA runs,
// then this step's d is read for the next step's scaling.  The scaled sums
// reach acc in block order; sk_loop adds the last step's after the loop.
// w4, sw: the weight block (both lane halves) and its exponent dword (byte
// SEL); sa: the digits' scale (2^4 hi, 2^0 lo).
template <int SEL, int NK>
__device__ __forceinline__ void sk_step(const u32x4_t &w4, uint32_t sw, skb &b, const uint32_t *cbuf, int st,
                                        const uint32_t *nbuf, int nst, bool next, int lane, int sa, f32x16_t &acc,
                                        f32x16_t &rp, f32x4_t (&dq)[NK]) {
  const i32x8_t wv = {(int)w4.x, (int)w4.y, (int)w4.z, (int)w4.w, 0, 0, 0, 0};
  const i32x8_t xv = {(int)b.lo.x, (int)b.lo.y, (int)b.lo.z, (int)b.lo.w,
                      (int)b.hi.x, (int)b.hi.y, (int)b.hi.z, (int)b.hi.w};
  f32x16_t z;
#pragma unroll
  for (int e = 0; e < 16; e++) z[e] = 0.0f;
  const f32x16_t r = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(xv, wv, z, 0, 4, 0, sa, SEL, (int)sw);
  __builtin_amdgcn_sched_barrier(0);
  if (next) load_skb_v(b, nbuf, lane, nst);
  __builtin_amdgcn_sched_barrier(0);
  sk_scale<NK>(acc, rp, dq);
  asm volatile("" : "+v"(acc));
  __builtin_amdgcn_sched_barrier(0);
  rp = r;
  load_skd<NK>(dq, cbuf, lane, st);
}

// Quad QL (0..3) of the 4-quad group G of the K loop; the group's chunks
// 2G and 2G + 1 are in buffers 0 and 1.  Every group but the last (LAST: G
// == NQ/4 - 1, known at compile time) runs the same code from a rolled loop:
// it stages the chunk after each of its chunks, loads the next group's
// exponents, keeps the weight ring 3 pairs ahead, and each chunk end waits
// for exactly the next chunk's staging (a constant count of younger loads).
// Weights are loaded with cache policy CPOL.
template <int QL, int NQ, int CPOL, int NK, bool LAST>
__device__ __forceinline__ void sk_quad(skring &r, const wstream (&ws)[1], const aoff32 &ao, const gsrc &src,
                                        const sdma &g, uint32_t *lds, int wave, int lane, int sa, int G,
                                        f32x16_t &acc, f32x16_t &rp, f32x4_t (&dq)[NK]) {
  constexpr int NG = NQ / 4, RP = MOE_SK_RP, c = QL >> 1, qc = QL & 1;  // chunk of the group, quad of the chunk
  static_assert(MOE_SK_CH == 2 && RP == 4, "a group is two chunks of two quads, the ring 4 pairs");
  constexpr bool next_chunk = !LAST || c == 0;  // chunk 2G + c + 1 exists
  const uint32_t *buf = lds + c * MOE_SK_BUF_DW;
  if constexpr (qc == 0 && next_chunk) {  // the next chunk's staging, straight into the other buffer
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    sdma_issue(g, src, lds + (c ^ 1) * MOE_SK_BUF_DW, wave, 2 * G + c + 1);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (QL == 0 && !LAST) load_sc32<1>(r.scn, ws, ao, G + 1);
  uint32_t e[4];  // this quad's group exponents, every lane block position 0..3
  dup_halves1(r.sc[0][0], e[0], e[1]);
  dup_halves1(r.sc[0][1], e[2], e[3]);
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int SL = 2 * QL + j + RP - 1;  // the pair 3 ahead, from the group's first pair
    if (!LAST || SL < 8) load_w32g<CPOL>(r.w[SL % RP], ws, ao, G, SL);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    u32x4_t w0, w1;
    dup_halves(r.w[(2 * QL + j) % RP], w0, w1);
    const int st = 4 * qc + 2 * j;  // block of the chunk
    sk_step<QL, NK>(w0, e[2 * j], r.b, buf, st, buf, st + 1, true, lane, sa, acc, rp, dq);
    const bool last_of_chunk = qc == 1 && j == 1;
    sk_step<QL, NK>(w1, e[2 * j + 1], r.b, buf, st + 1, buf, st + 2, !last_of_chunk, lane, sa, acc, rp, dq);
  }
  if constexpr (qc == 1 && next_chunk) {
    // the next chunk has landed in LDS (this wave's loads, then everyone's)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(sdma_after<(LAST ? 2 * (NG - 1) : 0) + c, NQ>()));
    lds_barrier();
    load_skb_v(r.b, lds + (c ^ 1) * MOE_SK_BUF_DW, lane, 0);
  }
}

template <int NQ, int CPOL, int NK, bool LAST>
__device__ __forceinline__ void sk_group(skring &r, const wstream (&ws)[1], const aoff32 &ao, const gsrc &src,
                                         const sdma &g, uint32_t *lds, int wave, int lane, int sa, int G,
                                         f32x16_t &acc, f32x16_t &rp, f32x4_t (&dq)[NK]) {
  sk_quad<0, NQ, CPOL, NK, LAST>(r, ws, ao, src, g, lds, wave, lane, sa, G, acc, rp, dq);
  sk_quad<1, NQ, CPOL, NK, LAST>(r, ws, ao, src, g, lds, wave, lane, sa, G, acc, rp, dq);
  sk_quad<2, NQ, CPOL, NK, LAST>(r, ws, ao, src, g, lds, wave, lane, sa, G, acc, rp, dq);
  sk_quad<3, NQ, CPOL, NK, LAST>(r, ws, ao, src, g, lds, wave, lane, sa, G, acc, rp, dq);
  if constexpr (!LAST) {
    r.sc[0][0] = r.scn[0][0];
    r.sc[0][1] = r.scn[0][1];
  }
}

// The K loop of one wave: its 32-row weight tile over NQ quads against the
// 32 staged tokens (xr: the staged row of token lane&31, < 0 absent).  acc:
// lane r + 32*gb, element 4i + j = weight row r, token 8i + 4gb + j (left 0
// for the groups i >= NK, which hold no token of the item).  CPOL: the
// weights' cache policy (non-temporal where no other item reads them).
template <int NQ, int CPOL, int NK>
__device__ __forceinline__ void sk_loop(const wstream (&ws)[1], const aoff32 &ao, const gsrc &src, int xr, int KB,
                                        bool block_major, int n_rows, uint32_t *lds, int wave, int lane,
                                        f32x16_t &acc) {
  static_assert(NQ % 4 == 0 && NQ >= 8, "whole groups, at least two");
  const sdma g = make_sdma(lane, xr, KB, block_major, n_rows);
  skring r;
  sdma_issue(g, src, lds, wave, 0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  load_sc32<1>(r.sc, ws, ao, 0);
#pragma unroll
  for (int i = 0; i + 1 < MOE_SK_RP; i++) load_w32g<CPOL>(r.w[i], ws, ao, 0, i);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  // chunk 0 has landed (2 exponent dwords and the first weight pairs went out after it)
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 + MOE_SK_RP - 1));
  lds_barrier();
  f32x16_t rp;
  f32x4_t dq[NK];
#pragma unroll
  for (int e = 0; e < 16; e++) {
    acc[e] = 0.0f;
    rp[e] = 0.0f;  // the first step scales a zero result: acc stays +0
  }
#pragma unroll
  for (int i = 0; i < NK; i++) dq[i] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  load_skb_v(r.b, lds, lane, 0);
  const int sa = (lane >> 5) ? 127 : 131;
#pragma unroll 1
  for (int G = 0; G + 1 < NQ / 4; G++) sk_group<NQ, CPOL, NK, false>(r, ws, ao, src, g, lds, wave, lane, sa, G, acc, rp, dq);
  sk_group<NQ, CPOL, NK, true>(r, ws, ao, src, g, lds, wave, lane, sa, NQ / 4 - 1, acc, rp, dq);
  sk_scale<NK>(acc, rp, dq);  // the last step's scaled sums
}

// sk_loop for the item's nk = ceil(rows / 8) groups of 8 tokens and weight
// cache policy (split: the default policy, else non-temporal).
template <int NQ>
__device__ __forceinline__ void sk_loop_any(const wstream (&ws)[1], const aoff32 &ao, const gsrc &src, int xr,
                                            int KB, bool block_major, int n_rows, uint32_t *lds, int wave, int lane,
                                            int nk, bool split, f32x16_t &acc) {
#define MOE_SK_LOOP(CP, K) sk_loop<NQ, CP, K>(ws, ao, src, xr, KB, block_major, n_rows, lds, wave, lane, acc)
  if (split) {
    switch (nk) {
      case 1: MOE_SK_LOOP(0, 1); break;
      case 2: MOE_SK_LOOP(0, 2); break;
      case 3: MOE_SK_LOOP(0, 3); break;
      default: MOE_SK_LOOP(0, 4); break;
    }
  } else {
    switch (nk) {
      case 1: MOE_SK_LOOP(MOE_CPOL_NT, 1); break;
      case 2: MOE_SK_LOOP(MOE_CPOL_NT, 2); break;
      case 3: MOE_SK_LOOP(MOE_CPOL_NT, 3); break;
      default: MOE_SK_LOOP(MOE_CPOL_NT, 4); break;
    }
  }
#undef MOE_SK_LOOP
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
  const int nk = __builtin_amdgcn_readfirstlane((nt + 7) >> 3);
  f32x16_t acc;
  // an expert of one item reads its tiles once: non-temporal, as in decode;
  // the items of a larger expert share them through L2
  sk_loop_any<NQ>(ws, ao, src, xr, KB, false, T, lds, wave, lane, nk, (it.w & MOE_ITEM_SPLIT) != 0, acc);
  lds_barrier();  // every wave is done with the chunk buffers
  float *red = reinterpret_cast<float *>(lds);  // [unit][gate/up][token][row]
#pragma unroll
  for (int e = 0; e < 16; e++)
    red[(((wave & 3) * 2 + (wave >> 2)) * 32 + 8 * (e >> 2) + 4 * gb + (e & 3)) * MOE_UNIT + n] = acc[e];
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
// capacity), 512 threads, LDS MOE_SK_DN_LDS_BYTES.  Requires F == 128 * NQ,
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
  const int nk = __builtin_amdgcn_readfirstlane((nt + 7) >> 3);
  f32x16_t acc;
  const int xr = n < nt ? row0 + n : -1;
  sk_loop_any<NQ>(ws, ao, src, xr, KB, true, n_rows, lds, wave, lane, nk, (it.w & MOE_ITEM_SPLIT) != 0, acc);
  // the router weight of token n, then of this lane's result tokens through
  // the wave's own 32 floats past the chunk buffers
  float *wtl = reinterpret_cast<float *>(lds + 2 * MOE_SK_BUF_DW) + 32 * wave;
  const float wt = (n < nt && !shared) ? wts[perm[row0 + n]] : 1.0f;
  if (gb == 0) wtl[n] = wt;
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  const f32x4_t *wq = reinterpret_cast<const f32x4_t *>(wtl + 4 * gb);
  float *dst = y + (size_t)row0 * H + (size_t)t32 * 32 + n;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    if (i >= nk) break;
    const f32x4_t w4 = wq[2 * i];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int t = 8 * i + 4 * gb + j;
      if (t < nt) dst[(size_t)t * H] = shared ? acc[4 * i + j] : __fmul_rn(acc[4 * i + j], w4[j]);
    }
  }
}
