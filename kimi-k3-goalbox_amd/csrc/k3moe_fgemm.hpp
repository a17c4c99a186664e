// Grouped expert GEMMs on the scaled FP4 MFMA (v_mfma_scale_f32_16x16x128_f8f6f4)
// for prefill-sized steps: the MXFP4 weights go to the MFMA as they are stored
// (E2M1 nibbles and their E8M0 block scales), the activations as two E4M3
// terms with E8M0 block scales.
//
// Activation format ("two-term MXFP8"): a block of 32 values v (bf16-exact)
// is stored as hi = E4M3(v / 2^eh) and lo = E4M3((v - hi 2^eh) / 2^el), where
// eh = floor(log2 max|v|) - 7 and el the same for the remainders, each scale
// one E8M0 byte per block. The MFMA runs once on hi and once on lo into the
// same fp32 accumulator. A bf16 value has 8 significant bits and E4M3 4, so
// hi + lo equals v for every element within 2^9 of its block's maximum
// (smaller ones lose only bits below 2^-17 of it): the products, accumulated
// in fp32, are those of the bf16 operands. A single E4M3 term would leave the
// reference's band (kimi.py:413-429) by a factor of about 7.
//
// Operand layouts of the 16x16x128 MFMA (one wave; measured on gfx950):
//   A (16 weight rows x 128 k, FP4): lane (row i = l % 16, q = l / 16) holds
//     k 32q .. 32q + 31 in 16 bytes, element 2j in the low nibble of byte j:
//     exactly MXFP4 block q of the k-step; its scale byte is that block's.
//   B (128 k x 16 token columns, FP8): lane (column j, q) holds k 16q .. 16q+15
//     in bytes 0-15 and k 64 + 16q .. 64 + 16q + 15 in bytes 16-31; its scale
//     byte is the one of block q (k 32q .. 32q + 31), whatever lane holds it.
//   D (16 x 16 fp32): lane (column j, q) holds rows 4q .. 4q + 3.
//
// Unit = (group j, row block nb) as in the bf16 grouped GEMMs: a group is up
// to kFM = 112 of one active expert's token-expert pairs; a row block is
// gate/up: 256 rows of I (gate rows and the same up rows), down: 512 rows of
// the hidden dimension. Four waves (one per SIMD, so each may hold 512
// registers): wave w owns 8 weight row tiles (gate/up: gate rows 64w .. 64w +
// 63 and the same up rows, so the activation is applied in registers; down:
// rows 128w .. 128w + 127) for every 16-token tile of the unit, up to 8 x 7 fp32
// accumulator tiles (in AGPRs).
// The unit's weights and activation rows (two terms) move through two LDS
// slots, filled by direct-to-LDS loads one k-step ahead (the compiler's own
// waits for loads into registers fall back to waiting for everything across
// the loop), one barrier per k-step. LDS slot: activation hi then lo, 128 rows
// x 128 bytes each, the 16-byte chunk c of row r at position c ^ ((r >> 1) & 7)
// (the B reads of 16 lanes then cover all 64 banks once); the activation scale
// dwords (blocks 4ks .. 4ks + 3) of each wave's 32 rows (hi at +0, lo at +128
// of the wave's 256-byte piece); the weight tiles in A-operand lane order; the
// weight scale dwords of each wave's 128 rows.
//
// Gate/up epilogue: h = act(bf16(gate), bf16(up)) in bf16 (kimi.py:322), split
// into two E4M3 terms per 32 columns of I (two gate tiles are one block) and
// stored for the down GEMM; down epilogue: bf16 y rows.
#pragma once

#include "k3moe_device.hpp"
#include "k3moe_plan.hpp"

namespace k3moe {

typedef __attribute__((ext_vector_type(8))) int i32x8;

constexpr int kFM = 112;                                  // tokens per unit (at most 7 tiles of 16)
constexpr int kFWaves = 4;                                // one wave per SIMD, 512 registers each
constexpr int kFThreads = kFWaves * 64;
constexpr int kFTiles = 8;                                // weight row tiles per wave
constexpr int kFRing = 2;                                 // k-step slots in LDS
constexpr int kFSlotX = 128 * 128;                        // one term's rows of a k-step (128 rows)
constexpr int kFOffXS = 2 * kFSlotX;                      // activation scale pieces (256 B per wave)
constexpr int kFOffW = kFOffXS + kFWaves * 256;           // weight tiles (1 KiB each, 8 per wave)
constexpr int kFOffWS = kFOffW + kFWaves * kFTiles * 1024;  // weight scale pieces (512 B per wave)
constexpr int kFSlot = kFOffWS + kFWaves * 512;           // 68608 bytes
constexpr int kFLds = kFRing * kFSlot;                    // 137216 bytes
constexpr int kFAhead = kFRing - 1;                       // k-steps of loads in flight beyond the current one

// ------------------------------------------------------ two-term MXFP8 --

// E8M0 byte of 2^(floor(log2 amax) - 7) for a block maximum amax >= 0 (0 for
// a zero or subnormal maximum).
__device__ __forceinline__ uint32_t mx8_scale(float amax) {
  const int be = (int)((__float_as_uint(amax) >> 23) & 255u);
  return be > 7 ? (uint32_t)(be - 7) : 0u;
}
// 2^(127 - s) and 2^(s - 127) for an E8M0 byte s <= 248.
__device__ __forceinline__ float mx8_inv(uint32_t s) { return __uint_as_float((254u - s) << 23); }
__device__ __forceinline__ float mx8_val(uint32_t s) { return s ? __uint_as_float(s << 23) : __uint_as_float(0x00400000u); }

// E4M3 bytes (round to nearest even) of four values, packed little-endian.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
}
__device__ __forceinline__ float e4m3_f32(uint32_t word, int byte) {
  switch (byte) {
    case 0: return __builtin_amdgcn_cvt_f32_fp8((int)word, 0);
    case 1: return __builtin_amdgcn_cvt_f32_fp8((int)word, 1);
    case 2: return __builtin_amdgcn_cvt_f32_fp8((int)word, 2);
    default: return __builtin_amdgcn_cvt_f32_fp8((int)word, 3);
  }
}

// Lane-group maximum of |v| over the lanes that xor-differ in `mask` bits
// (Masks: the xor distances, ascending).
template <int... Masks>
__device__ __forceinline__ float group_amax(float m) {
  ((m = fmaxf(m, shfl_xor(m, Masks))), ...);
  return m;
}

// Two-term split of the four values v of a lane; the block spans the lanes
// reached by Masks. Returns the hi and lo E4M3 words and the block's scale
// bytes.
template <int... Masks>
__device__ __forceinline__ void mx8_split4(const float v[4], uint32_t &hi, uint32_t &lo, uint32_t &sh, uint32_t &sl) {
  float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  sh = mx8_scale(group_amax<Masks...>(m));
  const float ih = mx8_inv(sh), vh = mx8_val(sh);
  hi = e4m3x4(v[0] * ih, v[1] * ih, v[2] * ih, v[3] * ih);
  float r[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) r[t] = __fsub_rn(v[t], __fmul_rn(e4m3_f32(hi, t), vh));  // exact
  m = fmaxf(fmaxf(fabsf(r[0]), fabsf(r[1])), fmaxf(fabsf(r[2]), fabsf(r[3])));
  sl = mx8_scale(group_amax<Masks...>(m));
  const float il = mx8_inv(sl);
  lo = e4m3x4(r[0] * il, r[1] * il, r[2] * il, r[3] * il);
}

// Expert inputs [n_rows, K] bf16 -> hi, lo [n_rows, K] E4M3 and shi, slo
// [n_rows, K/32] E8M0. 8 lanes per block of 32 (4 values each).
__global__ __launch_bounds__(256) void k_quant(const uint16_t *__restrict__ x, long n_blocks, uint8_t *__restrict__ hi,
                                               uint8_t *__restrict__ lo, uint8_t *__restrict__ shi,
                                               uint8_t *__restrict__ slo) {
  const int s = threadIdx.x & 7;
  const long stride = (long)gridDim.x * 32;
  for (long blk = (long)blockIdx.x * 32 + (threadIdx.x >> 3); blk < n_blocks; blk += stride) {
    const u32x2 w = *reinterpret_cast<const u32x2 *>(x + blk * 32 + 4 * s);
    const float v[4] = {bf16_bits_to_f32(w[0] & 0xFFFFu), bf16_bits_to_f32(w[0] >> 16),
                        bf16_bits_to_f32(w[1] & 0xFFFFu), bf16_bits_to_f32(w[1] >> 16)};
    uint32_t h, l, sh, sl;
    mx8_split4<1, 2, 4>(v, h, l, sh, sl);
    *reinterpret_cast<uint32_t *>(hi + blk * 32 + 4 * s) = h;
    *reinterpret_cast<uint32_t *>(lo + blk * 32 + 4 * s) = l;
    if (s == 0) {
      shi[blk] = (uint8_t)sh;
      slo[blk] = (uint8_t)sl;
    }
  }
}

// --------------------------------------------------------- grouped GEMM --

__device__ __forceinline__ f32x4 mfma_fp4x8(const u32x4 &a, const i32x8 &b, uint32_t sa, uint32_t sb, f32x4 c) {
  const i32x8 a8 = {(int)a[0], (int)a[1], (int)a[2], (int)a[3], 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8, b, c, 4, 0, 0, (int)sa, 0, (int)sb);
}

template <int N>
struct IntC {
  static constexpr int value = N;
};

// Activation operand arrays of one GEMM: rows of two E4M3 terms and their scales.
struct MxAct {
  const uint8_t *hi, *lo, *shi, *slo;
  int width;  // elements per row (the reduction length)
};

// GU: gate/up -> two-term h (pl.act applied); otherwise down -> bf16 y.
// a: activation rows (GU: token rows, gathered; down: pair rows of the
// grouped order); blk0/scl0 (+ blk1/scl1 for up): MXFP4 weights.
template <bool GU>
__global__ __launch_bounds__(kFThreads, 1) void k_fgemm(Plan pl, MxAct a, const uint8_t *__restrict__ blk0,
                                                       const uint8_t *__restrict__ scl0,
                                                       const uint8_t *__restrict__ blk1,
                                                       const uint8_t *__restrict__ scl1, char *ws) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  __shared__ int s_gstart[kMaxExperts + 1];  // first group of each active expert
  __shared__ int s_wsum[kFWaves];
  __shared__ int s_row[128];                 // activation row of each staged row (-1: none)
  const int tid = threadIdx.x, l = tid & 63, i = l & 15, q = l >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nact = *reinterpret_cast<const int *>(ws + pl.o_nact);
  const int *active = reinterpret_cast<const int *>(ws + pl.o_active);
  const int *aoff = reinterpret_cast<const int *>(ws + pl.o_aoff);
  const int *acnt = reinterpret_cast<const int *>(ws + pl.o_acnt);
  const int *ptok = reinterpret_cast<const int *>(ws + pl.o_ptok);
  const uint8_t *zero = reinterpret_cast<const uint8_t *>(ws + pl.o_zero);

  // groups per active expert, exclusive prefix (four experts per thread)
  {
    int t4[4], sum = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int dd = 4 * tid + u;
      t4[u] = dd < nact ? (acnt[dd] + kFM - 1) / kFM : 0;
      sum += t4[u];
    }
    const int incl = wave_incl_scan(sum);
    if (l == 63) s_wsum[w] = incl;
    __syncthreads();
    int base = 0;
    for (int ww = 0; ww < w; ++ww) base += s_wsum[ww];
    int excl = base + incl - sum;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int dd = 4 * tid + u;
      if (dd < nact) s_gstart[dd] = excl;
      excl += t4[u];
    }
    if (tid == kFThreads - 1) s_gstart[nact] = base + incl;
    __syncthreads();
  }
  const int J = s_gstart[nact];
  const int Kd = a.width;                  // reduction length, a multiple of 128
  const int KB = Kd / kBlockK, KS = Kd / 128;
  const int Nout = GU ? pl.I : pl.K;
  const int RPB = GU ? 256 : 512;          // output rows per unit
  const int NB = Nout / RPB;
  const int xcds = gridDim.x < 8 ? (int)gridDim.x : 8;
  const int xcd = blockIdx.x % xcds, nslot = gridDim.x / xcds, slot = blockIdx.x / xcds;
  if (slot >= nslot) return;  // (a grid that is not a multiple of the XCD count)
  uint8_t *const hq_hi = reinterpret_cast<uint8_t *>(ws + pl.o_hq);
  uint8_t *const hq_lo = hq_hi + (size_t)pl.P * pl.I;
  uint8_t *const hq_shi = hq_lo + (size_t)pl.P * pl.I;
  uint8_t *const hq_slo = hq_shi + (size_t)pl.P * (pl.I / kBlockK);
  uint16_t *const ybuf = reinterpret_cast<uint16_t *>(ws + pl.o_y);

  for (long v = slot;; v += nslot) {
    const long j = xcd + (long)xcds * (v / NB);
    if (j >= J) break;
    const int nb = (int)(v % NB);
    int lo_ = 0, hi_ = nact - 1;  // the group's expert: largest d with s_gstart[d] <= j
    while (lo_ < hi_) {
      const int mid = (lo_ + hi_ + 1) >> 1;
      if (s_gstart[mid] <= j) lo_ = mid; else hi_ = mid - 1;
    }
    const int d = lo_, mt = (int)j - s_gstart[d];
    const int e = active[d], p0 = aoff[d] + mt * kFM;
    const int m = min(kFM, acnt[d] - mt * kFM), T = (m + 15) / 16;
    wait_vm<0>();     // the previous unit's stores are done (the waits below count loads only)
    __syncthreads();  // the previous unit is done with the ring and s_row
    for (int r = tid; r < 128; r += kFThreads) s_row[r] = r < m ? (GU ? ptok[p0 + r] : p0 + r) : -1;
    __syncthreads();

    // this wave's 8 weight row tiles: gate/up: gate rows 64w + 16r (r < 4),
    // then the same up rows; down: rows 128w + 16r. Weight load r: lane (i, q)
    // takes block 4 ks + q of its row (16 bytes), landing at the tile's 1 KiB
    // in lane order, i.e. in the A-operand layout; scale load h: lane L takes
    // the dword of blocks 4 ks .. 4 ks + 3 of row L % 16 of tile 4 h + L / 16.
    // Addresses: a per-lane byte offset from a wave-uniform base, tiles a
    // wave-uniform stride apart.
    const size_t wrow = (size_t)e * Nout + nb * RPB + (GU ? 64 : 128) * w;
    const uint8_t *const wg = blk0 + (wrow * KB + q) * 16;                       // gate (down) tiles
    const uint8_t *const wu = (GU ? blk1 : blk0) + (wrow * KB + q) * 16 + (GU ? 0 : 64 * KB * 16);
    const uint32_t wlane = (uint32_t)i * KB * 16;                                // row i of a tile
    const size_t wtile = (size_t)16 * KB * 16;                                   // tile stride
    const uint8_t *const sg = scl0 + wrow * KB, *const su = (GU ? scl1 : scl0) + wrow * KB + (GU ? 0 : 64 * KB);
    const uint32_t slane = (uint32_t)(16 * (l >> 4) + (l & 15)) * KB;            // tile L/16, row L%16
    // this wave's activation rows 32 w .. 32 w + 31: lane L of load u (u < 4: hi,
    // u >= 4: lo, the same rows) covers row 32 w + 8 (u & 3) + L / 8 at chunk
    // position L % 8; scale load: lanes 0-31 the hi scale dwords of the rows,
    // lanes 32-63 the lo ones. Loads whose rows all lie past the unit's tokens
    // are not issued: the slot keeps stale bytes there, which reach only
    // accumulator columns of tokens that are not stored. Lanes of an issued
    // load whose row has no token read the zero area.
    uint32_t aoffs[4];
    bool arow[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int r = 32 * w + 8 * u + (l >> 3);
      const int c = (l & 7) ^ ((r >> 1) & 7);
      const int ar = s_row[r];
      arow[u] = ar >= 0;
      aoffs[u] = ar >= 0 ? (uint32_t)ar * (uint32_t)Kd + (uint32_t)c * 16 : (uint32_t)(l & 7) * 16;
    }
    const int sar = s_row[32 * w + (l & 31)];
    const bool srow = sar >= 0;
    const uint32_t soff = srow ? (uint32_t)sar * (uint32_t)KB : 0u;
    const uint8_t *const sbase = l < 32 ? a.shi : a.slo;
    int fill = 0;
    auto issue = [&](int ks) {
      char *base = lds + fill * kFSlot;
      fill ^= 1;
#pragma unroll
      for (int r = 0; r < kFTiles; ++r)
        load_lds<16>((r < 4 ? wg + r * wtile : wu + (r - 4) * wtile) + wlane + ks * 64,
                     base + kFOffW + (kFTiles * w + r) * 1024);
      load_lds<4>(sg + slane + 4 * ks, base + kFOffWS + w * 512);
      load_lds<4>(su + slane + 4 * ks, base + kFOffWS + w * 512 + 256);
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (32 * w + 8 * (u & 3) < m)  // wave-uniform
          load_lds<16>(arow[u & 3] ? (u < 4 ? a.hi : a.lo) + aoffs[u & 3] + ks * 128 : zero + aoffs[u & 3],
                       base + (u >= 4 ? kFSlotX : 0) + (32 * w + 8 * (u & 3)) * 128);
      if (32 * w < m) load_lds<4>(srow ? sbase + soff + 4 * ks : zero, base + kFOffXS + w * 256);
    };

    // The k-loop and the epilogue for NT token tiles (a compile-time count: the
    // accumulators of tiles past the unit's tokens are never touched, and no
    // control flow depends on the count inside the loop).
    auto run = [&](auto nt) {
      constexpr int NT = decltype(nt)::value;
      f32x4 acc[kFTiles][NT];
#pragma unroll
      for (int r = 0; r < kFTiles; ++r)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};

      static_assert(kFRing == 2 && kFAhead == 1, "one k-step of loads in flight");
      issue(0);
      int slot_rd = 0;
      for (int ks = 0; ks < KS; ++ks) {
        wait_vm<0>();    // this wave's loads of step ks have landed (none later are in flight)
        ring_barrier();  // everyone's have, and everyone is done with step ks - 1's slot
        if (ks + 1 < KS) issue(ks + 1);
        const char *base = lds + slot_rd * kFSlot;
        slot_rd ^= 1;
        u32x4 wa[kFTiles];
        uint32_t sa[kFTiles];
#pragma unroll
        for (int r = 0; r < kFTiles; ++r) {
          wa[r] = *reinterpret_cast<const u32x4 *>(base + kFOffW + (kFTiles * w + r) * 1024 + 16 * l);
          sa[r] = *reinterpret_cast<const uint8_t *>(base + kFOffWS + w * 512 + 4 * (16 * r + i) + q);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          // one token tile's operand reads at a time: hoisting every tile's reads
          // would not fit beside the accumulators
          __builtin_amdgcn_sched_barrier(0);
          const int row = 16 * t + i, sw = (row >> 1) & 7;
          const char *hr = base + row * 128, *lr = hr + kFSlotX;
          const u32x4 h0 = *reinterpret_cast<const u32x4 *>(hr + ((q ^ sw) * 16));
          const u32x4 h1 = *reinterpret_cast<const u32x4 *>(hr + (((4 + q) ^ sw) * 16));
          const u32x4 l0 = *reinterpret_cast<const u32x4 *>(lr + ((q ^ sw) * 16));
          const u32x4 l1 = *reinterpret_cast<const u32x4 *>(lr + (((4 + q) ^ sw) * 16));
          // rows 16t .. 16t + 15 were staged by wave t / 2, at row 16 (t & 1) + i of its piece
          const char *sp = base + kFOffXS + (t >> 1) * 256 + 4 * (16 * (t & 1) + i) + q;
          const uint32_t sbh = *reinterpret_cast<const uint8_t *>(sp);
          const uint32_t sbl = *reinterpret_cast<const uint8_t *>(sp + 128);
          const i32x8 bh = {(int)h0[0], (int)h0[1], (int)h0[2], (int)h0[3],
                            (int)h1[0], (int)h1[1], (int)h1[2], (int)h1[3]};
          const i32x8 bl = {(int)l0[0], (int)l0[1], (int)l0[2], (int)l0[3],
                            (int)l1[0], (int)l1[1], (int)l1[2], (int)l1[3]};
#pragma unroll
          for (int r = 0; r < kFTiles; ++r) acc[r][t] = mfma_fp4x8(wa[r], bh, sa[r], sbh, acc[r][t]);
#pragma unroll
          for (int r = 0; r < kFTiles; ++r) acc[r][t] = mfma_fp4x8(wa[r], bl, sa[r], sbl, acc[r][t]);
        }
      }

      // epilogue: lane (token column i, q) holds rows 4q .. 4q + 3 of each tile
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int jrow = 16 * t + i;
        const bool ok = jrow < m;
        const size_t p = (size_t)(p0 + (ok ? jrow : 0));
        if constexpr (GU) {
          // two 32-column blocks of I per token: gate tiles 2b, 2b + 1 with up tiles 4 + 2b, 5 + 2b
#pragma unroll
          for (int b = 0; b < 2; ++b) {
            float h[2][4];
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
              for (int vv = 0; vv < 4; ++vv)
                h[s][vv] = round_bf16(apply_act(pl.act, round_bf16(acc[2 * b + s][t][vv]),
                                                round_bf16(acc[4 + 2 * b + s][t][vv])));
            float m8 = 0.f;
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
              for (int vv = 0; vv < 4; ++vv) m8 = fmaxf(m8, fabsf(h[s][vv]));
            const uint32_t sh = mx8_scale(group_amax<16, 32>(m8));
            const float ih = mx8_inv(sh), vh = mx8_val(sh);
            uint32_t hw[2], lw[2];
            float rr[2][4];
#pragma unroll
            for (int s = 0; s < 2; ++s) {
              hw[s] = e4m3x4(h[s][0] * ih, h[s][1] * ih, h[s][2] * ih, h[s][3] * ih);
#pragma unroll
              for (int vv = 0; vv < 4; ++vv) rr[s][vv] = __fsub_rn(h[s][vv], __fmul_rn(e4m3_f32(hw[s], vv), vh));
            }
            float mr = 0.f;
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
              for (int vv = 0; vv < 4; ++vv) mr = fmaxf(mr, fabsf(rr[s][vv]));
            const uint32_t sl = mx8_scale(group_amax<16, 32>(mr));
            const float il = mx8_inv(sl);
#pragma unroll
            for (int s = 0; s < 2; ++s) lw[s] = e4m3x4(rr[s][0] * il, rr[s][1] * il, rr[s][2] * il, rr[s][3] * il);
            if (ok) {
              const int c0 = nb * RPB + 64 * w + 32 * b;  // the block's first column of I
#pragma unroll
              for (int s = 0; s < 2; ++s) {
                *reinterpret_cast<uint32_t *>(hq_hi + p * pl.I + c0 + 16 * s + 4 * q) = hw[s];
                *reinterpret_cast<uint32_t *>(hq_lo + p * pl.I + c0 + 16 * s + 4 * q) = lw[s];
              }
              if (q == 0) {
                hq_shi[p * (pl.I / kBlockK) + c0 / kBlockK] = (uint8_t)sh;
                hq_slo[p * (pl.I / kBlockK) + c0 / kBlockK] = (uint8_t)sl;
              }
            }
          }
        } else {
          if (ok) {
#pragma unroll
            for (int r = 0; r < kFTiles; ++r) {
              const f32x4 a4 = acc[r][t];
              const u32x2 packed = {(uint32_t)f32_to_bf16_bits(a4[0]) | ((uint32_t)f32_to_bf16_bits(a4[1]) << 16),
                                    (uint32_t)f32_to_bf16_bits(a4[2]) | ((uint32_t)f32_to_bf16_bits(a4[3]) << 16)};
              *reinterpret_cast<u32x2 *>(ybuf + p * pl.K + nb * RPB + 128 * w + 16 * r + 4 * q) = packed;
            }
          }
        }
      }
    };
    static_assert(kFM <= 112, "at most 7 token tiles: 8 x 7 accumulator tiles leave AGPRs to spare");
    switch (T) {  // 1 .. 7 (m in 1 .. kFM)
      case 1: run(IntC<1>{}); break;
      case 2: run(IntC<2>{}); break;
      case 3: run(IntC<3>{}); break;
      case 4: run(IntC<4>{}); break;
      case 5: run(IntC<5>{}); break;
      case 6: run(IntC<6>{}); break;
      default: run(IntC<7>{}); break;
    }
  }
}

}  // namespace k3moe
