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
// hi + lo equals v for every element within 2^8 of its block's maximum
// (smaller ones lose only bits below 2^-16 of it): the products, accumulated
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
// Unit = (group j, row block nb): a group is up to kFM = 96 of one active
// expert's token-expert pairs; a row block is gate/up: 128 rows of I (gate
// rows and the same up rows), down: 256 rows of the hidden dimension. Eight
// waves, two per SIMD: waves 0-3 run the MFMAs, waves 4-7 issue the loads. A
// vector-memory issue that waits for room in full memory queues then holds up
// only its loader wave; with one wave doing both, it held up the MFMAs of its
// SIMD too. MFMA wave w owns 4 weight row tiles (gate/up: gate rows 32w ..
// 32w + 31 and the same up rows, so the activation is applied in registers;
// down: rows 64w .. 64w + 63) for every 16-token tile of the unit, up to 4 x 6
// fp32 accumulator tiles; loader wave 4 + w fills the LDS pieces MFMA wave w
// reads. The unit's weights, activation rows (two terms) and scales move
// through kFRing LDS slots, filled by direct-to-LDS loads two k-steps ahead,
// one barrier per k-step. LDS slot: activation hi then lo, 96 rows x 128
// bytes each, the 16-byte chunk c of row r at position c ^ ((r >> 1) & 7) (the
// B reads of 16 lanes then cover all 64 banks once); the activation scale
// dwords (blocks 4ks .. 4ks + 3) of each loader's 24 rows (hi at +0, lo at
// +128 of its 256-byte piece); the weight tiles in A-operand lane order. The
// weight scales go through two further LDS buffers in chunks of 16 k-steps
// (64 bytes of each of the unit's weight rows): a scale row of a unit's 256
// weight rows is then read from memory in whole 64-byte pieces rather than 4
// bytes per k-step, whose 128-byte lines were fetched about ten times each.
//
// Gate/up epilogue: h = act(bf16(gate), bf16(up)) in bf16 (kimi.py:322; the
// activation from the hardware exponential and reciprocal, fast_act), split
// into two E4M3 terms per 32 columns of I (two gate tiles are one block) and
// stored for the down GEMM; down epilogue: bf16 y rows.
#pragma once

#include "k3moe_device.hpp"
#include "k3moe_plan.hpp"

namespace k3moe {

typedef __attribute__((ext_vector_type(8))) int i32x8;

constexpr int kFM = 96;                                   // tokens per unit (at most 6 tiles of 16)
constexpr int kFWaves = 4;                                // MFMA waves (one per SIMD) and as many loaders
constexpr int kFThreads = 2 * kFWaves * 64;
constexpr int kFTiles = 4;                                // weight row tiles per MFMA wave
constexpr int kFRing = 3;                                 // k-step slots in LDS
constexpr int kFSlotX = kFM * 128;                        // one term's rows of a k-step (96 rows)
constexpr int kFOffXS = 2 * kFSlotX;                      // activation scale pieces (256 B per loader)
constexpr int kFOffW = kFOffXS + kFWaves * 256;           // weight tiles (1 KiB each, kFTiles per wave)
constexpr int kFSlot = kFOffW + kFWaves * kFTiles * 1024;  // 41984 bytes
constexpr int kFScSteps = 16;                             // k-steps per weight-scale chunk (64 bytes of a row)
constexpr int kFScBuf = kFWaves * kFTiles * 16 * 64;      // one chunk of the unit's 256 weight rows (16 KiB)
constexpr int kFOffSc = kFRing * kFSlot;                  // the two chunk buffers
constexpr int kFLds = kFOffSc + 2 * kFScBuf;              // 158720 bytes
constexpr int kFAhead = kFRing - 1;                       // k-steps of loads issued ahead of the current one
constexpr int kFRowsL = kFM / kFWaves;                    // activation rows a loader stages (24)
static_assert(kFRowsL % 8 == 0, "8-row activation loads");

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

// s_waitcnt with lgkmcnt(0) and the other counters at their maxima (no wait on them)
constexpr int kLgkmZero = 0xC07F;

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
  __shared__ int s_wsum[2 * kFWaves];
  __shared__ int s_row[2][kFM];              // per unit parity: activation row of each staged row (-1: none)
  const int tid = threadIdx.x, l = tid & 63, i = l & 15, q = l >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool loader = wv >= kFWaves;
  const int w = wv & (kFWaves - 1);  // the MFMA wave (or the one this loader feeds)
  const int nact = *reinterpret_cast<const int *>(ws + pl.o_nact);
  const int *active = reinterpret_cast<const int *>(ws + pl.o_active);
  const int *aoff = reinterpret_cast<const int *>(ws + pl.o_aoff);
  const int *acnt = reinterpret_cast<const int *>(ws + pl.o_acnt);
  const int *ptok = reinterpret_cast<const int *>(ws + pl.o_ptok);
  const uint8_t *zero = reinterpret_cast<const uint8_t *>(ws + pl.o_zero);

  // groups per active expert, exclusive prefix (two experts per thread)
  {
    int t2[2], sum = 0;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int dd = 2 * tid + u;
      t2[u] = dd < nact ? (acnt[dd] + kFM - 1) / kFM : 0;
      sum += t2[u];
    }
    const int incl = wave_incl_scan(sum);
    if (l == 63) s_wsum[wv] = incl;
    __syncthreads();
    int base = 0;
    for (int ww = 0; ww < wv; ++ww) base += s_wsum[ww];
    int excl = base + incl - sum;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int dd = 2 * tid + u;
      if (dd < nact) s_gstart[dd] = excl;
      excl += t2[u];
    }
    if (tid == kFThreads - 1) s_gstart[nact] = base + incl;
    __syncthreads();
  }
  const int J = s_gstart[nact];
  const int Kd = a.width;                  // reduction length, a multiple of 128
  const int KB = Kd / kBlockK, KS = Kd / 128;
  const int Nout = GU ? pl.I : pl.K;
  const int RPB = GU ? 128 : 256;          // output rows per unit
  const int NB = Nout / RPB;
  const int xcds = gridDim.x < 8 ? (int)gridDim.x : 8;
  const int xcd = blockIdx.x % xcds, nslot = gridDim.x / xcds, slot = blockIdx.x / xcds;
  if (slot >= nslot) return;  // (a grid that is not a multiple of the XCD count)
  uint8_t *const hq_hi = reinterpret_cast<uint8_t *>(ws + pl.o_hq);
  uint8_t *const hq_lo = hq_hi + (size_t)pl.P * pl.I;
  uint8_t *const hq_shi = hq_lo + (size_t)pl.P * pl.I;
  uint8_t *const hq_slo = hq_shi + (size_t)pl.P * (pl.I / kBlockK);
  uint16_t *const ybuf = reinterpret_cast<uint16_t *>(ws + pl.o_y);

  // The unit of number v: group j, row block nb, expert e, pairs p0 .. p0 + m - 1.
  struct UnitP {
    int e, p0, m, nb;
  };
  auto unit_of = [&](long v, UnitP &U) -> bool {
    const long j = xcd + (long)xcds * (v / NB);
    if (j >= J) return false;
    U.nb = (int)(v % NB);
    int lo_ = 0, hi_ = nact - 1;  // the group's expert: largest d with s_gstart[d] <= j
    while (lo_ < hi_) {
      const int mid = (lo_ + hi_ + 1) >> 1;
      if (s_gstart[mid] <= j) lo_ = mid; else hi_ = mid - 1;
    }
    const int d = lo_, mt = (int)j - s_gstart[d];
    U.e = active[d];
    U.p0 = aoff[d] + mt * kFM;
    U.m = min(kFM, acnt[d] - mt * kFM);
    return true;
  };
  // a unit's staged rows, written one unit ahead (threads 0 .. kFM - 1, in the
  // MFMA waves) into the buffer of its parity, read by the loaders
  auto fill_rows = [&](const UnitP &U, int buf) {
    if (tid < kFM) s_row[buf][tid] = tid < U.m ? (GU ? ptok[U.p0 + tid] : U.p0 + tid) : -1;
  };

  // Loader 4 + w: MFMA wave w's 4 weight row tiles (gate/up: gate rows 32w +
  // 16r, r < 2, then the same up rows; down: rows 64w + 16r). Weight load r:
  // lane (i, q) takes block 4 ks + q of its row (16 bytes), landing at the
  // tile's 1 KiB in lane order, i.e. in the A-operand layout. Activation rows:
  // the 8-row blocks w + 4u, u < 3; lane L of load u (u < 3: hi, u >= 3: lo,
  // the same rows) covers row 8 (w + 4 (u % 3)) + L / 8 at chunk position L %
  // 8. Scale load (lane L lands at +4 L of the loader's 256-byte piece): lanes
  // 0-23 the hi scale dwords of rows 4 L + w, lanes 32-55 the lo ones (at
  // +128), the other lanes read the zero area; a token tile's scale addresses
  // then differ from the next tile's by a constant. Every load is issued (rows
  // without a token read the zero area), so that every k-step issues the same
  // number of them (and kFTiles more with a weight-scale chunk).
  const uint32_t wlane = (uint32_t)i * KB * 16 + q * 16;                 // row i of a tile, block q
  const size_t wtile = (size_t)16 * KB * 16;                             // tile stride
  const int sci = l >> 2, scp = 16 * (l & 3);
  const uint8_t *const sbase = l < 32 ? a.shi : a.slo;
  const int NSC = (KS + kFScSteps - 1) / kFScSteps;  // scale chunks of a unit
  // chunk c lands with the loads of step sc_step(c): 0 for the first, 2 steps
  // after the first step of chunk c - 1 for the others (its buffer held chunk
  // c - 2, whose last step is done once that step's barrier has passed)
  auto chunk_at = [&](int s) { return s == 0 || (s >= 2 && (s - 2) % kFScSteps == 0 && (s - 2) / kFScSteps + 1 < NSC); };
  constexpr int kNR = kFRowsL / 8;                  // 8-row loads per term
  constexpr int kLoads = 2 * kNR + 1 + kFTiles;     // a loader's loads per step (and kFTiles more with a chunk)
  struct LoadP {  // one unit's load addresses for this lane
    size_t wrow;
    uint32_t aoffs[kNR];
    bool arow[kNR];
    bool srow;
    uint32_t soff;
  };
  auto load_params = [&](const UnitP &U, int buf) {
    LoadP P;
    P.wrow = (size_t)U.e * Nout + U.nb * RPB + (GU ? 32 : 64) * w;
#pragma unroll
    for (int u = 0; u < kNR; ++u) {
      const int r = 8 * (w + kFWaves * u) + (l >> 3);
      const int c = (l & 7) ^ ((r >> 1) & 7);
      const int ar = s_row[buf][r];
      P.arow[u] = ar >= 0;
      P.aoffs[u] = ar >= 0 ? (uint32_t)ar * (uint32_t)Kd + (uint32_t)c * 16 : (uint32_t)(l & 7) * 16;
    }
    const int sar = (l & 31) < kFRowsL ? s_row[buf][kFWaves * (l & 31) + w] : -1;
    P.srow = sar >= 0;
    P.soff = P.srow ? (uint32_t)sar * (uint32_t)KB : 0u;
    return P;
  };
  // The loads of step ks of a unit (P) into ring slot g % kFRing, g the
  // workgroup's running step count; its weight-scale chunk c (if any) into
  // buffer (cb0 + c) & 1, cb0 the unit's first chunk number.
  auto issue = [&](const LoadP &P, int ks, int g, int cb0) {
    char *base = lds + (g % kFRing) * kFSlot;
    if (chunk_at(ks)) {
      const int c = ks == 0 ? 0 : (ks - 2) / kFScSteps + 1;
      const bool cin = 64 * c + scp < KB;  // lane L: bytes 64c + 16 (L % 4) .. of row L / 4 (zero area past the row)
#pragma unroll
      for (int r = 0; r < kFTiles; ++r) {
        const uint8_t *sp = GU ? (r < 2 ? scl0 : scl1) + (P.wrow + 16 * (r & 1) + sci) * KB + 64 * c + scp
                               : scl0 + (P.wrow + 16 * r + sci) * KB + 64 * c + scp;
        load_lds<16>(cin ? sp : zero, lds + kFOffSc + ((cb0 + c) & 1) * kFScBuf + (kFTiles * w + r) * 1024);
      }
    }
#pragma unroll
    for (int r = 0; r < kFTiles; ++r) {
      const uint8_t *tp = GU ? (r < 2 ? blk0 : blk1) + (P.wrow + 16 * (r & 1)) * KB * 16 + wlane
                             : blk0 + P.wrow * KB * 16 + r * wtile + wlane;
      load_lds<16>(tp + ks * 64, base + kFOffW + (kFTiles * w + r) * 1024);
    }
#pragma unroll
    for (int u = 0; u < 2 * kNR; ++u)
      load_lds<16>(P.arow[u % kNR] ? (u < kNR ? a.hi : a.lo) + P.aoffs[u % kNR] + ks * 128 : zero + P.aoffs[u % kNR],
                   base + (u >= kNR ? kFSlotX : 0) + 8 * (w + kFWaves * (u % kNR)) * 128);
    load_lds<4>(P.srow ? sbase + P.soff + 4 * ks : zero, base + kFOffXS + w * 256);
  };

  // Units follow each other without a pause in the loads: the loaders issue a
  // unit's first two steps during the previous unit's last two steps (ring
  // slots and chunk buffers are numbered over the workgroup's whole run), so
  // they land while the MFMA waves finish that unit's epilogue.
  UnitP U, Un;
  long v = slot;
  if (!unit_of(v, U)) return;  // (every wave of the workgroup alike)
  fill_rows(U, 0);
  __syncthreads();
  bool have_n = unit_of(v + nslot, Un);
  if (have_n) fill_rows(Un, 1);
  LoadP Pc, Pn;
  if (loader) {
    Pc = load_params(U, 0);
    issue(Pc, 0, 0, 0);
    issue(Pc, 1, 1, 0);
  }
  for (int uidx = 0;; ++uidx) {
    const int p0 = U.p0, m = U.m, nb = U.nb, T = (m + 15) / 16;
    const int g0 = uidx * KS, cb0 = uidx * NSC;  // the unit's first step and chunk numbers

    // The k-loop and the epilogue for NT token tiles (a compile-time count: the
    // accumulators of tiles past the unit's tokens are never touched, and no
    // control flow depends on the count inside the loop).
    auto run = [&](auto nt) {
      constexpr int NT = decltype(nt)::value;
      if (loader) {
        // two steps ahead: at the barrier of step ks the loads of ks have landed
        // and the MFMA waves are done with step ks - 1, whose slot takes the
        // running step after next (the next unit's first two at the end)
        static_assert(kFAhead == 2, "two k-steps ahead");
        for (int ks = 0; ks < KS; ++ks) {
          // step ks landed (the loads of the step after it may be in flight)
          if (ks + 1 < KS) {
            if (chunk_at(ks + 1)) wait_vm<kLoads + kFTiles>();
            else wait_vm<kLoads>();
          } else if (have_n) {
            wait_vm<kLoads + kFTiles>();  // the next unit's step 0 carries its first chunk
          } else {
            wait_vm<0>();
          }
          ring_barrier();
          if (ks + 2 < KS) {
            issue(Pc, ks + 2, g0 + ks + 2, cb0);
          } else if (have_n) {
            if (ks + 2 == KS) Pn = load_params(Un, (uidx + 1) & 1);  // written before this unit's first barrier
            issue(Pn, ks + 2 - KS, g0 + ks + 2, cb0 + NSC);
          }
        }
        return;
      }
      f32x4 acc[kFTiles][NT];
#pragma unroll
      for (int r = 0; r < kFTiles; ++r)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int ks = 0; ks < KS; ++ks) {
        ring_barrier();  // the loaders' loads of step ks have landed
        const char *base = lds + ((g0 + ks) % kFRing) * kFSlot;
        const char *scb = lds + kFOffSc + ((cb0 + ks / kFScSteps) & 1) * kFScBuf + kFTiles * w * 1024 + 64 * i +
                          4 * (ks % kFScSteps) + q;
        u32x4 wa[kFTiles];
        uint32_t sa[kFTiles];
#pragma unroll
        for (int r = 0; r < kFTiles; ++r) {
          wa[r] = *reinterpret_cast<const u32x4 *>(base + kFOffW + (kFTiles * w + r) * 1024 + 16 * l);
          sa[r] = *reinterpret_cast<const uint8_t *>(scb + r * 1024);
        }
        // token tile t's B operands (both terms) and scales; the reads of tile
        // t + 2 go out after the MFMAs of tile t, so that the MFMAs of tile
        // t + 1 cover their latency (with one MFMA wave per SIMD nothing else does)
        struct BTile {
          i32x8 h, l;
          uint32_t sh, sl;
        };
        auto read_b = [&](int t) {
          const int row = 16 * t + i, sw = (row >> 1) & 7;
          const char *hr = base + row * 128, *lr = hr + kFSlotX;
          const u32x4 h0 = *reinterpret_cast<const u32x4 *>(hr + ((q ^ sw) * 16));
          const u32x4 h1 = *reinterpret_cast<const u32x4 *>(hr + (((4 + q) ^ sw) * 16));
          const u32x4 l0 = *reinterpret_cast<const u32x4 *>(lr + ((q ^ sw) * 16));
          const u32x4 l1 = *reinterpret_cast<const u32x4 *>(lr + (((4 + q) ^ sw) * 16));
          // the scales of row 16t + i are in the piece of loader row % 4, at row / 4
          const char *sp = base + kFOffXS + (row % kFWaves) * 256 + 4 * (row / kFWaves) + q;
          BTile bt;
          bt.sh = *reinterpret_cast<const uint8_t *>(sp);
          bt.sl = *reinterpret_cast<const uint8_t *>(sp + 128);
          bt.h = i32x8{(int)h0[0], (int)h0[1], (int)h0[2], (int)h0[3], (int)h1[0], (int)h1[1], (int)h1[2], (int)h1[3]};
          bt.l = i32x8{(int)l0[0], (int)l0[1], (int)l0[2], (int)l0[3], (int)l1[0], (int)l1[1], (int)l1[2], (int)l1[3]};
          return bt;
        };
        auto mfma_hi = [&](const BTile &b, int t) {
#pragma unroll
          for (int r = 0; r < kFTiles; ++r) acc[r][t] = mfma_fp4x8(wa[r], b.h, sa[r], b.sh, acc[r][t]);
        };
        auto mfma_lo = [&](const BTile &b, int t) {
#pragma unroll
          for (int r = 0; r < kFTiles; ++r) acc[r][t] = mfma_fp4x8(wa[r], b.l, sa[r], b.sl, acc[r][t]);
        };
        // Tile t + 1's reads go out just before the MFMAs of tile t, which cover
        // their latency, after an explicit wait for tile t's: every wait is then
        // for everything outstanding, which is what the compiler can count.
        BTile bb[2];
        bb[0] = read_b(0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          __builtin_amdgcn_s_waitcnt(kLgkmZero);  // tile t's operands (and at t = 0 the weights) are in
          __builtin_amdgcn_sched_barrier(0);
          if (t + 1 < NT) bb[(t + 1) & 1] = read_b(t + 1);
          __builtin_amdgcn_sched_barrier(0);
          mfma_hi(bb[t & 1], t);
          mfma_lo(bb[t & 1], t);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      // (no barrier here: loaders and MFMA waves pass exactly KS barriers per unit)

      // epilogue: lane (token column i, q) holds rows 4q .. 4q + 3 of each tile
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int jrow = 16 * t + i;
        const bool ok = jrow < m;
        const size_t p = (size_t)(p0 + (ok ? jrow : 0));
        if constexpr (GU) {
          // one 32-column block of I per token: gate tiles 0, 1 with up tiles 2, 3
          float h[2][4];
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
            for (int vv = 0; vv < 4; ++vv)
              h[s2][vv] = round_bf16(fast_act(pl.act, round_bf16(acc[s2][t][vv]), round_bf16(acc[2 + s2][t][vv])));
          float m8 = 0.f;
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
            for (int vv = 0; vv < 4; ++vv) m8 = fmaxf(m8, fabsf(h[s2][vv]));
          const uint32_t sh = mx8_scale(group_amax<16, 32>(m8));
          const float ih = mx8_inv(sh), vh = mx8_val(sh);
          uint32_t hw[2], lw[2];
          float rr[2][4];
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            hw[s2] = e4m3x4(h[s2][0] * ih, h[s2][1] * ih, h[s2][2] * ih, h[s2][3] * ih);
#pragma unroll
            for (int vv = 0; vv < 4; ++vv) rr[s2][vv] = __fsub_rn(h[s2][vv], __fmul_rn(e4m3_f32(hw[s2], vv), vh));
          }
          float mr = 0.f;
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
            for (int vv = 0; vv < 4; ++vv) mr = fmaxf(mr, fabsf(rr[s2][vv]));
          const uint32_t sl = mx8_scale(group_amax<16, 32>(mr));
          const float il = mx8_inv(sl);
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) lw[s2] = e4m3x4(rr[s2][0] * il, rr[s2][1] * il, rr[s2][2] * il, rr[s2][3] * il);
          if (ok) {
            const int c0 = nb * RPB + 32 * w;  // the block's first column of I
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
              *reinterpret_cast<uint32_t *>(hq_hi + p * pl.I + c0 + 16 * s2 + 4 * q) = hw[s2];
              *reinterpret_cast<uint32_t *>(hq_lo + p * pl.I + c0 + 16 * s2 + 4 * q) = lw[s2];
            }
            if (q == 0) {
              hq_shi[p * (pl.I / kBlockK) + c0 / kBlockK] = (uint8_t)sh;
              hq_slo[p * (pl.I / kBlockK) + c0 / kBlockK] = (uint8_t)sl;
            }
          }
        } else {
          if (ok) {
#pragma unroll
            for (int r = 0; r < kFTiles; ++r) {
              const f32x4 a4 = acc[r][t];
              const u32x2 packed = {(uint32_t)f32_to_bf16_bits(a4[0]) | ((uint32_t)f32_to_bf16_bits(a4[1]) << 16),
                                    (uint32_t)f32_to_bf16_bits(a4[2]) | ((uint32_t)f32_to_bf16_bits(a4[3]) << 16)};
              *reinterpret_cast<u32x2 *>(ybuf + p * pl.K + nb * RPB + 64 * w + 16 * r + 4 * q) = packed;
            }
          }
        }
      }
    };
    static_assert(kFM == 96, "at most 6 token tiles");
    switch (T) {  // 1 .. 6 (m in 1 .. kFM)
      case 1: run(IntC<1>{}); break;
      case 2: run(IntC<2>{}); break;
      case 3: run(IntC<3>{}); break;
      case 4: run(IntC<4>{}); break;
      case 5: run(IntC<5>{}); break;
      default: run(IntC<6>{}); break;
    }
    if (!have_n) break;
    U = Un;
    if (loader) Pc = Pn;
    have_n = unit_of(v + (long)(uidx + 2) * nslot, Un);
    wait_vm<0>();     // the epilogue's stores (MFMA waves), the next unit's first steps (loaders)
    __syncthreads();  // the loaders are done with the rows of unit uidx, whose buffer takes unit uidx + 2's
    if (have_n) fill_rows(Un, uidx & 1);
  }
}

}  // namespace k3moe
