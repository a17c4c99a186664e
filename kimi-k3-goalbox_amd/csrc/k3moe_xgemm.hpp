// Grouped expert GEMMs for batches with many tokens per expert (prefill-sized
// steps of the general path): the gate/up and down projections of
// kimi.py:321-322 as one GEMM per active expert, MXFP4 weights decoded in
// registers, bf16 MFMA with fp32 accumulation.
//
// Unit = (group j, row block nb). A group is one active expert's tile of up to
// kXM = 128 of its tokens (pairs aoff[d] + 128 mt ..); a row block is a block
// of output rows: gate/up 128 rows of I (with the same 128 up rows: 256 weight
// rows), down 256 rows of the hidden dimension. One workgroup of 8 waves runs
// a unit: wave w takes 4 16-row weight tiles (row group w mod 4) for half of
// the unit's 16-token tiles (t = 2 tt + w / 4), so every weight byte of the
// unit is read once from memory and decoded by two waves.
//
// Operands move 128 k at a time ("k-step") through a ring of kXRing LDS slots
// filled by direct-to-LDS loads (global_load_lds), two k-steps ahead of the
// MFMAs; one barrier per k-step. Each wave loads 16 activation rows (only
// rows of the unit's tokens) and half of its row group's weight tiles. A slot
// holds
//   activations   128 token rows x 128 k bf16, 16-byte chunk c of row j at
//                 chunk position c ^ (j mod 16) (conflict-free reads);
//   weights       16 row tiles x (16 rows x 4 blocks x 16 B): lane (row i,
//                 block q) of a tile at position 16 q + i; then the scales,
//                 4 row groups x 64 rows x 4 bytes (blocks 4 ks .. 4 ks + 3).
// Rows and blocks past the data read the workspace's zero area instead.
//
// Schedule: a persistent grid; workgroup b works in XCD b mod 8 and takes the
// XCD's units (groups j = XCD, XCD + 8, ..; row blocks in order) in turn, so
// the row blocks of a group run on one XCD at about the same time and read the
// group's activation rows from that XCD's L2.
#pragma once

#include "k3moe_device.hpp"
#include "k3moe_plan.hpp"

namespace k3moe {

constexpr int kXM = 128;                                // tokens per unit
constexpr int kXThreads = 512;                          // 8 waves
constexpr int kXRing = 3;                               // k-step slots
constexpr int kXSlotX = kXM * 256;                      // activation tile bytes
constexpr int kXSlotW = 16 * 1024;                      // weight tiles
constexpr int kXSlot = kXSlotX + kXSlotW + 4 * 256;     // + scales: 50176 bytes
constexpr int kXLds = kXRing * kXSlot;                  // dynamic LDS, 150528 bytes


// GU: gate/up -> h (act = pl.act); otherwise down -> y.
template <bool GU>
__global__ __launch_bounds__(kXThreads, 1) void k_xgemm(Plan pl, const uint16_t *__restrict__ act,
                                                       const uint8_t *__restrict__ blk0,
                                                       const uint8_t *__restrict__ scl0,
                                                       const uint8_t *__restrict__ blk1,
                                                       const uint8_t *__restrict__ scl1, char *ws) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  __shared__ int s_gstart[kMaxExperts + 1];  // first group of each active expert
  __shared__ int s_wsum[kXThreads / kWave];
  __shared__ int s_tok[kXM];                 // gate/up: token of each activation row of the unit
  const int tid = threadIdx.x, l = tid & 63, i = l & 15, q = l >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = w & 3, half = w >> 2;
  const int nact = *reinterpret_cast<const int *>(ws + pl.o_nact);
  const int *active = reinterpret_cast<const int *>(ws + pl.o_active);
  const int *aoff = reinterpret_cast<const int *>(ws + pl.o_aoff);
  const int *acnt = reinterpret_cast<const int *>(ws + pl.o_acnt);
  const int *ptok = reinterpret_cast<const int *>(ws + pl.o_ptok);
  const uint8_t *zero = reinterpret_cast<const uint8_t *>(ws + pl.o_zero);
  uint16_t *out = reinterpret_cast<uint16_t *>(ws + (GU ? pl.o_h : pl.o_y));

  // groups per active expert, exclusive prefix (two experts per thread)
  {
    const int d0 = 2 * tid, d1 = d0 + 1;
    const int t0 = d0 < nact ? (acnt[d0] + kXM - 1) / kXM : 0;
    const int t1 = d1 < nact ? (acnt[d1] + kXM - 1) / kXM : 0;
    const int incl = wave_incl_scan(t0 + t1);
    if (l == 63) s_wsum[w] = incl;
    __syncthreads();
    int base = 0;
    for (int ww = 0; ww < w; ++ww) base += s_wsum[ww];
    const int excl = base + incl - t0 - t1;
    if (d0 < nact) s_gstart[d0] = excl;
    if (d1 < nact) s_gstart[d1] = excl + t0;
    if (tid == kXThreads - 1) s_gstart[nact] = base + incl;
    __syncthreads();
  }
  const int J = s_gstart[nact];
  const int Kd = GU ? pl.K : pl.I;  // reduction length (a multiple of 128 here)
  const int KB = Kd / kBlockK, KS = Kd / 128;
  const int Nout = GU ? pl.I : pl.K;
  const int RPB = GU ? 128 : 256;  // output rows per unit
  const int NB = (Nout + RPB - 1) / RPB;
  const int xcds = gridDim.x < 8 ? (int)gridDim.x : 8;
  const int xcd = blockIdx.x % xcds, nslot = gridDim.x / xcds, slot = blockIdx.x / xcds;
  if (slot >= nslot) return;  // (a grid that is not a multiple of the XCD count)

  for (long v = slot;; v += nslot) {
    const long j = xcd + (long)xcds * (v / NB);
    if (j >= J) break;
    const int nb = (int)(v % NB);
    int lo = 0, hi = nact - 1;  // the group's expert: largest d with s_gstart[d] <= j
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_gstart[mid] <= j) lo = mid; else hi = mid - 1;
    }
    const int d = lo, mt = (int)j - s_gstart[d];
    const int e = active[d], p0 = aoff[d] + mt * kXM;
    const int m = min(kXM, acnt[d] - mt * kXM), T = (m + 15) / 16;
    wait_vm<0>();     // the previous unit's stores are done (the waits below count loads only)
    __syncthreads();  // the previous unit is done with the ring and s_tok
    if (GU)
      for (int r = tid; r < kXM; r += kXThreads) s_tok[r] = r < m ? ptok[p0 + r] : 0;
    __syncthreads();

    // this wave's 4 weight row tiles: matrix, first row and validity
    const uint8_t *tb[4], *ts[4];
    bool tv[4];
    const int orow0 = nb * RPB + (GU ? 32 : 64) * rg;  // first output row of the row group
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int orow = GU ? orow0 + 16 * (r & 1) : orow0 + 16 * r;
      tv[r] = orow < Nout;
      const size_t row = (size_t)e * Nout + orow;  // tile's first row in the weight tensor
      tb[r] = (GU && r >= 2 ? blk1 : blk0) + row * KB * 16;
      ts[r] = (GU && r >= 2 ? scl1 : scl0) + row * KB;
    }

    // this wave's activation loads per k-step: its 4-row groups below m
    const int nx = min(4, max(0, (m - 16 * w + 3) / 4));
    auto issue = [&](int ks) {
      char *base = lds + (ks % kXRing) * kXSlot;
      // activation rows 16 w .. 16 w + 15 below m, four rows per load
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (u >= nx) break;  // wave-uniform
        const int row = 16 * w + 4 * u + (l >> 4), c = (l & 15) ^ (row & 15);
        const void *src = zero + l * 16;
        if (row < m) {
          const size_t arow = GU ? (size_t)s_tok[row] * pl.K : (size_t)(p0 + row) * pl.I;
          src = act + arow + ks * 128 + c * 8;
        }
        load_lds<16>(src, base + (16 * w + 4 * u) * 256);
      }
      // weight tiles 2 half, 2 half + 1 of the row group: lane (row i, block q)
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const uint8_t *b = half ? tb[2 + rr] : tb[rr];  // (constant indices: no scratch)
        const bool ok = half ? tv[2 + rr] : tv[rr];
        const void *src = ok ? (const void *)(b + ((size_t)i * KB + 4 * ks + q) * 16) : (const void *)(zero + l * 16);
        load_lds<16>(src, base + kXSlotX + (rg * 4 + 2 * half + rr) * 1024);
      }
      // scales of the 4 tiles: lane (tile q, row i), blocks 4 ks .. 4 ks + 3 (both halves load them)
      const uint8_t *sp = q == 0 ? ts[0] : q == 1 ? ts[1] : q == 2 ? ts[2] : ts[3];
      const bool ok = q == 0 ? tv[0] : q == 1 ? tv[1] : q == 2 ? tv[2] : tv[3];
      const void *src = ok ? (const void *)(sp + (size_t)i * KB + 4 * ks) : (const void *)(zero + l * 4);
      load_lds<4>(src, base + kXSlotX + kXSlotW + rg * 256);
    };

    f32x4 acc[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) acc[r][tt] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int s = 0; s < kXRing - 1 && s < KS; ++s) issue(s);
    for (int ks = 0; ks < KS; ++ks) {
      // this wave's loads of step ks are in LDS; those of step ks + 1 (nx + 3) may stay in flight
      switch (ks + 1 < KS ? nx + 3 : 0) {
        case 0: wait_vm<0>(); break;
        case 3: wait_vm<3>(); break;
        case 4: wait_vm<4>(); break;
        case 5: wait_vm<5>(); break;
        case 6: wait_vm<6>(); break;
        default: wait_vm<7>(); break;
      }
      static_assert(kXRing == 3, "the wait above keeps one later step in flight");
      ring_barrier();  // everyone's are, and everyone is done with step ks - 1's slot
      if (ks + kXRing - 1 < KS) issue(ks + kXRing - 1);
      const char *base = lds + (ks % kXRing) * kXSlot;
      const char *abase = base + kXSlotX;
      bf16x8 av[4][4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const u32x4 wv = *reinterpret_cast<const u32x4 *>(abase + (rg * 4 + r) * 1024 + l * 16);
        const uint32_t sw = *reinterpret_cast<const uint32_t *>(abase + kXSlotW + rg * 256 + (16 * r + i) * 4);
        convert_block_fast(wv, (sw >> (8 * q)) & 0xFFu, av[r]);
      }
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const int t = 2 * tt + half;
        if (t >= T) break;  // wave-uniform
        const char *xr = base + (16 * t + i) * 256;
        u32x4 b[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) b[kk] = *reinterpret_cast<const u32x4 *>(xr + (((4 * q + kk) ^ i) * 16));
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) acc[r][tt] = mfma16(av[r][kk], as_bf16x8(b[kk]), acc[r][tt]);
      }
    }

    // epilogue: lane holds rows 4 q + v of each tile for token column i
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int t = 2 * tt + half, jrow = 16 * t + i;
      if (t >= T || jrow >= m) continue;
      const size_t p = (size_t)(p0 + jrow);
      if (GU) {
#pragma unroll
        for (int sdx = 0; sdx < 2; ++sdx) {
          if (!tv[sdx]) continue;
          uint16_t hb[4];
#pragma unroll
          for (int vv = 0; vv < 4; ++vv)
            hb[vv] = f32_to_bf16_bits(apply_act(pl.act, round_bf16(acc[sdx][tt][vv]), round_bf16(acc[2 + sdx][tt][vv])));
          const u32x2 packed = {(uint32_t)hb[0] | ((uint32_t)hb[1] << 16), (uint32_t)hb[2] | ((uint32_t)hb[3] << 16)};
          *reinterpret_cast<u32x2 *>(out + p * pl.I + orow0 + 16 * sdx + 4 * q) = packed;
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (!tv[r]) continue;
          const f32x4 a4 = acc[r][tt];
          const u32x2 packed = {(uint32_t)f32_to_bf16_bits(a4[0]) | ((uint32_t)f32_to_bf16_bits(a4[1]) << 16),
                                (uint32_t)f32_to_bf16_bits(a4[2]) | ((uint32_t)f32_to_bf16_bits(a4[3]) << 16)};
          *reinterpret_cast<u32x2 *>(out + p * pl.K + orow0 + 16 * r + 4 * q) = packed;
        }
      }
    }
  }
}

}  // namespace k3moe
