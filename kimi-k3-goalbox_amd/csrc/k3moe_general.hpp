// General MoE-step path: a chain of six kernels, any token count.
//
//   k_router   router logits x . router^T on MFMA, split over k      (kimi.py:308)
//   k_topk     FP32 gating + top-k + renormalised weights, 1 wave/token (kimi.py:308-316)
//   k_group_*  expert histogram, active-expert list, token->expert pairs (kimi.py:319-320)
//   k_gateup   gate and up projections of every active expert, FP4 dequant in
//              registers, MFMA, activation epilogue -> bf16 h          (kimi.py:321-322)
//   k_down     down projection of every active expert -> bf16 y       (kimi.py:322)
//   k_combine  FP32 routing-weighted sum in ascending expert order    (kimi.py:318,323)
// plus k_decode, the exact MXFP4 decode (quantization.py:40-51).
#pragma once

#include "k3moe_device.hpp"
#include "k3moe_plan.hpp"

namespace k3moe {

// a ranks before b: NaN first, then the larger value, then the lower index
__device__ __forceinline__ bool ranks_before(float va, int ia, float vb, int ib) {
  const bool na = va != va, nb = vb != vb;
  if (na != nb) return na;
  if (!na && va != vb) return va > vb;
  return ia < ib;
}

// Router logits (kimi.py:308): partial[s][t][e] = sum over k-split s of
// x[t] . router[e], fp32 accumulation (bf16 MFMA 16x16x32).
// Workgroup tile = (kRM tokens, kRExperts experts, k split s): the tile's
// token rows move through a ring of kRRing LDS slots (direct-to-LDS loads two
// 128-k steps ahead; the 16-byte chunk c of row j at position c ^ (j & 15), so
// the B reads of 16 lanes hit distinct banks), and each of the 4 waves streams
// its kRTiles 16-expert row tiles from L2 / HBM straight to registers one step
// ahead. The router (a few MB) is re-read once per token tile; x once.
// Rows past E read the zero area; tokens past B stage zero rows.
constexpr int kRM = 64;                         // tokens per workgroup tile
constexpr int kRWaves = 4;
constexpr int kRTiles = 6;                      // expert row tiles per wave
constexpr int kRExperts = kRWaves * kRTiles * 16;  // 384 experts per workgroup tile
constexpr int kRRing = 3;
constexpr int kRSlot = kRM * 256;               // 64 token rows x 128 bf16
constexpr int kRLds = kRRing * kRSlot;          // 49152 bytes

__global__ __launch_bounds__(kRWaves * 64, 1) void k_router(Plan pl, const uint16_t *__restrict__ x,
                                                            const uint16_t *__restrict__ router, char *ws) {
  __shared__ __attribute__((aligned(16))) char lds[kRLds];
  const int tid = threadIdx.x, l = tid & 63, i = l & 15, q = l >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int TT = cdiv(pl.B, kRM), EG = cdiv(pl.E, kRExperts);
  const int tt = blockIdx.x % TT, eg = (blockIdx.x / TT) % EG, s = blockIdx.x / (TT * EG);
  const int ks0 = (int)((long)s * pl.KSr / pl.Sr), ks1 = (int)((long)(s + 1) * pl.KSr / pl.Sr);
  const int KB = pl.h / kBlockK;
  const uint8_t *zero = reinterpret_cast<const uint8_t *>(ws + pl.o_zero);
  // this wave's row tiles: experts eg * 384 + 96 w + 16 r + i
  const int e0 = eg * kRExperts + w * kRTiles * 16;
  const uint16_t *arow[kRTiles];
#pragma unroll
  for (int r = 0; r < kRTiles; ++r) {
    const int row = e0 + 16 * r + i;
    arow[r] = row < pl.E ? router + (size_t)row * pl.h : nullptr;
  }
  // staging: wave w loads token rows 16 w .. 16 w + 15; lane L of load u covers
  // row 16 w + 4 u + L / 16 at position L % 16
  const uint16_t *xrow[4];
  int xc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int r = 16 * w + 4 * u + (l >> 4), t = tt * kRM + r;
    xc[u] = (l & 15) ^ (r & 15);
    xrow[u] = t < pl.B ? x + (size_t)t * pl.h : nullptr;
  }
  auto issue_x = [&](int ks) {
    char *base = lds + ((ks - ks0) % kRRing) * kRSlot;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k = ks * 128 + 8 * xc[u];
      const void *src = (xrow[u] && k < pl.h) ? (const void *)(xrow[u] + k) : (const void *)(zero + 16 * (l & 15));
      load_lds<16>(src, base + (16 * w + 4 * u) * 256);
    }
  };
  u32x4 av[2][kRTiles][4];
  auto issue_a = [&](int ks, int sl) {
    const int kb = ks * 4 + q;
#pragma unroll
    for (int r = 0; r < kRTiles; ++r)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        av[sl][r][kk] = (arow[r] && kb < KB) ? load16(arow[r] + kb * kBlockK + kk * 8) : u32x4{0, 0, 0, 0};
  };
  f32x4 acc[kRTiles][kRM / 16];
#pragma unroll
  for (int r = 0; r < kRTiles; ++r)
#pragma unroll
    for (int t = 0; t < kRM / 16; ++t) acc[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int NS = ks1 - ks0;
  if (NS > 0) {
    issue_x(ks0);
    issue_a(ks0, 0);
    if (NS > 1) issue_x(ks0 + 1);
  }
  static_assert(kRRing == 3, "the waits below follow this issue order");
  // per step and wave the issue order is a(ks + 1) (4 kRTiles loads), then x(ks + 2) (4 loads)
  for (int j0 = 0; j0 < NS; j0 += 2) {
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int j = j0 + sub, ks = ks0 + j;
      if (j < NS) {
        if (j + 1 < NS) wait_vm<4>(); else wait_vm<0>();
        ring_barrier();  // everyone's x rows of step ks have landed; step ks - 1's slot is free
        if (j + 1 < NS) issue_a(ks + 1, sub ^ 1);
        if (j + 2 < NS) issue_x(ks + 2);
        const char *base = lds + (j % kRRing) * kRSlot;
#pragma unroll
        for (int t = 0; t < kRM / 16; ++t) {
          const int row = 16 * t + i;
          u32x4 b[4];
#pragma unroll
          for (int kk = 0; kk < 4; ++kk)
            b[kk] = *reinterpret_cast<const u32x4 *>(base + row * 256 + (((4 * q + kk) ^ (row & 15)) * 16));
#pragma unroll
          for (int r = 0; r < kRTiles; ++r)
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) acc[r][t] = mfma16(as_bf16x8(av[sub][r][kk]), as_bf16x8(b[kk]), acc[r][t]);
        }
      }
    }
  }
  // lane (token column i, q) holds experts e0 + 16 r + 4q .. + 3
  float *part = reinterpret_cast<float *>(ws + pl.o_logit);
#pragma unroll
  for (int t = 0; t < kRM / 16; ++t) {
    const int tok = tt * kRM + 16 * t + i;
    if (tok >= pl.B) continue;
#pragma unroll
    for (int r = 0; r < kRTiles; ++r) {
      if (e0 + 16 * r >= pl.Epad) break;  // wave-uniform
      *reinterpret_cast<f32x4 *>(part + ((size_t)s * pl.B + tok) * pl.Epad + e0 + 16 * r + 4 * q) = acc[r][t];
    }
  }
}

// Gating and top-k, one wave per token (kimi.py:308-316; distributed.py:174-176).
__global__ __launch_bounds__(kThreads) void k_topk(Plan pl, const float *__restrict__ bias,
                                                    const int64_t *__restrict__ routes, char *ws,
                                                    int64_t *__restrict__ out_ids, float *__restrict__ out_w,
                                                    float *__restrict__ out_short) {
  __shared__ float s_score[kWavesPerBlock][kMaxExperts];
  __shared__ float s_key[kWavesPerBlock][kMaxExperts];
  __shared__ uint32_t s_keyu[kWavesPerBlock][kMaxExperts];
  __shared__ int s_sel[kWavesPerBlock][kMaxTopk];
  const int wave = threadIdx.x / kWave, l = threadIdx.x % kWave;
  const int t = blockIdx.x * kWavesPerBlock + wave;
  if (t >= pl.B) return;
  const float *part = reinterpret_cast<const float *>(ws + pl.o_logit);
  const int E = pl.E, k = pl.k;
  for (int e = l; e < E; e += kWave) {
    float ps[kMaxRouterSplits];
#pragma unroll
    for (int s = 0; s < kMaxRouterSplits; ++s) ps[s] = s < pl.Sr ? part[((size_t)s * pl.B + t) * pl.Epad + e] : 0.f;
    float logit = ps[0];
#pragma unroll
    for (int s = 1; s < kMaxRouterSplits; ++s)
      if (s < pl.Sr) logit += ps[s];
    float score, kv;
    if (pl.gating == K3MOE_GATING_SIGMOID_BIAS) {
      score = 1.0f / (1.0f + expf(-logit));
      kv = bias ? __fadd_rn(score, bias[e]) : score;
    } else {
      score = logit;
      kv = logit;
    }
    s_score[wave][e] = score;
    s_key[wave][e] = kv;
    s_keyu[wave][e] = ordered_key(kv);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  wave_topk(s_keyu[wave], E, k, s_sel[wave]);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // chosen set in selection order (or the forced routes, in their order, when
  // the row is valid; an invalid row keeps its own top-k and sets the status word)
  int fid = 0;
  const bool forced = routes && forced_route(routes, t, k, E, &fid);
  if (routes && !forced && l == 0)
    __hip_atomic_fetch_or(reinterpret_cast<unsigned *>(ws + pl.o_ctl) + kCtlErr, (unsigned)kErrRoutes,
                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  int my_e = -1;
  float my_score = 0.f, my_key = 0.f;
  if (l < k) {
    my_e = forced ? fid : s_sel[wave][l];
    my_score = s_score[wave][my_e];
    my_key = s_key[wave][my_e];
  }
  // weights: sigmoid scores renormalised by their sum (+1e-20), or softmax of the logits
  float w = 0.f;
  if (pl.gating == K3MOE_GATING_SIGMOID_BIAS) {
    float sum = 0.f;
    for (int r = 0; r < k; ++r) sum = __fadd_rn(sum, lane_f32(my_score, r));
    w = my_score / __fadd_rn(sum, 1e-20f);
  } else {
    float mx = -INFINITY;
    for (int r = 0; r < k; ++r) mx = fmaxf(mx, lane_f32(my_score, r));
    const float ex = (l < k) ? expf(my_score - mx) : 0.f;
    float sum = 0.f;
    for (int r = 0; r < k; ++r) sum = __fadd_rn(sum, lane_f32(ex, r));
    w = ex / sum;
  }
  if (routes && out_short) {
    float mn = INFINITY;
    for (int r = 0; r < k; ++r) mn = fminf(mn, lane_f32(my_key, r));
    if (l == 0) out_short[t] = fmaxf(s_key[wave][s_sel[wave][k - 1]] - mn, 0.f);
  }
  // ascending expert order
  int rank = 0;
  for (int r = 0; r < k; ++r) rank += ((int)lane_u32((uint32_t)my_e, r) < my_e) ? 1 : 0;
  if (l < k) {
    const size_t o = (size_t)t * k + rank;
    out_ids[o] = my_e;
    out_w[o] = w;
    reinterpret_cast<int *>(ws + pl.o_ids)[o] = my_e;
    reinterpret_cast<float *>(ws + pl.o_w)[o] = w;
  }
}

// Grouping by expert (kimi.py:319-320) in three kernels over chunks of
// kGroupChunk tokens: the active experts ascending, each expert's pairs in a
// contiguous range with its tokens ascending (the order of `nonzero`), so the
// layout is deterministic.
//   k_group_count  one workgroup per chunk: the chunk's expert histogram
//                  (LDS atomics) -> cnt[chunk][e]
//   k_group_scan   one workgroup: per expert the chunks' counts summed in
//                  chunk order (exclusive prefix per chunk), then a scan over
//                  the experts of the totals and of the active flags; writes
//                  the active list, offsets and counts, and turns cnt into the
//                  absolute first position of each (chunk, expert) run; clears
//                  the gate/up split arrival counters for this step
//   k_group_place  one workgroup per chunk: a pair's rank among its expert's
//                  pairs in the chunk, from per-expert token bitmaps (popcounts
//                  of the bits below it), gives its position
__global__ __launch_bounds__(256) void k_group_count(Plan pl, char *ws) {
  __shared__ int s_cnt[kMaxExperts];
  const int tid = threadIdx.x, c = blockIdx.x;
  const int *ids = reinterpret_cast<const int *>(ws + pl.o_ids);
  for (int e = tid; e < pl.E; e += 256) s_cnt[e] = 0;
  __syncthreads();
  const int p0 = c * kGroupChunk * pl.k, p1 = min(pl.P, (c + 1) * kGroupChunk * pl.k);
  for (int p = p0 + tid; p < p1; p += 256) atomicAdd(&s_cnt[ids[p]], 1);
  __syncthreads();
  int *cnt = reinterpret_cast<int *>(ws + pl.o_gchunk) + (size_t)c * pl.E;
  for (int e = tid; e < pl.E; e += 256) cnt[e] = s_cnt[e];
}

__global__ __launch_bounds__(1024) void k_group_scan(Plan pl, char *ws) {
  __shared__ int s_off[kMaxExperts];
  __shared__ int s_act[kMaxExperts];
  const int tid = threadIdx.x, E = pl.E;
  const int nch = cdiv(pl.B, kGroupChunk);
  int *cnt = reinterpret_cast<int *>(ws + pl.o_gchunk);
  // per expert: chunk counts -> exclusive prefixes (relative to the expert's first pair)
  int total = 0;
  if (tid < E)
    for (int c = 0; c < nch; ++c) {
      const int v = cnt[(size_t)c * E + tid];
      cnt[(size_t)c * E + tid] = total;
      total += v;
    }
  // inclusive Hillis-Steele scans of the totals (s_off) and active flags (s_act);
  // the block has exactly kMaxExperts threads, one per expert slot
  s_off[tid] = total;
  s_act[tid] = total > 0 ? 1 : 0;
  __syncthreads();
  for (int d = 1; d < kMaxExperts; d <<= 1) {
    const int vo = tid >= d ? s_off[tid - d] : 0;
    const int va = tid >= d ? s_act[tid - d] : 0;
    __syncthreads();
    s_off[tid] += vo;
    s_act[tid] += va;
    __syncthreads();
  }
  if (tid == kMaxExperts - 1) *reinterpret_cast<int *>(ws + pl.o_nact) = s_act[tid];
  const int first = s_off[tid] - total;
  if (tid < E && total > 0) {
    const int d = s_act[tid] - 1;  // exclusive index of this active expert
    reinterpret_cast<int *>(ws + pl.o_active)[d] = tid;
    reinterpret_cast<int *>(ws + pl.o_aoff)[d] = first;
    reinterpret_cast<int *>(ws + pl.o_acnt)[d] = total;
  }
  if (tid < E)
    for (int c = 0; c < nch; ++c) cnt[(size_t)c * E + tid] += first;
  int *gcnt = reinterpret_cast<int *>(ws + pl.o_gcnt);
  for (int i = tid; i < pl.Dmax * pl.RTg; i += 1024) gcnt[i] = 0;
}

__global__ __launch_bounds__(256) void k_group_place(Plan pl, char *ws) {
  constexpr int W = kGroupChunk / 32;
  __shared__ uint32_t s_bits[kMaxExperts * W];
  const int tid = threadIdx.x, c = blockIdx.x, E = pl.E, k = pl.k;
  const int *ids = reinterpret_cast<const int *>(ws + pl.o_ids);
  const float *wts = reinterpret_cast<const float *>(ws + pl.o_w);
  const int *pos0 = reinterpret_cast<const int *>(ws + pl.o_gchunk) + (size_t)c * E;
  int *ptok = reinterpret_cast<int *>(ws + pl.o_ptok);
  float *pw = reinterpret_cast<float *>(ws + pl.o_pw);
  int *pof = reinterpret_cast<int *>(ws + pl.o_pof);
  for (int i = tid; i < E * W; i += 256) s_bits[i] = 0;
  __syncthreads();
  const int c0 = c * kGroupChunk, n = min(kGroupChunk, pl.B - c0) * k;
  for (int i = tid; i < n; i += 256) {
    const int tl = i / k;
    const int e = ids[(size_t)c0 * k + i];
    atomicOr(&s_bits[e * W + tl / 32], 1u << (tl % 32));
  }
  __syncthreads();
  for (int i = tid; i < n; i += 256) {
    const int tl = i / k, t = c0 + tl;
    const int e = ids[(size_t)c0 * k + i];
    int rank = 0;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const uint32_t bits = s_bits[e * W + w];
      if (w < tl / 32) rank += __popc(bits);
      else if (w == tl / 32) rank += __popc(bits & ((1u << (tl % 32)) - 1u));
    }
    const int pos = pos0[e] + rank;
    ptok[pos] = t;
    pw[pos] = wts[(size_t)c0 * k + i];
    pof[(size_t)c0 * k + i] = pos;
  }
}

// Gate/up epilogue for one lane: rows r0 .. r0+3 of token pair p.
__device__ __forceinline__ void gateup_store(const Plan &pl, char *ws, int p, int r0, const float g[4],
                                             const float u[4]) {
  uint16_t hb[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const float gb = round_bf16(g[v]), ub = round_bf16(u[v]);
    hb[v] = f32_to_bf16_bits(apply_act(pl.act, gb, ub));
  }
  uint16_t *h = reinterpret_cast<uint16_t *>(ws + pl.o_h) + (size_t)p * pl.I + r0;
  u32x2 packed = {(uint32_t)hb[0] | ((uint32_t)hb[1] << 16), (uint32_t)hb[2] | ((uint32_t)hb[3] << 16)};
  *reinterpret_cast<u32x2 *>(h) = packed;
}

// Gate and up projections with the activation epilogue (kimi.py:321-322).
// Wave item = (active expert d, 16-row tile of I, k split). Weights are
// streamed once per 16 tokens of the expert; k splits > 1 meet in a
// last-arriver reduction in a fixed split order.
__global__ __launch_bounds__(kThreads) void k_gateup(Plan pl, const uint16_t *__restrict__ xin,
                                                      const uint8_t *__restrict__ gblk,
                                                      const uint8_t *__restrict__ gscl,
                                                      const uint8_t *__restrict__ ublk,
                                                      const uint8_t *__restrict__ uscl, char *ws) {
  const int wave = threadIdx.x / kWave, l = threadIdx.x % kWave;
  const int item = blockIdx.x * kWavesPerBlock + wave;
  const int s = item % pl.Sg;
  const int rest = item / pl.Sg;
  const int rt = rest % pl.RTg, d = rest / pl.RTg;
  if (d >= pl.Dmax) return;
  const int nact = *reinterpret_cast<const int *>(ws + pl.o_nact);
  if (d >= nact) return;
  const int e = reinterpret_cast<const int *>(ws + pl.o_active)[d];
  const int p0 = reinterpret_cast<const int *>(ws + pl.o_aoff)[d];
  const int n = reinterpret_cast<const int *>(ws + pl.o_acnt)[d];
  const int *ptok = reinterpret_cast<const int *>(ws + pl.o_ptok);
  const int KB = pl.K / kBlockK;
  const int ks0 = (int)((long)s * pl.KSg / pl.Sg), ks1 = (int)((long)(s + 1) * pl.KSg / pl.Sg);
  const int i = l & 15, q = l >> 4;
  const size_t row = (size_t)e * pl.I + rt * 16 + i;
  const uint8_t *gb = gblk + row * KB * 16, *gs = gscl + row * KB;
  const uint8_t *ub = ublk + row * KB * 16, *us = uscl + row * KB;
  float *gpart = reinterpret_cast<float *>(ws + pl.o_gpart);
  const int r0 = rt * 16 + 4 * q;  // output rows of this lane
  for (int c = 0; c * 16 < n; ++c) {
    const int pj = c * 16 + i;
    const bool tok_ok = pj < n;
    const uint16_t *xr = xin + (size_t)(tok_ok ? ptok[p0 + pj] : 0) * pl.K;
    f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
    for (int ks = ks0; ks < ks1; ++ks) {
      const int kb = ks * 4 + q;
      const bool ok = kb < KB;
      const u32x4 wg = ok ? load16_nt(gb + kb * 16) : u32x4{0, 0, 0, 0};
      const u32x4 wu = ok ? load16_nt(ub + kb * 16) : u32x4{0, 0, 0, 0};
      const uint32_t sg = ok ? gs[kb] : 127u, su = ok ? us[kb] : 127u;
      u32x4 b[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        b[kk] = (ok && tok_ok) ? load16(xr + kb * kBlockK + kk * 8) : u32x4{0, 0, 0, 0};
      bf16x8 a[4];
      convert_block(wg, sg, a);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) ag = mfma16(a[kk], as_bf16x8(b[kk]), ag);
      convert_block(wu, su, a);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) au = mfma16(a[kk], as_bf16x8(b[kk]), au);
    }
    if (tok_ok) {
      if (pl.Sg == 1) {
        const float g[4] = {ag[0], ag[1], ag[2], ag[3]}, u[4] = {au[0], au[1], au[2], au[3]};
        gateup_store(pl, ws, p0 + pj, r0, g, u);
      } else {
        float *dst = gpart + (((size_t)s * pl.P + p0 + pj) * 2) * pl.I + r0;
        *reinterpret_cast<f32x4 *>(dst) = ag;
        *reinterpret_cast<f32x4 *>(dst + pl.I) = au;
      }
    }
  }
  if (pl.Sg == 1) return;
  // last arriver of the Sg splits of (d, rt) sums the partials in split order
  __threadfence();
  int old = 0;
  if (l == 0) old = atomicAdd(reinterpret_cast<int *>(ws + pl.o_gcnt) + (size_t)d * pl.RTg + rt, 1);
  old = __shfl(old, 0, kWave);
  if (old != pl.Sg - 1) return;
  __threadfence();
  for (int c = 0; c * 16 < n; ++c) {
    const int pj = c * 16 + i;
    if (pj >= n) continue;
    float g[4] = {0.f, 0.f, 0.f, 0.f}, u[4] = {0.f, 0.f, 0.f, 0.f};
    for (int sp = 0; sp < pl.Sg; ++sp) {
      const float *src = gpart + (((size_t)sp * pl.P + p0 + pj) * 2) * pl.I + r0;
      const f32x4 pg = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(src));
      const f32x4 pu = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(src + pl.I));
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        g[v] = __fadd_rn(g[v], pg[v]);
        u[v] = __fadd_rn(u[v], pu[v]);
      }
    }
    gateup_store(pl, ws, p0 + pj, r0, g, u);
  }
}

// Down projection (kimi.py:322): y[p][row] = bf16(h[p] . down[e][row]).
// Wave item = (active expert d, group of RPWd 16-row tiles of K).
__global__ __launch_bounds__(kThreads) void k_down(Plan pl, const uint8_t *__restrict__ dblk,
                                                    const uint8_t *__restrict__ dscl, char *ws) {
  constexpr int RPW = 4;
  const int wave = threadIdx.x / kWave, l = threadIdx.x % kWave;
  const int item = blockIdx.x * kWavesPerBlock + wave;
  const int rg = item % pl.RGd, d = item / pl.RGd;
  if (d >= pl.Dmax) return;
  const int nact = *reinterpret_cast<const int *>(ws + pl.o_nact);
  if (d >= nact) return;
  const int e = reinterpret_cast<const int *>(ws + pl.o_active)[d];
  const int p0 = reinterpret_cast<const int *>(ws + pl.o_aoff)[d];
  const int n = reinterpret_cast<const int *>(ws + pl.o_acnt)[d];
  const int KB = pl.I / kBlockK;
  const int i = l & 15, q = l >> 4;
  const uint16_t *hbuf = reinterpret_cast<const uint16_t *>(ws + pl.o_h);
  uint16_t *ybuf = reinterpret_cast<uint16_t *>(ws + pl.o_y);
  for (int c = 0; c * 16 < n; ++c) {
    const int pj = c * 16 + i;
    const bool tok_ok = pj < n;
    const uint16_t *hr = hbuf + (size_t)(p0 + (tok_ok ? pj : 0)) * pl.I;
    f32x4 acc[RPW];
#pragma unroll
    for (int t = 0; t < RPW; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int ks = 0; ks < pl.KSd; ++ks) {
      const int kb = ks * 4 + q;
      const bool ok = kb < KB;
      u32x4 b[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        b[kk] = (ok && tok_ok) ? load16(hr + kb * kBlockK + kk * 8) : u32x4{0, 0, 0, 0};
#pragma unroll
      for (int t = 0; t < RPW; ++t) {
        const int rtile = rg * RPW + t;
        if (rtile >= pl.RTd) break;
        const size_t row = (size_t)e * pl.K + rtile * 16 + i;
        const u32x4 w = ok ? load16_nt(dblk + (row * KB + kb) * 16) : u32x4{0, 0, 0, 0};
        const uint32_t sc = ok ? dscl[row * KB + kb] : 127u;
        bf16x8 a[4];
        convert_block(w, sc, a);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) acc[t] = mfma16(a[kk], as_bf16x8(b[kk]), acc[t]);
      }
    }
    if (!tok_ok) continue;
#pragma unroll
    for (int t = 0; t < RPW; ++t) {
      const int rtile = rg * RPW + t;
      if (rtile >= pl.RTd) break;
      uint16_t *y = ybuf + (size_t)(p0 + pj) * pl.K + rtile * 16 + 4 * q;
      u32x2 packed = {(uint32_t)f32_to_bf16_bits(acc[t][0]) | ((uint32_t)f32_to_bf16_bits(acc[t][1]) << 16),
                      (uint32_t)f32_to_bf16_bits(acc[t][2]) | ((uint32_t)f32_to_bf16_bits(acc[t][3]) << 16)};
      *reinterpret_cast<u32x2 *>(y) = packed;
    }
  }
}

// Weighted combine (kimi.py:318,323): expert_sum[t] = sum over the token's
// experts in ascending id order of float(y) * w, each product rounded to
// FP32 before the FP32 add, starting from zero. One thread per 8 columns
// (16-byte y loads, two 16-byte stores); K % 8 == 0.
__global__ __launch_bounds__(256) void k_combine(Plan pl, char *ws, float *__restrict__ out) {
  const int K8 = pl.K / 8;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)pl.B * K8) return;
  const int t = (int)(idx / K8), c = (int)(idx % K8) * 8;
  const int *pof = reinterpret_cast<const int *>(ws + pl.o_pof);
  const float *wts = reinterpret_cast<const float *>(ws + pl.o_w);
  const uint16_t *ybuf = reinterpret_cast<const uint16_t *>(ws + pl.o_y);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < pl.k; ++s) {
    const int p = pof[(size_t)t * pl.k + s];
    const float w = wts[(size_t)t * pl.k + s];
    const u32x4 yv = *reinterpret_cast<const u32x4 *>(ybuf + (size_t)p * pl.K + c);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      acc[2 * v] = __fadd_rn(acc[2 * v], __fmul_rn(bf16_bits_to_f32(yv[v] & 0xFFFFu), w));
      acc[2 * v + 1] = __fadd_rn(acc[2 * v + 1], __fmul_rn(bf16_bits_to_f32(yv[v] >> 16), w));
    }
  }
  float *o = out + (size_t)t * pl.K + c;
  *reinterpret_cast<f32x4 *>(o) = f32x4{acc[0], acc[1], acc[2], acc[3]};
  *reinterpret_cast<f32x4 *>(o + 4) = f32x4{acc[4], acc[5], acc[6], acc[7]};
}

// Exact MXFP4 decode, one thread per block byte (quantization.py:40-51).
__global__ __launch_bounds__(256) void k_decode(const uint8_t *__restrict__ blocks,
                                                const uint8_t *__restrict__ scales, int64_t n_blocks,
                                                int out_dtype, void *out) {
  const int64_t n = n_blocks * 16;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const uint32_t byte = blocks[i];
    const uint32_t s = scales[i / 16];
    const uint32_t lo = mxfp4_bits(byte & 15u, s), hi = mxfp4_bits(byte >> 4, s);
    if (out_dtype == K3MOE_DTYPE_F32) {
      reinterpret_cast<u32x2 *>(out)[i] = u32x2{lo, hi};
    } else {
      reinterpret_cast<uint32_t *>(out)[i] = (lo >> 16) | (hi & 0xFFFF0000u);
    }
  }
}

}  // namespace k3moe
