// General MoE-step path: a chain of six kernels, any token count.
//
//   k_router   router logits x . router^T on MFMA, split over k      (kimi.py:308)
//   k_topk     FP32 gating + top-k + renormalised weights, 1 wave/token (kimi.py:308-316)
//   k_group    expert histogram, active-expert list, token->expert pairs (kimi.py:319-320)
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

// Router logits: partial[s][t][e] = sum over k-split s of x[t] . router[e].
// Wave item = (k split, router row tile, token tile).
__global__ __launch_bounds__(kThreads) void k_router(Plan pl, const uint16_t *__restrict__ x,
                                                      const uint16_t *__restrict__ router, char *ws) {
  const int wave = threadIdx.x / kWave, l = threadIdx.x % kWave;
  const int item = blockIdx.x * kWavesPerBlock + wave;
  if (item >= pl.RTr * pl.TTr * pl.Sr) return;
  const int s = item % pl.Sr;
  const int rest = item / pl.Sr;
  const int rt = rest % pl.RTr, tt = rest / pl.RTr;
  const int ks0 = (int)((long)s * pl.KSr / pl.Sr), ks1 = (int)((long)(s + 1) * pl.KSr / pl.Sr);
  const int i = l & 15, q = l >> 4;
  const int row = rt * 16 + i, tok = tt * 16 + i;
  const bool row_ok = row < pl.E, tok_ok = tok < pl.B;
  const uint16_t *arow = router + (size_t)(row_ok ? row : 0) * pl.h;
  const uint16_t *brow = x + (size_t)(tok_ok ? tok : 0) * pl.h;
  const int KB = pl.h / kBlockK;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int ks = ks0; ks < ks1; ++ks) {
    const int kb = ks * 4 + q;
    const bool ok = kb < KB;
    u32x4 a[4], b[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      a[kk] = (ok && row_ok) ? load16(arow + kb * kBlockK + kk * 8) : u32x4{0, 0, 0, 0};
      b[kk] = (ok && tok_ok) ? load16(brow + kb * kBlockK + kk * 8) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) acc = mfma16(as_bf16x8(a[kk]), as_bf16x8(b[kk]), acc);
  }
  if (tok_ok) {
    // lane holds rows (experts) rt*16 + 4q + v of token column i
    float *dst = reinterpret_cast<float *>(ws + pl.o_logit) + ((size_t)s * pl.B + tok) * pl.Epad + rt * 16 + 4 * q;
    *reinterpret_cast<f32x4 *>(dst) = acc;
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
    float ps[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) ps[s] = s < pl.Sr ? part[((size_t)s * pl.B + t) * pl.Epad + e] : 0.f;
    float logit = ps[0];
#pragma unroll
    for (int s = 1; s < 4; ++s)
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

// Grouping by expert (kimi.py:319-320), one workgroup of 1024 threads:
// histogram, active-expert list in ascending order, and pairs grouped by
// expert with ascending token order inside an expert (placement by per-chunk
// token bitmaps, so the layout is deterministic). Also clears the gate/up
// split-k arrival counters for this step.
__global__ __launch_bounds__(1024) void k_group(Plan pl, char *ws) {
  __shared__ int s_cnt[kMaxExperts];
  __shared__ int s_off[kMaxExperts];
  __shared__ int s_act[kMaxExperts];
  __shared__ int s_cur[kMaxExperts];
  __shared__ uint32_t s_bits[kMaxExperts * (kGroupChunk / 32)];
  const int tid = threadIdx.x, nt = blockDim.x;
  const int E = pl.E, k = pl.k;
  const int *ids = reinterpret_cast<const int *>(ws + pl.o_ids);
  const float *wts = reinterpret_cast<const float *>(ws + pl.o_w);
  int *active = reinterpret_cast<int *>(ws + pl.o_active);
  int *aoff = reinterpret_cast<int *>(ws + pl.o_aoff);
  int *acnt = reinterpret_cast<int *>(ws + pl.o_acnt);
  int *ptok = reinterpret_cast<int *>(ws + pl.o_ptok);
  float *pw = reinterpret_cast<float *>(ws + pl.o_pw);
  int *pof = reinterpret_cast<int *>(ws + pl.o_pof);
  for (int e = tid; e < E; e += nt) s_cnt[e] = 0;
  __syncthreads();
  for (int p = tid; p < pl.P; p += nt) atomicAdd(&s_cnt[ids[p]], 1);
  __syncthreads();
  // inclusive Hillis-Steele scans of counts (s_off) and active flags (s_act);
  // the block has exactly kMaxExperts threads, one per expert slot
  const int c = tid < E ? s_cnt[tid] : 0;
  s_off[tid] = c;
  s_act[tid] = c > 0 ? 1 : 0;
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
  if (tid < E && c > 0) {
    const int d = s_act[tid] - 1;  // exclusive index of this active expert
    active[d] = tid;
    aoff[d] = s_off[tid] - c;
    acnt[d] = c;
  }
  if (tid < E) s_cur[tid] = s_off[tid] - c;
  __syncthreads();
  // stable placement, kGroupChunk tokens at a time
  constexpr int W = kGroupChunk / 32;
  for (int c0 = 0; c0 < pl.B; c0 += kGroupChunk) {
    for (int i = tid; i < E * W; i += nt) s_bits[i] = 0;
    __syncthreads();
    const int n = min(kGroupChunk, pl.B - c0) * k;
    for (int i = tid; i < n; i += nt) {
      const int tl = i / k, t = c0 + tl;
      const int e = ids[(size_t)t * k + (i % k)];
      atomicOr(&s_bits[e * W + tl / 32], 1u << (tl % 32));
    }
    __syncthreads();
    for (int i = tid; i < n; i += nt) {
      const int tl = i / k, t = c0 + tl, slot = i % k;
      const int e = ids[(size_t)t * k + slot];
      int rank = 0;
      for (int w = 0; w < W; ++w) {
        const uint32_t bits = s_bits[e * W + w];
        if (w < tl / 32) rank += __popc(bits);
        else if (w == tl / 32) rank += __popc(bits & ((1u << (tl % 32)) - 1u));
      }
      const int pos = s_cur[e] + rank;
      ptok[pos] = t;
      pw[pos] = wts[(size_t)t * k + slot];
      pof[(size_t)t * k + slot] = pos;
    }
    __syncthreads();
    for (int e = tid; e < E; e += nt) {
      int add = 0;
      for (int w = 0; w < W; ++w) add += __popc(s_bits[e * W + w]);
      s_cur[e] += add;
    }
    __syncthreads();
  }
  int *gcnt = reinterpret_cast<int *>(ws + pl.o_gcnt);
  for (int i = tid; i < pl.Dmax * pl.RTg; i += nt) gcnt[i] = 0;
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
// FP32 before the FP32 add, starting from zero.
__global__ __launch_bounds__(256) void k_combine(Plan pl, char *ws, float *__restrict__ out) {
  const int K4 = pl.K / 4;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)pl.B * K4) return;
  const int t = (int)(idx / K4), c = (int)(idx % K4) * 4;
  const int *pof = reinterpret_cast<const int *>(ws + pl.o_pof);
  const float *wts = reinterpret_cast<const float *>(ws + pl.o_w);
  const uint16_t *ybuf = reinterpret_cast<const uint16_t *>(ws + pl.o_y);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < pl.k; ++s) {
    const int p = pof[(size_t)t * pl.k + s];
    const float w = wts[(size_t)t * pl.k + s];
    const u32x2 yv = *reinterpret_cast<const u32x2 *>(ybuf + (size_t)p * pl.K + c);
    acc[0] = __fadd_rn(acc[0], __fmul_rn(bf16_bits_to_f32(yv[0] & 0xFFFFu), w));
    acc[1] = __fadd_rn(acc[1], __fmul_rn(bf16_bits_to_f32(yv[0] >> 16), w));
    acc[2] = __fadd_rn(acc[2], __fmul_rn(bf16_bits_to_f32(yv[1] & 0xFFFFu), w));
    acc[3] = __fadd_rn(acc[3], __fmul_rn(bf16_bits_to_f32(yv[1] >> 16), w));
  }
  *reinterpret_cast<f32x4 *>(out + (size_t)t * pl.K + c) = f32x4{acc[0], acc[1], acc[2], acc[3]};
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
