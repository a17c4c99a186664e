// k3moe: MXFP4 mixture-of-experts step for MI355X (gfx950).
//
// Replaces the MoE block of the reference's Kimi K3 decode oracle
// (megabench/tasks/kimi.py:307-324) and its MXFP4 decode
// (megabench/tasks/quantization.py:40-51). The C ABI is declared in
// include/k3moe.h.
//
// Pipeline of one step (all on the caller's stream, no host sync):
//   k_router   router logits x . router^T on MFMA, split over k      (kimi.py:308)
//   k_topk     FP32 gating + top-k + renormalised weights, 1 wave/token (kimi.py:308-316)
//   k_group    expert histogram, active-expert list, token->expert pairs (kimi.py:319-320)
//   k_gateup   gate and up projections of every active expert, FP4 dequant in
//              registers, MFMA, activation epilogue -> bf16 h          (kimi.py:321-322)
//   k_down     down projection of every active expert -> bf16 y       (kimi.py:322)
//   k_combine  FP32 routing-weighted sum in ascending expert order    (kimi.py:318,323)
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "../../include/k3moe.h"
#include "k3moe_device.hpp"

using namespace k3moe;

namespace {

// ------------------------------------------------------------------- plan --

constexpr int kWavesPerBlock = 4;
constexpr int kThreads = kWavesPerBlock * kWave;
constexpr int kMaxExperts = 1024;
constexpr int kMaxTopk = 32;
constexpr int kGroupChunk = 128;  // tokens per placement chunk in k_group

struct Plan {
  int B, E, k, h, K, I, gating, act;
  int P;       // token-expert pairs, B*k
  int Dmax;    // upper bound of distinct experts, min(E, P)
  int Epad;    // E rounded up to 16
  // router
  int RTr, TTr, KSr, Sr;
  // gate/up
  int RTg, KSg, Sg;
  // down
  int RTd, KSd, RPWd, RGd;
  // workspace byte offsets
  size_t o_logit, o_ids, o_w, o_nact, o_active, o_aoff, o_acnt, o_ptok, o_pw, o_pof, o_gpart, o_gcnt,
      o_h, o_y, total;
};

__host__ __device__ inline int cdiv(long a, long b) { return (int)((a + b - 1) / b); }

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

bool make_plan(const k3moe_dims &d, Plan &p) {
  p.B = d.tokens; p.E = d.experts; p.k = d.topk; p.h = d.hidden; p.K = d.latent; p.I = d.inter;
  p.gating = d.gating; p.act = d.activation;
  p.P = p.B * p.k;
  p.Dmax = p.E < p.P ? p.E : p.P;
  p.Epad = cdiv(p.E, 16) * 16;
  // router: (row tile, token tile, k split) wave items, about 1024 waves
  p.RTr = cdiv(p.E, 16);
  p.TTr = cdiv(p.B, 16);
  p.KSr = cdiv(p.h, kStepK);
  long base = (long)p.RTr * p.TTr;
  p.Sr = cdiv(1024, base);
  if (p.Sr > p.KSr) p.Sr = p.KSr;
  if (p.Sr < 1) p.Sr = 1;
  // gate/up: (active expert, 16-row tile, k split) wave items, about 2048 waves
  p.RTg = p.I / 16;
  p.KSg = cdiv(p.K, kStepK);
  base = (long)p.Dmax * p.RTg;
  p.Sg = cdiv(2048, base);
  if (p.Sg > p.KSg) p.Sg = p.KSg;
  if (p.Sg < 1) p.Sg = 1;
  // down: (active expert, group of RPWd 16-row tiles) wave items
  p.RTd = p.K / 16;
  p.KSd = cdiv(p.I, kStepK);
  p.RPWd = 4;
  p.RGd = cdiv(p.RTd, p.RPWd);
  // workspace
  size_t o = 0;
  auto take = [&](size_t bytes) { size_t at = o; o = align256(o + bytes); return at; };
  p.o_logit = take((size_t)p.Sr * p.B * p.Epad * 4);
  p.o_ids = take((size_t)p.P * 4);
  p.o_w = take((size_t)p.P * 4);
  p.o_nact = take(4);
  p.o_active = take((size_t)p.E * 4);
  p.o_aoff = take((size_t)p.E * 4);
  p.o_acnt = take((size_t)p.E * 4);
  p.o_ptok = take((size_t)p.P * 4);
  p.o_pw = take((size_t)p.P * 4);
  p.o_pof = take((size_t)p.P * 4);
  p.o_gpart = take(p.Sg > 1 ? (size_t)p.Sg * p.P * 2 * p.I * 4 : 0);
  p.o_gcnt = take((size_t)p.Dmax * p.RTg * 4);
  p.o_h = take((size_t)p.P * p.I * 2);
  p.o_y = take((size_t)p.P * p.K * 2);
  p.total = o;
  return true;
}

// ------------------------------------------------------------- errors --

thread_local char g_err[512];

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_dims(const k3moe_dims *d) {
  if (!d) return fail(K3MOE_EINVAL, "dims is NULL");
  if (d->tokens < 1) return fail(K3MOE_EINVAL, "tokens must be >= 1, got %d", d->tokens);
  if (d->experts < 1 || d->experts > kMaxExperts)
    return fail(K3MOE_EINVAL, "experts must be in [1, %d], got %d", kMaxExperts, d->experts);
  if (d->topk < 1 || d->topk > kMaxTopk || d->topk > d->experts)
    return fail(K3MOE_EINVAL, "topk must be in [1, min(%d, experts)], got %d", kMaxTopk, d->topk);
  if (d->hidden < 32 || d->hidden % 32)
    return fail(K3MOE_EINVAL, "hidden must be a positive multiple of 32, got %d", d->hidden);
  if (d->latent < 32 || d->latent % 32)
    return fail(K3MOE_EINVAL, "latent width must be a positive multiple of 32, got %d", d->latent);
  if (d->inter < 32 || d->inter % 32)
    return fail(K3MOE_EINVAL, "MXFP4 down-projection width (inter) must be a positive multiple of 32, got %d",
                d->inter);
  if (d->gating != K3MOE_GATING_SIGMOID_BIAS && d->gating != K3MOE_GATING_SOFTMAX)
    return fail(K3MOE_EINVAL, "unknown gating %d", d->gating);
  if (d->activation != K3MOE_ACT_SITU && d->activation != K3MOE_ACT_SILU)
    return fail(K3MOE_EINVAL, "unknown activation %d", d->activation);
  if (d->x_dtype != K3MOE_DTYPE_BF16) return fail(K3MOE_EINVAL, "x_dtype must be bf16 (%d)", K3MOE_DTYPE_BF16);
  if (d->reserved != 0) return fail(K3MOE_EINVAL, "reserved field must be 0");
  if ((long)d->tokens * d->topk > (1L << 30)) return fail(K3MOE_EINVAL, "tokens*topk too large");
  return K3MOE_OK;
}

// ------------------------------------------------------------ kernels --

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4 &v) { return __builtin_bit_cast(bf16x8, v); }

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

// a ranks before b: NaN first, then the larger value, then the lower index
__device__ __forceinline__ bool ranks_before(float va, int ia, float vb, int ib) {
  const bool na = va != va, nb = vb != vb;
  if (na != nb) return na;
  if (!na && va != vb) return va > vb;
  return ia < ib;
}

// Gating and top-k, one wave per token (kimi.py:308-316; distributed.py:174-176).
__global__ __launch_bounds__(kThreads) void k_topk(Plan pl, const float *__restrict__ bias,
                                                    const int64_t *__restrict__ routes, char *ws,
                                                    int64_t *__restrict__ out_ids, float *__restrict__ out_w,
                                                    float *__restrict__ out_short) {
  __shared__ float s_score[kWavesPerBlock][kMaxExperts];
  __shared__ float s_key[kWavesPerBlock][kMaxExperts];
  __shared__ int s_sel[kWavesPerBlock][kMaxTopk];
  __shared__ float s_selkey[kWavesPerBlock][kMaxTopk];
  const int wave = threadIdx.x / kWave, l = threadIdx.x % kWave;
  const int t = blockIdx.x * kWavesPerBlock + wave;
  if (t >= pl.B) return;
  const float *part = reinterpret_cast<const float *>(ws + pl.o_logit);
  const int E = pl.E, k = pl.k;
  constexpr int M = kMaxExperts / kWave;
  float key[M];
  uint32_t taken = 0;
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int e = l + kWave * m;
    key[m] = 0.f;
    if (e < E) {
      float logit = 0.f;
      for (int s = 0; s < pl.Sr; ++s) logit += part[((size_t)s * pl.B + t) * pl.Epad + e];
      float score, kv;
      if (pl.gating == K3MOE_GATING_SIGMOID_BIAS) {
        score = 1.0f / (1.0f + expf(-logit));
        kv = bias ? __fadd_rn(score, bias[e]) : score;
      } else {
        score = logit;
        kv = logit;
      }
      key[m] = kv;
      s_score[wave][e] = score;
      s_key[wave][e] = kv;
    } else {
      taken |= 1u << m;
    }
  }
  // k rounds of wave arg-max
  for (int r = 0; r < k; ++r) {
    float bv = 0.f;
    int bi = -1;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int e = l + kWave * m;
      if (!((taken >> m) & 1u) && (bi < 0 || ranks_before(key[m], e, bv, bi))) {
        bv = key[m];
        bi = e;
      }
    }
#pragma unroll
    for (int off = kWave / 2; off >= 1; off >>= 1) {
      const float ov = shfl_xor(bv, off);
      const int oi = shfl_xor(bi, off);
      if (oi >= 0 && (bi < 0 || ranks_before(ov, oi, bv, bi))) {
        bv = ov;
        bi = oi;
      }
    }
    if ((bi & (kWave - 1)) == l) taken |= 1u << (bi / kWave);
    if (l == 0) {
      s_sel[wave][r] = bi;
      s_selkey[wave][r] = bv;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // chosen set in selection order (or the forced routes, in their order)
  int my_e = -1;
  float my_score = 0.f, my_key = 0.f;
  if (l < k) {
    my_e = routes ? (int)routes[(size_t)t * k + l] : s_sel[wave][l];
    my_score = s_score[wave][my_e];
    my_key = s_key[wave][my_e];
  }
  // weights: sigmoid scores renormalised by their sum (+1e-20), or softmax of the logits
  float w = 0.f;
  if (pl.gating == K3MOE_GATING_SIGMOID_BIAS) {
    float sum = 0.f;
    for (int r = 0; r < k; ++r) sum = __fadd_rn(sum, __shfl(my_score, r, kWave));
    w = my_score / __fadd_rn(sum, 1e-20f);
  } else {
    float mx = -INFINITY;
    for (int r = 0; r < k; ++r) mx = fmaxf(mx, __shfl(my_score, r, kWave));
    const float ex = (l < k) ? expf(my_score - mx) : 0.f;
    float sum = 0.f;
    for (int r = 0; r < k; ++r) sum = __fadd_rn(sum, __shfl(ex, r, kWave));
    w = ex / sum;
  }
  if (routes && out_short) {
    float mn = INFINITY;
    for (int r = 0; r < k; ++r) mn = fminf(mn, __shfl(my_key, r, kWave));
    if (l == 0) out_short[t] = fmaxf(s_selkey[wave][k - 1] - mn, 0.f);
  }
  // ascending expert order
  int rank = 0;
  for (int r = 0; r < k; ++r) rank += (__shfl(my_e, r, kWave) < my_e) ? 1 : 0;
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

int launch_check(const char *what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(K3MOE_EHIP, "%s launch failed: %s", what, hipGetErrorString(err));
  return K3MOE_OK;
}

}  // namespace

// ----------------------------------------------------------------- C ABI --

extern "C" {

const char *k3moe_last_error(void) { return g_err; }

const char *k3moe_version(void) { return "k3moe 0.1 gfx950"; }

int k3moe_workspace_bytes(const k3moe_dims *dims, size_t *bytes) {
  g_err[0] = 0;
  int rc = check_dims(dims);
  if (rc) return rc;
  if (!bytes) return fail(K3MOE_EINVAL, "bytes is NULL");
  Plan p;
  make_plan(*dims, p);
  *bytes = p.total;
  return K3MOE_OK;
}

int k3moe_moe_step(const k3moe_dims *dims, const void *x, const void *latent, const void *router,
                   const float *router_bias, const uint8_t *gate_blocks, const uint8_t *gate_scales,
                   const uint8_t *up_blocks, const uint8_t *up_scales, const uint8_t *down_blocks,
                   const uint8_t *down_scales, const int64_t *routes, float *expert_sum, int64_t *expert_ids,
                   float *route_weights, float *shortfall, void *workspace, size_t workspace_bytes,
                   void *stream) {
  g_err[0] = 0;
  int rc = check_dims(dims);
  if (rc) return rc;
  if (!x || !router || !gate_blocks || !gate_scales || !up_blocks || !up_scales || !down_blocks ||
      !down_scales || !expert_sum || !expert_ids || !route_weights)
    return fail(K3MOE_EINVAL, "a required pointer is NULL");
  if (!latent && dims->latent != dims->hidden)
    return fail(K3MOE_EINVAL, "latent width %d differs from hidden %d but no latent input was given",
                dims->latent, dims->hidden);
  Plan p;
  make_plan(*dims, p);
  if (!workspace || workspace_bytes < p.total)
    return fail(K3MOE_EWORKSPACE, "workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
                p.total);
  if (reinterpret_cast<uintptr_t>(workspace) % 256)
    return fail(K3MOE_EWORKSPACE, "workspace must be 256-byte aligned");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char *ws = reinterpret_cast<char *>(workspace);
  const uint16_t *xin = reinterpret_cast<const uint16_t *>(latent ? latent : x);

  const int nr = p.RTr * p.TTr * p.Sr;
  hipLaunchKernelGGL(k_router, dim3(cdiv(nr, kWavesPerBlock)), dim3(kThreads), 0, st, p,
                     reinterpret_cast<const uint16_t *>(x), reinterpret_cast<const uint16_t *>(router), ws);
  if ((rc = launch_check("router"))) return rc;
  hipLaunchKernelGGL(k_topk, dim3(cdiv(p.B, kWavesPerBlock)), dim3(kThreads), 0, st, p, router_bias, routes, ws,
                     expert_ids, route_weights, shortfall);
  if ((rc = launch_check("topk"))) return rc;
  hipLaunchKernelGGL(k_group, dim3(1), dim3(1024), 0, st, p, ws);
  if ((rc = launch_check("group"))) return rc;
  const long ng = (long)p.Dmax * p.RTg * p.Sg;
  hipLaunchKernelGGL(k_gateup, dim3(cdiv(ng, kWavesPerBlock)), dim3(kThreads), 0, st, p, xin, gate_blocks,
                     gate_scales, up_blocks, up_scales, ws);
  if ((rc = launch_check("gateup"))) return rc;
  const long nd = (long)p.Dmax * p.RGd;
  hipLaunchKernelGGL(k_down, dim3(cdiv(nd, kWavesPerBlock)), dim3(kThreads), 0, st, p, down_blocks, down_scales,
                     ws);
  if ((rc = launch_check("down"))) return rc;
  const long nc = (long)p.B * (p.K / 4);
  hipLaunchKernelGGL(k_combine, dim3(cdiv(nc, 256)), dim3(256), 0, st, p, ws, expert_sum);
  if ((rc = launch_check("combine"))) return rc;
  return K3MOE_OK;
}

int k3moe_mxfp4_decode(const uint8_t *blocks, const uint8_t *scales, int64_t n_blocks, int32_t out_dtype,
                       void *out, void *stream) {
  g_err[0] = 0;
  if (n_blocks < 0) return fail(K3MOE_EINVAL, "n_blocks must be >= 0");
  if (out_dtype != K3MOE_DTYPE_F32 && out_dtype != K3MOE_DTYPE_BF16)
    return fail(K3MOE_EINVAL, "out_dtype must be f32 or bf16, got %d", out_dtype);
  if (n_blocks == 0) return K3MOE_OK;
  if (!blocks || !scales || !out) return fail(K3MOE_EINVAL, "a required pointer is NULL");
  const int64_t n = n_blocks * 16;
  long grid = (long)((n + 255) / 256);
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(k_decode, dim3((unsigned)grid), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), blocks,
                     scales, n_blocks, out_dtype, out);
  return launch_check("decode");
}

}  // extern "C"
