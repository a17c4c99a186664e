// The latent MoE block around the routed experts of a Kimi K3 layer
// (kimi.py:317, 325-328), as two persistent weight-streaming kernels:
//
//   k_latent<0>  latent   = bf16(x @ latent_down.T)                         kimi.py:317
//                shared_h = bf16(act(bf16(x @ shared_gate.T),
//                                    bf16(x @ shared_up.T)))                 kimi.py:326-327
//   k_latent<1>  en       = bf16(bf16(rms_normalize(bf16(expert_sum))) * latent_norm)
//                                                              kimi.py:325, common.py:13-21
//                out      = bf16(bf16(en @ latent_up.T) + bf16(shared_h @ shared_down.T))
//                                                                          kimi.py:325-328
//
// Both are skinny bf16 GEMMs: B <= 64 tokens against 10-50 MB weight
// matrices, HBM-bound, every weight byte read once. The output rows form 16-row
// tiles (k_latent<0>: latent_down, shared_gate, shared_up rows in turn;
// k_latent<1>: the h output rows, each with two parts: k over latent_up then
// k over shared_down, rounded separately). The k axis is cut into SP splits
// of 128-k steps. Workgroup b takes split s = b mod SP and the row tiles
// b / SP + j G / SP ("units"):
//   - it stages the activation rows of its split (all tokens) in LDS once;
//   - the 8 waves take the split's k-steps in turn (wave w: k0 + w, k0 + w + 8),
//     each loading 16 rows x 128 k of bf16 weights per k-step (64 bytes per
//     lane) into a register ring three units deep, so the weight stream of
//     the next two units is in flight while one is multiplied (MFMA
//     16x16x32 bf16, token tiles of 16 as the B operand from LDS);
//   - the waves' fp32 tiles meet in LDS (wave order) and the split's partial
//     of each (token, row) goes to the workspace with device-coherent stores.
// At the end each workgroup counts its units in on a per-tile counter; the
// workgroup that completes a tile sums its partials in split order and writes
// the bf16 outputs (with the activation for a shared gate/up tile pair, which
// shares one counter), then puts the counter back to zero. k_latent<1> first
// normalises the expert sum: workgroup t < B computes token t's en row into
// the workspace (followed by a copy of its shared_h row), while every
// workgroup already streams its first two units' weights, and a grid barrier
// separates that from the staging.
//
// Accumulation order is fixed (k-step order per wave, wave order, split
// order), so results do not depend on timing.
#pragma once

#include <stddef.h>

#include "k3moe_barrier.hpp"
#include "k3moe_decode.hpp"
#include "k3moe_device.hpp"
#include "k3moe_plan.hpp"

namespace k3moe {

constexpr int kLatMaxTokens = 64;
constexpr int kLatWaves = 8;
constexpr int kLatThreads = kLatWaves * 64;
constexpr int kLatKW = 2;          // k-steps per wave and unit, at most
constexpr int kLatXChunks = 16;    // 16-byte activation chunks per thread when staging, at most
constexpr int kLatMaxLds = kDecMaxLds - 1024;  // dynamic LDS (the static LDS stays under 1 KiB)
constexpr int kLatMaxUnits = 64;   // units per workgroup, at most
constexpr int kLatMaxSplits = 16;  // k-splits, at most
constexpr int kLatNormPairs = 8;   // k_latent<1>: expert-sum pairs per thread of a normalising workgroup
constexpr float kLatRmsEps = 1e-5f;  // kimi.py:325

struct LatPlan {
  int B, h, lh, S, act;
  int out;     // 0: k_latent<0> (before the experts), 1: k_latent<1> (after)
  int TT;      // 16-token tiles
  int G;       // persistent workgroups (a power of two)
  int RT;      // 16-row output tiles
  int KS0, KS; // 128-k steps of part 0 and of both parts
  int SP;      // k-splits (a power of two <= G)
  int J;       // units of the busiest workgroup
  int kwmax;   // k-steps of the largest split
  int xpitch;  // staged activation row pitch, elements
  int lds_x, lds_total;
  int ntile0;  // k_latent<0>: latent_down row tiles (the shared tiles follow)
  long o_cnt, o_part0, o_part1, o_en, total;
};

// The arguments of both kernels.
struct LatArgs {
  const uint16_t *x;     // <0>: x [B, h]                   <1>: shared_h [B, S]
  const float *esum;     //                                 <1>: expert_sum [B, lh]
  const uint16_t *norm;  //                                 <1>: latent_norm [lh]
  const uint16_t *wa;    // <0>: latent_down [lh, h]        <1>: latent_up [h, lh]
  const uint16_t *wb;    // <0>: shared_gate [S, h]         <1>: shared_down [h, S]
  const uint16_t *wc;    // <0>: shared_up [S, h]
  uint16_t *ya;          // <0>: latent [B, lh]             <1>: out [B, h]
  uint16_t *yb;          // <0>: shared_h [B, S]
  char *ws;
};

// Split s covers k-steps [lat_k0(s), lat_k0(s + 1)).
__host__ __device__ inline int lat_k0(int s, int KS, int SP) { return (int)((long)s * KS / SP); }

// Plan of k_latent<out> for the given geometry; null on success, else why it does not fit.
inline const char *latent_plan(const k3moe_latent_dims &d, int n_cus, int out, LatPlan &p) {
  p.B = d.tokens; p.h = d.hidden; p.lh = d.latent; p.S = d.shared; p.act = d.activation; p.out = out;
  p.TT = cdiv(p.B, 16);
  p.G = 1;
  while (p.G * 2 <= n_cus && p.G * 2 <= 1024) p.G *= 2;
  p.ntile0 = p.lh / 16;
  int ncnt;
  if (!out) {
    p.RT = (p.lh + 2 * p.S) / 16; p.KS0 = p.KS = p.h / kStepK;
    ncnt = p.lh / 16 + p.S / 16;
  } else {
    p.RT = p.h / 16; p.KS0 = p.lh / kStepK; p.KS = p.KS0 + p.S / kStepK;
    ncnt = p.RT;
    if (p.lh > 2 * kLatNormPairs * kLatThreads || p.S > 2 * kLatNormPairs * kLatThreads)
      return "latent or shared width too large for the normalisation";
  }
  const int parts = out ? 2 : 1;
  const int red = parts * p.TT * kLatWaves * 1024;
  p.SP = 0;
  for (int sp = 4; sp <= kLatMaxSplits && !p.SP; sp *= 2) {
    int s = sp;
    while (s > p.KS) s >>= 1;  // at least one k-step per split
    const int kw = cdiv(p.KS, s);
    const int lx = p.B * (kw * kStepK + 8) * 2;
    if (kw <= kLatWaves * kLatKW && p.B * kw <= kLatXChunks * kLatThreads / 16 && lx + red <= kLatMaxLds) p.SP = s;
    if (s < sp) break;
  }
  if (!p.SP) return "the staged activation slice does not fit in LDS";
  if (p.SP > p.G) return "too few compute units for the k-splits";
  p.kwmax = cdiv(p.KS, p.SP);
  p.xpitch = p.kwmax * kStepK + 8;
  p.lds_x = p.B * p.xpitch * 2;
  p.lds_total = p.lds_x + red;
  p.J = cdiv(p.RT, p.G / p.SP);
  if (p.J > kLatMaxUnits) return "too many row tiles per workgroup";
  if (ncnt * 4 > kLatCntBytes) return "too many row tiles for the counter area";
  long o = 0;
  auto take = [&](long bytes) { long at = o; o = (long)align256((size_t)(o + bytes)); return at; };
  take(kInitBytes - kLatCntBytes);
  p.o_cnt = take(kLatCntBytes);
  const long part = (long)p.SP * p.RT * p.B * 16 * 4;
  p.o_part0 = take(part);
  p.o_part1 = out ? take(part) : 0;
  p.o_en = out ? take((long)p.B * (p.lh + p.S) * 2) : 0;
  p.total = o;
  return nullptr;
}

// The first bf16 of lane (row i, block q)'s 64 bytes of k-step ks of row tile rt.
__device__ __forceinline__ const uint16_t *lat_src(const LatPlan &pl, const LatArgs &a, int rt, int ks, int i, int q) {
  const long r = (long)rt * 16 + i;
  const int kq = q * 32;
  if (!pl.out) {
    const uint16_t *row = r < pl.lh ? a.wa + r * pl.h
                          : r < pl.lh + pl.S ? a.wb + (r - pl.lh) * pl.h
                                             : a.wc + (r - pl.lh - pl.S) * pl.h;
    return row + ks * kStepK + kq;
  }
  return ks < pl.KS0 ? a.wa + r * pl.lh + ks * kStepK + kq : a.wb + r * pl.S + (ks - pl.KS0) * kStepK + kq;
}

__device__ __forceinline__ float bload4_dev(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, kCpolDevice));
}

template <int OUT>
__global__ __launch_bounds__(kLatThreads, 1) void k_latent(LatPlan pl, LatArgs a) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  uint16_t *xs = reinterpret_cast<uint16_t *>(lds);                 // [B][xpitch] activation slice
  float *red = reinterpret_cast<float *>(lds + pl.lds_x);          // [parts][TT][8 waves][256]
  __shared__ int s_fin[kLatMaxUnits];
  __shared__ int s_nfin;
  __shared__ float s_wsum[kLatWaves];

  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int i = l & 15, q = l >> 4;
  const int B = pl.B, TT = pl.TT, SP = pl.SP;
  const int s = blockIdx.x % SP;
  const int k0 = lat_k0(s, pl.KS, SP), k1 = lat_k0(s + 1, pl.KS, SP), nk = k1 - k0;
  const int rstep = gridDim.x / SP, rt0 = blockIdx.x / SP;
  const int J = rt0 < pl.RT ? cdiv(pl.RT - rt0, rstep) : 0;
  const bool touch0 = k0 < pl.KS0, touch1 = OUT && k1 > pl.KS0;  // parts with k-steps in this split
  unsigned *ctl = reinterpret_cast<unsigned *>(a.ws);
  unsigned *cnt = reinterpret_cast<unsigned *>(a.ws + pl.o_cnt);
  const uint16_t *zlane = reinterpret_cast<const uint16_t *>(a.ws + 4096 + l * 64);  // 64 zero bytes
  const uint32_t part_bytes = (uint32_t)((long)SP * pl.RT * B * 64);
  const __amdgpu_buffer_rsrc_t rp0 = make_rsrc(a.ws + pl.o_part0, part_bytes);
  const __amdgpu_buffer_rsrc_t rp1 = make_rsrc(a.ws + (OUT ? pl.o_part1 : pl.o_part0), part_bytes);
  BarrierBase bb{0u, 0u};
  if (OUT && tid == 0) bb = barrier_base(ctl);

  // weight ring: unit j's k-steps of this wave; past the units or the split, the zero area
  auto issue = [&](int j, u32x4 (&buf)[kLatKW][4]) {
    const int rt = rt0 + rstep * j;
#pragma unroll
    for (int m = 0; m < kLatKW; ++m) {
      const int ks = k0 + w + kLatWaves * m;
      const uint16_t *src = (j < J && ks < k1) ? lat_src(pl, a, rt, ks, i, q) : zlane;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) buf[m][kk] = load16(src + kk * 8);
    }
  };

  // the activation slice of this split: x (<0>) or [en | shared_h] (<1>), all tokens
  const int cpt = nk * (kStepK / 8);  // 16-byte chunks per token
  u32x4 xc[kLatXChunks];
  const int erow = pl.lh + pl.S;  // <1>: workspace row of a token, [en | shared_h]
  const __amdgpu_buffer_rsrc_t ren = make_rsrc(a.ws + pl.o_en, OUT ? (uint32_t)(B * erow * 2) : 0u);
  auto stage_load = [&]() {
#pragma unroll
    for (int c = 0; c < kLatXChunks; ++c) {
      const int idx = tid + c * kLatThreads;
      const int t = idx / cpt, cc = idx - t * cpt;
      const int ks = k0 + (cc >> 4), e = (cc & 15) * 8;
      if (!OUT) {
        const uint16_t *src = t < B ? a.x + (long)t * pl.h + ks * kStepK + e : zlane;
        xc[c] = load16(src);
      } else {
        xc[c] = bload16_dev(ren, t < B ? (uint32_t)(((long)t * erow + ks * kStepK + e) * 2) : kOffNone);
      }
    }
  };
  auto stage_store = [&]() {
#pragma unroll
    for (int c = 0; c < kLatXChunks; ++c) {
      const int idx = tid + c * kLatThreads;
      const int t = idx / cpt, cc = idx - t * cpt;
      if (t < B) *reinterpret_cast<u32x4 *>(xs + t * pl.xpitch + cc * 8) = xc[c];
    }
  };

  u32x4 b0[kLatKW][4], b1[kLatKW][4], b2[kLatKW][4];
  if (!OUT) {
    stage_load();  // first, so that its wait below does not include the weight loads
    issue(0, b0);
    issue(1, b1);
    stage_store();
    ring_barrier();
  } else {
    // Workgroup t < B normalises token t's expert sum: en = bf16(bf16(e r) w),
    // e = bf16(expert_sum), r = 1/sqrt(mean(e^2) + eps), and writes the
    // workspace row [en | shared_h] the splits stage from. Its loads go first,
    // then the first two units' weight loads.
    const bool norm_wg = (int)blockIdx.x < B;
    const int t = norm_wg ? (int)blockIdx.x : 0;
    float2 ev[kLatNormPairs];
    uint32_t wv[kLatNormPairs], hv[kLatNormPairs];
    if (norm_wg) {
#pragma unroll
      for (int m = 0; m < kLatNormPairs; ++m) {
        const int k = 2 * (tid + m * kLatThreads);
        const int kc = k < pl.lh ? k : 0, kh = k < pl.S ? k : 0;
        ev[m] = *reinterpret_cast<const float2 *>(a.esum + (long)t * pl.lh + kc);
        wv[m] = *reinterpret_cast<const uint32_t *>(a.norm + kc);
        hv[m] = *reinterpret_cast<const uint32_t *>(a.x + (long)t * pl.S + kh);
      }
    }
    issue(0, b0);
    issue(1, b1);
    if (norm_wg) {
      float ss = 0.f;
#pragma unroll
      for (int m = 0; m < kLatNormPairs; ++m) {
        if (2 * (tid + m * kLatThreads) < pl.lh) {
          const float e0 = round_bf16(ev[m].x), e1 = round_bf16(ev[m].y);
          ss += e0 * e0;
          ss += e1 * e1;
        }
      }
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) ss += shfl_xor(ss, m);
      if (l == 0) s_wsum[w] = ss;
      ring_barrier();
      float tot = s_wsum[0];
#pragma unroll
      for (int v = 1; v < kLatWaves; ++v) tot += s_wsum[v];
      const float r = 1.0f / __fsqrt_rn(tot / (float)pl.lh + kLatRmsEps);
#pragma unroll
      for (int m = 0; m < kLatNormPairs; ++m) {
        const int k = 2 * (tid + m * kLatThreads);
        const float n0 = round_bf16(round_bf16(ev[m].x) * r), n1 = round_bf16(round_bf16(ev[m].y) * r);
        const uint32_t o0 = f32_to_bf16_bits(n0 * bf16_bits_to_f32(wv[m] & 0xFFFFu));
        const uint32_t o1 = f32_to_bf16_bits(n1 * bf16_bits_to_f32(wv[m] >> 16));
        st_dev32(ren, k < pl.lh ? (uint32_t)(((long)t * erow + k) * 2) : kOffNone, o0 | (o1 << 16));
        st_dev32(ren, k < pl.S ? (uint32_t)(((long)t * erow + pl.lh + k) * 2) : kOffNone, hv[m]);
      }
    }
    grid_barrier(ctl, bb, 1);
    stage_load();
    stage_store();
    ring_barrier();
  }

  // one unit: the split's k-steps of row tile rt0 + rstep j from `buf`, partials out
  auto unit = [&](int j, const u32x4 (&buf)[kLatKW][4]) {
    const int rt = rt0 + rstep * j;
    f32x4 acc0[4], acc1[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) acc0[tt] = acc1[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < kLatKW; ++m) {
      const int ks = k0 + w + kLatWaves * m;
      if (ks >= k1) continue;
      const bool p1 = OUT && ks >= pl.KS0;
      const uint16_t *xrow = xs + (ks - k0) * kStepK + q * 32;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        if (tt >= TT) continue;
        const int tok = tt * 16 + i;
        u32x4 bv[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          bv[kk] = tok < B ? *reinterpret_cast<const u32x4 *>(xrow + tok * pl.xpitch + kk * 8) : u32x4{0, 0, 0, 0};
        if (p1) {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) acc1[tt] = mfma16(as_bf16x8(buf[m][kk]), as_bf16x8(bv[kk]), acc1[tt]);
        } else {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) acc0[tt] = mfma16(as_bf16x8(buf[m][kk]), as_bf16x8(bv[kk]), acc0[tt]);
        }
      }
    }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      if (tt >= TT) continue;
      if (touch0) *reinterpret_cast<f32x4 *>(red + ((0 * TT + tt) * kLatWaves + w) * 256 + l * 4) = acc0[tt];
      if (touch1) *reinterpret_cast<f32x4 *>(red + ((1 * TT + tt) * kLatWaves + w) * 256 + l * 4) = acc1[tt];
    }
    ring_barrier();
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      if (p == 0 ? !touch0 : !touch1) continue;
#pragma unroll
      for (int c = 0; c < 2; ++c) {  // TT * 256 <= 2 * kLatThreads items
        const int it = tid + c * kLatThreads;
        if (it >= TT * 256) continue;
        const int t = it >> 4, r = it & 15;
        const float v = red_sum(red + (p * TT + (t >> 4)) * kLatWaves * 256, tile_index(r, t & 15));
        const uint32_t off = t < B ? (uint32_t)((((long)s * pl.RT + rt) * B + t) * 64 + r * 4) : kOffNone;
        st_dev32(p == 0 ? rp0 : rp1, off, __float_as_uint(v));
      }
    }
    ring_barrier();
  };

  for (int j = 0; j < J; j += 3) {
    issue(j + 2, b2);
    unit(j, b0);
    if (j + 1 >= J) break;
    issue(j + 3, b0);
    unit(j + 1, b1);
    if (j + 2 >= J) break;
    issue(j + 4, b1);
    unit(j + 2, b2);
  }

  // count the units in (one lane of wave 0 per unit, all atomics in flight
  // together); the workgroup that completes a tile finishes it
  if (tid == 0) s_nfin = 0;
  wait_vmem();  // this wave's partial stores are complete
  __syncthreads();
  if (tid < J) {
    const int rt = rt0 + rstep * tid;
    int ci = rt, need = SP;
    if (!OUT && rt >= pl.ntile0) {  // a shared gate tile and its up tile share a counter
      ci = pl.ntile0 + (rt - pl.ntile0) % (pl.S / 16);
      need = 2 * SP;
    }
    const unsigned old = __hip_atomic_fetch_add(cnt + ci, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == (unsigned)need - 1u) {
      __hip_atomic_store(cnt + ci, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_fin[atomicAdd(&s_nfin, 1)] = ci;
    }
  }
  __syncthreads();
  const int nfin = s_nfin;
  if (nfin) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  int s0 = 0, last0 = SP;  // <1>: splits [0, last0) have part-0 k-steps, [s0, SP) part-1 k-steps
  if (OUT) {
    while (s0 < SP && lat_k0(s0 + 1, pl.KS, SP) <= pl.KS0) ++s0;
    last0 = lat_k0(s0, pl.KS, SP) < pl.KS0 ? s0 + 1 : s0;
  }
  for (int f = 0; f < nfin; ++f) {
    const int ci = s_fin[f];
#pragma unroll
    for (int c = 0; c < 2; ++c) {  // B * 16 <= 2 * kLatThreads outputs
      const int it = tid + c * kLatThreads;
      if (it >= B * 16) continue;
      const int t = it >> 4, r = it & 15;
      // every split's partials are loaded first, then summed in split order
      auto off = [&](int ss, int rt) { return (uint32_t)((((long)ss * pl.RT + rt) * B + t) * 64 + r * 4); };
      float va[kLatMaxSplits], vb[kLatMaxSplits];
      const int rta = ci, rtb = !OUT ? ci + pl.S / 16 : ci;
      const bool two = OUT || ci >= pl.ntile0;
#pragma unroll
      for (int ss = 0; ss < kLatMaxSplits; ++ss) {
        va[ss] = vb[ss] = 0.f;
        if (ss < SP) {
          va[ss] = bload4_dev(rp0, off(ss, rta));
          if (two) vb[ss] = bload4_dev(OUT ? rp1 : rp0, off(ss, rtb));
        }
      }
      float sa = 0.f, sb = 0.f;
#pragma unroll
      for (int ss = 0; ss < kLatMaxSplits; ++ss) {
        if (ss < SP && ss < last0) sa += va[ss];
        if (ss < SP && (OUT ? ss >= s0 : two)) sb += vb[ss];
      }
      if (!OUT) {
        if (ci < pl.ntile0)
          a.ya[(long)t * pl.lh + ci * 16 + r] = f32_to_bf16_bits(sa);
        else
          a.yb[(long)t * pl.S + (ci - pl.ntile0) * 16 + r] =
              f32_to_bf16_bits(apply_act(pl.act, round_bf16(sa), round_bf16(sb)));
      } else {
        a.ya[(long)t * pl.h + ci * 16 + r] = f32_to_bf16_bits(round_bf16(sa) + round_bf16(sb));
      }
    }
  }
}

}  // namespace k3moe
