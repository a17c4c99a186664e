// Decode path: the whole MoE step in one persistent kernel (B <= 64 tokens).
//
// One 512-thread workgroup (8 waves) per CU. Phases, separated by grid
// barriers where a phase needs every workgroup's results:
//   R   router logits on MFMA. Workgroup unit = (16 router rows, k-split s)
//       for every token tile; each wave takes a 128-k step of the split with
//       all its loads in flight, the waves meet in LDS and one partial per
//       (split, logit) reaches memory.                          (kimi.py:308)
//   --- barrier 1
//   T   gating and top-k: partials summed in split order, sigmoid + bias (or
//       softmax), the k largest by the workgroup's threshold-and-rank
//       selection (block_topk), weights renormalised, ids sorted; token t is
//       routed by workgroup t, which publishes its pairs.     (kimi.py:308-316)
//   --- barrier 2 (only when tokens are routed by different workgroups)
//   G   every workgroup rebuilds the expert grouping in its own LDS (active
//       experts ascending, token pairs ascending inside an expert, chunk
//       offsets), so no barrier is needed after it.            (kimi.py:319-320)
//   GU  gate/up: stream-K over groups of (expert, token chunk, 8 gate + 8 up
//       rows) units with the chunks' activation rows staged in LDS; SiTU /
//       SiLU epilogue; bf16 h to memory.                       (kimi.py:321-322)
//   --- barrier 3 (general row-tile down only; the other down paths wait on
//       per-expert counts of finished gate/up units)
//   DN  many active experts: expert-major (expert, 16-row tile) ranges per
//       wave, bf16 y per pair staged in LDS and written out in bulk, then
//       barrier 4 and the combine (w * bf16(y), ascending expert order).
//       Few active experts: each workgroup takes 16 output rows of every
//       active expert and sums w * bf16(y) in LDS; with at most 8 (one per
//       wave) and two row tiles per workgroup, a wave's weights for both
//       tiles are loaded while its expert's gate/up completes.  (kimi.py:318-323)
// The barrier spin is bounded: a workgroup that waits too long sets the
// error word and every workgroup runs to the end.
#pragma once

#include <stddef.h>

#include <type_traits>

#include "k3moe_barrier.hpp"
#include "k3moe_device.hpp"
#include "k3moe_general.hpp"
#include "k3moe_plan.hpp"

namespace k3moe {

constexpr int kDnDepth = 2;                // down k-steps per pipelined item
constexpr int kDnExpertMajorMin = 32;      // more active experts: expert-major down + combine

struct DecodeArgs {
  const uint16_t *x;     // [B, h] router input
  const uint16_t *xin;   // [B, K] expert input (x or latent)
  const uint16_t *router;
  const float *bias;
  const uint8_t *gblk, *gscl, *ublk, *uscl, *dblk, *dscl;
  const int64_t *routes;
  float *out;
  int64_t *out_ids;
  float *out_w;
  float *out_short;
  char *ws;
  // the latent block's input projections (Plan::lat_in): latent_down [K, h],
  // shared_gate / shared_up [S, h] (bf16) and shared_h [B, S] (bf16 out); the
  // latent itself goes to xin
  const uint16_t *lat_ld, *lat_sg, *lat_su;
  uint16_t *lat_sh;
  // the single-token kernel's latent block output (Plan::lat_out): latent_norm
  // [K], latent_up [h, K], shared_down [h, S] (bf16) and the block's output [h] (bf16)
  const uint16_t *lat_norm, *lat_up, *lat_sd;
  uint16_t *lat_y;
};

// The memory pipeline serves older waves first, so in a stream split evenly
// over the waves the younger ones fall behind. Each wave publishes its
// progress (in 1/4096 of its range) in prog[8] and raises its issue priority
// while it is behind the workgroup's mean. The branch is wave-uniform:
// s_setprio ignores the exec mask.
__device__ __forceinline__ void balance_waves(int *prog, int done, int total) {
  const int w = wave_id();
  const int mine = total > 0 ? done * 4096 / total : 4096;
  if ((threadIdx.x & 63) == 0) __hip_atomic_store(prog + w, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  // relaxed atomic loads: read afresh each call, and (unlike volatile ones,
  // which keep a generic address) compiled as LDS reads, which wait for
  // nothing but LDS; a flat read would wait for the wave's weight loads
  int sum = 0;
#pragma unroll
  for (int j = 0; j < kDecWaves; ++j) sum += __hip_atomic_load(prog + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  if (__builtin_amdgcn_readfirstlane(mine * kDecWaves < sum ? 1 : 0)) __builtin_amdgcn_s_setprio(2);
  else __builtin_amdgcn_s_setprio(0);
}

// The first 8-byte aligned address at or after p (an LDS pointer), derived from
// p by pointer arithmetic so that it stays an LDS pointer for the compiler (an
// integer round trip would make its accesses flat ones, which also wait for
// the wave's global loads).
__device__ __forceinline__ uint64_t *lds_align8(int *p) {
  char *c = reinterpret_cast<char *>(p);
  return reinterpret_cast<uint64_t *>(c + ((8 - (reinterpret_cast<uintptr_t>(c) & 7)) & 7));
}

// The first 16-byte aligned address at or after p (an LDS pointer; see lds_align8).
__device__ __forceinline__ char *lds_align16(int *p) {
  char *c = reinterpret_cast<char *>(p);
  return c + ((16 - (reinterpret_cast<uintptr_t>(c) & 15)) & 15);
}

// Trace slots of workgroup blockIdx.x starting at `slot`, or null when not tracing.
__device__ __forceinline__ uint64_t *trace_slots(const Plan &pl, char *ws, int slot) {
  return pl.o_trace ? reinterpret_cast<uint64_t *>(ws + pl.o_trace) + blockIdx.x * kTraceSlots + slot : nullptr;
}

// Phase timestamps (100 MHz real-time counter) of workgroup blockIdx.x, when
// the plan carries a trace area; slot n of kTraceSlots.
__device__ __forceinline__ void trace_mark(const Plan &pl, char *ws, int n) {
  if (pl.o_trace && threadIdx.x == 0)
    reinterpret_cast<uint64_t *>(ws + pl.o_trace)[blockIdx.x * kTraceSlots + n] = __builtin_amdgcn_s_memrealtime();
}

__device__ __forceinline__ void wave_lds_order() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Sum of the 8 per-wave tiles at element `idx` of the LDS reduction area, in wave order.
__device__ __forceinline__ float red_sum(const float *red, int idx) {
  float s = red[idx];
#pragma unroll
  for (int w = 1; w < kDecWaves; ++w) s += red[w * 256 + idx];
  return s;
}

// Position of element (row, col) of a 16x16 MFMA result in a wave's 256-float tile.
__device__ __forceinline__ int tile_index(int row, int col) { return (col + 16 * (row >> 2)) * 4 + (row & 3); }

// ------------------------------------------------------- workgroup top-k --
// LDS of block_topk: the group maxima of the 32-bit keys and of the 64-bit
// values ([group][wave] each), the candidates, their counts.
struct BlockTopk {
  uint32_t gmax[32 * kDecWaves];
  uint64_t gmax64[32 * kDecWaves];
  uint64_t cand[kMaxExperts];
  int count, count64;
};
constexpr int kTopkCandCap = 64;  // more candidates than this after the 32-bit threshold: the 64-bit one

// One DPP step of a 64-bit maximum or minimum with the lane the control selects.
template <int Ctrl, bool Max>
__device__ __forceinline__ uint64_t dpp_fold64(uint64_t v) {
  const uint64_t o = ((uint64_t)dpp<Ctrl, 0xF>((uint32_t)(v >> 32)) << 32) | dpp<Ctrl, 0xF>((uint32_t)v);
  return Max ? (o > v ? o : v) : (o < v ? o : v);
}

// Folds v over aligned runs of n consecutive lanes (n a power of two up to 64):
// every lane of a run ends with the run's maximum (Max) or minimum. Runs of up
// to 16 lanes use DPP (quad swaps, then the half-row and row mirrors, which
// pair every lane with one of the other half once the halves are uniform);
// longer runs add cross-row shuffles.
template <bool Max>
__device__ __forceinline__ uint64_t fold_runs(uint64_t v, int n) {
  if (n >= 2) v = dpp_fold64<kDppQuadXor1, Max>(v);
  if (n >= 4) v = dpp_fold64<kDppQuadXor2, Max>(v);
  if (n >= 8) v = dpp_fold64<kDppHalfMirror, Max>(v);
  if (n >= 16) v = dpp_fold64<kDppMirror, Max>(v);
#pragma unroll
  for (int d = 16; d < 64; d *= 2) {
    if (n > d) {
      const uint64_t o = ((uint64_t)(uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), d, kWave) << 32) |
                         (uint32_t)__shfl_xor((int)(uint32_t)v, d, kWave);
      v = Max ? (o > v ? o : v) : (o < v ? o : v);
    }
  }
  return v;
}
// The same for 32-bit values.
template <bool Max>
__device__ __forceinline__ uint32_t fold_runs32(uint32_t v, int n) {
  auto op = [](uint32_t x, uint32_t y) { return Max ? (x > y ? x : y) : (x < y ? x : y); };
  if (n >= 2) v = op(v, dpp<kDppQuadXor1, 0xF>(v));
  if (n >= 4) v = op(v, dpp<kDppQuadXor2, 0xF>(v));
  if (n >= 8) v = op(v, dpp<kDppHalfMirror, 0xF>(v));
  if (n >= 16) v = op(v, dpp<kDppMirror, 0xF>(v));
#pragma unroll
  for (int d = 16; d < 64; d *= 2)
    if (n > d) v = op(v, (uint32_t)__shfl_xor((int)v, d, kWave));
  return v;
}
__device__ __forceinline__ uint64_t lane0_u64(uint64_t v) {
  return ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32)) << 32) |
         (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
}

// Top-k (1 <= k <= 32) of the ordered keys key0 (expert tid) and key1 (expert
// tid + 512) of every thread (E <= 1024 experts), with the order of wave_topk:
// larger keys first, equal keys in ascending expert order, i.e. the k largest
// of the distinct 64-bit values key << 32 | ~expert; sel[0..k) gets the
// experts in that rank order.
//   1. Threshold: with G the power of two >= k, group g is the experts whose
//      thread's lane lies in the g-th run of 64 / G lanes; T = the smallest of
//      the G group maxima of the keys. At least G >= k experts have a key >= T
//      (each group's maximum is an expert's key; a group without experts has
//      maximum 0, and then every key is >= T), so the k-th largest key is >= T
//      and every top-k expert is a candidate (key >= T). Group maxima are taken
//      in DPP runs and over the waves ([group][wave] in LDS, two 16-byte reads).
//      When exact ties leave more than kTopkCandCap candidates, the threshold
//      is taken again on the 64-bit values: their G group maxima are distinct,
//      so at most ~G + 64 values reach it whatever the ties.
//   2. Candidates are appended to an LDS list (order free: a rank does not
//      depend on it).
//   3. Ranks: wave w takes candidates 8w + 64 c .. (8 lanes each, c = 0, 1, ..);
//      lane part p of a candidate counts the candidates j = p mod 8 above it
//      (four reads in flight), the 8 lanes add their counts (DPP), and ranks
//      below k are written to sel.
// Every thread of the workgroup calls it; it ends with a barrier after sel is written.
__device__ __forceinline__ void block_topk(uint32_t key0, uint32_t key1, int E, int k, int *sel, BlockTopk &tk) {
  const int tid = threadIdx.x, w = wave_id(), l = tid & 63;
  int G = 1;
  while (G < k) G <<= 1;
  const int run = 64 / G;
  const int e0 = tid, e1 = tid + kDecThreads;
  const bool ok0 = e0 < E, ok1 = e1 < E;
  {
    const uint32_t a0 = ok0 ? key0 : 0u, a1 = ok1 ? key1 : 0u;
    const uint32_t m = fold_runs32<true>(a0 > a1 ? a0 : a1, run);
    if ((l & (run - 1)) == 0) tk.gmax[(l / run) * kDecWaves + w] = m;
  }
  if (tid == 0) {
    tk.count = 0;
    tk.count64 = 0;
  }
  __syncthreads();
  // lane g < G: group g's maximum over the waves; then the minimum over lanes 0 .. G - 1
  uint32_t g = 0xFFFFFFFFu;
  if (l < G) {
    const u32x4 p0 = *reinterpret_cast<const u32x4 *>(tk.gmax + l * kDecWaves);
    const u32x4 p1 = *reinterpret_cast<const u32x4 *>(tk.gmax + l * kDecWaves + 4);
    g = p0[0];
#pragma unroll
    for (int t = 1; t < 4; ++t) g = p0[t] > g ? p0[t] : g;
#pragma unroll
    for (int t = 0; t < 4; ++t) g = p1[t] > g ? p1[t] : g;
  }
  const uint32_t T = (uint32_t)__builtin_amdgcn_readfirstlane((int)fold_runs32<false>(g, G));
  const uint64_t v0 = ok0 ? ((uint64_t)key0 << 32) | (uint32_t)~e0 : 0ull;
  const uint64_t v1 = ok1 ? ((uint64_t)key1 << 32) | (uint32_t)~e1 : 0ull;
  // appends the values with flag f0 / f1 to the candidate list, counted on cnt
  auto append = [&](bool f0, bool f1, int &cnt) {
    const uint64_t b0 = __ballot(f0), b1 = __ballot(f1);
    const int n0 = __popcll(b0), n = n0 + __popcll(b1);
    int base = 0;
    if (n > 0) {
      if (l == 0) base = atomicAdd(&cnt, n);
      base = __builtin_amdgcn_readfirstlane(base);
    }
    const int below0 = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b0 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b0, 0u));
    const int below1 = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b1 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b1, 0u));
    if (f0) tk.cand[base + below0] = v0;
    if (f1) tk.cand[base + n0 + below1] = v1;
  };
  append(ok0 && key0 >= T, ok1 && key1 >= T, tk.count);
  __syncthreads();
  int nc = __builtin_amdgcn_readfirstlane(tk.count);
  if (nc > kTopkCandCap) {  // workgroup-uniform: exact ties; the threshold on the distinct 64-bit values
    const uint64_t m = fold_runs<true>(v0 > v1 ? v0 : v1, run);
    if ((l & (run - 1)) == 0) tk.gmax64[(l / run) * kDecWaves + w] = m;
    __syncthreads();  // also: every thread has read the first count, so the list is free
    uint64_t g64 = ~0ull;
    if (l < G) {
      const u32x4 *p = reinterpret_cast<const u32x4 *>(tk.gmax64 + l * kDecWaves);
      u32x4 q4[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) q4[t] = p[t];
      g64 = 0ull;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint64_t oa = ((uint64_t)q4[t][1] << 32) | q4[t][0], ob = ((uint64_t)q4[t][3] << 32) | q4[t][2];
        g64 = oa > g64 ? oa : g64;
        g64 = ob > g64 ? ob : g64;
      }
    }
    const uint64_t T64 = lane0_u64(fold_runs<false>(g64, G));
    append(ok0 && v0 >= T64, ok1 && v1 >= T64, tk.count64);
    __syncthreads();
    nc = __builtin_amdgcn_readfirstlane(tk.count64);
  }
  const int cc = l >> 3, part = l & 7;
  for (int c0 = 8 * w; c0 < nc; c0 += 8 * kDecWaves) {  // wave-uniform
    const int c = c0 + cc;
    const uint64_t me = tk.cand[c < nc ? c : 0];
    int rank = 0;
    for (int j0 = 0; j0 < nc; j0 += 32) {
      uint64_t o[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int j = j0 + 8 * u + part;
        o[u] = tk.cand[j < nc ? j : 0];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) rank += (j0 + 8 * u + part < nc && o[u] > me) ? 1 : 0;
    }
    rank += (int)dpp<kDppQuadXor1, 0xF>((uint32_t)rank);
    rank += (int)dpp<kDppQuadXor2, 0xF>((uint32_t)rank);
    rank += (int)dpp<kDppHalfMirror, 0xF>((uint32_t)rank);
    if (part == 0 && c < nc && rank < k) sel[rank] = (int)~(uint32_t)me;
  }
  __syncthreads();
}

// ---------------------------------------------------------------- gate/up --
// A unit is 8 gate + 8 up rows of one (active expert, chunk of up to NX
// tokens): one 16x16 MFMA tile. Units form groups of W (W = 2 when the grid
// has at least two units per workgroup and pairs balance, gu_pairs; else 1), ordered expert-major, chunk,
// unit. Workgroup b takes groups [NG b / G, NG (b + 1) / G) in rounds; a round
// is a run of whole chunks whose token rows fit the LDS staging area (NX
// rows), copied there once, so the MFMA B operand comes from LDS. Inside a
// round the (group, super-step) pairs -- a super-step is 16 MXFP4 blocks, 512
// k -- are cut into 8 equal contiguous ranges, one per wave: a wave streams its
// range with the next super-step's loads in flight, finishes every group it
// covers whole and leaves partial tiles of the groups cut by its range ends in
// LDS; after a barrier, the wave holding a cut group's first part adds the
// other parts in ascending k order and finishes it.
// Lane (i, q) covers row i of a tile and, at k-step t of super-step ss, block
// 16 ss + 4 t + q: a load instruction reads 64 contiguous bytes of 16 rows,
// and the lane's 4 scales of a super-step are byte q of the dwords of one
// 16-byte load (K a multiple of 512; otherwise per-lane byte loads).
template <int W>
struct GuSS {
  u32x4 a[W][4];  // per unit, k-steps t = 0..3
  u32x4 s[W];     // per unit, dword t holds the scale of this lane's block in byte q
};

struct GuChunk {  // one chunk of the current round (LDS)
  int e;          // expert id
  int pbase;      // pair index of the chunk's first token
  int n;          // tokens in the chunk
  int xrow;       // first staged row
};

template <int W, bool AL>
__device__ __forceinline__ void gu_issue(GuSS<W> &B, const uint8_t *const (&wr)[W], const uint8_t *const (&sr)[W],
                                         int ss, int KB) {
  const int q = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int u = 0; u < W; ++u) {
    if (AL) {
#pragma unroll
      for (int t = 0; t < 4; ++t) B.a[u][t] = load16(wr[u] + (16 * ss + 4 * t + q) * 16);
      B.s[u] = load16(sr[u] + 16 * ss);
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int kb = 16 * ss + 4 * t + q;
        const bool ok = kb < KB;
        B.a[u][t] = ok ? load16(wr[u] + kb * 16) : u32x4{0, 0, 0, 0};
        B.s[u][t] = ok ? (uint32_t)sr[u][kb] << (8 * q) : 0u;
      }
    }
  }
}

// acc[u] += tile u over super-step ss; xrow: this lane's staged token row (LDS).
// The scale words enter here through an empty asm: loads issued early (before
// the round table, or a super-step ahead) would otherwise have their scale
// conversion hoisted next to them, and the wave would wait there for them.
template <int W, bool AL>
__device__ __forceinline__ void gu_compute(const GuSS<W> &B, const uint16_t *xrow, int ss, int KB, f32x4 (&acc)[W]) {
  const int q = (threadIdx.x & 63) >> 4;
  u32x4 sc[W];
#pragma unroll
  for (int u = 0; u < W; ++u) {
    sc[u] = B.s[u];
    asm volatile("" : "+v"(sc[u]));
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if (!AL && 16 * ss + 4 * t >= KB) break;  // wave-uniform: nothing left in this super-step
    const int kb = 16 * ss + 4 * t + q;
    const bool ok = AL || kb < KB;
    u32x4 b[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      b[kk] = ok ? *reinterpret_cast<const u32x4 *>(xrow + kb * kBlockK + kk * 8) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < W; ++u) {
      bf16x8 av[4];
      convert_block_fast(B.a[u][t], (sc[u][t] >> (8 * q)) & 0xFFu, av);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) acc[u] = mfma16(av[kk], as_bf16x8(b[kk]), acc[u]);
    }
  }
}

// n * b / gridDim.x, rounded down, for the persistent grid (a power of two):
// a shift instead of a 64-bit division (whose expansion is long, and first
// executed code costs instruction fetches).
__device__ __forceinline__ int grid_share(int n, unsigned b) {
  return (int)(((uint64_t)(unsigned)n * b) >> __builtin_ctz(gridDim.x));
}

// n * w / kDecWaves, rounded down (n >= 0).
__device__ __forceinline__ int wave_share(int n, int w) {
  return (int)(((uint64_t)(unsigned)n * (unsigned)w) >> 3);
}
static_assert(kDecWaves == 8, "wave_share divides by 8");

// Gate/up groups of two units (W = 2) for nu units over the grid: when there
// are at least two units per workgroup, and the whole groups balance as well
// as single units or there are at least 8 units per workgroup (one group more
// or less then costs at most an eighth).
__device__ __forceinline__ bool gu_pairs(int nu) {
  const int G = (int)gridDim.x;
  if (nu < 2 * G) return false;
  return cdiv(cdiv(nu, 2), G) * 2 <= cdiv(nu, G) || nu >= 8 * G;
}

// Activation epilogue of a full-K unit tile held by one wave: lanes 0-31 hold
// the gate rows, lanes 32-63 the up rows of the same (row, token); lanes 0-31
// write h[p][row0 .. row0+7] for their token column.
__device__ __forceinline__ void gu_finish_wave(const Plan &pl, uint16_t *hbuf, const f32x4 &acc, int p,
                                               bool tok_ok, int row0) {
  const int l = threadIdx.x & 63;
  float up[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) up[v] = __shfl_xor(acc[v], 32, 64);
  if (l < 32 && tok_ok) {
    uint16_t hb[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) hb[v] = f32_to_bf16_bits(apply_act(pl.act, round_bf16(acc[v]), round_bf16(up[v])));
    u32x2 packed = {(uint32_t)hb[0] | ((uint32_t)hb[1] << 16), (uint32_t)hb[2] | ((uint32_t)hb[3] << 16)};
    st_dev64(make_rsrc(hbuf, (uint32_t)pl.P * pl.I * 2), (uint32_t)((size_t)p * pl.I + row0 + 4 * (l >> 4)) * 2,
             packed);
  }
}

// The gate/up phase of one workgroup (see the comment above GuSS).
template <int W, bool AL>
__device__ __forceinline__ void gu_phase(const Plan &pl, const DecodeArgs &a, float *red, const int *g_act,
                                      const int *g_aoff, const int *g_acnt, const int *g_coff, const int *g_cexp,
                                      const int *g_ptok,
                                      uint16_t *xs, GuChunk *tab, int *s_round, int *s_rowtok, int *s_prog, int D,
                                      uint16_t *hbuf, const u32x4 (&xpre)[2], bool xpre_ok) {
  const int tid = threadIdx.x, w = wave_id(), l = tid & 63, i = l & 15;
  const int KB = pl.K / kBlockK, NSS = (KB + 15) / 16, K8 = pl.K / 8;
  const int GPC = pl.U8 / W;  // groups per chunk
  const int NG = g_coff[D] * GPC;
  const int ga = grid_share(NG, blockIdx.x), gb = grid_share(NG, blockIdx.x + 1);
  auto slot = [&](int wv, int which, int u) { return red + ((wv * 2 + which) * 2 + u) * 256 + l * 4; };
  // unit rows: lanes 0-7 gate, 8-15 up
  const uint8_t *const lane_blk = i >= 8 ? a.ublk : a.gblk;
  const uint8_t *const lane_scl = i >= 8 ? a.uscl : a.gscl;
  // The first round usually holds all of this workgroup's groups: assuming it
  // does, each wave's range and first expert are known before the round table,
  // so its first super-step's weight loads are issued first and the table is
  // built while they are in flight. They are the loads the round needs when
  // the wave's range starts at the same position (always when the assumption
  // holds); otherwise they are issued again.
  GuSS<W> B0, B1;
  int s_pre = -1;
  // Whole 512-column row chunks (K a multiple of 512, more than one token):
  // each round's activation rows are loaded straight into LDS before its
  // first weights, and only the rows are waited for; no weights go out before
  // the round table (their issue would hold up the table's barrier).
  const bool dma_rows = AL && !xpre_ok;
  trace_mark(pl, a.ws, 12);
  if (!dma_rows && ga < gb) {
    const int work = (gb - ga) * NSS;
    const int s = wave_share(work, w), e = wave_share(work, w + 1);
    if (s < e) {
      const int G = ga + s / NSS, ci = G / GPC, pg = G % GPC;
      const int lo = g_cexp[ci];  // active expert of chunk ci
      const uint8_t *wr[W], *sr[W];
#pragma unroll
      for (int u = 0; u < W; ++u) {
        const size_t row = (size_t)g_act[lo] * pl.I + (pg * W + u) * 8 + (i & 7);
        wr[u] = lane_blk + row * KB * 16;
        sr[u] = lane_scl + row * KB;
      }
      gu_issue<W, AL>(B0, wr, sr, s % NSS, KB);
      s_pre = s;
    }
  }
  trace_mark(pl, a.ws, 13);
  for (int g0 = ga; g0 < gb;) {
    const int ci0 = g0 / GPC;
    // LDS-only barriers in the round (no vector-memory wait): the previous round is
    // done with the table, the staged rows and the partial tiles
    ring_barrier();
    if (g0 == ga) trace_mark(pl, a.ws, 45);
    if (w == 0) {
      // lane j < 16 takes chunk ci0 + j; the round is the prefix of chunks whose rows fit
      const int ci = ci0 + l;
      const bool in = l < 16 && ci * GPC < gb;
      int n = 0, e = 0, pbase = 0;
      if (in) {
        const int lo = g_cexp[ci];  // active expert of chunk ci
        const int c = ci - g_coff[lo];
        e = g_act[lo];
        pbase = g_aoff[lo] + c * pl.NX;
        n = min(pl.NX, g_acnt[lo] - c * pl.NX);
      }
      if (g0 == ga && pl.o_trace && l == 0)
        reinterpret_cast<uint64_t *>(a.ws + pl.o_trace)[blockIdx.x * kTraceSlots + 46] =
            __builtin_amdgcn_s_memrealtime() + (uint64_t)(n & 0);
      const int pre = wave_incl_scan(n);  // inclusive prefix of the token counts (lanes >= 16 add 0)
      const bool fits = in && pre <= pl.NX;
      const int nch = __popcll(__ballot(fits));  // >= 1: one chunk never exceeds NX rows
      const int rows = __builtin_amdgcn_readlane(pre, nch - 1);
      if (fits) tab[l] = GuChunk{e, pbase, n, pre - n};
      // staged row l's chunk: the number of chunks that end at or before it
      int j = 0;
      for (int jj = 0; jj + 1 < nch; ++jj) j += __builtin_amdgcn_readlane(pre, jj) <= l ? 1 : 0;
      wave_lds_order();
      if (l < rows) s_rowtok[l] = g_ptok[tab[j].pbase + l - tab[j].xrow];  // staged row l: token of its chunk
      if (l == 0) {
        s_round[0] = nch;
        s_round[1] = rows;
      }
      if (g0 == ga) trace_mark(pl, a.ws, 47);
    }
    ring_barrier();
    if (g0 == ga) trace_mark(pl, a.ws, 32);
    const int nch = s_round[0], rows = s_round[1];
    const int g1 = min(gb, (ci0 + nch) * GPC);
    const int work = (g1 - g0) * NSS;
    const int s = wave_share(work, w), e = wave_share(work, w + 1);
    // unit rows of group gg of the round (relative to g0)
    auto rows_of = [&](int gg, const uint8_t *(&wr)[W], const uint8_t *(&sr)[W]) {
      const int G = g0 + gg, j = G / GPC - ci0, pg = G % GPC;
      const int ex = tab[j].e;
#pragma unroll
      for (int u = 0; u < W; ++u) {
        const size_t row = (size_t)ex * pl.I + (pg * W + u) * 8 + (i & 7);
        wr[u] = lane_blk + row * KB * 16;
        sr[u] = lane_scl + row * KB;
      }
    };
    auto xrow_of = [&](int gg) {
      const GuChunk ch = tab[(g0 + gg) / GPC - ci0];
      return (const uint16_t *)(xs + (size_t)(ch.xrow + min(i, ch.n - 1)) * pl.xpitch);
    };
    auto finish = [&](int gg, const f32x4 (&acc)[W]) {
      const int G = g0 + gg, pg = G % GPC;
      const GuChunk ch = tab[G / GPC - ci0];
#pragma unroll
      for (int u = 0; u < W; ++u) gu_finish_wave(pl, hbuf, acc[u], ch.pbase + i, i < ch.n, (pg * W + u) * 8);
    };
    const uint8_t *iwr[W], *isr[W];
    int ig = s / NSS, iss = s % NSS;  // issue cursor
    if (dma_rows) {
      // the round's rows (1 KiB of a row per instruction, spread over the waves), then the weights
      const int per_row = pl.K / 512;
      for (int c = w; c < rows * per_row; c += kDecWaves) {
        const int r = c / per_row, j = c - r * per_row;
        load_lds<16>(a.xin + (size_t)s_rowtok[r] * pl.K + j * 512 + l * 8,
                     reinterpret_cast<char *>(xs + (size_t)r * pl.xpitch + j * 512));
      }
      asm volatile("" ::: "memory");  // the row loads stay ahead of the weights
    }
    if (s < e) {
      rows_of(ig, iwr, isr);
      if (s != s_pre) gu_issue<W, AL>(B0, iwr, isr, iss, KB);  // else issued before the table, the same loads
    }
    s_pre = -1;  // later rounds issue their own
    // progress of each wave's range in 1/4096 (empty ranges count as done);
    // visible to the workgroup's other waves after the staging barrier
    if (l == 0) __hip_atomic_store(s_prog + w, s < e ? 0 : 4096, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    // stage the round's activation rows (eight rows per pass, every load in flight);
    // a single token's row was loaded into xpre after the first barrier (every
    // staged row of a round is then that token's)
    for (int r = 0; xpre_ok && r < rows; ++r) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int c = hh * kDecThreads + tid;
        if (c < K8) *reinterpret_cast<u32x4 *>(xs + (size_t)r * pl.xpitch + c * 8) = xpre[hh];
      }
    }
    if (dma_rows) {  // wait for the rows only: after them each wave issued 5 W weight loads, or none
      if (s < e) wait_vm<5 * W>();
      else wait_vm<0>();
    }
    for (int r0 = 0; !xpre_ok && !dma_rows && r0 < rows; r0 += 8) {
      for (int c0 = 0; c0 < K8; c0 += 2 * kDecThreads) {
        u32x4 v[8][2];
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) {
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const int c = c0 + hh * kDecThreads + tid;
            const bool ok = r0 + rr < rows && c < K8;
            v[rr][hh] = ok ? load16(a.xin + (size_t)s_rowtok[r0 + rr] * pl.K + c * 8) : u32x4{0, 0, 0, 0};
          }
        }
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) {
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const int c = c0 + hh * kDecThreads + tid;
            if (r0 + rr < rows && c < K8) *reinterpret_cast<u32x4 *>(xs + (size_t)(r0 + rr) * pl.xpitch + c * 8) = v[rr][hh];
          }
        }
      }
    }
    ring_barrier();  // staged rows visible; each wave's compute waits for its own weight loads
    if (g0 == ga) trace_mark(pl, a.ws, 33);
    if (s < e) {
      int cg = ig, css = iss;  // compute cursor
      const uint16_t *xrow = xrow_of(cg);
      f32x4 acc[W];
#pragma unroll
      for (int u = 0; u < W; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
      // step(pos): issue super-step pos + 1 (always: past the range end the
      // range's last super-step again, an L2 hit), then compute pos if it is in
      // the range. An issue under a condition would make the compiler's wait for
      // pos's data cover the loads just issued (vmcnt(0) at the join), and the
      // stream would run one super-step deep.
      auto step = [&](GuSS<W> &cur, GuSS<W> &nxt, int pos) {
        if (pos + 1 < e) {
          if (++iss == NSS) {
            iss = 0;
            rows_of(++ig, iwr, isr);
          }
        }
        gu_issue<W, AL>(nxt, iwr, isr, iss, KB);
        if (pos >= e) return;  // wave-uniform: the odd step past an odd range
        gu_compute<W, AL>(cur, xrow, css, KB, acc);
        balance_waves(s_prog, pos + 1 - s, e - s);
        if (++css == NSS || pos + 1 == e) {
          const bool started_here = cg * NSS >= s;
          if (started_here && css == NSS) {
            finish(cg, acc);
          } else {
#pragma unroll
            for (int u = 0; u < W; ++u) *reinterpret_cast<f32x4 *>(slot(w, started_here ? 1 : 0, u)) = acc[u];
          }
#pragma unroll
          for (int u = 0; u < W; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
          if (css == NSS && pos + 1 < e) {
            css = 0;
            xrow = xrow_of(++cg);
          }
        }
      };
      for (int pos = s; pos < e; pos += 2) {
        step(B0, B1, pos);
        step(B1, B0, pos + 1);
      }
    }
    __builtin_amdgcn_s_setprio(0);
    if (g0 == ga) trace_mark(pl, a.ws, 34);
    if (g0 == ga && pl.o_trace && l == 0)  // every wave's stream end
      reinterpret_cast<uint64_t *>(a.ws + pl.o_trace)[blockIdx.x * kTraceSlots + 36 + w] = __builtin_amdgcn_s_memrealtime();
    __syncthreads();
    if (g0 == ga) trace_mark(pl, a.ws, 35);
    // a group cut by wave ranges: the wave holding its first part adds the rest in wave (= k) order
    if (s < e) {
      const int gl = (e - 1) / NSS;
      if (gl * NSS >= s && e < (gl + 1) * NSS) {
        // the parts of later waves, all reads in flight, added in wave order
        f32x4 sum[W], part[kDecWaves - 1][W];
        bool has[kDecWaves - 1];
#pragma unroll
        for (int j = 0; j < kDecWaves - 1; ++j) {
          const int w2 = w + 1 + j;
          const int s2 = wave_share(work, w2), e2 = wave_share(work, w2 + 1);
          has[j] = w2 < kDecWaves && s2 < (gl + 1) * NSS && e2 > s2;
#pragma unroll
          for (int u = 0; u < W; ++u)
            part[j][u] = has[j] ? *reinterpret_cast<const f32x4 *>(slot(w2, 0, u)) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < W; ++u) {
          sum[u] = *reinterpret_cast<const f32x4 *>(slot(w, 1, u));
#pragma unroll
          for (int j = 0; j < kDecWaves - 1; ++j)
            if (has[j]) {
#pragma unroll
              for (int vv = 0; vv < 4; ++vv) sum[u][vv] += part[j][u][vv];
            }
        }
        finish(gl, sum);
      }
    }
    if (g0 == ga) trace_mark(pl, a.ws, 14);
    g0 = g1;
  }
  trace_mark(pl, a.ws, 15);
}

// ------------------------------------------------------ gate/up, pinned --
// For batches whose token rows all fit in LDS (xs, row t at t * xpitch): the
// gate/up units (8 gate + 8 up rows of one chunk of up to 16 of an active
// expert's tokens; unit u = chunk u / U8, rows 8 (u mod U8) ..) are shared out
// over all waves of the grid as contiguous ranges of whole units: global wave
// gw = 8 b + w takes units [NU gw / 8G, NU (gw + 1) / 8G). First the rows of
// the tokens in the workgroup's chunks go to LDS (direct-to-LDS loads, 1 KiB
// of a row per instruction, spread over the waves), each wave issuing its share
// before its first three super-steps of weights, so that waiting for its rows
// (vmcnt) leaves the weights in flight; a barrier publishes the rows. Then a
// wave streams its units' super-steps (16 MXFP4 blocks of 16 rows, 512 k) with
// four in flight and finishes each unit itself (activation, bf16 h): it
// shares nothing with the workgroup's other waves and moves on to the down
// phase as soon as its units are done. Every wave of the workgroup calls it;
// it returns after the wave's h stores have completed.
template <bool AL>
__device__ __forceinline__ void gu_pinned(const Plan &pl, const DecodeArgs &a, const int *g_act, const int *g_aoff,
                                          const int *g_acnt, const int *g_coff, const int *g_cexp, const int *g_ptok,
                                          uint16_t *xs, int *s_prog, uint16_t *hbuf, int ua, int ub, int wa, int wb,
                                          bool staged, bool coherent) {
  static_assert(AL, "pinned rows are loaded in whole 512-column chunks");
  const int w = wave_id(), l = threadIdx.x & 63, i = l & 15;
  const int KB = pl.K / kBlockK, NSS = KB / 16, U8 = pl.U8;
  const int n = (ub - ua) * NSS;  // this wave's super-steps
  const uint8_t *const lane_blk = i >= 8 ? a.ublk : a.gblk;
  const uint8_t *const lane_scl = i >= 8 ? a.uscl : a.gscl;
  // chunk c of active expert d = g_cexp[c]: pairs pbase .. pbase + nt - 1 of the expert
  auto chunk = [&](int c, int &pbase, int &nt) {
    const int d = g_cexp[c];
    pbase = g_aoff[d] + (c - g_coff[d]) * 16;
    nt = min(16, g_aoff[d] + g_acnt[d] - pbase);
  };
  trace_mark(pl, a.ws, 12);
  // the workgroup's token rows: tokens of its chunks (units [wa, wb)), as a bit set (B <= 64);
  // none when every token's row is in LDS already (staged)
  uint64_t rows = 0;
  if (!staged && wa < wb) {
    for (int c = wa / U8; c <= (wb - 1) / U8; ++c) {
      int pbase, nt;
      chunk(c, pbase, nt);
      const int t = l < nt ? g_ptok[pbase + l] : 0;
      const uint64_t bit = l < nt ? 1ull << t : 0ull;  // each lane's token bit, OR-ed over the wave
      rows |= ((uint64_t)wave_or_u32((uint32_t)(bit >> 32)) << 32) | wave_or_u32((uint32_t)bit);
    }
  }
  {
    const int per_row = pl.K / 512, nrows = __popcll(rows);
    uint64_t left = rows;
    int r = 0, rr = -1;
    for (int c = w; c < nrows * per_row; c += kDecWaves) {
      const int want = c / per_row;  // the want-th set bit of rows
      while (rr < want) {
        r = __builtin_ctzll(left);
        left &= left - 1;
        ++rr;
      }
      const int j = c - want * per_row;
      const uint16_t *src = a.xin + (size_t)r * pl.K + j * 512 + l * 8;
      char *dst = reinterpret_cast<char *>(xs + (size_t)r * pl.xpitch + j * 512);
      if (coherent) load_lds<16, kCpolDevice>(src, dst);  // (written in this launch by other workgroups)
      else load_lds<16>(src, dst);
    }
  }
  asm volatile("" ::: "memory");  // the row loads stay ahead of the weights
  auto rows_of = [&](int u, const uint8_t *(&wr)[1], const uint8_t *(&sr)[1]) {
    const int c = u / U8;
    const size_t row = (size_t)g_act[g_cexp[c]] * pl.I + (u - c * U8) * 8 + (i & 7);
    wr[0] = lane_blk + row * KB * 16;
    sr[0] = lane_scl + row * KB;
  };
  auto xrow_of = [&](int u) {  // lane column i: token i of the unit's chunk (the last one again past its end)
    int pbase, nt;
    chunk(u / U8, pbase, nt);
    return (const uint16_t *)(xs + (size_t)g_ptok[pbase + min(i, nt - 1)] * pl.xpitch);
  };
  // issue cursor: position ip (unit iu, super-step iss); past the last position it stays there
  // (an unconditional issue of an L2-resident step keeps the compiler's waits exact)
  const uint8_t *iwr[1], *isr[1];
  int ip = 0, iu = ua, iss = 0;
  auto issue = [&](GuSS<1> &buf) {
    gu_issue<1, AL>(buf, iwr, isr, iss, KB);
    if (ip + 1 < n) {
      ++ip;
      if (++iss == NSS) {
        iss = 0;
        rows_of(++iu, iwr, isr);
      }
    }
  };
  GuSS<1> R0, R1, R2, R3;
  if (n > 0) {
    rows_of(iu, iwr, isr);
    issue(R0);
    issue(R1);
    issue(R2);
    if (!staged) wait_vm<3 * 5>();  // this wave's row loads have landed; the 3 super-steps (5 loads each) stay in flight
  } else {
    if (!staged) wait_vm<0>();
  }
  trace_mark(pl, a.ws, 13);
  if (!staged) ring_barrier();  // every wave's rows are in LDS (staged: published by earlier barriers)
  trace_mark(pl, a.ws, 33);
  if (n <= 0) return;
  int cu = ua, css = 0;
  const uint16_t *xrow = xrow_of(cu);
  f32x4 acc[1] = {f32x4{0.f, 0.f, 0.f, 0.f}};
  // step(pos): issue position pos + 3 into nxt, then compute position pos from cur
  auto step = [&](GuSS<1> &cur, GuSS<1> &nxt, int pos) {
    issue(nxt);
    if (pos >= n) return;  // wave-uniform: the tail of the last group of four
    gu_compute<1, AL>(cur, xrow, css, KB, acc);
    balance_waves(s_prog, pos + 1, n);
    if (++css == NSS) {
      int pbase, nt;
      chunk(cu / U8, pbase, nt);
      gu_finish_wave(pl, hbuf, acc[0], pbase + i, i < nt, (cu % U8) * 8);
      acc[0] = f32x4{0.f, 0.f, 0.f, 0.f};
      css = 0;
      if (pos + 1 < n) xrow = xrow_of(++cu);
    }
  };
  for (int pos = 0; pos < n; pos += 4) {
    step(R0, R3, pos);
    step(R1, R0, pos + 1);
    step(R2, R1, pos + 2);
    step(R3, R2, pos + 3);
  }
  __builtin_amdgcn_s_setprio(0);
  trace_mark(pl, a.ws, 34);
  wait_vmem();  // the h stores (device-coherent) have completed
}

// ---------------------------------------------------- down, expert-major --
// For many active experts: a wave streams a contiguous run of (expert, 16-row
// tile) items; the B operand (the expert's h rows, KSD = I / 128 k-steps) is
// loaded once per expert and token chunk; bf16 y goes to the pair buffer and
// a combine phase sums it. Tiles come in batches of dn_tiles(KSD), two in flight.
__host__ __device__ constexpr int dn_tiles(int ksd) { return ksd == 2 ? 4 : ksd == 3 ? 3 : 2; }

template <int KSD>
struct DnTileBatch {
  u32x4 a[dn_tiles(KSD)][KSD];
  uint32_t s[dn_tiles(KSD)][KSD];
};

// wrow/srow: this lane's row (tile rt0) + 16 KSD q / + KSD q bytes: lane
// group q owns blocks KSD q .. KSD q + KSD - 1 of the row (k-step ks takes
// block KSD q + ks), so a row's 4 lane groups read it whole and contiguous.
// Rows of later tiles are 16 rows further each; tiles at or past rt1 read the
// zero area.
template <int KSD>
__device__ __forceinline__ void dnc_issue(DnTileBatch<KSD> &bt, const Plan &pl, const uint8_t *wrow,
                                          const uint8_t *srow, const uint8_t *zero, int rt0, int rt1) {
  constexpr int T = dn_tiles(KSD), KB = 4 * KSD;
  constexpr size_t tstride = (size_t)16 * KB * 16, sstride = (size_t)16 * KB;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const bool ok = rt0 + t < rt1;  // wave-uniform
    // unconditional loads (a tile past the last reads the zero area): a load
    // under a condition is joined by a copy that waits for it at once
    const uint8_t *sp = ok ? srow + t * sstride : zero;
    uint32_t sc;
    if constexpr (KSD == 2) sc = *reinterpret_cast<const uint16_t *>(sp);
    else if constexpr (KSD == 4) sc = *reinterpret_cast<const uint32_t *>(sp);
    else sc = (uint32_t)sp[0] | ((uint32_t)sp[1] << 8) | ((uint32_t)sp[2] << 16);
#pragma unroll
    for (int ks = 0; ks < KSD; ++ks) {
      bt.a[t][ks] = load16(ok ? wrow + t * tstride + ks * 16 : zero);
      bt.s[t][ks] = (sc >> (8 * ks)) & 0xFFu;
    }
  }
}

// y of a pair's 16-row tile goes to a per-wave LDS buffer of kDnStage
// entries (bf16 rows + a (pair, row tile) tag) instead of memory: stores in the
// weight stream would queue behind (and hold up) its loads. The buffer is
// written out with 16-byte stores when full and at the end of the wave's range.
struct DnStage {
  uint16_t *rows;  // [cap][16] bf16
  int *tag;        // [cap] pair << 16 | row tile
  int fill;
  int cap;         // rows the stage holds (kDnStage, or what the pinned rows leave)
};

__device__ __forceinline__ void dn_flush(DnStage &st, const Plan &pl, uint16_t *ybuf) {
  const int l = threadIdx.x & 63;
  wave_lds_order();
  for (int c = l; c < 2 * st.fill; c += 64) {
    const int ent = c >> 1, half = c & 1, tag = st.tag[ent];
    const u32x4 v = *reinterpret_cast<const u32x4 *>(st.rows + ent * 16 + half * 8);
    st_dev128(make_rsrc(ybuf, (uint32_t)pl.P * pl.K * 2),
              (uint32_t)((size_t)(tag >> 16) * pl.K + (tag & 0xFFFF) * 16 + half * 8) * 2, v);
  }
  wave_lds_order();
  st.fill = 0;
}

// Tiles rt .. of a batch for token chunk columns [0, ncol) (pairs p0c + column):
// MFMA over the KSD k-steps, bf16 y rows into the stage.
template <int KSD>
__device__ __forceinline__ void dnc_compute(const DnTileBatch<KSD> &bt, const Plan &pl, const u32x4 (&hb)[KSD][4],
                                            DnStage &st, uint16_t *ybuf, int rt0, int rt1, int p0c, int ncol) {
  const int l = threadIdx.x & 63, i = l & 15, q = l >> 4;
#pragma unroll
  for (int t = 0; t < dn_tiles(KSD); ++t) {
    if (rt0 + t >= rt1) break;  // wave-uniform
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KSD; ++ks) {
      bf16x8 av[4];
      uint32_t sc = bt.s[t][ks];
      asm volatile("" : "+v"(sc));  // no conversion hoisted next to the (early) load
      convert_block_fast(bt.a[t][ks], sc, av);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) acc = mfma16(av[kk], as_bf16x8(hb[ks][kk]), acc);
    }
    if (st.fill + ncol > st.cap) dn_flush(st, pl, ybuf);
    if (i < ncol) {
      const u32x2 packed = {(uint32_t)f32_to_bf16_bits(acc[0]) | ((uint32_t)f32_to_bf16_bits(acc[1]) << 16),
                            (uint32_t)f32_to_bf16_bits(acc[2]) | ((uint32_t)f32_to_bf16_bits(acc[3]) << 16)};
      *reinterpret_cast<u32x2 *>(st.rows + (st.fill + i) * 16 + 4 * q) = packed;
      if (q == 0) st.tag[st.fill + i] = ((p0c + i) << 16) | (rt0 + t);
    }
    st.fill += ncol;
  }
}

// One wave's expert-major down range: items t in [ta, tb) of (active expert,
// 16-row tile), expert-major; for each expert and 16-token chunk the h rows
// (B operand) are loaded once, and the weight tiles stream in batches. The
// waves balance their progress in prog[8] (balance_waves; a wave with no items
// counts as done, one not yet here as not started, so a wave still in gate/up
// never loses its priority to the down waves).
template <int KSD, class WaitExpert>
__device__ __forceinline__ void dn_expert_major(const Plan &pl, const DecodeArgs &a, const int *g_act,
                                                const int *g_aoff, const int *g_acnt, const uint8_t *zero,
                                                __amdgpu_buffer_rsrc_t hrs, DnStage &st, uint16_t *ybuf, int ta,
                                                int tb, const WaitExpert &wait_expert, int *prog) {
  constexpr int T = dn_tiles(KSD), KB = 4 * KSD;
  const int l = threadIdx.x & 63, i = l & 15, q = l >> 4;
  if (ta >= tb && l == 0) __hip_atomic_store(prog + wave_id(), 4096, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  for (int t = ta; t < tb;) {
    const int d = t / pl.RTd;
    const int rt0 = t % pl.RTd, rt1 = min(pl.RTd, rt0 + (tb - t));
    const int e = g_act[d], p0 = g_aoff[d], n = g_acnt[d];
    const size_t row0 = (size_t)e * pl.K + rt0 * 16 + i;
    const uint8_t *wrow = a.dblk + row0 * KB * 16 + q * 16 * KSD, *srow = a.dscl + row0 * KB + q * KSD;
    const size_t tstride = (size_t)16 * KB * 16, sstride = (size_t)16 * KB;
    for (int c = 0; c * 16 < n; ++c) {
      const int pj = c * 16 + i;
      const bool tok_ok = pj < n;
      const int ncol = min(16, n - c * 16);
      // lane group q feeds blocks KSD q + ks (k-step ks) of the h row (64 bytes each)
      const uint32_t hoff = tok_ok ? (uint32_t)(p0 + pj) * pl.I * 2 + q * 64 * KSD : kOffNone;
      DnTileBatch<KSD> b0, b1;
      dnc_issue<KSD>(b0, pl, wrow, srow, zero, rt0, rt1);  // weights do not depend on h
      if (c == 0) wait_expert(d);  // the expert's gate/up units are all done
      u32x4 hb[KSD][4];
#pragma unroll
      for (int ks = 0; ks < KSD; ++ks) {
        const uint32_t ho = hoff + ks * 64;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) hb[ks][kk] = bload16_dev(hrs, ho + kk * 16);  // device-coherent
      }
      // the next batch is always issued (tiles at or past rt1 read the zero
      // area): an issue under a condition would make the wait for the current
      // batch cover it (vmcnt(0) at the join)
      for (int rt = rt0; rt < rt1; rt += 2 * T) {
        const int o1 = rt + T - rt0, o2 = rt + 2 * T - rt0;
        balance_waves(prog, t - ta + (rt - rt0), tb - ta);
        dnc_issue<KSD>(b1, pl, wrow + o1 * tstride, srow + o1 * sstride, zero, rt + T, rt1);
        dnc_compute<KSD>(b0, pl, hb, st, ybuf, rt, rt1, p0 + c * 16, ncol);
        dnc_issue<KSD>(b0, pl, wrow + o2 * tstride, srow + o2 * sstride, zero, rt + 2 * T, rt1);
        if (rt + T < rt1) dnc_compute<KSD>(b1, pl, hb, st, ybuf, rt + T, rt1, p0 + c * 16, ncol);
      }
    }
    t += rt1 - rt0;
  }
  __builtin_amdgcn_s_setprio(0);
}

// Loads of one down-projection item: up to kDnDepth k-steps of A (weights and
// scales) and B (the activated h of the item's 16-token chunk).
struct DnLoad {
  u32x4 w[kDnDepth];
  uint32_t s[kDnDepth];   // the aligned dword holding the scale byte
  uint32_t sh[kDnDepth];  // the byte's bit offset in it
  u32x4 b[kDnDepth][4];
};

// Scale byte j of a down item. The byte is loaded as its aligned dword (a
// dword never crosses a page, so the load stays in mapped memory) and taken
// apart here, at its use: a byte load's value is zero-extended where the
// compiler places it, which can be a loop latch ahead of the next issue, and
// that wait would then hold up the next item's loads.
__device__ __forceinline__ uint32_t dn_scale(const DnLoad &L, int j) {
  uint32_t v = L.s[j];
  asm volatile("" : "+v"(v));
  return (v >> L.sh[j]) & 0xffu;
}

// Weights and scales of a down item (they do not depend on h): exactly
// 2 kDnDepth loads per lane, k-steps past I and row tiles past the last read
// from the zero area.
__device__ __forceinline__ void dn_issue_w(const Plan &pl, const DecodeArgs &a, const uint8_t *zero,
                                           const int *g_act, int rt, int d, int kc, int KB, DnLoad &L) {
  const int l = threadIdx.x & 63, i = l & 15, q = l >> 4;
  const bool rt_ok = rt < pl.RTd;
  const size_t row = (size_t)g_act[d] * pl.K + (rt_ok ? rt : 0) * 16 + i;
#pragma unroll
  for (int j = 0; j < kDnDepth; ++j) {
    const int kb = (kc + j) * 4 + q;
    const bool ok = rt_ok && kc + j < pl.KSd && kb < KB;
    L.w[j] = load16(ok ? a.dblk + (row * KB + kb) * 16 : zero);
    const uint8_t *sp = ok ? a.dscl + row * KB + kb : zero;
    const uint32_t mis = (uint32_t)reinterpret_cast<uintptr_t>(sp) & 3u;
    L.s[j] = *reinterpret_cast<const uint32_t *>(sp - mis);  // (pointer arithmetic keeps it a global load)
    L.sh[j] = mis * 8u;
  }
}

// The row-tile down reads h with device-coherent loads, and leaves its grid
// barrier without an L2 invalidate, when all of h is at most this many bytes;
// a larger h is read through the L2 (every workgroup reads all of it).
constexpr long kHDevBytes = 131072;
__device__ __forceinline__ bool dn_h_dev(const Plan &pl) { return (long)pl.P * pl.I * 2 <= kHDevBytes; }

// The activated h rows (B operand) of a down item: token chunk c of active expert d.
__device__ __forceinline__ void dn_issue_h(const Plan &pl, const uint16_t *hbuf, const uint8_t *zero,
                                           const int *g_aoff, const int *g_acnt, int d, int c, int kc, int KB,
                                           DnLoad &L) {
  const int l = threadIdx.x & 63, i = l & 15, q = l >> 4;
  const int p0 = g_aoff[d], n = g_acnt[d];
  const int pj = c * 16 + i;
  const bool tok_ok = pj < n;
  if (dn_h_dev(pl)) {
    const __amdgpu_buffer_rsrc_t hrs = make_rsrc(hbuf, (uint32_t)pl.P * pl.I * 2);
#pragma unroll
    for (int j = 0; j < kDnDepth; ++j) {
      const int kb = (kc + j) * 4 + q;
      const bool ok = tok_ok && kc + j < pl.KSd && kb < KB;
      const uint32_t off = ok ? (uint32_t)(((p0 + pj) * pl.I + kb * kBlockK) * 2) : kOffNone;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) L.b[j][kk] = bload16_dev(hrs, off + kk * 16);
    }
    return;
  }
  const uint16_t *hr = hbuf + (size_t)(p0 + (tok_ok ? pj : 0)) * pl.I;
#pragma unroll
  for (int j = 0; j < kDnDepth; ++j) {
    const int kb = (kc + j) * 4 + q;
    const bool ok = kc + j < pl.KSd && kb < KB;
    // out-of-range lanes read the zero area rather than skip the load: a
    // skipped load is joined by a copy that waits for it at once
    const uint8_t *src = (ok && tok_ok) ? reinterpret_cast<const uint8_t *>(hr + kb * kBlockK) : zero;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) L.b[j][kk] = load16(src + kk * 16);
  }
}

// The same h rows (k-steps 0 .. kDnDepth - 1) with device-coherent loads, for
// a wave that waited on the expert's count instead of a grid barrier.
__device__ __forceinline__ void dn_issue_h_dev(const Plan &pl, const uint16_t *hbuf, const int *g_aoff,
                                               const int *g_acnt, int d, DnLoad &L) {
  const int l = threadIdx.x & 63, i = l & 15, q = l >> 4;
  const __amdgpu_buffer_rsrc_t hrs = make_rsrc(hbuf, (uint32_t)pl.P * pl.I * 2);
  const int KB = pl.I / kBlockK;
  const bool tok_ok = i < g_acnt[d];
#pragma unroll
  for (int j = 0; j < kDnDepth; ++j) {
    const int kb = j * 4 + q;
    const bool ok = tok_ok && j < pl.KSd && kb < KB;
    const uint32_t off = ok ? (uint32_t)(((g_aoff[d] + i) * pl.I + kb * kBlockK) * 2) : kOffNone;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) L.b[j][kk] = bload16_dev(hrs, off + kk * 16);
  }
}

__device__ __forceinline__ void dn_issue(const Plan &pl, const DecodeArgs &a, const uint16_t *hbuf,
                                         const uint8_t *zero, const int *g_act, const int *g_aoff,
                                         const int *g_acnt, int rt, int d, int c, int kc, int KB, DnLoad &L) {
  dn_issue_w(pl, a, zero, g_act, rt, d, kc, KB, L);
  dn_issue_h(pl, hbuf, zero, g_aoff, g_acnt, d, c, kc, KB, L);
}

// The latent block's input projections (kimi.py:317, 326) in the decode
// kernel (Plan::lat_in, at most 8 tokens): latent = bf16(x @ latent_down.T)
// into xin and shared_h = bf16(act(bf16(x @ shared_gate.T), bf16(x @ shared_up.T))).
// The rows are latent_down's lh rows, then the shared pairs (gate s, up s) as
// rows lh + 2 s, lh + 2 s + 1; the workgroups that route no token share them
// out in whole pairs, workgroup j of the NW taking rows [2 U j / NW, 2 U (j + 1)
// / NW) (U = (lh + 2 S) / 2; at most 32 rows, two 16-row MFMA tiles, rows past
// the range reading the zero area). The tokens' rows of x go to LDS first
// (after kLatRedBytes, clear of the reduction area; row pitch h + 8;
// direct-to-LDS loads: the workgroup's LDS holds nothing else yet); the 8
// waves split h in 128-column steps (MFMA 16x16x32 bf16: the weights as the A
// operand from global memory, four steps in flight, the tokens as the B
// operand from LDS); the waves' tiles meet in LDS in wave order. The latent
// goes out with device-coherent stores (read by every workgroup after the
// latent barrier), shared_h with plain ones (read by the next kernel).
__device__ __forceinline__ void dec_latent_rows(const Plan &pl, const DecodeArgs &a, char *lds, const uint8_t *zero,
                                                int j, int NW) {
  const int w = wave_id(), l = threadIdx.x & 63, i = l & 15, q = l >> 4, tid = threadIdx.x;
  const int h = pl.h, lh = pl.K, B = pl.B, S = pl.lat_S, hp = h + 8;
  float *red = reinterpret_cast<float *>(lds);                    // [2 tiles][8 waves][256]
  uint16_t *xs = reinterpret_cast<uint16_t *>(lds + kLatRedBytes);  // [B][h + 8], clear of the reduction area
  const int U = (lh + 2 * S) / 2;
  const int r0 = 2 * (int)((long)U * j / NW), n = 2 * (int)((long)U * (j + 1) / NW) - r0;
  auto row_ptr = [&](int r) -> const uint16_t * {  // row r of the projections (r < lh + 2 S)
    if (r < lh) return a.lat_ld + (size_t)r * h;
    const int s = (r - lh) >> 1;
    return (((r - lh) & 1) ? a.lat_su : a.lat_sg) + (size_t)s * h;
  };
  const uint16_t *rowa = i < n ? row_ptr(r0 + i) : nullptr, *rowb = 16 + i < n ? row_ptr(r0 + 16 + i) : nullptr;
  const int KS = h / 128, ka = KS * w / kDecWaves, kb = KS * (w + 1) / kDecWaves;
  struct Step {
    u32x4 wa[4], wb[4];
  };
  // step ks, MFMA kk: lane (i, q) holds columns 128 ks + 32 kk + 8 q .. + 7 of
  // row i (weights) and of token i (x), so that one load instruction reads 64
  // contiguous bytes of each of the 16 rows
  auto issue = [&](int ks, Step &st) {  // steps past the wave's range read the zero area
    const bool in = ks < kb;
    const int off = ks * 128 + q * 8;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      st.wa[kk] = load16((in && rowa) ? reinterpret_cast<const uint8_t *>(rowa + off + kk * 32) : zero);
      st.wb[kk] = load16((in && rowb) ? reinterpret_cast<const uint8_t *>(rowb + off + kk * 32) : zero);
    }
  };
  Step s0, s1, s2, s3;
  issue(ka, s0);
  issue(ka + 1, s1);
  issue(ka + 2, s2);
  issue(ka + 3, s3);
  // the tokens' rows of x into LDS (1 KiB of a row per instruction), after the first weight loads
  const int per_row = h / 512;
  for (int c = w; c < B * per_row; c += kDecWaves) {
    const int t = c / per_row, jj = c - t * per_row;
    load_lds<16>(a.x + (size_t)t * h + jj * 512 + l * 8, reinterpret_cast<char *>(xs + (size_t)t * hp + jj * 512));
  }
  wait_vm<0>();
  __syncthreads();
  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  auto compute = [&](int ks, const Step &st) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const u32x4 xv = i < B ? *reinterpret_cast<const u32x4 *>(xs + (size_t)i * hp + ks * 128 + kk * 32 + q * 8)
                             : u32x4{0u, 0u, 0u, 0u};
      acc[0] = mfma16(as_bf16x8(st.wa[kk]), as_bf16x8(xv), acc[0]);
      acc[1] = mfma16(as_bf16x8(st.wb[kk]), as_bf16x8(xv), acc[1]);
    }
  };
  for (int ks = ka; ks < kb; ks += 4) {  // (the first four steps have landed with the rows of x)
    wait_vm<24>();
    compute(ks, s0);
    issue(ks + 4, s0);
    wait_vm<24>();
    if (ks + 1 < kb) compute(ks + 1, s1);  // wave-uniform
    issue(ks + 5, s1);
    wait_vm<24>();
    if (ks + 2 < kb) compute(ks + 2, s2);
    issue(ks + 6, s2);
    wait_vm<24>();
    if (ks + 3 < kb) compute(ks + 3, s3);
    issue(ks + 7, s3);
  }
  wait_vm<0>();
#pragma unroll
  for (int t = 0; t < 2; ++t) *reinterpret_cast<f32x4 *>(red + (t * kDecWaves + w) * 256 + l * 4) = acc[t];
  __syncthreads();
  if (tid < 256) {
    // thread tid: tile tid >> 7, elements 2 p and 2 p + 1 of its 16x16 tile
    // (p = tid & 127): rows 2 v, 2 v + 1 (a latent pair or a shared gate/up
    // pair, the range being pair-aligned) of token column c
    const int t = tid >> 7, idx = 2 * (tid & 127), ln = idx >> 2, v = idx & 3;
    const int rr = t * 16 + 4 * (ln >> 4) + v, c = ln & 15;
    if (rr < n && c < B) {
      const float v0 = red_sum(red + t * kDecWaves * 256, idx), v1 = red_sum(red + t * kDecWaves * 256, idx + 1);
      const int row = r0 + rr;
      if (row < lh) {
        const uint32_t pair = (uint32_t)f32_to_bf16_bits(v0) | ((uint32_t)f32_to_bf16_bits(v1) << 16);
        st_dev32(make_rsrc(a.xin, (uint32_t)B * lh * 2), (uint32_t)((c * lh + row) * 2), pair);
      } else {
        const uint16_t hv = f32_to_bf16_bits(apply_act(pl.act, round_bf16(v0), round_bf16(v1)));
        const size_t at = (size_t)c * S + ((row - lh) >> 1);
        if (pl.lat_out) {  // (read in this launch by dec_latent_out: device-coherent, a 16-bit store)
          __builtin_amdgcn_raw_buffer_store_b16(hv, make_rsrc(a.lat_sh, (uint32_t)B * S * 2), (uint32_t)(at * 2), 0,
                                                kCpolDevice);
        } else {
          a.lat_sh[at] = hv;
        }
      }
    }
  }
  wait_vmem();  // the latent's stores have completed (the latent barrier publishes them)
  __syncthreads();
}

// The latent block's output (kimi.py:325-328) in the decode kernel
// (Plan::lat_out, at most 8 tokens, after the step's expert sum): out =
// bf16(bf16(en @ latent_up.T) + bf16(shared_h @ shared_down.T)), en =
// bf16(bf16(e r) w) with e = bf16(expert_sum), r = 1 / sqrt(mean(e^2) + 1e-5),
// w = latent_norm. Workgroup b takes a contiguous share of the h output rows
// (at most 32: two 16-row MFMA tiles), the 8 waves split the K + S columns of
// [latent_up | shared_down] in 128-column steps (K and S multiples of 128, so a
// step lies in one part; one accumulator per part and tile; workgroups below
// wg0, which write the expert sum after a grid barrier, take no rows); the
// workgroup publishes its expert-sum stores (`arrive`), issues the first four
// steps' weights and then waits until every workgroup has published (`wait`),
// latent_norm and shared_h (published at the latent barrier) going straight to
// LDS before the weights; then the expert-sum loads go out; wave t < B
// normalises token t (the bf16 copy of its expert
// sum, written by the combine at o_ebf, read with device-coherent loads; the
// sum of squares in k_latent<1>'s order) and writes en beside shared_h in LDS
// after kLatRedBytes (the step is over: nothing else lives in LDS any more);
// the waves' tiles meet in LDS in wave order and the two parts are rounded
// apart. Returns false when the wait gave up.
template <class Arrive, class Wait>
__device__ __forceinline__ bool dec_latent_out(const Plan &pl, const DecodeArgs &a, char *lds, const uint8_t *zero,
                                               int wg0, Arrive &&arrive, Wait &&wait) {
  const int w = wave_id(), l = threadIdx.x & 63, i = l & 15, q = l >> 4, tid = threadIdx.x;
  const int h = pl.h, K = pl.K, B = pl.B, S = pl.lat_S, KT = K + S, xp = KT + 8;
  float *red = reinterpret_cast<float *>(lds);                    // [2 parts][2 tiles][8 waves][256]
  uint16_t *xs = reinterpret_cast<uint16_t *>(lds + kLatRedBytes);  // [B][K + S + 8]: en, then shared_h
  char *nw = lds + kLatRedBytes + align16((size_t)B * (K + S + 8) * 2);  // latent_norm, kLatOutMaxK bf16
  const int G = (int)gridDim.x - wg0, rpw = (h + G - 1) / G, row0 = ((int)blockIdx.x - wg0) * rpw;
  const int n = h > row0 ? min(rpw, h - row0) : 0;
  const int KS = KT / 128, KS0 = K / 128, ka = KS * w / kDecWaves, kb = KS * (w + 1) / kDecWaves;
  const bool ra = i < n, rb = 16 + i < n;
  struct Step {
    u32x4 wa[4], wb[4];
  };
  // step ks, MFMA kk: lane (i, q) holds columns 128 ks + 32 kk + 8 q .. + 7 of
  // output row row0 + i (tile a) / row0 + 16 + i (tile b) and of token i
  auto issue = [&](int ks, Step &st) {  // steps past the wave's range read the zero area
    const bool in = ks < kb;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int c = ks * 128 + kk * 32 + q * 8;
      const uint16_t *pa = c < K ? a.lat_up + (size_t)(row0 + i) * K + c : a.lat_sd + (size_t)(row0 + i) * S + (c - K);
      const uint16_t *pb = c < K ? a.lat_up + (size_t)(row0 + 16 + i) * K + c
                                 : a.lat_sd + (size_t)(row0 + 16 + i) * S + (c - K);
      st.wa[kk] = load16((in && ra) ? reinterpret_cast<const uint8_t *>(pa) : zero);
      st.wb[kk] = load16((in && rb) ? reinterpret_cast<const uint8_t *>(pb) : zero);
    }
  };
  // publish first (the expert-sum stores have completed); before waiting,
  // stage what does not depend on the other workgroups' expert sums
  // (latent_norm; shared_h, published at the latent barrier, read
  // device-coherent) straight into LDS and issue the first four steps' weights
  arrive();
  if (w < B)
    for (int c = 0; c < S; c += 128)  // 64 lanes x 2 values
      load_lds<4, kCpolDevice>(a.lat_sh + (size_t)w * S + c + 2 * l, reinterpret_cast<char *>(xs + (size_t)w * xp + K + c));
  {
    const int o = w * 1024 + l * 16;  // 8 waves x 64 lanes x 16 bytes = kLatOutMaxK bf16
    load_lds<16>(o < 2 * K ? reinterpret_cast<const uint8_t *>(a.lat_norm) + o : zero, nw + w * 1024);
  }
  Step s0, s1, s2, s3;
  issue(ka, s0);
  issue(ka + 1, s1);
  issue(ka + 2, s2);
  issue(ka + 3, s3);
  wait_vm<32>();  // the LDS loads, issued before the 32 weight loads, have landed (the wait's sync publishes them)
  if (!wait()) return false;
  // (trace slots 36-38 also hold the stream-K gate/up's per-wave ends: never in one launch with these)
  trace_mark(pl, a.ws, 36);  // every expert-sum share published
  const __amdgpu_buffer_rsrc_t er = make_rsrc(a.ws + pl.o_ebf, (uint32_t)((size_t)B * K * 2));
  u32x2 ec[kLatOutMaxK / 256];  // bf16 expert sum, 4 values a load
#pragma unroll
  for (int m = 0; m < kLatOutMaxK / 256; ++m)  // (no loads for waves w >= B: the offsets are past the end)
    ec[m] = bload8_dev(er, w < B && 4 * (l + 64 * m) < K ? (uint32_t)(((size_t)w * K + 4 * (l + 64 * m)) * 2) : kOffNone);
  if (w < B) {  // token w: en into LDS
    float ss = 0.f;
#pragma unroll
    for (int m = 0; m < kLatOutMaxK / 256; ++m) {
      if (4 * (l + 64 * m) < K) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float e = bf16_bits_to_f32(v & 1 ? ec[m][v >> 1] >> 16 : ec[m][v >> 1] & 0xFFFFu);
          ss += e * e;
        }
      }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss += shfl_xor(ss, m);
    const float r = 1.0f / __fsqrt_rn(ss / (float)K + kLatOutRmsEps);
#pragma unroll
    for (int m = 0; m < kLatOutMaxK / 256; ++m) {
      const int k = 4 * (l + 64 * m);
      if (k < K) {
        const u32x2 wp = *reinterpret_cast<const u32x2 *>(nw + 2 * k);
        uint32_t o[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const uint32_t wb = v & 1 ? wp[v >> 1] >> 16 : wp[v >> 1] & 0xFFFFu;
          const uint32_t eb = v & 1 ? ec[m][v >> 1] >> 16 : ec[m][v >> 1] & 0xFFFFu;
          o[v] = f32_to_bf16_bits(round_bf16(bf16_bits_to_f32(eb) * r) * bf16_bits_to_f32(wb));
        }
        *reinterpret_cast<u32x2 *>(xs + (size_t)w * xp + k) = u32x2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
      }
    }
  }
  __syncthreads();
  trace_mark(pl, a.ws, 37);  // en in LDS
  f32x4 acc[2][2] = {{f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}},
                     {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}}};
  auto compute = [&](int ks, const Step &st) {
    const int part = ks < KS0 ? 0 : 1;  // wave-uniform
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const u32x4 xv = i < B ? *reinterpret_cast<const u32x4 *>(xs + (size_t)i * xp + ks * 128 + kk * 32 + q * 8)
                             : u32x4{0u, 0u, 0u, 0u};
      if (part == 0) {
        acc[0][0] = mfma16(as_bf16x8(st.wa[kk]), as_bf16x8(xv), acc[0][0]);
        acc[0][1] = mfma16(as_bf16x8(st.wb[kk]), as_bf16x8(xv), acc[0][1]);
      } else {
        acc[1][0] = mfma16(as_bf16x8(st.wa[kk]), as_bf16x8(xv), acc[1][0]);
        acc[1][1] = mfma16(as_bf16x8(st.wb[kk]), as_bf16x8(xv), acc[1][1]);
      }
    }
  };
  // Steps past the wave's last one are not issued in the loop (their zero-area
  // loads would only add latency at the end); before computing step ks, the
  // wave's real steps after it, up to three, are the loads allowed in flight
  // (any other load issued after them only makes the wait stricter).
  auto wait_after = [](int later) {
    if (later >= 3) wait_vm<24>();
    else if (later == 2) wait_vm<16>();
    else if (later == 1) wait_vm<8>();
    else wait_vm<0>();
  };
  for (int ks = ka; ks < kb; ks += 4) {  // (wave-uniform conditions)
    wait_after(kb - 1 - ks);
    compute(ks, s0);
    if (ks + 4 < kb) issue(ks + 4, s0);
    if (ks + 1 >= kb) break;
    wait_after(kb - 2 - ks);
    compute(ks + 1, s1);
    if (ks + 5 < kb) issue(ks + 5, s1);
    if (ks + 2 >= kb) break;
    wait_after(kb - 3 - ks);
    compute(ks + 2, s2);
    if (ks + 6 < kb) issue(ks + 6, s2);
    if (ks + 3 >= kb) break;
    wait_after(kb - 4 - ks);
    compute(ks + 3, s3);
    if (ks + 7 < kb) issue(ks + 7, s3);
  }
  if (kb - ka < 4) wait_vm<0>();  // the first four's zero-area loads past kb
  trace_mark(pl, a.ws, 38);  // this wave-0 k-range done
  __syncthreads();  // (the reduction area held nothing of this phase before: its LDS was only read)
#pragma unroll
  for (int pt = 0; pt < 2; ++pt)
#pragma unroll
    for (int t = 0; t < 2; ++t)
      *reinterpret_cast<f32x4 *>(red + ((pt * 2 + t) * kDecWaves + w) * 256 + l * 4) = acc[pt][t];
  __syncthreads();
  {
    const int t = tid >> 8, idx = tid & 255, ln = idx >> 2, v = idx & 3;
    const int rr = t * 16 + 4 * (ln >> 4) + v, c = ln & 15;
    if (rr < n && c < B) {
      const float s0 = red_sum(red + (0 * 2 + t) * kDecWaves * 256, idx);
      const float s1 = red_sum(red + (1 * 2 + t) * kDecWaves * 256, idx);
      a.lat_y[(size_t)c * h + row0 + rr] = f32_to_bf16_bits(round_bf16(s0) + round_bf16(s1));
    }
  }
  return true;
}

static_assert(sizeof(Plan) % alignof(DecodeArgs) == 0, "DecodeArgs follows Plan in the argument segment");

// The DecodeArgs at constant address `at`; every pointer is device (global) memory.
__device__ __forceinline__ DecodeArgs load_args(uint64_t at) {
  DecodeArgs a;
#define K3_FIELD(f) a.f = global_field<std::remove_pointer_t<decltype(a.f)>>(at + offsetof(DecodeArgs, f))
  K3_FIELD(x);
  K3_FIELD(xin);
  K3_FIELD(router);
  K3_FIELD(bias);
  K3_FIELD(gblk);
  K3_FIELD(gscl);
  K3_FIELD(ublk);
  K3_FIELD(uscl);
  K3_FIELD(dblk);
  K3_FIELD(dscl);
  K3_FIELD(routes);
  K3_FIELD(out);
  K3_FIELD(out_ids);
  K3_FIELD(out_w);
  K3_FIELD(out_short);
  K3_FIELD(ws);
  K3_FIELD(lat_ld);
  K3_FIELD(lat_sg);
  K3_FIELD(lat_su);
  K3_FIELD(lat_sh);
  K3_FIELD(lat_norm);
  K3_FIELD(lat_up);
  K3_FIELD(lat_sd);
  K3_FIELD(lat_y);
#undef K3_FIELD
  static_assert(sizeof(DecodeArgs) == 24 * sizeof(void *), "every field read");
  return a;
}

// AL: K is a multiple of 512 (whole 16-block super-steps in gate/up); KSD: the
// expert-major down path's k-steps per row (I / 128 for I = 256, 384, 512; 0:
// that path is not used). Each instantiation holds one variant of each, which
// keeps the kernel's code (and its instruction-cache footprint) small.
template <bool AL, int KSD, bool LAT>
__global__ __launch_bounds__(kDecThreads, 1) void k_moe_decode(Plan pl_arg, DecodeArgs a_arg) {
  const uint64_t t_entry = __builtin_amdgcn_s_memrealtime();  // (stored when tracing)
  // The arguments, read through the touched segment (pl_arg at offset 0, a_arg after it).
  const uint64_t kargs = touch_kernargs<sizeof(Plan) + sizeof(DecodeArgs)>();
  const Plan pl = load_const<Plan>(kargs);
  const DecodeArgs a = load_args(kargs + sizeof(Plan));
  // the latent block's phases only in the LAT instantiations (the plain step's
  // code then carries none of them)
  const bool lat_in = LAT && pl.lat_in != 0, lat_out = LAT && pl.lat_out != 0;
  (void)pl_arg;
  (void)a_arg;
  extern __shared__ __attribute__((aligned(16))) char lds[];
  float *red = reinterpret_cast<float *>(lds);
  int *g_act = reinterpret_cast<int *>(lds + pl.lds_red);
  int *g_aoff = g_act + pl.Dmax;
  int *g_acnt = g_aoff + pl.Dmax;
  int *g_coff = g_acnt + pl.Dmax;  // [Dmax + 1] gate/up chunks (NX tokens) before each active expert
  int *g_ptok = g_coff + pl.Dmax + 1;
  float *g_pw = reinterpret_cast<float *>(g_ptok + pl.P);
  int *g_pof = reinterpret_cast<int *>(g_pw + pl.P);  // pair index of (token, slot)
  int *g_cexp = g_pof + pl.P;  // [P] active expert (index into g_act) of each gate/up chunk
  char *scr = lds + pl.lds_red + pl.lds_grp;
  uint16_t *xpin = reinterpret_cast<uint16_t *>(scr + pl.lds_scr);  // pinned: every token's expert-input row
  __shared__ int s_nact;
  __shared__ GuChunk s_tab[16];
  __shared__ int s_round[2], s_rowtok[16];
  __shared__ __attribute__((aligned(16))) int s_prog[kDecWaves];
  __shared__ __attribute__((aligned(16))) int s_dprog[kDecWaves];  // expert-major down progress
  __shared__ uint32_t s_tag;
  __shared__ int s_fail;

  const int tid = threadIdx.x, w = wave_id(), l = tid & 63;
  const int i = l & 15, q = l >> 4;
  unsigned *ctl = reinterpret_cast<unsigned *>(a.ws + pl.o_ctl);
  // Workgroups hand the router partials, the routed pairs and the gate/up
  // completions to each other through tagged 8-byte slots {payload, tag} in
  // the tag area; the tag numbers the launch (launches so far on this
  // workspace + 1, from the launch counters every workgroup of the decode and
  // single-token kernels adds to when it leaves), so a reader polls the data
  // itself until it carries this launch's tag, and no slot needs clearing.
  const __amdgpu_buffer_rsrc_t tagr = make_rsrc(a.ws + kOffTag, kTagBytes);
  uint32_t launches = 0u;  // wave 0, lane g < kEpochCounters: launch counter g
  if (w == 0 && l < kEpochCounters)
    launches = __hip_atomic_load(ctl + kCtlEpoch + l * kCtlEpochStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  bool tag_made = false;
  auto make_tag = [&]() {  // wave 0, once, after the router's loads are issued
    if (tag_made || w != 0) return;
    tag_made = true;
    uint32_t sum = 0u;
#pragma unroll
    for (int g = 0; g < kEpochCounters; ++g) sum += lane_u32(launches, g);
    if (l == 0) {
      s_tag = (sum >> __builtin_ctz(gridDim.x)) + 1u;
      s_fail = 0;
    }
  };
  // this workgroup's count on its launch counter: once, on every way out
  auto leave = [&]() {
    if (tid == 0)
      __hip_atomic_fetch_add(ctl + kCtlEpoch + (blockIdx.x % kEpochCounters) * kCtlEpochStride, 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  };
  uint16_t *hbuf = reinterpret_cast<uint16_t *>(a.ws + pl.o_h);
  const uint8_t *zero = reinterpret_cast<const uint8_t *>(a.ws + pl.o_zero);  // kZeroBytes of zeros
  const int B = pl.B, E = pl.E, k = pl.k;
  trace_mark(pl, a.ws, 0);
  if (pl.o_trace && tid == 0)
    reinterpret_cast<uint64_t *>(a.ws + pl.o_trace)[blockIdx.x * kTraceSlots + kTraceEntry] = t_entry;
  // The gating bias of experts tid and tid + 512: a token's one-logit-per-thread
  // gather uses exactly these, and loading them now keeps a cold HBM round trip
  // out of the top-k phase.
  float bias_pre[2] = {0.f, 0.f};
  if (a.bias) {
    if (tid < pl.E) bias_pre[0] = a.bias[tid];
    if (tid + kDecThreads < pl.E) bias_pre[1] = a.bias[tid + kDecThreads];
  }
  // this launch's barrier targets (thread 0 arrives for the workgroup)
  const BarrierBase bb = tid == 0 ? barrier_base(ctl) : BarrierBase{0u, 0u, 0u};
  __shared__ unsigned s_abort0;  // the abort counter at the start, for every thread's bounded waits
  if (tid == 0) s_abort0 = bb.abort;

  // Code warm-up: a step runs much of this kernel's code once, and after other
  // work has evicted it every new stretch stalls on instruction fetches from
  // HBM. The last workgroup to leave records the kernel's code range in the
  // control block; at the next launch with the same code the last wave of
  // each workgroup loads eight 1 KiB chunks of that range as data, so that it
  // sits in its XCD's L2 (the 32 workgroups b, b + 8, .. of an XCD cover up to
  // 256 KiB). The range is read only if its recorded start is this launch's
  // and never past its recorded end. That wave takes no router k-steps, so the
  // router's waits never include these loads (nor the range read they
  // depend on).
  uint64_t *crange = reinterpret_cast<uint64_t *>(ctl + kCtlCode);
  const uint64_t pc0 = program_counter();
  u32x4 code_probe = {0, 0, 0, 0};
  if (w == kDecWaves - 1) {
    const uint64_t c0 = crange[0], c1 = crange[1];
    if (c0 == pc0 && c1 > pc0 && c1 - pc0 < (1u << 20)) {
      const uint64_t lo = pc0 & ~(uint64_t)1023;
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const uint64_t addr = lo + (uint64_t)((blockIdx.x >> 3) * 8 + m) * 1024 + l * 16;
        // out of range: the kernel's own first bytes
        const uint64_t at = addr + 16 <= c1 ? addr : (pc0 & ~(uint64_t)15);
        code_probe ^= *reinterpret_cast<const __attribute__((address_space(1))) u32x4 *>(at);
      }
    }
  }

  if (l == 0) __hip_atomic_store(s_prog + w, 4096, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  if (l == 0) __hip_atomic_store(s_dprog + w, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);

  // ------------------------------------------------------------ R: router --
  // Workgroup unit = (16 router rows, k-split s) for every token tile: the
  // first 7 waves take consecutive k-steps of the split, load the row tile once and
  // every token tile with all loads in flight, and meet in LDS; the sum over
  // waves is written as partial s of each logit.
  {
    const int NU = pl.RTr * pl.Srw;
    const int KB = pl.h / kBlockK;
    for (int u = blockIdx.x; u < NU; u += gridDim.x) {
      const int s = u % pl.Srw, rt = u / pl.Srw;
      const int k0 = (int)((unsigned)(s * pl.KSr) / (unsigned)pl.Srw), k1 = (int)((unsigned)((s + 1) * pl.KSr) / (unsigned)pl.Srw);
      constexpr int RW = kDecWaves - 1;  // router waves (the last one warms the code)
      const int ka = w < RW ? k0 + (k1 - k0) * w / RW : k1, kb1 = w < RW ? k0 + (k1 - k0) * (w + 1) / RW : k1;
      const int row = rt * 16 + i;
      const bool row_ok = row < E;
      const uint16_t *arow = a.router + (size_t)(row_ok ? row : 0) * pl.h;
      f32x4 acc[kDecMaxTokens / 16];
#pragma unroll
      for (int tt = 0; tt < kDecMaxTokens / 16; ++tt) acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int ks = ka; ks < kb1; ++ks) {
        const int kb = ks * 4 + q;
        const bool ok = kb < KB;
        u32x4 va[4], vb[kDecMaxTokens / 16][4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) va[kk] = (ok && row_ok) ? load16(arow + kb * kBlockK + kk * 8) : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int tt = 0; tt < kDecMaxTokens / 16; ++tt) {
          const int tok = tt * 16 + i;
          const bool tok_ok = ok && tt < pl.TTr && tok < B;
          const uint16_t *brow = a.x + (size_t)(tok_ok ? tok : 0) * pl.h + kb * kBlockK;
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) vb[tt][kk] = tok_ok ? load16(brow + kk * 8) : u32x4{0, 0, 0, 0};
        }
        make_tag();
#pragma unroll
        for (int tt = 0; tt < kDecMaxTokens / 16; ++tt) {
          if (tt < pl.TTr) {
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) acc[tt] = mfma16(as_bf16x8(va[kk]), as_bf16x8(vb[tt][kk]), acc[tt]);
          }
        }
      }
      make_tag();
      if (u == (int)blockIdx.x) trace_mark(pl, a.ws, 31);
#pragma unroll
      for (int tt = 0; tt < kDecMaxTokens / 16; ++tt)
        if (tt < pl.TTr) *reinterpret_cast<f32x4 *>(red + (tt * kDecWaves + w) * 256 + l * 4) = acc[tt];
      __syncthreads();
      // partial s of logit (t, e): slot kTagDecPart + ((t Srw + s) Epad + e) 8
      for (int j = tid; j < pl.TTr * 256; j += kDecThreads) {
        const int tt = j >> 8, ln = (j >> 2) & 63, v = j & 3;
        const int r = 4 * (ln >> 4) + v, c = ln & 15;
        const int t = tt * 16 + c, e = rt * 16 + r;
        if (t < B)
          st_dev64(tagr, (uint32_t)(kTagDecPart + (((size_t)t * pl.Srw + s) * pl.Epad + e) * 8),
                   u32x2{__float_as_uint(red_sum(red + tt * kDecWaves * 256, j & 255)), s_tag});
      }
      __syncthreads();
    }
  }
  make_tag();
  trace_mark(pl, a.ws, 1);
  asm volatile("" ::"v"(code_probe));  // the warm-up loads complete here
  __syncthreads();  // s_tag, s_fail, s_abort0
  const uint32_t tag = s_tag;
  const unsigned abort0 = s_abort0;
  unsigned nbar = 0;  // grid barriers of this launch passed so far
  unsigned nb_late = 0;  // a barrier this workgroup arrived at without waiting (0: none)
  // a wait of this launch gave up: NaN in this workgroup's share of the output, and leave
  auto give_up = [&]() {
    poison_share<false>(a.out, (long)B * pl.K);
    if (lat_out) poison_share<true>(a.lat_y, (long)B * pl.h);
    leave();
  };
  trace_mark(pl, a.ws, 2);
  // A single token's expert-input row is known from the start: its loads are
  // issued here and arrive during the top-k and grouping phases; gate/up then
  // writes it to LDS instead of loading it (two 16-byte chunks per thread, the
  // chunk mapping of the gate/up staging).
  const bool xpre_ok = B == 1 && pl.K / 8 <= 2 * kDecThreads;
  u32x4 xpre[2] = {u32x4{0, 0, 0, 0}, u32x4{0, 0, 0, 0}};
  if (xpre_ok) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int c = hh * kDecThreads + tid;
      if (c < pl.K / 8) xpre[hh] = load16(a.xin + c * 8);
    }
  }

  // -------------------------------------------------------- T: top-k/gating --
  // One token: every workgroup routes it itself (the grouping reads its own
  // LDS). More tokens: token t is routed by workgroup t, which publishes its
  // (id, weight) pairs in tagged slots that every workgroup polls.
  const bool redundant = pl.redundant;
  int *rid = reinterpret_cast<int *>(scr);     // [P] expert ids, ascending per token
  float *rw = reinterpret_cast<float *>(rid + pl.P);  // [P] weights aligned with rid
  char *scr2 = scr + 8 * pl.P;
  {
    const int nt = redundant ? B : 1;  // tokens routed per pass of this workgroup
    uint32_t *kyl = reinterpret_cast<uint32_t *>(scr2);  // [nt][E] ordered keys
    float *kyf = reinterpret_cast<float *>(kyl + nt * E);  // [nt][E] keys as float
    float *scl = kyf + nt * E;                           // [nt][E] scores (sigmoid or logits)
    int *sel = reinterpret_cast<int *>(scl + nt * E);    // [8 waves][kMaxTopk]
    for (int t0 = redundant ? 0 : blockIdx.x; t0 < B; t0 += redundant ? B : gridDim.x) {
      auto gate = [&](int f, float logit, float bias) {
        float score, key;
        if (pl.gating == K3MOE_GATING_SIGMOID_BIAS) {
          score = 1.0f / (1.0f + expf(-logit));
          key = a.bias ? __fadd_rn(score, bias) : score;
        } else {
          score = logit;
          key = logit;
        }
        scl[f] = score;
        kyf[f] = key;
        const uint32_t o = ordered_key(key);
        kyl[f] = o;
        return o;
      };
      uint32_t key0 = 0u, key1 = 0u;  // this thread's ordered keys (experts tid, tid + 512)
      // logits of token t0: thread e polls the partial slots of experts e and
      // e + 512 (every split's 8-byte load per round) until each carries this
      // launch's tag, then sums them in split order
      {
        const int e0 = tid, e1 = tid + kDecThreads;
        const int n0 = e0 < E ? pl.Srw : 0, n1 = e1 < E ? pl.Srw : 0;
        const uint32_t pbase = (uint32_t)(kTagDecPart + (size_t)t0 * pl.Srw * pl.Epad * 8);
        const uint32_t sstride = (uint32_t)pl.Epad * 8;
        u32x2 v0[kDecMaxSplits], v1[kDecMaxSplits];
#pragma unroll
        for (int sp = 0; sp < kDecMaxSplits; ++sp) v0[sp] = v1[sp] = u32x2{0u, tag};
        bool ok = true;
        unsigned spins = 0;
        // a wave without experts to poll skips the loop (wave-uniform): its
        // waits would also cover loads it issued earlier (the pinned rows)
        for (; w * 64 < E;) {
#pragma unroll
          for (int sp = 0; sp < kDecMaxSplits; ++sp) {
            v0[sp] = sp < n0 ? bload8_dev(tagr, pbase + sp * sstride + e0 * 8) : u32x2{0u, tag};
            v1[sp] = sp < n1 ? bload8_dev(tagr, pbase + sp * sstride + e1 * 8) : u32x2{0u, tag};
          }
          bool ready = pl.stall == 0;  // (a test hook: the wait never ends and gives up)
#pragma unroll
          for (int sp = 0; sp < kDecMaxSplits; ++sp) ready = ready && v0[sp][1] == tag && v1[sp][1] == tag;
          if (spins == 0 && w == 0) trace_mark(pl, a.ws, 44);
          if (__ballot(!ready) == 0) break;
          ++spins;
          if ((spins & 63u) == 0u && aborted(ctl, abort0)) {
            ok = false;
            break;
          }
          if (spins > (pl.stall ? (unsigned)pl.stall : kSpinLimit)) {
            if (l == 0) raise_timeout(ctl);
            ok = false;
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
        if (!ok) s_fail = 1;
        float lg0 = __uint_as_float(v0[0][0]), lg1 = __uint_as_float(v1[0][0]);
#pragma unroll
        for (int sp = 1; sp < kDecMaxSplits; ++sp)
          if (sp < pl.Srw) {
            lg0 += __uint_as_float(v0[sp][0]);
            lg1 += __uint_as_float(v1[sp][0]);
          }
        if (n0) key0 = gate(e0, lg0, bias_pre[0]);
        if (n1) key1 = gate(e1, lg1, bias_pre[1]);
      }
      // One token per pass: the workgroup's threshold-and-rank selection
      // (block_topk, E <= 1024, k <= 32) on the keys in registers; its
      // barriers publish s_fail, the scores and keys. Several tokens per
      // pass: one wave per token runs wave_topk on the keys in LDS.
      const bool coop = nt == 1;
      if (!coop) {
        __syncthreads();
        if (s_fail) return give_up();
      }
      trace_mark(pl, a.ws, 10);
      for (int tg = 0; tg < nt; tg += kDecWaves) {
        if (coop) {
          block_topk(key0, key1, E, k, sel, *reinterpret_cast<BlockTopk *>(lds_align16(sel + kDecWaves * kMaxTopk)));
          if (s_fail) return give_up();
        }
        const int tl = tg + w;
        if (tl >= nt) continue;
        const int t = t0 + tl;
        int *mysel = sel + w * kMaxTopk;
        if (!coop) wave_topk(kyl + tl * E, E, k, mysel);
        wave_lds_order();
        trace_mark(pl, a.ws, 30);
        const bool writer = redundant ? blockIdx.x == 0 : true;
        // forced routes replace the selection when the row is valid; an invalid
        // row keeps its own top-k and sets the status word
        int fid = 0;
        const bool forced = a.routes && forced_route(a.routes, t, k, E, &fid);
        if (a.routes && !forced && l == 0 && writer)
          __hip_atomic_fetch_or(ctl + kCtlErr, (unsigned)kErrRoutes, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        int my_e = -1;
        float my_score = 0.f, my_key = 0.f;
        if (l < k) {
          my_e = forced ? fid : mysel[l];
          my_score = scl[tl * E + my_e];
          my_key = kyf[tl * E + my_e];
        }
        float wt = 0.f;
        if (pl.gating == K3MOE_GATING_SIGMOID_BIAS) {
          float sum = 0.f;
          for (int r = 0; r < k; ++r) sum = __fadd_rn(sum, lane_f32(my_score, r));
          wt = my_score / __fadd_rn(sum, 1e-20f);
        } else {
          float mx = -INFINITY;
          for (int r = 0; r < k; ++r) mx = fmaxf(mx, lane_f32(my_score, r));
          const float ex = (l < k) ? expf(my_score - mx) : 0.f;
          float sum = 0.f;
          for (int r = 0; r < k; ++r) sum = __fadd_rn(sum, lane_f32(ex, r));
          wt = ex / sum;
        }
        if (a.routes && a.out_short) {
          float mn = INFINITY;
          for (int r = 0; r < k; ++r) mn = fminf(mn, lane_f32(my_key, r));
          if (l == 0 && writer) a.out_short[t] = fmaxf(kyf[tl * E + mysel[k - 1]] - mn, 0.f);
        }
        int rank = 0;
        for (int r = 0; r < k; ++r) rank += ((int)lane_u32((uint32_t)my_e, r) < my_e) ? 1 : 0;
        if (l < k) {
          const size_t o = (size_t)t * k + rank;
          if (writer) {
            a.out_ids[o] = my_e;
            a.out_w[o] = wt;
          }
          if (redundant) {
            rid[o] = my_e;
            rw[o] = wt;
          } else {  // pair slot o: {id, tag, weight, tag}
            st_dev128(tagr, (uint32_t)(kTagDecPairs + o * 16), u32x4{(uint32_t)my_e, tag, __float_as_uint(wt), tag});
          }
        }
      }
      trace_mark(pl, a.ws, 11);
      __syncthreads();
    }
  }
  trace_mark(pl, a.ws, 3);
  // The latent block's input projections (Plan::lat_in): the workgroups that
  // routed no token compute them now (the routed pairs arrive meanwhile); every
  // workgroup arrives at the latent barrier here and waits at it before its
  // gate/up rows are loaded.
  unsigned lat_bar = 0;
  if (lat_in) {
    if ((int)blockIdx.x >= B) dec_latent_rows(pl, a, lds, zero, (int)blockIdx.x - B, (int)gridDim.x - B);
    trace_mark(pl, a.ws, 16);
    lat_bar = ++nbar;
    if (tid == 0) barrier_arrive(ctl, bb, lat_bar, nullptr);
  }
  // Pinned gate/up in a workgroup that routed no token: it would wait here
  // for the routed pairs with nothing to load, so it loads every token's row
  // into its pinned rows now (1 KiB of a row per instruction, spread over the
  // waves) and gate/up starts on its weights without a row wait. The pair
  // poll below waits for these loads too (vmcnt counts in order); they land
  // long before the pairs are published.
  bool rows_staged = false;
  if constexpr (AL) {
    if (pl.pinned && !redundant && !lat_in && (int)blockIdx.x >= B) {
      rows_staged = true;
      const int per_row = pl.K / 512;
      for (int c = w; c < B * per_row; c += kDecWaves) {
        const int r = c / per_row, j = c - r * per_row;
        load_lds<16>(a.xin + (size_t)r * pl.K + j * 512 + l * 8,
                     reinterpret_cast<char *>(xpin + (size_t)r * pl.xpitch + j * 512));
      }
      wait_vm<0>();  // before the barriers below publish them
    }
  }
  if (!redundant) {
    // every pair's slot (pairs tid and tid + 512), polled until both halves carry this launch's tag
    u32x4 pv[2] = {u32x4{0u, tag, 0u, tag}, u32x4{0u, tag, 0u, tag}};
    bool ok = true;
    unsigned spins = 0;
    for (; w * 64 < pl.P;) {  // waves without pairs to poll skip it (see the logit poll)
      bool ready = true;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int p = tid + j * kDecThreads;
        pv[j] = p < pl.P ? bload16_dev(tagr, (uint32_t)(kTagDecPairs + p * 16)) : u32x4{0u, tag, 0u, tag};
        ready = ready && pv[j][1] == tag && pv[j][3] == tag;
      }
      if (__ballot(!ready) == 0) break;
      ++spins;
      if ((spins & 63u) == 0u && aborted(ctl, abort0)) {
        ok = false;
        break;
      }
      if (spins > kSpinLimit) {
        if (l == 0) raise_timeout(ctl);
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (!ok) s_fail = 1;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int p = tid + j * kDecThreads;
      if (p < pl.P) {
        rid[p] = (int)pv[j][0];
        rw[p] = __uint_as_float(pv[j][2]);
      }
    }
    __syncthreads();
    if (s_fail) return give_up();
  }
  trace_mark(pl, a.ws, 4);

  // ------------------------------------------------- G: grouping (in LDS) --
  if (B == 1) {
    // one token: its k distinct experts, ascending, are the active list, with
    // one pair and one chunk each
    if (tid < k) {
      g_act[tid] = rid[tid];
      g_aoff[tid] = tid;
      g_acnt[tid] = 1;
      g_coff[tid] = tid;
      g_ptok[tid] = 0;
      g_pw[tid] = rw[tid];
      g_pof[tid] = tid;
      g_cexp[tid] = tid;
    }
    if (tid == 0) {
      s_nact = k;
      g_coff[k] = k;
    }
    __syncthreads();
  } else {
    int *cnt = reinterpret_cast<int *>(scr2);  // [E]
    int *off = cnt + E;                        // [E]
    uint32_t *bits = reinterpret_cast<uint32_t *>(off + E);  // [E][2] token bitmaps (B <= 64)
    for (int e = tid; e < E; e += kDecThreads) {
      cnt[e] = 0;
      bits[2 * e] = 0;
      bits[2 * e + 1] = 0;
    }
    __syncthreads();
    for (int p = tid; p < pl.P; p += kDecThreads) {
      const int e = rid[p];
      const int t = p / k;
      atomicAdd(&cnt[e], 1);
      atomicOr(&bits[2 * e + (t >> 5)], 1u << (t & 31));
    }
    __syncthreads();
    trace_mark(pl, a.ws, 28);
    {
      // exclusive prefix, in ascending expert order, of the pair counts, the
      // active flags and the gate/up chunk counts: thread tid owns experts
      // 2 tid and 2 tid + 1 (E <= 1024); wave scans, then the wave totals
      int *wsum = reinterpret_cast<int *>(bits + 2 * E);  // [8 waves][3]
      const int e0 = 2 * tid, e1 = e0 + 1;
      const int c0 = e0 < E ? cnt[e0] : 0, c1 = e1 < E ? cnt[e1] : 0;
      const int n0 = (c0 + pl.NX - 1) / pl.NX, n1 = (c1 + pl.NX - 1) / pl.NX;
      const int tp = c0 + c1, ta = (c0 > 0) + (c1 > 0), tc = n0 + n1;
      const int sp = wave_incl_scan(tp), sa = wave_incl_scan(ta), sc = wave_incl_scan(tc);
      if (l == 63) {
        wsum[3 * w] = sp;
        wsum[3 * w + 1] = sa;
        wsum[3 * w + 2] = sc;
      }
      __syncthreads();
      int bp = 0, ba = 0, bc = 0;
      for (int ww = 0; ww < w; ++ww) {
        bp += wsum[3 * ww];
        ba += wsum[3 * ww + 1];
        bc += wsum[3 * ww + 2];
      }
      int op = bp + sp - tp, oa = ba + sa - ta, oc = bc + sc - tc;
      if (e0 < E) {
        off[e0] = op;
        if (c0 > 0) {
          g_act[oa] = e0;
          g_aoff[oa] = op;
          g_acnt[oa] = c0;
          g_coff[oa] = oc;
          for (int c = 0; c < n0; ++c) g_cexp[oc + c] = oa;
          ++oa;
          oc += n0;
        }
      }
      op += c0;
      if (e1 < E) {
        off[e1] = op;
        if (c1 > 0) {
          g_act[oa] = e1;
          g_aoff[oa] = op;
          g_acnt[oa] = c1;
          g_coff[oa] = oc;
          for (int c = 0; c < n1; ++c) g_cexp[oc + c] = oa;
        }
      }
      if (tid == kDecThreads - 1) {  // totals
        s_nact = ba + sa;
        g_coff[ba + sa] = bc + sc;
      }
    }
    __syncthreads();
    trace_mark(pl, a.ws, 29);
    for (int p = tid; p < pl.P; p += kDecThreads) {
      const int e = rid[p], t = p / k;
      const uint32_t lo = bits[2 * e], hi = bits[2 * e + 1];
      const int rank = t < 32 ? __popc(lo & ((1u << t) - 1u)) : __popc(lo) + __popc(hi & ((1u << (t - 32)) - 1u));
      const int pos = off[e] + rank;
      g_ptok[pos] = t;
      g_pw[pos] = rw[p];
      g_pof[p] = pos;
    }
    __syncthreads();
  }
  const int D = s_nact;
  trace_mark(pl, a.ws, 5);

  if (lat_in) {  // every workgroup's latent rows are out (read with device-coherent loads)
    if (tid == 0 && !barrier_wait(ctl, bb, lat_bar, nullptr, false)) s_fail = 1;
    __syncthreads();
    if (s_fail) return give_up();
    trace_mark(pl, a.ws, 17);
  }

  // ------------------------------------------------------------ GU: gate/up --
  // pinned: this wave's range of whole units (global wave gw of 8 G)
  const unsigned gw = blockIdx.x * kDecWaves + w;
  const int pin_nu = g_coff[D] * pl.U8;
  auto wave_unit = [&](unsigned v) {  // NU v / 8G for the persistent grid (a power of two)
    return (int)(((uint64_t)(unsigned)pin_nu * v) >> (__builtin_ctz(gridDim.x) + 3));
  };
  const int pin_ua = wave_unit(gw), pin_ub = wave_unit(gw + 1);
  bool pinned_done = false;  // (pinned plans have K a multiple of 512: AL)
  if constexpr (AL) {
    if (pl.pinned) {
      gu_pinned<AL>(pl, a, g_act, g_aoff, g_acnt, g_coff, g_cexp, g_ptok, xpin, s_prog, hbuf, pin_ua, pin_ub,
                    wave_unit(blockIdx.x * kDecWaves), wave_unit((blockIdx.x + 1) * kDecWaves), rows_staged,
                    lat_in != 0);
      pinned_done = true;
    }
  }
  if (!pinned_done) {
    uint16_t *xs = reinterpret_cast<uint16_t *>(scr);  // staged activation rows (the scratch is free now)
    if (gu_pairs(g_coff[D] * pl.U8))
      gu_phase<2, AL>(pl, a, red, g_act, g_aoff, g_acnt, g_coff, g_cexp, g_ptok, xs, s_tab, s_round, s_rowtok, s_prog, D, hbuf, xpre, xpre_ok);
    else
      gu_phase<1, AL>(pl, a, red, g_act, g_aoff, g_acnt, g_coff, g_cexp, g_ptok, xs, s_tab, s_round, s_rowtok, s_prog, D, hbuf, xpre, xpre_ok);
  }
  trace_mark(pl, a.ws, 6);
  // Expert-major down reads an expert's h only after its gate/up units are
  // done: instead of a grid barrier, each workgroup that finished gate/up
  // units of active expert d (after its h stores have completed) writes the
  // tagged slot d + b (b: the workgroup; unique, since a later expert's
  // workgroups never come before an earlier one's), and a down wave polls the
  // slots of the workgroups whose gate/up range holds a group of its expert.
  // The paired row-tile path below (at most one expert per wave) waits the
  // same way; the general row-tile path needs every expert in every workgroup
  // and keeps the barrier.
  const bool expert_major = KSD > 0 && D > kDnExpertMajorMin && pl.o_y;
  // Paired row-tile down: at most one active expert per wave, one token
  // chunk per expert, I <= 256 and at most two row tiles per workgroup (small
  // batches). Wave w takes its expert's item in both row tiles; the weights
  // do not depend on h, so they are loaded while the expert's gate/up units
  // complete.
  const int dn_da = D * w / kDecWaves, dn_db = D * (w + 1) / kDecWaves;
  const bool dn_pair = !expert_major && D <= kDecWaves && B <= 16 && pl.KSd <= kDnDepth &&
                       pl.RTd <= 2 * (int)gridDim.x;
  // gate/up groups (as in the gate/up phase): W units each, NG in all; workgroup
  // b's range is [NG b / G, NG (b + 1) / G)
  const int gu_w = gu_pairs(g_coff[D] * pl.U8) ? 2 : 1;
  const int ngu = g_coff[D] * (pl.U8 / gu_w);
  // the workgroup whose range holds group x: the largest b with NG b / G <= x
  auto wg_of = [&](unsigned x) { return (int)(((x + 1u) * gridDim.x - 1u) / (unsigned)ngu); };
  // pinned: the wave whose range holds unit u: the largest gw with NU gw / 8G <= u
  auto wave_of = [&](unsigned u) {
    return (int)(((uint64_t)(u + 1u) * (gridDim.x * kDecWaves) - 1u) / (unsigned)pin_nu);
  };
  auto wait_expert = [&](int d) {  // bounded: a timeout sets the status word; gives up with the launch
    const unsigned gpc = (unsigned)(pl.U8 / gu_w);
    // the slots to poll: workgroups b0 .. b1 (slot d + b), or, pinned, waves b0 .. b1 (slot gw)
    const int b0 = pl.pinned ? wave_of((unsigned)g_coff[d] * pl.U8) : wg_of((unsigned)g_coff[d] * gpc);
    const int b1 = pl.pinned ? wave_of((unsigned)g_coff[d + 1] * pl.U8 - 1u)
                             : wg_of((unsigned)g_coff[d + 1] * gpc - 1u);
    unsigned spins = 0;
    for (int bs = b0; bs <= b1; bs += 64) {
      const int b = bs + l;
      // workgroups (waves) in [b0, b1] with an empty range (fewer groups than workgroups) write no slot
      const bool need = b <= b1 && (pl.pinned ? wave_unit(b) < wave_unit(b + 1)
                                              : grid_share(ngu, b) < grid_share(ngu, b + 1));
      const uint32_t slot = (uint32_t)(kTagDecDone + (pl.pinned ? b : d + b) * 8);
      for (;;) {
        const u32x2 v = need ? bload8_dev(tagr, slot) : u32x2{0u, tag};
        if (__ballot(v[1] != tag) == 0) break;
        ++spins;
        if ((spins & 63u) == 0u && aborted(ctl, abort0)) return;
        if (spins > kSpinLimit) {
          if (l == 0) raise_timeout(ctl);
          return;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    // the h loads after the wait stay after it (the hardware issues in
    // order; this keeps the compiler from hoisting them)
    asm volatile("" ::: "memory");
  };
  if ((expert_major || dn_pair) && pl.pinned) {
    // this wave's units are done (gu_pinned waited for its h stores): its slot gw
    if (pin_ua < pin_ub && l == 0) st_dev64(tagr, (uint32_t)(kTagDecDone + gw * 8), u32x2{0u, tag});
  } else if (expert_major || dn_pair) {
    wait_vmem();
    __syncthreads();
    const int ga = grid_share(ngu, blockIdx.x), gb = grid_share(ngu, blockIdx.x + 1);
    if (ga < gb) {
      const int ua = ga * gu_w, ub = gb * gu_w;  // this workgroup's units, chunk-major (chunk * U8 + unit)
      const int d0 = g_cexp[ua / pl.U8], d1 = g_cexp[(ub - 1) / pl.U8];
      for (int d = d0 + tid; d <= d1; d += kDecThreads)
        st_dev64(tagr, (uint32_t)(kTagDecDone + (d + (int)blockIdx.x) * 8), u32x2{0u, tag});
    }
  }
  DnLoad pf[2];
  if (dn_pair && dn_da < dn_db) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)  // a row tile past the last reads the zero area
      dn_issue_w(pl, a, zero, g_act, (int)blockIdx.x + tt * (int)gridDim.x, dn_da, 0, pl.I / kBlockK, pf[tt]);
  } else if (!expert_major && !dn_pair) {
    if (!grid_barrier(ctl, bb, ++nbar, trace_slots(pl, a.ws, 20), !dn_h_dev(pl))) return give_up();
  }
  trace_mark(pl, a.ws, 7);
  // expert_sum stores; when the latent block's output follows in this launch,
  // also its bf16 rounding (what the output's norm reads) at o_ebf, written
  // device-coherent (other workgroups read it after a grid barrier)
  const __amdgpu_buffer_rsrc_t ebr = make_rsrc(a.ws + pl.o_ebf, (uint32_t)((size_t)B * pl.K * 2));
  auto put_out = [&](size_t at, f32x4 v) {
    *reinterpret_cast<f32x4 *>(a.out + at) = v;
    if (lat_out)
      st_dev64(ebr, (uint32_t)(at * 2), u32x2{f32_to_bf16_bits(v[0]) | ((uint32_t)f32_to_bf16_bits(v[1]) << 16),
                                              f32_to_bf16_bits(v[2]) | ((uint32_t)f32_to_bf16_bits(v[3]) << 16)});
  };
  auto put_out1 = [&](size_t at, float v) {
    a.out[at] = v;
    if (lat_out) __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(v), ebr, (int)(at * 2), 0, kCpolDevice);
  };

  // ------------------------------------------------------- DN: down+combine --
  if (expert_major) {
    uint16_t *ybuf = reinterpret_cast<uint16_t *>(a.ws + pl.o_y);
    const __amdgpu_buffer_rsrc_t hrs = make_rsrc(hbuf, (uint32_t)pl.P * pl.I * 2);
    const int NT = D * pl.RTd;  // (expert, 16-row tile) items, expert-major
    const int gw = blockIdx.x * kDecWaves + w;
    const int ta = grid_share(NT, gw) >> 3, tb = grid_share(NT, gw + 1) >> 3;  // NT * gw / (8 G)
    DnStage st;  // this wave's y stage in the scratch area (free after the grouping)
    st.cap = pl.dn_cap;
    st.rows = reinterpret_cast<uint16_t *>(scr) + w * st.cap * 16;
    st.tag = reinterpret_cast<int *>(scr + kDecWaves * st.cap * 32) + w * st.cap;
    st.fill = 0;
    if constexpr (KSD > 0) dn_expert_major<KSD>(pl, a, g_act, g_aoff, g_acnt, zero, hrs, st, ybuf, ta, tb, wait_expert, s_dprog);
    if (pl.o_trace && l == 0)  // every wave's stream end (before its y flush)
      reinterpret_cast<uint64_t *>(a.ws + pl.o_trace)[blockIdx.x * kTraceSlots + 48 + w] = __builtin_amdgcn_s_memrealtime();
    dn_flush(st, pl, ybuf);
    trace_mark(pl, a.ws, 9);
    // (no acquire: the combine reads y only, with device-coherent loads; an
    // agent-scope acquire would invalidate the XCD's L2 first). With the latent
    // block's output following, a workgroup with no combine share only arrives
    // and goes on to stream its output weights; it waits for the barrier later,
    // before any other barrier (the group counters count arrivals in order).
    const unsigned nb4 = ++nbar;
    if (lat_out && blockIdx.x * kDecThreads >= (unsigned)(B * (pl.K / 4))) {
      wait_vmem();  // this wave's y stores have completed
      __syncthreads();
      if (tid == 0) barrier_arrive(ctl, bb, nb4, trace_slots(pl, a.ws, 24));
      nb_late = nb4;
    } else if (!grid_barrier(ctl, bb, nb4, trace_slots(pl, a.ws, 24), false)) {
      return give_up();
    }
    // combine (kimi.py:318,323): expert_sum[t][col] = sum over the token's
    // experts in ascending id order of w * bf16(y), from zero, FP32 adds
    const int K4 = pl.K / 4;
    const __amdgpu_buffer_rsrc_t yrs = make_rsrc(ybuf, (uint32_t)pl.P * pl.K * 2);
    for (unsigned idx = blockIdx.x * kDecThreads + tid; idx < (unsigned)(B * K4); idx += gridDim.x * kDecThreads) {
      const int t = (int)(idx / (unsigned)K4), c4 = ((int)idx - t * K4) * 4;
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      for (int sl = 0; sl < k; ++sl) {
        const int p = g_pof[t * k + sl];
        const float wt = g_pw[p];
        const u32x2 yv = bload8_dev(yrs, (uint32_t)((size_t)p * pl.K + c4) * 2);
        acc[0] = __fadd_rn(acc[0], __fmul_rn(bf16_bits_to_f32(yv[0] & 0xFFFFu), wt));
        acc[1] = __fadd_rn(acc[1], __fmul_rn(bf16_bits_to_f32(yv[0] >> 16), wt));
        acc[2] = __fadd_rn(acc[2], __fmul_rn(bf16_bits_to_f32(yv[1] & 0xFFFFu), wt));
        acc[3] = __fadd_rn(acc[3], __fmul_rn(bf16_bits_to_f32(yv[1] >> 16), wt));
      }
      put_out((size_t)t * pl.K + c4, f32x4{acc[0], acc[1], acc[2], acc[3]});
    }
  } else if (dn_pair) {
    // wave w: its expert's item in both row tiles, h loaded once after the barrier
    float *acc_lds = reinterpret_cast<float *>(scr);  // [2 row tiles][8 waves][B][16]
    const int BS = B * 16;
    for (int j = l; j < 2 * BS; j += 64) {
      const int tt = j >= BS ? 1 : 0;
      acc_lds[(tt * kDecWaves + w) * BS + j - tt * BS] = 0.f;
    }
    wave_lds_order();
    if (dn_da < dn_db) {
      const int d = dn_da;
      wait_expert(d);  // the expert's gate/up units are all done
      dn_issue_h_dev(pl, hbuf, g_aoff, g_acnt, d, pf[0]);
      f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
        for (int j = 0; j < kDnDepth; ++j) {
          if (j >= pl.KSd) break;
          bf16x8 av[4];
          convert_block_fast(pf[tt].w[j], dn_scale(pf[tt], j), av);  // the weights were loaded before the wait
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) acc[tt] = mfma16(av[kk], as_bf16x8(pf[0].b[j][kk]), acc[tt]);
        }
      }
      const int p0 = g_aoff[d];
      if (i < g_acnt[d]) {  // w * bf16(y) of the expert's token i, from zero
        const int t = g_ptok[p0 + i];
        const float wt = g_pw[p0 + i];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          float *dst = acc_lds + (tt * kDecWaves + w) * BS + t * 16 + 4 * q;
#pragma unroll
          for (int v = 0; v < 4; ++v) dst[v] = __fadd_rn(dst[v], __fmul_rn(round_bf16(acc[tt][v]), wt));
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int rt = (int)blockIdx.x + tt * (int)gridDim.x;
      if (rt >= pl.RTd) break;
      for (int j = tid; j < BS; j += kDecThreads) {
        float sum = acc_lds[tt * kDecWaves * BS + j];
#pragma unroll
        for (int ww = 1; ww < kDecWaves; ++ww) sum = __fadd_rn(sum, acc_lds[(tt * kDecWaves + ww) * BS + j]);
        put_out1((size_t)(j >> 4) * pl.K + rt * 16 + (j & 15), sum);
      }
    }
  } else
  {
    const int KB = pl.I / kBlockK;
    // [P pairs][16]: w * bf16(y) of each (token, expert) pair of the row tile;
    // every pair is written once per row tile, then each token's pairs are
    // summed from zero in ascending expert order (the order of kimi.py:319-323)
    float *pv = reinterpret_cast<float *>(scr);
    const int da = D * w / kDecWaves, db = D * (w + 1) / kDecWaves;
    // The wave walks items (expert d, 16-token chunk c, k-steps kc..kc+1) in
    // order with the next item's loads in flight while the current one runs,
    // across row tiles too (the next row tile's first item is issued before
    // the current one's reduction).
    // Two load buffers in turn (a copy of the next item's registers into the
    // current one would wait for its loads). The wave's item list of a row
    // tile is padded to an even length n2 with a filler (k-step KSd:
    // zero-area reads), so a tile starts with its first item in L0 and the
    // loop over item pairs has one exit: a path that re-enters the loop from
    // an exit test makes the compiler wait on the buffer being reissued.
    // `item` runs item `it` (loaded in X) and issues item it + 1 into Y: the
    // wave's next item, the filler, the next row tile's first item, or an
    // empty one. Every k-step is computed, those past KSd on zero-area
    // operands that add zero: a load left unread keeps its register busy.
    const int ksi = (pl.KSd + kDnDepth - 1) / kDnDepth;
    int n = 0;
    for (int d = da; d < db; ++d) n += (g_acnt[d] + 15) / 16 * ksi;
    n = __builtin_amdgcn_readfirstlane(n);
    const int n2 = (n + 1) & ~1;
    DnLoad L0, L1;
    auto item = [&](DnLoad &X, DnLoad &Y, int rt, int it, int &d, int &c, int &kc, f32x4 &acc) {
      int nd = d, nc = c, nkc = kc + kDnDepth;
      if (nkc >= pl.KSd) {
        nkc = 0;
        if (++nc * 16 >= g_acnt[d]) {
          nc = 0;
          ++nd;
        }
      }
      const bool more = it + 1 < n, filler = !more && it + 1 < n2;
      const bool next_rt = !more && !filler && rt + (int)gridDim.x < pl.RTd;
      dn_issue(pl, a, hbuf, zero, g_act, g_aoff, g_acnt, next_rt ? rt + (int)gridDim.x : rt, more ? nd : da,
               more ? nc : 0, more ? nkc : (next_rt ? 0 : pl.KSd), KB, Y);
#pragma unroll
      for (int j = 0; j < kDnDepth; ++j) {
        bf16x8 av[4];
        convert_block_fast(X.w[j], dn_scale(X, j), av);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) acc = mfma16(av[kk], as_bf16x8(X.b[j][kk]), acc);
      }
      if (it < n && nkc == 0) {  // (d, c) complete: w * bf16(y) of its pairs
        const int p0 = g_aoff[d], pj = c * 16 + i;
        if (pj < g_acnt[d]) {
          const float wt = g_pw[p0 + pj];
          *reinterpret_cast<f32x4 *>(pv + (p0 + pj) * 16 + 4 * q) =
              f32x4{__fmul_rn(round_bf16(acc[0]), wt), __fmul_rn(round_bf16(acc[1]), wt),
                    __fmul_rn(round_bf16(acc[2]), wt), __fmul_rn(round_bf16(acc[3]), wt)};
        }
        acc = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      if (more) {
        d = nd;
        c = nc;
        kc = nkc;
      }
    };
    if (n > 0) dn_issue(pl, a, hbuf, zero, g_act, g_aoff, g_acnt, blockIdx.x, da, 0, 0, KB, L0);
    for (int rt = blockIdx.x; rt < pl.RTd; rt += gridDim.x) {
      int d = da, c = 0, kc = 0;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      for (int it = 0; it < n2; it += 2) {
        item(L0, L1, rt, it, d, c, kc, acc);
        item(L1, L0, rt, it + 1, d, c, kc, acc);
      }
      __syncthreads();
      for (int j = tid; j < B * 16; j += kDecThreads) {
        const int t = j >> 4;
        float sum = 0.f;
        for (int sl = 0; sl < k; ++sl) sum = __fadd_rn(sum, pv[g_pof[t * k + sl] * 16 + (j & 15)]);
        put_out1((size_t)t * pl.K + rt * 16 + (j & 15), sum);
      }
      __syncthreads();
    }
  }

  // ------------------------------------------------------------------ exit --
  __syncthreads();
  // a wait of this launch gave up (the down-phase waits have no barrier after
  // them); with the latent block's output, checked after it
  if (!lat_out && aborted(ctl, abort0)) {
    give_up();
    return;
  }
  trace_mark(pl, a.ws, 8);
  if (lat_out) {
    // the latent block's output once every workgroup has published its
    // expert-sum stores: workgroup b's slot kTagDecFlags + 8 b carries this
    // launch's tag after its stores completed (workgroups without a share
    // publish at once)
    auto arrive = [&]() {
      wait_vmem();  // this wave's expert-sum stores have completed
      __syncthreads();
      if (tid == 0) st_dev64(tagr, (uint32_t)(kTagDecFlags + blockIdx.x * 8), u32x2{0u, tag});
    };
    // the abort counter, read by wave 0 once every slot is seen (every
    // workgroup is past its down phase then, whose waits have no barrier
    // after them) and used at the end, so that the read overlaps the output
    unsigned abort_end = abort0;
    auto wait = [&]() {  // wave 0 polls every workgroup's slot (bounded)
      if (w == 0) {
        unsigned spins = 0;
        for (;;) {
          bool ready = true;
#pragma unroll
          for (int m = 0; m < kLatFlagsMax / 64; ++m) {
            const unsigned f = (unsigned)(l + 64 * m);
            const u32x2 v = bload8_dev(tagr, f < gridDim.x ? (uint32_t)(kTagDecFlags + f * 8) : kOffNone);
            ready = ready && (f >= gridDim.x || v[1] == tag);
          }
          if (__ballot(!ready) == 0) break;
          ++spins;
          if ((spins & 63u) == 0u && aborted(ctl, abort0)) {
            if (l == 0) s_fail = 1;
            break;
          }
          if (spins > kSpinLimit) {
            if (l == 0) {
              raise_timeout(ctl);
              s_fail = 1;
            }
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
        abort_end = __hip_atomic_load(ctl + kCtlAbort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      return s_fail == 0;
    };
    // expert-major: the workgroups with a combine share (below ncomb) write
    // their expert sum only after barrier 4; the output rows go to the others
    // when at most 32 rows each
    const int ncomb = (B * (pl.K / 4) + kDecThreads - 1) / kDecThreads;
    const int wg0 = expert_major && ncomb < (int)gridDim.x && cdiv(pl.h, (int)gridDim.x - ncomb) <= 32 ? ncomb : 0;
    if ((int)blockIdx.x < wg0) {
      arrive();
      // (its own down phase and combine are done; another workgroup's wait
      // that gives up later poisons its own share and this workgroup's output
      // is the expert sum only, which that workgroup's readers then poison)
      if (aborted(ctl, abort0)) return give_up();
    } else {
      if (!dec_latent_out(pl, a, lds, zero, wg0, arrive, wait)) return give_up();
      if (tid == 0 && abort_end != abort0) s_fail = 1;
      __syncthreads();
      if (s_fail) return give_up();
    }
    trace_mark(pl, a.ws, 18);
  }
  if (blockIdx.x == 0 && tid == 0) {  // this kernel's code range, for the next launch's warm-up
    crange[0] = pc0;
    crange[1] = program_counter();
  }
  if (tag == last_tag_of_cycle()) {
    if (nb_late) {  // the barrier this workgroup only arrived at, before its next arrival
      if (tid == 0 && !barrier_wait(ctl, bb, nb_late, nullptr, false)) s_fail = 1;
      __syncthreads();
      if (s_fail) return give_up();
    }
    if (!clear_tag_area(ctl, bb, ++nbar, tagr)) return give_up();
  }
  leave();
  trace_mark(pl, a.ws, kTraceExit);
}

}  // namespace k3moe
