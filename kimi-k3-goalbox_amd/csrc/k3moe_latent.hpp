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
// tiles (k_latent<0>: the latent_down rows, then "pair" tiles of 8 shared_gate
// rows and the same 8 shared_up rows; k_latent<1>: the h output rows, each with
// two parts: k over latent_up then k over shared_down, rounded separately). The
// k axis is cut into SP splits of 128-k steps. Workgroup b takes split
// s = b mod SP and the row tiles b / SP + j G / SP ("units"), so the SP
// consecutive workgroups of a group share their tiles:
//   - it stages the activation rows of its split (all tokens) in LDS once;
//   - the 8 waves take the split's k-steps in turn (wave w: k0 + w, k0 + w + 8),
//     each loading 16 rows x 128 k of bf16 weights per k-step (64 bytes per
//     lane, 4 loads of 16 rows x 64 contiguous bytes) into a register ring three units deep,
//     refilled as soon as a unit is multiplied, so three units' weights are in
//     flight (MFMA 16x16x32 bf16, token tiles of 16 as the B operand from LDS);
//   - the waves' fp32 tiles meet in LDS (wave order) and the split's partial
//     of each (token, row) goes to the workspace with device-coherent stores.
// After its units the group meets at a counter of its own (a barrier of SP
// workgroups); member s then sums the partials of the group's tiles
// j = s, s + SP, .. in split order and writes the bf16 outputs (with the
// activation for a pair tile). k_latent<1> normalises the expert sum first:
// for up to 8 tokens every workgroup does it itself for its split's k range,
// for more workgroup t < B writes token t's row to the workspace and a grid
// barrier separates that from the staging.
//
// Accumulation order is fixed (k-step order per wave, wave order, split
// order), so results do not depend on timing.
#pragma once

#include <stddef.h>

#include <type_traits>

#include "k3moe_barrier.hpp"
#include "k3moe_decode.hpp"
#include "k3moe_device.hpp"
#include "k3moe_plan.hpp"

namespace k3moe {

constexpr int kLatMaxTokens = 64;
constexpr int kLatWaves = 8;
constexpr int kLatThreads = kLatWaves * 64;
constexpr int kLatKW = 2;          // k-steps per wave and unit, at most
constexpr int kLatMaxLds = kDecMaxLds - 1024;  // dynamic LDS (the static LDS stays under 1 KiB)
constexpr int kLatMaxUnits = 64;   // units per workgroup, at most
constexpr int kLatMaxSplits = 16;  // k-splits, at most
constexpr int kLatLocalNorm = 8;   // k_latent<1>: up to this many tokens every workgroup normalises
constexpr int kLatNormChunks = 16; // ... from 16-byte chunks, 64 lanes x 16 x 4 = latent widths up to 4096
constexpr float kLatRmsEps = 1e-5f;  // kimi.py:325
constexpr int kLatGrpStride = 16;    // words between group counters (64 bytes)
// streamed kernels (k_latent_sk)
// (steps go in pairs: one barrier per two 128-k steps)
constexpr int kSkAPairs = 2;                    // activation step pairs loaded ahead of the current one
constexpr int kSkSlots = 2 * (kSkAPairs + 1);   // activation ring slots, one step of 64 tokens (16 KiB) each
constexpr int kSkSlotBytes = kLatMaxTokens * kStepK * 2;
constexpr int kSkWPairs = 5;                    // weight step pairs loaded ahead (HBM latency)
constexpr int kSkWSlots = 2 * (kSkWPairs + 1);  // weight ring slots, one row tile's step (4 KiB) each
constexpr int kSkWSlotBytes = 16 * kStepK * 2;
constexpr int kSkCntWord = 2048;        // first counter word (per row tile and token tile) in the latent counter area
constexpr unsigned kLatGrpTotal = 1024;  // a group counter grows by this much per launch, whatever SP is

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
  int ntile0;  // k_latent<0>: latent_down row tiles (the shared pair tiles follow)
  int local_norm;  // k_latent<1>: every workgroup normalises the expert sum (no grid barrier)
  int sk;          // 1: the streamed kernel k_latent_sk (no k-splits; G workgroups share the (tile, k-step) items)
  long o_cnt, o_part0, o_part1, o_en, o_trace, total;
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

// Split s covers k-steps [lat_k0(s), lat_k0(s + 1)) (SP a power of two: a shift).
__host__ __device__ inline int lat_k0(int s, int KS, int SP) {
  return (int)(((unsigned)s * (unsigned)KS) >> __builtin_ctz((unsigned)SP));
}

// Plan of k_latent<out> for the given geometry; null on success, else why it does not fit.
inline const char *latent_plan(const k3moe_latent_dims &d, int n_cus, int out, LatPlan &p) {
  p.B = d.tokens; p.h = d.hidden; p.lh = d.latent; p.S = d.shared; p.act = d.activation; p.out = out;
  p.TT = cdiv(p.B, 16);
  p.G = 1;
  while (p.G * 2 <= n_cus && p.G * 2 <= 1024) p.G *= 2;
  p.ntile0 = p.lh / 16;
  if (!out) {
    p.RT = p.lh / 16 + p.S / 8; p.KS0 = p.KS = p.h / kStepK;
  } else {
    p.RT = p.h / 16; p.KS0 = p.lh / kStepK; p.KS = p.KS0 + p.S / kStepK;
  }
  p.local_norm = out && p.B <= kLatLocalNorm && p.lh <= 64 * 4 * kLatNormChunks;

  const int parts = out ? 2 : 1;
  // Past the batches that normalise locally, the streamed kernel: the staged
  // one's split partials would move 8 SP B / K of the weights' bytes (0.5 at
  // 64 tokens), the streamed one's move a row tile's partial at most once per
  // workgroup. Its grid is at most the row tile count (each workgroup's run of
  // (tile, k-step) items then spans a whole tile's worth, so a tile is cut at
  // most once). Measured at 64 tokens on a TP8 rank's geometry: <1> 36 us
  // against the staged kernel's 66, <0> 39 us against 45. <1> takes it only
  // with the full grid (its grid barrier counts arrivals in groups, and every
  // launch on a workspace that uses one must use the same grid size for the
  // counts of earlier launches to round off); <0>, which has no grid barrier,
  // from 64 workgroups on.
  p.sk = 0;
  if (p.B > kLatLocalNorm) {
    int g = 1;
    while (g * 2 <= p.G && g * 2 <= p.RT) g *= 2;
    if ((out ? g == p.G && g >= p.B : g >= 64) && p.RT * 4 <= kLatCntBytes / 4 - kSkCntWord) {
      p.sk = 1;
      p.G = g;
      p.SP = 1;
      p.J = 0;
      p.kwmax = 0;
      p.xpitch = 0;
      p.lds_x = kSkSlots * kSkSlotBytes + kSkWSlots * kSkWSlotBytes;  // 144 KiB
      p.lds_total = p.lds_x;
      long o = 0;
      auto take = [&](long bytes) { long at = o; o = (long)align256((size_t)(o + bytes)); return at; };
      take(kOffLatCnt);
      p.o_cnt = take(kLatCntBytes);
      take(kTagBytes);
      p.o_part0 = take((long)p.RT * 2 * parts * 4 * 1024);  // [tile][segment][part][token tile] 16 x 16 fp32
      p.o_part1 = 0;
      p.o_en = out ? take((long)p.B * (p.lh + p.S) * 2) : 0;
      p.o_trace = 0;
      p.total = o;
      return nullptr;
    }
  }
  const int red = parts * p.TT * kLatWaves * 1024;
  p.SP = 0;
  for (int sp = 4; sp <= kLatMaxSplits && !p.SP; sp *= 2) {
    int s = sp;
    while (s > p.KS) s >>= 1;  // at least one k-step per split
    const int kw = cdiv(p.KS, s);
    const int lx = p.B * (kw * kStepK + 8) * 2;
    if (kw <= kLatWaves * kLatKW && lx + red <= kLatMaxLds) p.SP = s;
    if (s < sp) break;
  }
  if (!p.SP) return "the staged activation slice does not fit in LDS";
  if (p.SP > p.G) return "too few compute units for the k-splits";
  p.kwmax = cdiv(p.KS, p.SP);
  p.xpitch = p.kwmax * kStepK + 8;
  p.lds_x = p.B * p.xpitch * 2;
  p.lds_total = p.lds_x + red;
  // the group counters stay below the streamed kernels' counters (kSkCntWord
  // on): only a single-step <0> has more groups (k_latent<1> has at least two
  // steps, so SP >= 2), and <0> has no grid barrier, so its grid may shrink
  if (!out || p.local_norm)
    while (p.G > p.SP && (p.G / p.SP) * kLatGrpStride > kSkCntWord) p.G /= 2;
  p.J = cdiv(p.RT, p.G / p.SP);
  if (p.J > kLatMaxUnits) return "too many row tiles per workgroup";
  if ((p.G / p.SP) * kLatGrpStride > kSkCntWord) return "too many workgroup groups for the counter area";
  long o = 0;
  auto take = [&](long bytes) { long at = o; o = (long)align256((size_t)(o + bytes)); return at; };
  take(kOffLatCnt);
  p.o_cnt = take(kLatCntBytes);
  take(kTagBytes);
  const long part = (long)p.SP * p.RT * p.B * 16 * 4;
  p.o_part0 = take(part);
  p.o_part1 = out ? take(part) : 0;
  p.o_en = out ? take((long)p.B * (p.lh + p.S) * 2) : 0;
  p.o_trace = 0;  // a trace area, when wanted, follows the larger of the two kernels' layouts
  p.total = o;
  return nullptr;
}

// Lane (row i, group q) of k-step ks of row tile rt: MFMA kk of the step takes
// k = 32 kk + 8 q .. + 7, so the 4 lanes of a row read 64 contiguous bytes per
// load (half a 128-byte line). Returns the lane's first bf16 (kk = 0). `pair`
// is this lane's matrix in a <0> pair tile (shared_gate for rows i < 8,
// shared_up for i >= 8), chosen once per lane by the caller.
__device__ __forceinline__ const uint16_t *lat_src(const LatPlan &pl, const LatArgs &a, const uint16_t *pair, int rt,
                                                   int ks, int i, int q) {
  const long r = (long)rt * 16 + i;
  const int kq = q * 8;
  if (!pl.out) {
    // pair tile p: rows i < 8 are shared_gate row 8 p + i, rows i >= 8 shared_up row 8 p + i - 8
    const long sr = 8L * (rt - pl.ntile0) + (i & 7);
    const uint16_t *row = rt < pl.ntile0 ? a.wa + r * pl.h : pair + sr * pl.h;
    return row + ks * kStepK + kq;
  }
  return ks < pl.KS0 ? a.wa + r * pl.lh + ks * kStepK + kq : a.wb + r * pl.S + (ks - pl.KS0) * kStepK + kq;
}

__device__ __forceinline__ float bload4_dev(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, kCpolDevice));
}

static_assert(sizeof(LatPlan) % alignof(LatArgs) == 0, "LatArgs follows LatPlan in the argument segment");

// The LatArgs at constant address `at`; every pointer is device (global) memory.
__device__ __forceinline__ LatArgs lat_args(uint64_t at) {
  LatArgs a;
#define K3_FIELD(f) a.f = global_field<std::remove_pointer_t<decltype(a.f)>>(at + offsetof(LatArgs, f))
  K3_FIELD(x);
  K3_FIELD(esum);
  K3_FIELD(norm);
  K3_FIELD(wa);
  K3_FIELD(wb);
  K3_FIELD(wc);
  K3_FIELD(ya);
  K3_FIELD(yb);
  K3_FIELD(ws);
#undef K3_FIELD
  static_assert(sizeof(LatArgs) == 9 * sizeof(void *), "every field read");
  return a;
}

template <int OUT>
__global__ __launch_bounds__(kLatThreads, 1) void k_latent(LatPlan pl_arg, LatArgs a_arg) {
  // the arguments, read through the touched segment (all its lines requested at once)
  const uint64_t kargs = touch_kernargs<sizeof(LatPlan) + sizeof(LatArgs)>();
  const LatPlan pl = load_const<LatPlan>(kargs);
  const LatArgs a = lat_args(kargs + sizeof(LatPlan));
  (void)pl_arg;
  (void)a_arg;
  extern __shared__ __attribute__((aligned(16))) char lds[];
  uint16_t *xs = reinterpret_cast<uint16_t *>(lds);                 // [B][xpitch] activation slice
  float *red = reinterpret_cast<float *>(lds + pl.lds_x);          // [parts][TT][8 waves][256]
  __shared__ float s_wsum[kLatWaves];

  const int tid = threadIdx.x, w = wave_id(), l = tid & 63;
  const int i = l & 15, q = l >> 4;
  const int B = pl.B, TT = pl.TT, SP = pl.SP;
  const int lsp = __builtin_ctz(SP), lstep = __builtin_ctz(gridDim.x) - lsp;  // SP and the grid are powers of two
  const int s = blockIdx.x & (SP - 1);
  const int k0 = (s * pl.KS) >> lsp, k1 = ((s + 1) * pl.KS) >> lsp, nk = k1 - k0;
  const int rstep = 1 << lstep, rt0 = blockIdx.x >> lsp;
  const int J = rt0 < pl.RT ? (pl.RT - rt0 + rstep - 1) >> lstep : 0;
  const bool touch0 = k0 < pl.KS0, touch1 = OUT && k1 > pl.KS0;  // parts with k-steps in this split
  const bool local = OUT && pl.local_norm;  // <1>: every workgroup normalises the expert sum itself
  unsigned *ctl = reinterpret_cast<unsigned *>(a.ws);
  unsigned *gcnt = reinterpret_cast<unsigned *>(a.ws + pl.o_cnt) + rt0 * kLatGrpStride;  // this group's counter
  const uint16_t *zlane = reinterpret_cast<const uint16_t *>(a.ws + 4096 + l * 64);  // 64 zero bytes
  const uint32_t part_bytes = (uint32_t)((long)SP * pl.RT * B * 64);
  const __amdgpu_buffer_rsrc_t rp0 = make_rsrc(a.ws + pl.o_part0, part_bytes);
  const __amdgpu_buffer_rsrc_t rp1 = make_rsrc(a.ws + (OUT ? pl.o_part1 : pl.o_part0), part_bytes);
  // this kernel's code into L2 before the weight loads (the range its last launch recorded)
  const uint64_t pc0 = program_counter();
  uint64_t *const crange = reinterpret_cast<uint64_t *>(ctl + kCtlCodeLatent + 4 * OUT);
  const u32x4 code_probe = warm_code_range(crange, pc0);
  BarrierBase bb{0u, 0u, 0u};
  if (OUT && !local && tid == 0) bb = barrier_base(ctl);
  // the group counter before this launch: no member can have added a whole kLatGrpTotal yet
  const unsigned gbase =
      tid == 0 ? __hip_atomic_load(gcnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & ~(kLatGrpTotal - 1u) : 0u;
  // phase timestamps (100 MHz) when the plan carries a trace area: 0 start, 1 staged,
  // 2 + j unit j done (j < 40), 45 units done, 46 group met, 47 end; <1>: 48 normalised, 49 barrier
  auto mark = [&](int n) {
    if (pl.o_trace && tid == 0)
      reinterpret_cast<uint64_t *>(a.ws + pl.o_trace)[blockIdx.x * kTraceSlots + n] = __builtin_amdgcn_s_memrealtime();
  };
  mark(0);

  const uint16_t *pair = i < 8 ? a.wb : a.wc;  // <0>: this lane's matrix in a pair tile
  // weight ring: unit j's k-steps of this wave; past the units or the split, the zero area
  auto issue = [&](int j, u32x4 (&buf)[kLatKW][4]) {
    const int rt = rt0 + rstep * j;
#pragma unroll
    for (int m = 0; m < kLatKW; ++m) {
      const int ks = k0 + w + kLatWaves * m;
      const uint16_t *src = (j < J && ks < k1) ? lat_src(pl, a, pair, rt, ks, i, q) : zlane;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) buf[m][kk] = load16(src + kk * 32);
    }
  };

  // The activation slice of this split (all tokens) loaded straight into LDS,
  // one 16-byte chunk per lane: wave u takes (token t, group g), the chunks
  // 64 g .. 64 g + 63 of token t's cpt chunks. <0>: x; <1>: [en | shared_h]
  // from the workspace rows, or with local normalisation the shared_h chunks
  // only (the normalisation writes the en chunks). Waited for with wait_vm.
  const int cpt = nk * (kStepK / 8);  // chunks per token
  const int ngrp = (cpt + 63) >> 6;
  const int erow = pl.lh + pl.S;      // <1>: workspace row of a token, [en | shared_h]
  auto stage = [&]() {
    for (int u = w; u < B * ngrp; u += kLatWaves) {
      const int t = u / ngrp, g = u - t * ngrp;
      const int cc = g * 64 + l;
      const int ks = k0 + (cc >> 4), e = (cc & 15) * 8;
      char *dst = reinterpret_cast<char *>(xs + t * pl.xpitch) + g * 64 * 16;
      if (cc < cpt) {
        if (!OUT)
          load_lds<16>(a.x + (long)t * pl.h + ks * kStepK + e, dst);
        else if (!local)
          load_lds<16, kCpolDevice>(a.ws + pl.o_en + ((long)t * erow + ks * kStepK + e) * 2, dst);
        else if (ks >= pl.KS0)
          load_lds<16>(a.x + (long)t * pl.S + (ks - pl.KS0) * kStepK + e, dst);
      }
    }
  };
  constexpr int kRingLoads = 3 * kLatKW * 4;  // weight loads of the three prologue units, per wave

  u32x4 b0[kLatKW][4], b1[kLatKW][4], b2[kLatKW][4];
  if (!OUT) {
    stage();  // first, so that its wait below does not include the weight loads
    issue(0, b0);
    issue(1, b1);
    issue(2, b2);
    wait_vm<kRingLoads>();
    ring_barrier();
  } else if (local) {
    // Small batches: wave t < B normalises token t in every workgroup, from
    // 16-byte chunks k = 4 (l + 64 m) of its expert-sum row:
    //   en = bf16(bf16(e r) w), e = bf16(expert_sum), r = 1/sqrt(mean(e^2) + eps),
    // and writes the chunks in this split's latent range to the slice. The
    // shared_h chunks, the expert sum and the norm weights of the range are
    // loaded before the first units' weights; the staging goes first (its
    // number of loads varies), so that the expert sum's use waits for a fixed
    // count of later loads and not for the weights.
    const int t = w;
    const int kr0 = k0 * kStepK, kr1 = (touch0 ? (k1 < pl.KS0 ? k1 : pl.KS0) : k0) * kStepK;
    stage();
    f32x4 ec[kLatNormChunks];
#pragma unroll
    for (int m = 0; m < kLatNormChunks; ++m) ec[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (t < B) {  // wave-uniform: the other waves load nothing here
#pragma unroll
      for (int m = 0; m < kLatNormChunks; ++m) {
        const int k = 4 * (l + 64 * m);
        ec[m] = *reinterpret_cast<const f32x4 *>(k < pl.lh ? a.esum + (long)t * pl.lh + k
                                                           : reinterpret_cast<const float *>(zlane));
      }
    }
    const u32x4 wnv = load16(tid * 8 < kr1 - kr0 ? a.norm + kr0 + tid * 8 : zlane);
    issue(0, b0);
    issue(1, b1);
    issue(2, b2);
    float r = 0.f;
    if (t < B) {
      float ss = 0.f;
#pragma unroll
      for (int m = 0; m < kLatNormChunks; ++m) {
        if (4 * (l + 64 * m) < pl.lh) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float e = round_bf16(ec[m][v]);
            ss += e * e;
          }
        }
      }
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) ss += shfl_xor(ss, m);
      r = 1.0f / __fsqrt_rn(ss / (float)pl.lh + kLatRmsEps);
    }
    uint16_t *wn_lds = reinterpret_cast<uint16_t *>(red);  // the range's norm weights (red is free until the units)
    if (tid * 8 < kr1 - kr0) *reinterpret_cast<u32x4 *>(wn_lds + tid * 8) = wnv;
    wait_vm<kRingLoads>();
    ring_barrier();
    if (t < B) {
#pragma unroll
      for (int m = 0; m < kLatNormChunks; ++m) {
        const int k = 4 * (l + 64 * m);
        if (k >= kr0 && k < kr1) {
          const u32x2 wp = *reinterpret_cast<const u32x2 *>(wn_lds + (k - kr0));
          uint32_t o[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const uint32_t wb = v & 1 ? wp[v >> 1] >> 16 : wp[v >> 1] & 0xFFFFu;
            o[v] = f32_to_bf16_bits(round_bf16(round_bf16(ec[m][v]) * r) * bf16_bits_to_f32(wb));
          }
          *reinterpret_cast<u32x2 *>(xs + t * pl.xpitch + (k - kr0)) = u32x2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
        }
      }
    }
    ring_barrier();
    mark(48);
  } else {
    issue(0, b0);
    issue(1, b1);
    issue(2, b2);
    if ((int)blockIdx.x < B) {
      // Workgroup t < B normalises token t's expert sum into the workspace row
      // [en | shared_h] the splits stage from (as above, one workgroup per token).
      const int t = blockIdx.x;
      float ss = 0.f;
      for (int k = 2 * tid; k < pl.lh; k += 2 * kLatThreads) {
        const float2 v = *reinterpret_cast<const float2 *>(a.esum + (long)t * pl.lh + k);
        const float e0 = round_bf16(v.x), e1 = round_bf16(v.y);
        ss += e0 * e0;
        ss += e1 * e1;
      }
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) ss += shfl_xor(ss, m);
      if (l == 0) s_wsum[w] = ss;
      __syncthreads();
      float tot = s_wsum[0];
#pragma unroll
      for (int v = 1; v < kLatWaves; ++v) tot += s_wsum[v];
      const float r = 1.0f / __fsqrt_rn(tot / (float)pl.lh + kLatRmsEps);
      const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.ws + pl.o_en, (uint32_t)(B * erow * 2));
      for (int k = 2 * tid; k < pl.lh; k += 2 * kLatThreads) {
        const float2 v = *reinterpret_cast<const float2 *>(a.esum + (long)t * pl.lh + k);
        const uint32_t wn = *reinterpret_cast<const uint32_t *>(a.norm + k);
        const float n0 = round_bf16(round_bf16(v.x) * r), n1 = round_bf16(round_bf16(v.y) * r);
        const uint32_t o0 = f32_to_bf16_bits(n0 * bf16_bits_to_f32(wn & 0xFFFFu));
        const uint32_t o1 = f32_to_bf16_bits(n1 * bf16_bits_to_f32(wn >> 16));
        st_dev32(rw, (uint32_t)(((long)t * erow + k) * 2), o0 | (o1 << 16));
      }
      for (int k = 2 * tid; k < pl.S; k += 2 * kLatThreads)
        st_dev32(rw, (uint32_t)(((long)t * erow + pl.lh + k) * 2),
                 *reinterpret_cast<const uint32_t *>(a.x + (long)t * pl.S + k));
    }
    mark(48);
    // (no acquire: the rows are read with device-coherent loads)
    if (!grid_barrier(ctl, bb, 1, nullptr, false)) {  // a wait of this launch gave up: the rows are incomplete
      poison_share<true>(a.ya, (long)B * pl.h);
      return;
    }
    mark(49);
    stage();
    wait_vm<0>();
    ring_barrier();
  }

  // one unit: the split's k-steps of row tile rt0 + rstep j from `buf`, partials
  // out; `buf` takes unit j + 3 as soon as this wave's products are done (before
  // the unit's barriers, which wait for the workgroup's slowest wave)
  auto unit = [&](int j, u32x4 (&buf)[kLatKW][4]) {
    const int rt = rt0 + rstep * j;
    f32x4 acc0[4], acc1[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) acc0[tt] = acc1[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < kLatKW; ++m) {
      const int ks = k0 + w + kLatWaves * m;
      if (ks >= k1) continue;
      const bool p1 = OUT && ks >= pl.KS0;
      const uint16_t *xrow = xs + (ks - k0) * kStepK + q * 8;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        if (tt >= TT) continue;
        const int tok = tt * 16 + i;
        u32x4 bv[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          bv[kk] = tok < B ? *reinterpret_cast<const u32x4 *>(xrow + tok * pl.xpitch + kk * 32) : u32x4{0, 0, 0, 0};
        if (p1) {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) acc1[tt] = mfma16(as_bf16x8(buf[m][kk]), as_bf16x8(bv[kk]), acc1[tt]);
        } else {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) acc0[tt] = mfma16(as_bf16x8(buf[m][kk]), as_bf16x8(bv[kk]), acc0[tt]);
        }
      }
    }
    if (j + 3 < J) issue(j + 3, buf);
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
    if (j < 40) mark(2 + j);
  };

  mark(1);
  asm volatile("" ::"v"(code_probe));  // (issued first: complete with the staging)
  // three units in flight: a buffer is refilled with unit j + 3 once this wave has multiplied unit j
  for (int j = 0; j < J; j += 3) {
    unit(j, b0);
    if (j + 1 >= J) break;
    unit(j + 1, b1);
    if (j + 2 >= J) break;
    unit(j + 2, b2);
  }
  mark(45);

  // the group's barrier: every member's partial stores are complete
  __shared__ int s_gave_up;
  wait_vmem();
  __syncthreads();
  if (tid == 0) {
    s_gave_up = 0;
    __hip_atomic_fetch_add(gcnt, kLatGrpTotal >> lsp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned target = gbase + kLatGrpTotal;
    unsigned spins = 0;
    while ((int)(__hip_atomic_load(gcnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - target) < 0) {
      __builtin_amdgcn_s_sleep(1);
      if (++spins > kSpinLimit) {
        raise_timeout(ctl);
        s_gave_up = 1;
        break;
      }
    }
    // no acquire fence: the partials are read with device-coherent loads
  }
  __syncthreads();
  mark(46);
  int s0 = 0, last0 = SP;  // <1>: splits [0, last0) have part-0 k-steps, [s0, SP) part-1 k-steps
  if (OUT) {
    while (s0 < SP && (((s0 + 1) * pl.KS) >> lsp) <= pl.KS0) ++s0;
    last0 = ((s0 * pl.KS) >> lsp) < pl.KS0 ? s0 + 1 : s0;
  }
  // member s finishes the group's tiles j = s, s + SP, ..: output item it of
  // the nj tiles' nj x B x 16 (tile jj = it / (16 B), token, row) goes to a
  // thread, so the partial loads of all its tiles are in flight together; per
  // output, every split's partial is loaded before the sum (in split order)
  const int nj = J > s ? (J - s + SP - 1) >> lsp : 0;
  const int per_tile = B * 16, items = nj * per_tile;
  for (int it0 = 0; it0 < items; it0 += 2 * kLatThreads) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int it = it0 + tid + c * kLatThreads;
      const int jj = it / per_tile, rem = it - jj * per_tile;
      const int t = rem >> 4, r = rem & 15;
      const int rt = rt0 + rstep * (s + SP * jj);
      const bool pair = !OUT && rt >= pl.ntile0;
      const bool ok = it < items && (!pair || r < 8);
      // (only the splits that wrote a part: <1>'s part 1 lives in the last few)
      float va[kLatMaxSplits], vb[kLatMaxSplits];
#pragma unroll
      for (int ss = 0; ss < kLatMaxSplits; ++ss) {
        va[ss] = vb[ss] = 0.f;
        if (ss < SP) {
          const uint32_t o = ok ? (uint32_t)((((long)ss * pl.RT + rt) * B + t) * 64 + r * 4) : 0u;
          va[ss] = bload4_dev(rp0, ok && ss < last0 ? o : kOffNone);
          vb[ss] = bload4_dev(OUT ? rp1 : rp0, ok && (OUT ? ss >= s0 : pair) ? o + (OUT ? 0 : 32) : kOffNone);
        }
      }
      if (!ok) continue;
      float sa = 0.f, sb = 0.f;
#pragma unroll
      for (int ss = 0; ss < kLatMaxSplits; ++ss) {
        if (ss < SP && ss < last0) sa += va[ss];
        if (ss < SP && ss >= s0) sb += vb[ss];
      }
      if (OUT)
        a.ya[(long)t * pl.h + rt * 16 + r] = f32_to_bf16_bits(round_bf16(sa) + round_bf16(sb));
      else if (!pair)
        a.ya[(long)t * pl.lh + rt * 16 + r] = f32_to_bf16_bits(sa);
      else
        a.yb[(long)t * pl.S + (rt - pl.ntile0) * 8 + r] =
            f32_to_bf16_bits(apply_act(pl.act, round_bf16(sa), round_bf16(sb)));
    }
  }
  if (s_gave_up) {  // the group's partials were incomplete: NaN in this workgroup's share of the outputs
    __syncthreads();
    poison_share<true>(a.ya, (long)B * (OUT ? pl.h : pl.lh));
    if (!OUT) poison_share<true>(a.yb, (long)B * pl.S);
  }
  if (blockIdx.x == 0 && tid == 0) {  // this kernel's code range, for the next launch's warm-up
    crange[0] = pc0;
    crange[1] = program_counter();
  }
  mark(47);
}


// ---------------------------------------------------------------- streamed --
// k_latent_sk<OUT>: the same outputs for batches past kLatLocalNorm tokens,
// without k-splits. The (row tile, 128-k step) items, tile-major, are cut
// into G equal runs, one per workgroup; a run covers at least one tile's worth
// of steps, so a tile is either whole in one run or cut once, into segments 0
// and 1 of two neighbouring runs. Eight waves:
//   - waves 4-7 load each step's operands into two LDS rings by direct-to-LDS
//     loads: the row tile's weights (16 rows x 256 bytes) 2 kSkWPairs steps
//     ahead (the HBM stream) and the activation rows (all tokens) 2 kSkAPairs
//     steps ahead (read from L2); in both, 16-byte chunk c of row r sits at
//     position c ^ (r & 15) of its 256-byte row, so the operand reads of 16
//     rows cover all 64 banks; one barrier per pair of steps;
//   - wave tt < 4 multiplies token tile tt: four 16x16x32 MFMAs per step, MFMA
//     c taking k 32q + 8c .. + 7 of both operands in lane (row or token i, q)
//     (the same permutation of the step's 128 k in A and B).
// At the end of a segment the wave writes its tile's outputs, or, for a cut
// tile, its fp32 partial (device-coherent), and counts itself in on the
// (tile, token tile) counter; the second of the two finishes the tile:
// segment 0's sum plus segment 1's, each in step order (and per MFMA c, summed
// in c order), so the result does not depend on which arrives last. It then
// clears the counter.
// k_latent<1> first normalises the expert sums into the workspace rows
// [en | shared_h] (workgroup t for token t) behind a grid barrier.

// Row i's first bf16 of step ks of row tile rt (plus 32 q); wa, wb, wc: the
// weight pointers of LatArgs, passed as values (a choice between members of
// the argument struct by address would keep the struct in scratch memory and
// put a scratch load, and a wait for every load in flight, before each load).
__device__ __forceinline__ const uint16_t *sk_src(const LatPlan &pl, const uint16_t *wa, const uint16_t *wb,
                                                  const uint16_t *wc, int rt, int ks, int i, int q) {
  const long r = (long)rt * 16 + i;
  const int kq = q * 32;
  if (!pl.out) {
    // pair tile p: rows i < 8 are shared_gate row 8 p + i, rows i >= 8 shared_up row 8 p + i - 8
    const long sr = 8L * (rt - pl.ntile0) + (i & 7);
    const uint16_t *row = rt < pl.ntile0 ? wa + r * pl.h : (i < 8 ? wb : wc) + sr * pl.h;
    return row + ks * kStepK + kq;
  }
  return ks < pl.KS0 ? wa + r * pl.lh + ks * kStepK + kq : wb + r * pl.S + (ks - pl.KS0) * kStepK + kq;
}

// A run's items in processing order: entry 0 the last tile's head [0, ks_end)
// when that tile is cut, entry 1 the first tile's tail [ks_lo, KS) when that
// one is, entry 2 the whole tiles between, so that a cut tile's partial is
// stored early and both segments' counts and the sum come off the run's end.
// (A run spans at least one tile's steps, so a run within one tile is that
// whole tile.) The run's bounds are passed as values: choosing between
// variables by reference would keep them in scratch memory.
struct SkCursor {
  int e, rt, r1, ks, k0, k1;  // entry, tile, the entry's last tile, step, the tile's first step and end
};
// the first item of entry e, or of the first non-empty entry after it
__device__ __forceinline__ SkCursor sk_entry(int e, int rt_lo, int ks_lo, int rt_hi, int ks_end, int KS) {
  const int cut_first = ks_lo > 0, cut_last = rt_hi != rt_lo && ks_end < KS;
  if (e == 0 && cut_last) return SkCursor{0, rt_hi, rt_hi, 0, 0, ks_end};
  if (e <= 1 && cut_first) return SkCursor{1, rt_lo, rt_lo, ks_lo, ks_lo, KS};
  if (e <= 2 && rt_lo + cut_first <= rt_hi - cut_last) return SkCursor{2, rt_lo + cut_first, rt_hi - cut_last, 0, 0, KS};
  return SkCursor{3, 0, 0, 0, 0, KS};  // past the run (its loads read the zero area)
}
__device__ __forceinline__ void sk_next(SkCursor &c, int rt_lo, int ks_lo, int rt_hi, int ks_end, int KS) {
  if (++c.ks < c.k1) return;
  if (c.rt < c.r1) {  // entry 2's next whole tile
    ++c.rt;
    c.ks = 0;
  } else if (c.e < 3) {
    c = sk_entry(c.e + 1, rt_lo, ks_lo, rt_hi, ks_end, KS);
  }
}

template <int OUT>
__global__ __launch_bounds__(kLatThreads, 1) void k_latent_sk(LatPlan pl_arg, LatArgs a_arg) {
  const uint64_t kargs = touch_kernargs<sizeof(LatPlan) + sizeof(LatArgs)>();
  const LatPlan pl = load_const<LatPlan>(kargs);
  const LatArgs a = lat_args(kargs + sizeof(LatPlan));
  (void)pl_arg;
  (void)a_arg;
  // kSkSlots x [64 tokens][256 B] activation steps, then kSkWSlots x [16 rows][256 B] weight steps
  extern __shared__ __attribute__((aligned(16))) char lds[];
  char *const wring = lds + kSkSlots * kSkSlotBytes;
  __shared__ float s_wsum[kLatWaves];

  const int tid = threadIdx.x, w = wave_id(), l = tid & 63;
  const int i = l & 15, q = l >> 4;
  const int B = pl.B, KS = pl.KS;
  const long NI = (long)pl.RT * KS;
  const long lo = NI * blockIdx.x / gridDim.x, hi = NI * (blockIdx.x + 1) / gridDim.x;
  const int n = (int)(hi - lo);  // this workgroup's steps
  const bool loader = w >= 4;
  const int tt = w & 3;          // compute wave: its token tile; loader: which quarter of the loads
  unsigned *ctl = reinterpret_cast<unsigned *>(a.ws);
  const uint16_t *zlane = reinterpret_cast<const uint16_t *>(a.ws + 4096 + l * 64);  // 64 zero bytes
  const int erow = pl.lh + pl.S;  // <1>: workspace row of a token, [en | shared_h]
  const int rt_lo = (int)(lo / KS), ks_lo = (int)(lo - (long)rt_lo * KS);  // the run's first item
  const int rt_hi = (int)((hi - 1) / KS), ks_end = (int)(hi - 1 - (long)rt_hi * KS) + 1;  // its last, + 1
  auto cur_from = [&](int e) __attribute__((always_inline)) { return sk_entry(e, rt_lo, ks_lo, rt_hi, ks_end, KS); };
  auto cur_next = [&](SkCursor &c) __attribute__((always_inline)) { sk_next(c, rt_lo, ks_lo, rt_hi, ks_end, KS); };
  // Waves 4-5 load the weights (two loads of 4 rows, 1 KiB, per step each) from
  // the kernel's start, ahead of the <1> normalisation's grid barrier.
  const int lw = w & 1;
  const uint16_t *const wa = a.wa, *const wb = a.wb, *const wc = a.wc;
  SkCursor wcur = cur_from(0);
  auto issue_w = [&](int s) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = 2 * lw + u;  // rows 4j .. 4j + 3
      const int r = 4 * j + (l >> 4), p = l & 15, c = p ^ r;
      const uint16_t *src = s < n ? sk_src(pl, wa, wb, wc, wcur.rt, wcur.ks, r, 0) + c * 8 : zlane;
      load_lds<16>(src, wring + (s % kSkWSlots) * kSkWSlotBytes + j * 1024);
    }
    cur_next(wcur);
  };
  const bool wl = w == 4 || w == 5;
  if (wl)
    for (int s = 0; s < 2 * kSkWPairs; ++s) issue_w(s);

  if (OUT) {
    BarrierBase bb{0u, 0u, 0u};
    if (tid == 0) bb = barrier_base(ctl);
    if ((int)blockIdx.x < B) {  // token t's [en | shared_h] row (as k_latent<1> for larger batches)
      const int t = blockIdx.x;
      // the row's first kHeld float pairs per thread (and their norm weights)
      // stay in registers between the two passes; sums in ascending k as ever
      constexpr int kHeld = 4;
      float2 vh[kHeld];
      uint32_t wh[kHeld];
#pragma unroll
      for (int j = 0; j < kHeld; ++j) {
        const int k = 2 * tid + j * 2 * kLatThreads;
        vh[j] = k < pl.lh ? *reinterpret_cast<const float2 *>(a.esum + (long)t * pl.lh + k) : float2{0.f, 0.f};
        wh[j] = k < pl.lh ? *reinterpret_cast<const uint32_t *>(a.norm + k) : 0u;
      }
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < kHeld; ++j) {
        if (2 * tid + j * 2 * kLatThreads >= pl.lh) break;
        const float e0 = round_bf16(vh[j].x), e1 = round_bf16(vh[j].y);
        ss += e0 * e0;
        ss += e1 * e1;
      }
      for (int k = 2 * tid + kHeld * 2 * kLatThreads; k < pl.lh; k += 2 * kLatThreads) {
        const float2 v = *reinterpret_cast<const float2 *>(a.esum + (long)t * pl.lh + k);
        const float e0 = round_bf16(v.x), e1 = round_bf16(v.y);
        ss += e0 * e0;
        ss += e1 * e1;
      }
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) ss += shfl_xor(ss, m);
      if (l == 0) s_wsum[w] = ss;
      __syncthreads();
      float tot = s_wsum[0];
#pragma unroll
      for (int v = 1; v < kLatWaves; ++v) tot += s_wsum[v];
      const float r = 1.0f / __fsqrt_rn(tot / (float)pl.lh + kLatRmsEps);
      const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.ws + pl.o_en, (uint32_t)(B * erow * 2));
      auto put = [&](int k, float2 v, uint32_t wn) __attribute__((always_inline)) {
        const float n0 = round_bf16(round_bf16(v.x) * r), n1 = round_bf16(round_bf16(v.y) * r);
        const uint32_t o0 = f32_to_bf16_bits(n0 * bf16_bits_to_f32(wn & 0xFFFFu));
        const uint32_t o1 = f32_to_bf16_bits(n1 * bf16_bits_to_f32(wn >> 16));
        st_dev32(rw, (uint32_t)(((long)t * erow + k) * 2), o0 | (o1 << 16));
      };
#pragma unroll
      for (int j = 0; j < kHeld; ++j) {
        const int k = 2 * tid + j * 2 * kLatThreads;
        if (k < pl.lh) put(k, vh[j], wh[j]);
      }
      for (int k = 2 * tid + kHeld * 2 * kLatThreads; k < pl.lh; k += 2 * kLatThreads)
        put(k, *reinterpret_cast<const float2 *>(a.esum + (long)t * pl.lh + k), *reinterpret_cast<const uint32_t *>(a.norm + k));
      for (int k = 2 * tid; k < pl.S; k += 2 * kLatThreads)
        st_dev32(rw, (uint32_t)(((long)t * erow + pl.lh + k) * 2),
                 *reinterpret_cast<const uint32_t *>(a.x + (long)t * pl.S + k));
    }
    // (no acquire: the rows are read with device-coherent loads)
    if (!grid_barrier(ctl, bb, 1, nullptr, false)) {  // a wait of this launch gave up: the rows are incomplete
      poison_share<true>(a.ya, (long)B * pl.h);
      return;
    }
  }

  if (loader) {
    // Waves 4-5 load the weights, waves 6-7 the activations (eight loads of 4
    // token rows each; rows past the batch from the zero area): loads complete
    // in issue order within a wave, so the weight stream, further ahead, does
    // not hold up the activation loads. Past the run the loads read the zero
    // area, so that every step issues the same number. A slot is free at the
    // barrier after its last reader (the pair of steps a ring's length before).
    SkCursor cur = cur_from(0);
    auto issue_a = [&](int s) __attribute__((always_inline)) {
      const int ks = cur.ks;
      cur_next(cur);
      char *slot = lds + (s % kSkSlots) * kSkSlotBytes;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int g = lw + 2 * u;             // token group: tokens 4g .. 4g + 3
        const int t = 4 * g + (l >> 4), p = l & 15;
        const int c = p ^ (t & 15);           // the global 16-byte chunk landing at position p
        const uint16_t *src = (t >= B || s >= n) ? zlane
                              : !OUT ? a.x + (long)t * pl.h + ks * kStepK + c * 8
                                     : reinterpret_cast<const uint16_t *>(a.ws + pl.o_en) + (long)t * erow + ks * kStepK + c * 8;
        load_lds<16, OUT ? kCpolDevice : 0>(src, slot + g * 1024);  // one instruction for all lanes
      }
    };
    // at the barrier of pair p its loads have landed: what may be outstanding
    // is what this wave issued after them (the later pairs' loads)
    const int np = (n + 1) / 2;
    if (wl) {  // (the first 2 kSkWPairs steps issued at the start)
      for (int p = 0; p < np; ++p) {
        wait_vm<4 * (kSkWPairs - 1)>();
        ring_barrier();
        issue_w(2 * (p + kSkWPairs));
        issue_w(2 * (p + kSkWPairs) + 1);
      }
    } else {
      for (int s = 0; s < 2 * kSkAPairs; ++s) issue_a(s);
      for (int p = 0; p < np; ++p) {
        wait_vm<16 * (kSkAPairs - 1)>();
        ring_barrier();
        issue_a(2 * (p + kSkAPairs));
        issue_a(2 * (p + kSkAPairs) + 1);
      }
    }
    wait_vm<0>();  // no load lands after the workgroup is done
    return;
  }

  // compute wave tt: token tile tt, token 16 tt + i (B operand lane (i, q))
  const bool active = tt < pl.TT;
  const int parts = OUT ? 2 : 1;
  const __amdgpu_buffer_rsrc_t rpart = make_rsrc(a.ws + pl.o_part0, (uint32_t)((long)pl.RT * 2 * parts * 4 * 1024));
  unsigned *cnt = reinterpret_cast<unsigned *>(a.ws + pl.o_cnt) + kSkCntWord;
  const int tok = 16 * tt + i;
  // four accumulators per part (MFMA c of every step), so that a step's four
  // MFMAs do not wait for each other; summed in c order at the segment's end
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  f32x4 c0[4], c1[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) c0[c] = c1[c] = f32x4{0.f, 0.f, 0.f, 0.f};

  // the outputs of row tile rt for this token tile from the finished sums
  auto write_out = [&](int rt, const f32x4 &s0, const f32x4 &s1) __attribute__((always_inline)) {
    // lane (token i, q): rows 4q .. 4q + 3 of the tile
    if (OUT) {
      uint32_t o[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) o[v] = f32_to_bf16_bits(round_bf16(s0[v]) + round_bf16(s1[v]));
      if (tok < B)
        *reinterpret_cast<u32x2 *>(a.ya + (long)tok * pl.h + rt * 16 + 4 * q) = u32x2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
    } else if (rt < pl.ntile0) {
      uint32_t o[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) o[v] = f32_to_bf16_bits(s0[v]);
      if (tok < B)
        *reinterpret_cast<u32x2 *>(a.ya + (long)tok * pl.lh + rt * 16 + 4 * q) = u32x2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
    } else {
      // pair tile: rows 0-7 shared_gate, rows 8-15 the same shared_up rows; lane
      // q < 2 holds gate rows 4q .., lane q + 2 (lane + 32) the matching up rows
      f32x4 up;
#pragma unroll
      for (int v = 0; v < 4; ++v) up[v] = shfl_xor(s0[v], 32);
      uint32_t o[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) o[v] = f32_to_bf16_bits(apply_act(pl.act, round_bf16(s0[v]), round_bf16(up[v])));
      if (q < 2 && tok < B)
        *reinterpret_cast<u32x2 *>(a.yb + (long)tok * pl.S + (rt - pl.ntile0) * 8 + 4 * q) =
            u32x2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
    }
  };
  auto part_off = [&](int rt, int seg, int p) __attribute__((always_inline)) {
    return (uint32_t)((((((long)rt * 2 + seg) * parts + p) * 4 + tt) * 256 + l * 4) * 4);
  };
  // parts with steps in [k_a, k_b) (<1>: part 0 below KS0, part 1 from it)
  auto has0 = [&](int k_a) __attribute__((always_inline)) { return !OUT || k_a < pl.KS0; };
  auto has1 = [&](int k_b) __attribute__((always_inline)) { return OUT && k_b > pl.KS0; };
  // A cut tile's segment stores its fp32 partial; kLagStore steps later (the
  // stores done by then) it counts itself in on the (tile, token tile) counter;
  // kLag steps after that the count's answer is back, and the second of the
  // tile's two counts loads both segments' partials, which
  // kLagLoad steps later still it sums (segment 0 + segment 1) into the
  // outputs, then clears the counter: the round trips overlap the step stream.
  // Cut tiles come first in a run, so a wave holds at most two, in slots ca and
  // cb. (A compute wave's only loads are these, so waiting for the stores waits
  // for nothing else.)
  constexpr int kLagStore = 8, kLag = 8, kLagLoad = 8;
  struct CutSlot {
    int st;        // 0 unused, 1 partial stored, 2 counted, 3 partials loading, 4 done
    int rt, kc;    // the tile; segment 0 holds steps [0, kc), segment 1 [kc, KS)
    int at;        // the first step at which the next stage may run
    unsigned old;  // the count's answer (lane 0)
    f32x4 s0, s1, t0, t1;
  };
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  CutSlot ca{0, 0, 0, 0, 0u, z4, z4, z4, z4}, cb{0, 0, 0, 0, 0u, z4, z4, z4, z4};
  int count_at = 0;
  auto finish = [&](int rt, int k_a, int k_b, int s) __attribute__((always_inline)) {
    if (k_a == 0 && k_b == KS) {
      write_out(rt, acc0, acc1);
      return;
    }
    const int seg = k_a == 0 ? 0 : 1;
    if (has0(k_a)) st_dev128(rpart, part_off(rt, seg, 0), __builtin_bit_cast(u32x4, acc0));
    if (has1(k_b)) st_dev128(rpart, part_off(rt, seg, 1), __builtin_bit_cast(u32x4, acc1));
    if (ca.st == 0) {
      ca.st = 1;
      ca.rt = rt;
      ca.kc = seg ? k_a : k_b;
    } else {
      cb.st = 1;
      cb.rt = rt;
      cb.kc = seg ? k_a : k_b;
    }
    count_at = s + kLagStore;
  };
  auto count_in = [&](int s) __attribute__((always_inline)) {
    wait_vmem();  // the partials are stored before the counts
    if (ca.st == 1) {
      if (l == 0) ca.old = __hip_atomic_fetch_add(cnt + ca.rt * 4 + tt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ca.st = 2;
      ca.at = s + kLag;
    }
    if (cb.st == 1) {
      if (l == 0) cb.old = __hip_atomic_fetch_add(cnt + cb.rt * 4 + tt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      cb.st = 2;
      cb.at = s + kLag;
    }
  };
  // the next stage of slot c: the answer (first count: done, the other
  // segment's wave finishes the tile), or the sum of the loaded partials
  auto advance = [&](CutSlot &c, int s) __attribute__((always_inline)) {
    if (c.st == 2) {
      if (__builtin_amdgcn_readfirstlane(c.old) == 0u) {
        c.st = 4;
        return;
      }
      // no acquire fence: the partials are read with device-coherent loads,
      // issued after the answer showed the other segment's count, whose
      // device-coherent stores had completed before it counted (an agent-scope
      // acquire would invalidate the XCD's L2, several us mid-stream)
      if (has0(0)) c.s0 = __builtin_bit_cast(f32x4, bload16_dev(rpart, part_off(c.rt, 0, 0)));
      if (has1(c.kc)) c.s1 = __builtin_bit_cast(f32x4, bload16_dev(rpart, part_off(c.rt, 0, 1)));
      if (has0(c.kc)) c.t0 = __builtin_bit_cast(f32x4, bload16_dev(rpart, part_off(c.rt, 1, 0)));
      if (has1(KS)) c.t1 = __builtin_bit_cast(f32x4, bload16_dev(rpart, part_off(c.rt, 1, 1)));
      c.st = 3;
      c.at = s + kLagLoad;
      return;
    }
    f32x4 s0 = c.s0, s1 = c.s1;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      s0[v] += c.t0[v];
      s1[v] += c.t1[v];
    }
    write_out(c.rt, s0, s1);
    if (l == 0) __hip_atomic_store(cnt + c.rt * 4 + tt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    c.st = 4;
  };

  // operand reads: row (weight row i, or token tok) of a slot, the 16-byte
  // chunk 4q + c at its swizzled position
  const int bq = tok * 256;
  SkCursor cc = cur_from(0);  // the current item
  for (int s2 = 0; s2 < n; s2 += 2) {
    ring_barrier();  // the loaders' steps s2, s2 + 1 have landed
    if (active) {
      if ((ca.st == 1 || cb.st == 1) && s2 >= count_at) count_in(s2);
      if ((ca.st == 2 || ca.st == 3) && s2 >= ca.at) advance(ca, s2);
      if ((cb.st == 2 || cb.st == 3) && s2 >= cb.at) advance(cb, s2);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int s = s2 + h;
      if (s >= n) break;
      const char *aslot = lds + (s % kSkSlots) * kSkSlotBytes;
      const char *wslot = wring + (s % kSkWSlots) * kSkWSlotBytes;
      const int rt = cc.rt, ks = cc.ks, k0 = cc.k0, k1 = cc.k1;
      cur_next(cc);
      if (active) {
        u32x4 av[4], bv[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          av[c] = *reinterpret_cast<const u32x4 *>(wslot + i * 256 + (((4 * q + c) ^ i) * 16));
          bv[c] = *reinterpret_cast<const u32x4 *>(aslot + bq + (((4 * q + c) ^ i) * 16));
        }
        if (OUT && ks >= pl.KS0) {
#pragma unroll
          for (int c = 0; c < 4; ++c) c1[c] = mfma16(as_bf16x8(av[c]), as_bf16x8(bv[c]), c1[c]);
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c) c0[c] = mfma16(as_bf16x8(av[c]), as_bf16x8(bv[c]), c0[c]);
        }
      }
      if (ks + 1 == k1) {  // the tile's segment ends here
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          acc0[v] = ((c0[0][v] + c0[1][v]) + c0[2][v]) + c0[3][v];
          acc1[v] = ((c1[0][v] + c1[1][v]) + c1[2][v]) + c1[3][v];
        }
        if (active) finish(rt, k0, k1, s);
#pragma unroll
        for (int c = 0; c < 4; ++c) c0[c] = c1[c] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  }
  if (!active) return;
  // what the run's end left: both slots' loads first, then the sums
  if (ca.st == 1 || cb.st == 1) count_in(n);
  if (ca.st == 2) advance(ca, n);
  if (cb.st == 2) advance(cb, n);
  if (ca.st == 3) advance(ca, n);
  if (cb.st == 3) advance(cb, n);
}

}  // namespace k3moe
