// Single-token MoE step: the whole step for one token (the decode batch of 1)
// in one persistent launch with no grid barrier.
//
// Workgroups hand data to each other through tagged 8-byte slots {payload,
// tag} in the workspace's tag area. The tag numbers the launch, so a reader
// polls the data itself until every slot it needs carries this launch's tag:
// one memory round trip after the last write, where a grid barrier costs its
// counter round trips and then a separate gather.
//
//   R   router logits (kimi.py:308): unit = (16 router rows, k-split s) as in
//       the general persistent kernel; each (expert, split) partial goes to
//       its tagged slot.
//   T   every workgroup polls the partials of the experts its threads hold
//       (thread e: expert e), sums them in split order, gates them (sigmoid
//       + bias, or the logits; kimi.py:308-315, tasks/distributed.py:174-176)
//       and selects the top k (k <= 8) with the workgroup's threshold-and-rank
//       selection (block_topk);
//       valid forced routes replace the selection (kimi.py:311-313).
//   GU  gate/up (kimi.py:321-322): the k x I/8 units (8 gate + 8 up rows of
//       one chosen expert) go to the workgroups in turn (exactly one each at
//       top-8, I = 256 on a grid of 256); the 8 waves split the unit's K
//       evenly and issue all their weight loads as soon as the ids are known;
//       the waves' partial tiles meet in LDS in wave order, the activation is
//       applied, and the unit's 8 bf16 h values go to tagged slots.
//   DN  down and combine (kimi.py:322-323): wave j takes the j-th chosen
//       expert (ascending ids) in the workgroup's one or two 16-row output
//       tiles; its weights are loaded once the gate/up data has arrived (they
//       then arrive while h is exchanged), it polls the expert's h,
//       multiplies, and the waves' w x bf16(y) rows are summed in LDS from zero
//       in ascending expert order.
// Each workgroup adds one to a launch counter when it leaves, on every path;
// the counters' sum at a launch's start, over the grid size, numbers the
// launch, and its tag is that number + 1 (a zeroed slot never matches).
// Every wait is bounded: a workgroup that gives up sets the status word,
// leaves NaN in its share of the output and leaves.
#pragma once

#include "k3moe_barrier.hpp"
#include "k3moe_decode.hpp"
#include "k3moe_device.hpp"
#include "k3moe_plan.hpp"

namespace k3moe {

constexpr int kTagPartials = 0;  // tag area: router partials, [E][8 splits] slots
constexpr uint32_t kTraceSingle = 0x5349u;  // trace slot 55 of the single-token kernel's rows

// Fixed LDS scratch of the single-token kernel, after the keys and the staged row.
struct SingleScratch {
  int sel[kDecWaves * kMaxTopk];         // selection output (sel[0..k) in rank order)
  float rred[kDecWaves * 16];            // router: the waves' 16 partial logits
  float gred[kDecWaves * 16];            // gate/up: the waves' 16 partial rows
  uint16_t hs[8 * 256];                  // down: each chosen expert's h (bf16)
  float dacc[2 * kDecWaves * 16];        // down: w x bf16(y) per row tile, wave, row
  int ids[8];                            // chosen experts, ascending
  float wts[8];                          // their gating weights
};
static_assert(sizeof(SingleScratch) <= 8192, "single_lds reserves 8 KiB of scratch");
static_assert(sizeof(SingleScratch) % 16 == 0 && sizeof(BlockTopk) <= kBlockTopkBytes, "single_lds layout");

// Polls tagged slots until every lane's `n` slots (n in 0..2, read as one
// 16-byte device-coherent load at byte offset `off` of `r`) carry `tag`;
// wave-uniform. Returns false when the wait gave up (a timeout, which it
// records, or another wait of this launch that gave up).
__device__ __forceinline__ bool poll_tagged(__amdgpu_buffer_rsrc_t r, uint32_t off, int n, uint32_t tag,
                                            unsigned *ctl, unsigned abort0, u32x4 &v) {
  unsigned spins = 0;
  for (;;) {
    v = n > 0 ? bload16_dev(r, off) : u32x4{0, 0, 0, 0};
    const bool ok = (n < 1 || v[1] == tag) && (n < 2 || v[3] == tag);
    if (__ballot(!ok) == 0) return true;
    ++spins;
    if ((spins & 63u) == 0u && aborted(ctl, abort0)) return false;
    if (spins > kSpinLimit) {
      if ((threadIdx.x & 63) == 0) raise_timeout(ctl);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

__global__ __launch_bounds__(kDecThreads, 1) void k_moe_single(Plan pl_arg, DecodeArgs a_arg) {
  const uint64_t kargs = touch_kernargs<sizeof(Plan) + sizeof(DecodeArgs)>();
  const Plan pl = load_const<Plan>(kargs);
  const DecodeArgs a = load_args(kargs + sizeof(Plan));
  (void)pl_arg;
  (void)a_arg;
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int E = pl.E, k = pl.k, K = pl.K, I = pl.I;
  uint32_t *kyl = reinterpret_cast<uint32_t *>(lds);  // [E] ordered keys
  float *kyf = reinterpret_cast<float *>(kyl + E);    // [E] keys
  float *scl = kyf + E;                               // [E] scores
  uint16_t *xs = reinterpret_cast<uint16_t *>(lds + align16(12 * E));  // [K] the token's expert-input row
  SingleScratch &sh = *reinterpret_cast<SingleScratch *>(lds + align16(12 * E) + 2 * K);
  BlockTopk &tk = *reinterpret_cast<BlockTopk *>(lds + align16(12 * E) + 2 * K + sizeof(SingleScratch));
  __shared__ uint32_t s_tag, s_abort0;
  __shared__ int s_fail;

  const int tid = threadIdx.x, w = wave_id(), l = tid & 63, i = l & 15, q = l >> 4;
  unsigned *ctl = reinterpret_cast<unsigned *>(a.ws + pl.o_ctl);
  char *tag_area = a.ws + kOffTag;
  const __amdgpu_buffer_rsrc_t tagr = make_rsrc(tag_area, kTagBytes);
  // tag area: the router partials, kTagCopies copies of [8 splits][E] slots
  // (split-major: one poll instruction reads 64 consecutive experts' slots of a
  // split; workgroup b polls copy b mod 8, the copy of its XCD: fewer readers
  // per line), then the h slots, [k][I/2]
  const uint32_t copy_bytes = (uint32_t)E * kDecMaxSplits * 8;
  const uint32_t my_copy = (blockIdx.x % kTagCopies) * copy_bytes;
  const uint32_t h_base = kTagCopies * copy_bytes;
  const uint8_t *zero = reinterpret_cast<const uint8_t *>(a.ws + pl.o_zero);
  trace_mark(pl, a.ws, 0);

  // Leaves the kernel: NaN in this workgroup's share of the output when a wait
  // gave up, and this workgroup's count on its launch counter (every path).
  auto leave = [&](bool gave_up) {
    if (gave_up) poison_share<false>(a.out, (long)K);
    if (tid == 0)
      __hip_atomic_fetch_add(ctl + kCtlEpoch + (blockIdx.x % kEpochCounters) * kCtlEpochStride, 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  };

  // wave 0: the launch counters and the abort counter (lanes 0-15, 16), first
  uint32_t cnt = 0u;
  if (w == 0 && l <= kEpochCounters)
    cnt = __hip_atomic_load(l < kEpochCounters ? ctl + kCtlEpoch + l * kCtlEpochStride : ctl + kCtlAbort,
                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // the token's expert-input row (two 16-byte chunks per thread), the gating
  // bias of experts tid and tid + 512: both needed later, loaded now
  u32x4 xpre[2] = {u32x4{0, 0, 0, 0}, u32x4{0, 0, 0, 0}};
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int c = hh * kDecThreads + tid;
    if (c < K / 8) xpre[hh] = load16(a.xin + c * 8);
  }
  float bias_pre[2] = {0.f, 0.f};
  if (a.bias) {
    if (tid < E) bias_pre[0] = a.bias[tid];
    if (tid + kDecThreads < E) bias_pre[1] = a.bias[tid + kDecThreads];
  }
  bool tagged = false;
  auto make_tag = [&]() {  // wave 0, once: tag = launches so far + 1
    if (tagged || w != 0) return;
    tagged = true;
    uint32_t sum = 0u;
#pragma unroll
    for (int g = 0; g < kEpochCounters; ++g) sum += lane_u32(cnt, g);
    if (l == 0) {
      s_tag = (sum >> __builtin_ctz(gridDim.x)) + 1u;
      s_abort0 = lane_u32(cnt, kEpochCounters);
      s_fail = 0;
    }
  };

  // Code warm-up (as in the general persistent kernel): each workgroup loads a
  // slice of the code range the previous launch recorded, so that later
  // phases' instruction fetches hit L2; issued after the router's loads.
  uint64_t *crange = reinterpret_cast<uint64_t *>(ctl + kCtlCodeSingle);
  const uint64_t pc0 = program_counter();
  u32x4 code_probe = {0, 0, 0, 0};
  bool warm = false;
  auto warm_code = [&]() {
    if (warm) return;
    warm = true;
    const uint64_t c0 = crange[0], c1 = crange[1];
    if (c0 == pc0 && c1 > pc0 && c1 - pc0 < (1u << 20)) {
      const uint64_t lo = pc0 & ~(uint64_t)1023;
      const uint64_t addr = lo + (uint64_t)((blockIdx.x >> 3) + 32 * w) * 1024 + l * 16;
      const uint64_t at = addr + 16 <= c1 ? addr : (pc0 & ~(uint64_t)15);  // unconditional (see k_moe_decode)
      code_probe = *reinterpret_cast<const __attribute__((address_space(1))) u32x4 *>(at);
    }
  };

  // ------------------------------------------------------------ R: router --
  {
    const int NU = pl.RTr * pl.Srw, KB = pl.h / kBlockK;
    for (int u = blockIdx.x; u < NU; u += gridDim.x) {
      const int s = u % pl.Srw, rt = u / pl.Srw;
      const int k0 = (int)((unsigned)(s * pl.KSr) / (unsigned)pl.Srw);
      const int k1 = (int)((unsigned)((s + 1) * pl.KSr) / (unsigned)pl.Srw);
      const int ka = k0 + (k1 - k0) * w / kDecWaves, kb1 = k0 + (k1 - k0) * (w + 1) / kDecWaves;
      const int row = rt * 16 + i;
      const bool row_ok = row < E;
      const uint16_t *arow = a.router + (size_t)(row_ok ? row : 0) * pl.h;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      for (int ks = ka; ks < kb1; ++ks) {
        const int kb = ks * 4 + q;
        const bool ok = kb < KB;
        u32x4 va[4], vb[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          va[kk] = (ok && row_ok) ? load16(arow + kb * kBlockK + kk * 8) : u32x4{0, 0, 0, 0};
          vb[kk] = (ok && i == 0) ? load16(a.x + kb * kBlockK + kk * 8) : u32x4{0, 0, 0, 0};
        }
        warm_code();
        make_tag();
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) acc = mfma16(as_bf16x8(va[kk]), as_bf16x8(vb[kk]), acc);
      }
      make_tag();
      if (i == 0) {  // column 0 (the token): rows 4q .. 4q + 3
#pragma unroll
        for (int v = 0; v < 4; ++v) sh.rred[w * 16 + 4 * q + v] = acc[v];
      }
      __syncthreads();
      if (tid < 16 * kTagCopies && rt * 16 + (tid & 15) < E) {
        // the split's partial of expert rt * 16 + (tid & 15), waves in order, into copy tid / 16
        const int r = tid & 15;
        float sum = sh.rred[r];
#pragma unroll
        for (int ww = 1; ww < kDecWaves; ++ww) sum += sh.rred[ww * 16 + r];
        st_dev64(tagr, (uint32_t)(kTagPartials + (tid >> 4) * copy_bytes + (s * E + rt * 16 + r) * 8),
                 u32x2{__float_as_uint(sum), s_tag});
      }
      __syncthreads();
    }
  }
  warm_code();
  make_tag();
  trace_mark(pl, a.ws, 1);
  // the staged row for gate/up (its loads have long arrived)
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int c = hh * kDecThreads + tid;
    if (c < K / 8) *reinterpret_cast<u32x4 *>(xs + c * 8) = xpre[hh];
  }
  __syncthreads();  // s_tag, s_abort0, the staged row
  asm volatile("" ::"v"(code_probe));
  const uint32_t tag = s_tag, abort0 = s_abort0;

  // -------------------------------------------------------- T: top-k/gating --
  int w0_rank = 0, w0_e = -1;  // wave 0, lane l < k: the l-th chosen expert and its ascending rank
  {
    // thread e polls expert e's partials (splits 0 .. Srw - 1, slot s E + e of
    // its copy), every split's 8-byte load per round, then sums them in split order
    float logit = 0.f;
    bool ok = true;
    {
      const int ns = tid < E ? pl.Srw : 0;
      u32x2 v[kDecMaxSplits];
      unsigned spins = 0;
      for (;;) {
        bool ready = true;
#pragma unroll
        for (int sp = 0; sp < kDecMaxSplits; ++sp)
          v[sp] = sp < ns ? bload8_dev(tagr, (uint32_t)(kTagPartials + my_copy + (sp * E + tid) * 8)) : u32x2{0, 0};
#pragma unroll
        for (int sp = 0; sp < kDecMaxSplits; ++sp) ready = ready && (sp >= ns || v[sp][1] == tag);
        if (spins == 0 && w == 0) trace_mark(pl, a.ws, 10);
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
#pragma unroll
      for (int sp = 0; sp < kDecMaxSplits; ++sp)
        if (sp < ns) logit = sp == 0 ? __uint_as_float(v[0][0]) : logit + __uint_as_float(v[sp][0]);
      if (pl.o_trace && tid == 0)
        reinterpret_cast<uint64_t *>(a.ws + pl.o_trace)[blockIdx.x * kTraceSlots + 11] = spins + 1;
    }
    if (!ok) s_fail = 1;
    trace_mark(pl, a.ws, 2);
    if (tid < E) {  // gating (kimi.py:308-309; tasks/distributed.py:174)
      float score, key;
      if (pl.gating == K3MOE_GATING_SIGMOID_BIAS) {
        score = 1.0f / (1.0f + expf(-logit));
        key = a.bias ? __fadd_rn(score, bias_pre[0]) : score;
      } else {
        score = logit;
        key = logit;
      }
      scl[tid] = score;
      kyf[tid] = key;
      kyl[tid] = ordered_key(key);
    }
    __syncthreads();
    if (s_fail) return leave(true);
    trace_mark(pl, a.ws, 3);
    // the workgroup's top-k: a threshold from group maxima, then exact ranks among the candidates
    block_topk(kyl, E, k, sh.sel, tk);
    trace_mark(pl, a.ws, 4);
    if (w == 0) {
      // forced routes replace the selection when the row is valid (kimi.py:311-313)
      int fid = 0;
      const bool forced = a.routes && forced_route(a.routes, 0, k, E, &fid);
      if (a.routes && !forced && l == 0 && blockIdx.x == 0)
        __hip_atomic_fetch_or(ctl + kCtlErr, (unsigned)kErrRoutes, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int my_e = l < k ? (forced ? fid : sh.sel[l]) : -1;
      int rank = 0;
      for (int r = 0; r < k; ++r) rank += ((int)lane_u32((uint32_t)my_e, r) < my_e) ? 1 : 0;
      if (l < k) sh.ids[rank] = my_e;
      w0_rank = rank;  // kept in registers for the weights, after the loads are issued
      w0_e = my_e;
    }
    __syncthreads();
  }
  trace_mark(pl, a.ws, 5);

  // ------------------------------------------------------------- GU issue --
  // gate/up unit u: chosen expert j = u / U8 (ascending ids), rows 8 rg .. 8 rg + 7
  // of gate (lanes i < 8) and of up (lanes i >= 8). The rows' K / 512
  // super-steps of 16 MXFP4 blocks are shared out over the 8 waves (at most
  // kSingleMaxSS each: the CU's bytes in flight, not one wave's, set the
  // time). Per super-step a lane loads blocks 16 ss + 4 t + q (t = 0..3; a wave
  // instruction covers 64 contiguous bytes of 16 rows) and the row's 16 scale
  // bytes in one 16-byte load, of which it uses byte 4 t + q of dword t.
  const int KB = K / kBlockK, NSS = KB / 16, U8 = pl.U8, NU = k * U8;
  const int ss0 = NSS * w / kDecWaves, ss1 = NSS * (w + 1) / kDecWaves;
  const uint8_t *const lane_blk = i >= 8 ? a.ublk : a.gblk;
  const uint8_t *const lane_scl = i >= 8 ? a.uscl : a.gscl;
  u32x4 ga[kSingleMaxSS][4], gsc[kSingleMaxSS];
  auto gu_issue1 = [&](int u) {
    const int j = u / U8, rg = u % U8;
    const size_t row = (size_t)sh.ids[j] * I + rg * 8 + (i & 7);
    const uint8_t *wr = lane_blk + row * KB * 16, *sr = lane_scl + row * KB;
#pragma unroll
    for (int m = 0; m < kSingleMaxSS; ++m) {
      if (ss0 + m < ss1) {
        const int ss = ss0 + m;
#pragma unroll
        for (int t = 0; t < 4; ++t) ga[m][t] = load16(wr + (16 * ss + 4 * t + q) * 16);
        gsc[m] = load16(sr + 16 * ss);
      }
    }
  };
  int u0 = blockIdx.x;
  if (u0 < NU) gu_issue1(u0);
  trace_mark(pl, a.ws, 9);

  if (w == 0) {
    // the gating weights, while the loads are in flight; the down phase reads
    // them after the gate/up phase's LDS barriers
    const int rank = w0_rank, my_e = w0_e;
    const float my_score = l < k ? scl[my_e] : 0.f, my_key = l < k ? kyf[my_e] : 0.f;
    {
      // weights in selection order (kimi.py:314-315; tasks/distributed.py:176)
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
      if (l < k) sh.wts[rank] = wt;
      if (blockIdx.x == 0) {
        if (l < k) {
          a.out_ids[rank] = my_e;
          a.out_w[rank] = wt;
        }
        if (a.routes && a.out_short) {  // kimi.py:313
          float mn = INFINITY;
          for (int r = 0; r < k; ++r) mn = fminf(mn, lane_f32(my_key, r));
          if (l == 0) a.out_short[0] = fmaxf(kyf[sh.sel[k - 1]] - mn, 0.f);
        }
      }
    }
  }

  // ----------------------------------------------------------- GU compute --
  // The down weights of this workgroup's row tiles (blockIdx.x, blockIdx.x + G)
  // for wave w's expert are issued once the gate/up data has arrived, so that
  // the gate/up stream has the memory system to itself; they arrive while h is
  // exchanged. A tile past the last reads the zero area.
  DnLoad pf[2];
  bool dn_issued = false;
  auto dn_issue = [&]() {
    if (dn_issued) return;
    dn_issued = true;
    if (w < k) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
        dn_issue_w(pl, a, zero, sh.ids, (int)blockIdx.x + tt * (int)gridDim.x, w, 0, I / kBlockK, pf[tt]);
    }
  };
  for (; u0 < NU; u0 += gridDim.x) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < kSingleMaxSS; ++m) {
      if (ss0 + m < ss1) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int kb = 16 * (ss0 + m) + 4 * t + q;
          bf16x8 av[4];
          convert_block_fast(ga[m][t], (gsc[m][t] >> (8 * q)) & 0xFFu, av);
#pragma unroll
          for (int kk = 0; kk < 4; ++kk)
            acc = mfma16(av[kk], as_bf16x8(*reinterpret_cast<const u32x4 *>(xs + kb * kBlockK + kk * 8)), acc);
        }
      }
    }
    if (u0 == (int)blockIdx.x) trace_mark(pl, a.ws, 12);
    if (i == 0) {  // column 0: rows 4q .. 4q + 3 (0-7 gate, 8-15 up)
#pragma unroll
      for (int v = 0; v < 4; ++v) sh.gred[w * 16 + 4 * q + v] = acc[v];
    }
    ring_barrier();  // every wave's gate/up data has arrived
    dn_issue();
    if (u0 == (int)blockIdx.x) trace_mark(pl, a.ws, 13);
    if (u0 + (int)gridDim.x < NU) gu_issue1(u0 + gridDim.x);  // the next unit's loads (grids smaller than k I / 8)
    if (w == 0) {
      // h = act(bf16(gate), bf16(up)) of the unit's 8 rows: lane r < 16 sums
      // row r over the waves in order (gate rows 0-7, up rows 8-15); the
      // activation's transcendental factors run in separate lanes (act_parts)
      // and lane r < 8 combines them in the reference's order
      const int r = l & 15;
      float v = sh.gred[r];
#pragma unroll
      for (int ww = 1; ww < kDecWaves; ++ww) v += sh.gred[ww * 16 + r];
      v = round_bf16(v);
      const float g = __shfl(v, l & 7, kWave), up = __shfl(v, 8 + (l & 7), kWave);
      const float hv = act_parts(pl.act, g, up);
      const uint32_t hb = f32_to_bf16_bits(hv);
      const uint32_t pair = hb | ((uint32_t)__shfl_down((int)hb, 1, kWave) << 16);
      const int j = u0 / U8, rg = u0 % U8;
      if (l < 8 && (l & 1) == 0)
        st_dev64(tagr, h_base + (uint32_t)((j * (I / 2) + rg * 4 + (l >> 1)) * 8), u32x2{pair, tag});
      if (u0 == (int)blockIdx.x) trace_mark(pl, a.ws, 14);
    }
    ring_barrier();  // gred is free again
  }
  dn_issue();    // a workgroup without a gate/up unit
  ring_barrier();  // wave 0's gating weights (sh.wts) are visible to the down phase
  trace_mark(pl, a.ws, 6);

  // ------------------------------------------------------- DN: down+combine --
  const int KBd = I / kBlockK;
  bool ok = true;
  if (w < k) {
    // expert w's h: lane l holds h values 4 l .. 4 l + 3 (slots 2 l, 2 l + 1)
    const int n = 4 * l < I ? 2 : 0;
    u32x4 v;
    ok = poll_tagged(tagr, h_base + (uint32_t)((w * (I / 2) + 2 * l) * 8), n, tag, ctl, abort0, v);
    if (n > 0) *reinterpret_cast<u32x2 *>(sh.hs + w * 256 + 4 * l) = u32x2{v[0], v[2]};
    wave_lds_order();
    if (w == 0) trace_mark(pl, a.ws, 7);
    // B operand: k-step jj covers blocks 4 jj + q of h (lane group q)
    u32x4 hb[kDnDepth][4];
#pragma unroll
    for (int jj = 0; jj < kDnDepth; ++jj) {
      const int kb = jj * 4 + q;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        hb[jj][kk] = kb < KBd ? *reinterpret_cast<const u32x4 *>(sh.hs + w * 256 + kb * kBlockK + kk * 8)
                              : u32x4{0, 0, 0, 0};
    }
    const float wt = sh.wts[w];
    // The down scale bytes are taken apart only here, after the h poll
    // (dn_scale): the compiler would otherwise convert them right where they
    // are loaded and wait there for the loads, which are meant to arrive
    // while h is exchanged.
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int jj = 0; jj < kDnDepth; ++jj) {
        if (jj >= pl.KSd) break;
        bf16x8 av[4];
        convert_block_fast(pf[tt].w[jj], dn_scale(pf[tt], jj), av);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) acc = mfma16(av[kk], as_bf16x8(hb[jj][kk]), acc);
      }
      if (i == 0) {  // column 0: rows 4q .. 4q + 3 of the tile
#pragma unroll
        for (int vv = 0; vv < 4; ++vv) sh.dacc[(tt * kDecWaves + w) * 16 + 4 * q + vv] = __fmul_rn(round_bf16(acc[vv]), wt);
      }
    }
  }
  if (!ok) s_fail = 1;
  __syncthreads();
  if (s_fail) return leave(true);
  if (tid < 32) {  // row tile blockIdx.x + tt G, row r: the chosen experts in ascending order, from zero
    const int tt = tid >> 4, r = tid & 15, rt = (int)blockIdx.x + tt * (int)gridDim.x;
    if (rt < pl.RTd) {
      float sum = 0.f;
      for (int j = 0; j < k; ++j) sum = __fadd_rn(sum, sh.dacc[(tt * kDecWaves + j) * 16 + r]);
      a.out[rt * 16 + r] = sum;
    }
  }
  trace_mark(pl, a.ws, 8);
  if (pl.o_trace && tid == 0)
    reinterpret_cast<uint64_t *>(a.ws + pl.o_trace)[blockIdx.x * kTraceSlots + 55] = kTraceSingle;
  if (blockIdx.x == 0 && tid == 0) {  // this kernel's code range, for the next launch's warm-up
    crange[0] = pc0;
    crange[1] = program_counter();
  }
  leave(false);
}

}  // namespace k3moe
