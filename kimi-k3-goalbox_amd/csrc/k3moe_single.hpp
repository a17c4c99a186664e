// Single-token MoE step: the whole step for one token (the decode batch of 1)
// in one persistent launch with no grid barrier.
//
// Workgroups hand data to each other through tagged 8-byte slots {payload,
// tag} in the workspace's tag area. The tag numbers the launch, so a reader
// polls the data itself until every slot it needs carries this launch's tag:
// one memory round trip after the last write, where a grid barrier costs its
// counter round trips and then a separate gather.
//
//   R   router logits (kimi.py:308): workgroup b computes the whole logits
//       of experts b, b + G, .. (at most 4 rows, FP32 sums of the bf16
//       products); each goes to its tagged slot, one copy per XCD.
//   T   every workgroup polls the logits of the experts its threads hold
//       (thread e: experts e, e + 512), gates them (sigmoid
//       + bias, or the logits; kimi.py:308-315, tasks/distributed.py:174-176)
//       and selects the top k (k <= 16) with the workgroup's threshold-and-rank
//       selection (block_topk);
//       valid forced routes replace the selection (kimi.py:311-313).
//   GU  gate/up (kimi.py:321-322): the k x I/8 units (8 gate + 8 up rows of
//       one chosen expert) go to the workgroups in turn (unit u to workgroup
//       u mod G: exactly one each at top-8, I = 256 on a grid of 256, at most
//       4); the 8 waves split the K axis evenly and issue the weight loads of
//       all the workgroup's units at once as soon as the ids are known; the
//       waves' partial tiles meet in LDS, wave m sums unit m's in wave order,
//       applies the activation, and writes the unit's 8 bf16 h values to
//       tagged slots. Chosen expert j is the j-th of the selection (or of a
//       forced route row), so the loads go out right after the selection.
//   DN  down and combine (kimi.py:322-323): wave w takes the chosen experts
//       w, w + 8 (selection order) in the workgroup's one or two 16-row output
//       tiles; its weights are loaded once the gate/up data has arrived (they
//       then arrive while h is exchanged), it polls all its experts' h slots
//       together, multiplies, and the waves' w x bf16(y) rows are summed in
//       LDS from zero in ascending expert order.
// Each workgroup adds one to a launch counter when it leaves, on every path;
// the counters' sum at a launch's start, over the grid size, numbers the
// launch, and its tag is that number + 1 (a zeroed slot never matches).
// Every wait is bounded: a workgroup that gives up sets the status word,
// leaves NaN in its share of the output and leaves. The launch whose tag is
// the last of the 32-bit cycle clears the tag area behind a grid barrier, so
// that no slot written a whole cycle earlier carries a current tag.
#pragma once

#include <type_traits>

#include "k3moe_barrier.hpp"
#include "k3moe_decode.hpp"
#include "k3moe_device.hpp"
#include "k3moe_plan.hpp"

namespace k3moe {

constexpr int kTagPartials = 0;  // tag area: router logits, kTagCopies copies of [E] slots
constexpr uint32_t kTraceSingle = 0x5349u;  // trace slot 55 of the single-token kernel's rows

// Fixed LDS scratch of the single-token kernel, after the keys and the staged
// row; then the top-k's (BlockTopk), the chosen experts' h ([k][I] bf16) and
// the down products ([2 row tiles][k][16] fp32).
struct SingleScratch {
  int sel[kDecWaves * kMaxTopk];         // selection output (sel[0..k) in rank order)
  float rred[kDecWaves * 16];            // router: the waves' partial logits
  float gred[kSingleSlots * kDecWaves * 16];  // gate/up: per unit, the waves' 16 partial rows
  int ids[kSingleMaxTopk];               // forced routes: the chosen experts, in the row's order
  float wts[kSingleMaxTopk];             // gating weight of chosen expert j (selection order)
  int ord[kSingleMaxTopk];               // ord[r]: the chosen expert of ascending rank r (its j)
};
static_assert(sizeof(SingleScratch) % 16 == 0 && sizeof(SingleScratch) <= kSingleScratchBytes, "single_lds layout");
static_assert(sizeof(BlockTopk) <= kBlockTopkBytes, "single_lds layout");

// Down weights of one (expert, row tile) for KSD k-steps: a lane's 16 bytes
// and the aligned dword holding its scale byte (taken apart at use, as DnLoad).
template <int KSD>
struct SgDn {
  u32x4 w[KSD];
  uint32_t s[KSD], sh[KSD];
};

// JE: chosen experts per wave in the down phase (k <= 8 JE); KSD: the down
// projection's k-steps of 128 (I <= 128 KSD).
template <int JE, int KSD, bool LAT>
__global__ __launch_bounds__(kDecThreads, 1) void k_moe_single(Plan pl_arg, DecodeArgs a_arg) {
  const uint64_t t_entry = __builtin_amdgcn_s_memrealtime();  // (stored when tracing)
  const uint64_t kargs = touch_kernargs<sizeof(Plan) + sizeof(DecodeArgs)>();
  const Plan pl = load_const<Plan>(kargs);
  // the latent block's phases only in the LAT instantiations (the plain step's
  // code then carries none of them)
  const bool lat_in = LAT && pl.lat_in != 0, lat_out = LAT && pl.lat_out != 0;
  const DecodeArgs a = load_args(kargs + sizeof(Plan));
  (void)pl_arg;
  (void)a_arg;
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int E = pl.E, k = pl.k, K = pl.K, I = pl.I;
  uint32_t *kyl = reinterpret_cast<uint32_t *>(lds);  // [E] ordered keys
  float *kyf = reinterpret_cast<float *>(kyl + E);    // [E] keys
  float *scl = kyf + E;                               // [E] scores
  uint16_t *xs = reinterpret_cast<uint16_t *>(lds + align16(12 * E));  // [K] the token's expert-input row
  char *fixed = lds + align16(12 * E) + 2 * K;
  SingleScratch &sh = *reinterpret_cast<SingleScratch *>(fixed);
  BlockTopk &tk = *reinterpret_cast<BlockTopk *>(fixed + kSingleScratchBytes);
  uint16_t *hs = reinterpret_cast<uint16_t *>(fixed + kSingleScratchBytes + kBlockTopkBytes);  // [k][I]
  float *dacc = reinterpret_cast<float *>(fixed + kSingleScratchBytes + kBlockTopkBytes + align16(2 * k * I));
  __shared__ uint32_t s_tag, s_abort0;
  __shared__ int s_fail;

  const int tid = threadIdx.x, w = wave_id(), l = tid & 63, i = l & 15, q = l >> 4;
  unsigned *ctl = reinterpret_cast<unsigned *>(a.ws + pl.o_ctl);
  char *tag_area = a.ws + kOffTag;
  const __amdgpu_buffer_rsrc_t tagr = make_rsrc(tag_area, kTagBytes);
  // tag area: the logits, kTagCopies copies of [E] slots (workgroup b polls
  // copy b mod 8, the copy of its XCD: fewer readers per line), then the h
  // slots, [k][I/2]
  const uint32_t copy_bytes = (uint32_t)E * 8;
  const uint32_t my_copy = (blockIdx.x % kTagCopies) * copy_bytes;
  const uint32_t h_base = kTagCopies * copy_bytes;
  const uint8_t *zero = reinterpret_cast<const uint8_t *>(a.ws + pl.o_zero);
  trace_mark(pl, a.ws, 0);
  if (pl.o_trace && threadIdx.x == 0)
    reinterpret_cast<uint64_t *>(a.ws + pl.o_trace)[blockIdx.x * kTraceSlots + kTraceEntry] = t_entry;

  // Leaves the kernel: NaN in this workgroup's share of the output when a wait
  // gave up, and this workgroup's count on its launch counter (every path).
  auto leave = [&](bool gave_up) {
    if (gave_up) poison_share<false>(a.out, (long)K);
    if (gave_up && lat_out) poison_share<true>(a.lat_y, (long)pl.h);
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
  if (!lat_in) {  // (with the latent block's inputs, the kernel computes the row itself)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int c = hh * kDecThreads + tid;
      if (c < K / 8) xpre[hh] = load16(a.xin + c * 8);
    }
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
  // Workgroup b computes the whole logits (kimi.py:308) of experts b, b + G, ..
  // (at most kSingleRouterRows): wave w takes the w-th eighth of the h / 8
  // 16-byte chunks of x and of each row (at most two per lane), each lane sums
  // its bf16 products in FP32, the wave sums its lanes (a fixed DPP tree) and
  // the waves meet in LDS, summed in wave order; each logit goes to its tagged
  // slot in every copy.
  // wave w's share of h (16-byte chunks hc0 .. hc1 - 1; lane l takes hc0 + l
  // and hc0 + l + 64) and its chunks of x, kept for the latent block's inputs
  const int hc0 = (pl.h / 8) * w / kDecWaves, hc1 = (pl.h / 8) * (w + 1) / kDecWaves;
  u32x4 xv[2];
  // The latent block's input rows (Plan::lat_in; used in phase L below): this
  // workgroup's rows, their two first batches issued with the router's loads
  constexpr int RB = 4;
  const int G = (int)gridDim.x, b = (int)blockIdx.x, h = pl.h, S = pl.lat_S;
  const int nlp = K / 2 > b ? (K / 2 - b + G - 1) / G : 0, ns = S > b ? (S - b + G - 1) / G : 0;
  const int n = 2 * (nlp + ns), nb = (n + RB - 1) / RB;
  float *lred = sh.gred;  // [8 waves][kLatRowsMax]: the waves' partial sums (gate/up's area, free until then)
  auto row_ptr = [&](int r) -> const uint16_t * {
    if (r < 2 * nlp) return a.lat_ld + ((size_t)2 * (b + G * (r >> 1)) + (r & 1)) * h;
    const int rs = r - 2 * nlp;
    return ((rs & 1) ? a.lat_su : a.lat_sg) + (size_t)(b + G * (rs >> 1)) * h;
  };
  auto issue = [&](int bi, u32x4 (&buf)[RB][2]) {
#pragma unroll
    for (int rr = 0; rr < RB; ++rr) {
      const int r = bi * RB + rr;
      const uint16_t *row = r < n ? row_ptr(r) : nullptr;
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const int c = hc0 + l + 64 * m;
        buf[rr][m] = load16((row && c < hc1) ? reinterpret_cast<const uint8_t *>(row + c * 8) : zero);
      }
    }
  };
  auto compute = [&](int bi, const u32x4 (&buf)[RB][2]) {
#pragma unroll
    for (int rr = 0; rr < RB; ++rr) {
      float p = 0.f;
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t av = buf[rr][m][d], bv = xv[m][d];
          p = fmaf(bf16_bits_to_f32(av & 0xFFFFu), bf16_bits_to_f32(bv & 0xFFFFu), p);
          p = fmaf(bf16_bits_to_f32(av >> 16), bf16_bits_to_f32(bv >> 16), p);
        }
      p = wave_sum_f32(p);
      if (l == 0 && bi * RB + rr < n) lred[w * kLatRowsMax + bi * RB + rr] = p;
    }
  };
  u32x4 ba[RB][2], bb[RB][2];
  {
    const int c0 = hc0, c1 = hc1;
    u32x4 rv[kSingleRouterRows][2];
#pragma unroll
    for (int r = 0; r < kSingleRouterRows; ++r) {
      const int e = (int)blockIdx.x + r * (int)gridDim.x;
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const int c = c0 + l + 64 * m;
        rv[r][m] = (e < E && c < c1) ? load16(a.router + (size_t)e * pl.h + c * 8) : u32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int c = c0 + l + 64 * m;
      xv[m] = c < c1 ? load16(a.x + c * 8) : u32x4{0, 0, 0, 0};
    }
    if (lat_in) {
      issue(0, ba);
      issue(1, bb);
    }
    warm_code();
    make_tag();
#pragma unroll
    for (int r = 0; r < kSingleRouterRows; ++r) {
      if ((int)blockIdx.x + r * (int)gridDim.x >= E) break;  // workgroup-uniform
      float p = 0.f;
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t av = rv[r][m][d], bv = xv[m][d];
          p = __fadd_rn(p, __fmul_rn(bf16_bits_to_f32(av & 0xFFFFu), bf16_bits_to_f32(bv & 0xFFFFu)));
          p = __fadd_rn(p, __fmul_rn(bf16_bits_to_f32(av >> 16), bf16_bits_to_f32(bv >> 16)));
        }
      p = wave_sum_f32(p);
      if (l == 0) sh.rred[w * kSingleRouterRows + r] = p;
    }
    make_tag();
    __syncthreads();
    if (tid < kSingleRouterRows * kTagCopies) {
      const int r = tid % kSingleRouterRows, e = (int)blockIdx.x + r * (int)gridDim.x;
      if (e < E) {
        float sum = sh.rred[r];
#pragma unroll
        for (int ww = 1; ww < kDecWaves; ++ww) sum = __fadd_rn(sum, sh.rred[ww * kSingleRouterRows + r]);
        st_dev64(tagr, (uint32_t)(kTagPartials + (tid / kSingleRouterRows) * copy_bytes + e * 8),
                 u32x2{__float_as_uint(sum), s_tag});
      }
    }
  }
  warm_code();
  make_tag();
  trace_mark(pl, a.ws, 1);
  // the staged row for gate/up (its loads have long arrived)
  if (!lat_in) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int c = hh * kDecThreads + tid;
      if (c < K / 8) *reinterpret_cast<u32x4 *>(xs + c * 8) = xpre[hh];
    }
  }
  __syncthreads();  // s_tag, s_abort0, the staged row
  asm volatile("" ::"v"(code_probe));
  const uint32_t tag = s_tag, abort0 = s_abort0;
  const uint32_t lat_base = lat_slot_base(pl);  // the latent's row-pair slots, [K / 2]

  // ------------------------------------------------ L: latent block inputs --
  // With Plan::lat_in (kimi.py:317, 326): latent = bf16(x @ latent_down.T)
  // and shared_h = bf16(act(bf16(x @ shared_gate.T), bf16(x @ shared_up.T))).
  // Workgroup b takes latent row pairs b, b + G, .. and shared pairs b, b + G,
  // ..; its waves take the router's shares of h (x already in registers), in
  // batches of 4 rows with two batches in flight (rows past the workgroup's
  // read the zero area, so every batch is 8 loads a lane and the waits are
  // exact); each lane's 16 products are summed in FP32 (exact products, fused
  // adds), the wave's lanes by the DPP tree and the waves in order in LDS. The
  // latent goes to xin and, as bf16 pairs, to tagged slots that every
  // workgroup polls before its gate/up products; shared_h goes to lat_sh.
  if (lat_in) {
    for (int bi = 0; bi < nb; bi += 2) {  // batches past nb read the zero area
      wait_vm<2 * RB>();
      compute(bi, ba);
      issue(bi + 2, ba);
      wait_vm<2 * RB>();
      compute(bi + 1, bb);
      issue(bi + 3, bb);
    }
    wait_vm<0>();
    __syncthreads();
    if (tid < nlp) {  // latent rows 2 jp, 2 jp + 1
      const int jp = b + G * tid;
      float v0 = lred[2 * tid], v1 = lred[2 * tid + 1];
#pragma unroll
      for (int ww = 1; ww < kDecWaves; ++ww) {
        v0 = __fadd_rn(v0, lred[ww * kLatRowsMax + 2 * tid]);
        v1 = __fadd_rn(v1, lred[ww * kLatRowsMax + 2 * tid + 1]);
      }
      const uint32_t pair = (uint32_t)f32_to_bf16_bits(v0) | ((uint32_t)f32_to_bf16_bits(v1) << 16);
      *reinterpret_cast<uint32_t *>(const_cast<uint16_t *>(a.xin) + 2 * jp) = pair;
      st_dev64(tagr, lat_base + (uint32_t)jp * 8, u32x2{pair, tag});
    } else if (tid >= 64 && tid < 64 + ns) {  // shared gate and up rows of pair s
      const int j = tid - 64, r = 2 * nlp + 2 * j, sj = b + G * j;
      float g = lred[r], u = lred[r + 1];
#pragma unroll
      for (int ww = 1; ww < kDecWaves; ++ww) {
        g = __fadd_rn(g, lred[ww * kLatRowsMax + r]);
        u = __fadd_rn(u, lred[ww * kLatRowsMax + r + 1]);
      }
      const uint16_t hv = f32_to_bf16_bits(apply_act(pl.act, round_bf16(g), round_bf16(u)));
      a.lat_sh[sj] = hv;
      if (lat_out) st_dev64(tagr, lat_base + (uint32_t)(K / 2 + sj) * 8, u32x2{hv, tag});
    }
    trace_mark(pl, a.ws, 16);
  }

  // -------------------------------------------------------- T: top-k/gating --
  {
    // thread e polls the logits of experts e and e + 512 (slot e of its copy)
    float logit0 = 0.f, logit1 = 0.f;
    bool ok = true;
    // TWO: experts past 512 exist (a second expert per thread); a separate
    // loop without them otherwise
    auto poll = [&](auto two_) {
      constexpr bool TWO = decltype(two_)::value;
      const int e0 = tid, e1 = tid + kDecThreads;
      const bool n0 = e0 < E, n1 = TWO && e1 < E;
      u32x2 v0 = {0, 0}, v1 = {0, 0};
      unsigned spins = 0;
      for (;;) {
        v0 = n0 ? bload8_dev(tagr, (uint32_t)(kTagPartials + my_copy + e0 * 8)) : u32x2{0, tag};
        if constexpr (TWO) v1 = n1 ? bload8_dev(tagr, (uint32_t)(kTagPartials + my_copy + e1 * 8)) : u32x2{0, tag};
        bool ready = v0[1] == tag && pl.stall == 0;  // (a test hook: the wait never ends and gives up)
        if constexpr (TWO) ready = ready && v1[1] == tag;
        if (spins == 0 && w == 0) trace_mark(pl, a.ws, 10);
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
      logit0 = __uint_as_float(v0[0]);
      if constexpr (TWO) logit1 = __uint_as_float(v1[0]);
      if (pl.o_trace && tid == 0)
        reinterpret_cast<uint64_t *>(a.ws + pl.o_trace)[blockIdx.x * kTraceSlots + 11] = spins + 1;
    };
    if (E > kDecThreads) poll(std::true_type{});
    else poll(std::false_type{});
    if (!ok) s_fail = 1;
    trace_mark(pl, a.ws, 2);
    // gating (kimi.py:308-309; tasks/distributed.py:174); returns the ordered key
    auto gate = [&](int e, float logit, float bias) {
      float score, key;
      if (pl.gating == K3MOE_GATING_SIGMOID_BIAS) {
        score = 1.0f / (1.0f + expf(-logit));
        key = a.bias ? __fadd_rn(score, bias) : score;
      } else {
        score = logit;
        key = logit;
      }
      scl[e] = score;
      kyf[e] = key;
      return ordered_key(key);
    };
    uint32_t key0 = 0u, key1 = 0u;
    if (tid < E) key0 = gate(tid, logit0, bias_pre[0]);
    if (tid + kDecThreads < E) key1 = gate(tid + kDecThreads, logit1, bias_pre[1]);
    trace_mark(pl, a.ws, 3);
    // the workgroup's top-k: a threshold from group maxima, then exact ranks
    // among the candidates (its barriers also publish s_fail, the scores and keys)
    block_topk(key0, key1, E, k, sh.sel, tk);
    if (s_fail) return leave(true);
    trace_mark(pl, a.ws, 4);
    if (a.routes) {  // kernel-uniform
      // forced routes replace the selection when the row is valid (kimi.py:311-313)
      if (w == 0) {
        int fid = 0;
        const bool forced = forced_route(a.routes, 0, k, E, &fid);
        if (!forced && l == 0 && blockIdx.x == 0)
          __hip_atomic_fetch_or(ctl + kCtlErr, (unsigned)kErrRoutes, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (l < k) sh.ids[l] = forced ? fid : sh.sel[l];
      }
      __syncthreads();
    }
  }
  // the chosen experts in selection order: chosen expert j of the gate/up
  // units, the h slots and the down waves (the combine adds them in ascending
  // expert order through sh.ord)
  const int *const chosen = a.routes ? sh.ids : sh.sel;
  trace_mark(pl, a.ws, 5);

  // ------------------------------------------------------------- GU issue --
  // gate/up unit u: chosen expert j = u / U8 (selection order), rows 8 rg .. 8 rg + 7
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
  // This workgroup's units are b, b + G, .. (nu of them); their loads are all
  // issued at once, in kSingleSlots register slots: slot sl holds unit
  // b + (sl / ssw) G, super-step ss0 + sl mod ssw (ssw = 1 or 2 super-steps per
  // wave), so one memory round trip brings every unit's rows.
  const int ssw = NSS > kDecWaves ? 2 : 1, lg_ssw = ssw - 1;
  const int nu = (NU - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
  u32x4 ga[kSingleSlots][4], gsc[kSingleSlots];
#pragma unroll
  for (int sl = 0; sl < kSingleSlots; ++sl) {
    const int mu = sl >> lg_ssw, ss = ss0 + (sl & lg_ssw);
    if (mu < nu && ss < ss1) {  // wave-uniform
      const int u = (int)blockIdx.x + mu * (int)gridDim.x, j = u / U8, rg = u - j * U8;
      const size_t row = (size_t)chosen[j] * I + rg * 8 + (i & 7);
      const uint8_t *wr = lane_blk + row * KB * 16, *sr = lane_scl + row * KB;
#pragma unroll
      for (int t = 0; t < 4; ++t) ga[sl][t] = load16(wr + (16 * ss + 4 * t + q) * 16);
      gsc[sl] = load16(sr + 16 * ss);
    }
  }
  trace_mark(pl, a.ws, 9);

  if (w == 0) {
    // the gating weights, while the loads are in flight; the down phase reads
    // them after the gate/up phase's LDS barriers
    const int my_e = l < k ? chosen[l] : -1;
    int rank = 0;  // ascending rank of my_e among the chosen
    for (int r = 0; r < k; ++r) rank += ((int)lane_u32((uint32_t)my_e, r) < my_e) ? 1 : 0;
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
      if (l < k) {
        sh.wts[l] = wt;
        sh.ord[rank] = l;
      }
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

  if (lat_in) {
    // the latent row (the experts' input) from every workgroup's tagged row-pair
    // slots (thread tid: pairs tid + 512 m), polled until each carries this
    // launch's tag; its first check waits for this wave's gate/up loads too
    // (issued before it), which are needed next anyway
    const int lp = K / 2;
    u32x2 v[kSingleMaxK / 1024];
    bool ok = true;
    unsigned spins = 0;
    for (;;) {
      bool ready = true;
#pragma unroll
      for (int m = 0; m < kSingleMaxK / 1024; ++m) {
        const int c = tid + kDecThreads * m;
        v[m] = c < lp ? bload8_dev(tagr, lat_base + (uint32_t)c * 8) : u32x2{0u, tag};
        ready = ready && v[m][1] == tag;
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
#pragma unroll
    for (int m = 0; m < kSingleMaxK / 1024; ++m) {
      const int c = tid + kDecThreads * m;
      if (c < lp) *reinterpret_cast<uint32_t *>(xs + 2 * c) = v[m][0];
    }
    if (!ok) s_fail = 1;
    __syncthreads();
    if (s_fail) return leave(true);
  }

  // The latent block's output rows (phase O below): wave w's first two rows'
  // weights go out once the gate/up data has arrived, with the down weights,
  // so that they stream while h is exchanged and the down products run; the
  // first into registers, the second straight into LDS (kLatOutRow1Bytes
  // after the expert sum and [en | shared_h]), which the down phase leaves
  // free of registers.
  struct OutRow {
    u32x4 v[kLatOutChunks];
  };
  const int o_nro = pl.h > (int)blockIdx.x ? (pl.h - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x : 0;
  auto out_issue = [&](int m, OutRow &rw) {  // wave w's m-th row (row b + G (w + 8 m)); past its rows: the zero area
    const int KC = K / 8, NC = (K + pl.lat_S) / 8;
    const int ri = w + kDecWaves * m, ro = (int)blockIdx.x + (int)gridDim.x * ri;
#pragma unroll
    for (int jc = 0; jc < kLatOutChunks; ++jc) {
      const int c = l + 64 * jc;
      const uint16_t *src = c < KC ? a.lat_up + (size_t)ro * K + c * 8 : a.lat_sd + (size_t)ro * pl.lat_S + (c - KC) * 8;
      rw.v[jc] = load16((ri < o_nro && c < NC) ? reinterpret_cast<const uint8_t *>(src) : zero);
    }
  };
  OutRow r0w, r1w;
  char *const o_row1 = lds + single_lds_base(pl) + align16(4 * K) + align16(2 * (K + pl.lat_S)) +
                       w * kLatOutChunks * 1024;  // wave w's second row (chunk jc at jc KiB, lane l at 16 l)

  // ----------------------------------------------------------- GU compute --
  // The down weights of this workgroup's row tiles (blockIdx.x, blockIdx.x + G)
  // for wave w's expert are issued once the gate/up data has arrived, so that
  // the gate/up stream has the memory system to itself; they arrive while h is
  // exchanged. A tile past the last reads the zero area.
  SgDn<KSD> pf[JE][2];
  bool dn_issued = false;
  const int KBd = I / kBlockK;
  auto dn_issue = [&]() {
    if (dn_issued) return;
    dn_issued = true;
#pragma unroll
    for (int je = 0; je < JE; ++je) {
      const int j = w + kDecWaves * je;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int rt = (int)blockIdx.x + tt * (int)gridDim.x;
        const bool rt_ok = j < k && rt < pl.RTd;  // wave-uniform
        const size_t row = (size_t)(rt_ok ? chosen[j] : 0) * K + (rt_ok ? rt : 0) * 16 + i;
#pragma unroll
        for (int ks = 0; ks < KSD; ++ks) {
          const int kb = ks * 4 + q;
          const bool okb = rt_ok && kb < KBd;
          // unconditional loads: a skipped one is joined by a copy that waits for it at once
          pf[je][tt].w[ks] = load16(okb ? a.dblk + (row * KBd + kb) * 16 : zero);
          const uint8_t *sp = okb ? a.dscl + row * KBd + kb : zero;
          const uint32_t mis = (uint32_t)reinterpret_cast<uintptr_t>(sp) & 3u;
          pf[je][tt].s[ks] = *reinterpret_cast<const uint32_t *>(sp - mis);
          pf[je][tt].sh[ks] = mis * 8u;
        }
      }
    }
  };
  // every unit's partial rows (this wave's super-steps), then one barrier; wave
  // mu finishes unit mu
#pragma unroll
  for (int mu = 0; mu < kSingleSlots; ++mu) {
    if (mu >= nu) break;  // wave-uniform
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sl = 0; sl < kSingleSlots; ++sl) {
      const int ss = ss0 + (sl & lg_ssw);
      if ((sl >> lg_ssw) == mu && ss < ss1) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int kb = 16 * ss + 4 * t + q;
          bf16x8 av[4];
          convert_block_fast(ga[sl][t], (gsc[sl][t] >> (8 * q)) & 0xFFu, av);
#pragma unroll
          for (int kk = 0; kk < 4; ++kk)
            acc = mfma16(av[kk], as_bf16x8(*reinterpret_cast<const u32x4 *>(xs + kb * kBlockK + kk * 8)), acc);
        }
      }
    }
    if (i == 0) {  // column 0: rows 4q .. 4q + 3 (0-7 gate, 8-15 up)
#pragma unroll
      for (int v = 0; v < 4; ++v) sh.gred[(mu * kDecWaves + w) * 16 + 4 * q + v] = acc[v];
    }
  }
  trace_mark(pl, a.ws, 12);
  ring_barrier();  // every wave's gate/up data has arrived
  dn_issue();
  trace_mark(pl, a.ws, 13);
  if (w < nu) {
    // h = act(bf16(gate), bf16(up)) of unit w's 8 rows: lane r < 16 sums row r
    // over the waves in order (gate rows 0-7, up rows 8-15); the activation's
    // transcendental factors run in separate lanes (act_parts) and lane r < 8
    // combines them in the reference's order
    const int u0 = (int)blockIdx.x + w * (int)gridDim.x;
    const float *red = sh.gred + w * kDecWaves * 16;
    const int r = l & 15;
    float v = red[r];
#pragma unroll
    for (int ww = 1; ww < kDecWaves; ++ww) v += red[ww * 16 + r];
    v = round_bf16(v);
    const float g = __shfl(v, l & 7, kWave), up = __shfl(v, 8 + (l & 7), kWave);
    const float hv = act_parts(pl.act, g, up);
    const uint32_t hb = f32_to_bf16_bits(hv);
    const uint32_t pair = hb | ((uint32_t)__shfl_down((int)hb, 1, kWave) << 16);
    const int j = u0 / U8, rg = u0 % U8;
    if (l < 8 && (l & 1) == 0)
      st_dev64(tagr, h_base + (uint32_t)((j * (I / 2) + rg * 4 + (l >> 1)) * 8), u32x2{pair, tag});
    if (w == 0) trace_mark(pl, a.ws, 14);
  }
  dn_issue();    // a workgroup without a gate/up unit
  if (lat_out) {
    out_issue(0, r0w);
    const int KC = K / 8, NC = (K + pl.lat_S) / 8, ri = w + kDecWaves, ro = (int)blockIdx.x + (int)gridDim.x * ri;
#pragma unroll
    for (int jc = 0; jc < kLatOutChunks; ++jc) {
      const int c = l + 64 * jc;
      const uint16_t *src = c < KC ? a.lat_up + (size_t)ro * K + c * 8 : a.lat_sd + (size_t)ro * pl.lat_S + (c - KC) * 8;
      load_lds<16>((ri < o_nro && c < NC) ? reinterpret_cast<const uint8_t *>(src) : zero, o_row1 + jc * 1024);
    }
  }
  ring_barrier();  // wave 0's gating weights (sh.wts) are visible to the down phase
  trace_mark(pl, a.ws, 6);

  // ------------------------------------------------------- DN: down+combine --
  // wave w: chosen experts w, w + 8, .. (JE of them); each expert's h is polled
  // (lane l: values 4 l .. 4 l + 3 and 256 + 4 l .., two 8-byte slots each),
  // put in LDS and read back as the B operand
  // all of a wave's h slots are polled together: every load of a round in flight at once
  bool ok = true;
  {
    u32x4 hv[JE][2];
    int hn[JE][2];
#pragma unroll
    for (int je = 0; je < JE; ++je)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int j = w + kDecWaves * je, v0 = hh * 256 + 4 * l;
        hn[je][hh] = (j < k && v0 < I) ? 2 : 0;
        hv[je][hh] = u32x4{0, 0, 0, 0};
      }
    unsigned spins = 0;
    for (;;) {
      bool ready = true;
#pragma unroll
      for (int je = 0; je < JE; ++je)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int j = w + kDecWaves * je, v0 = hh * 256 + 4 * l;
          hv[je][hh] = hn[je][hh] ? bload16_dev(tagr, h_base + (uint32_t)((j * (I / 2) + v0 / 2) * 8)) : u32x4{0, tag, 0, tag};
        }
#pragma unroll
      for (int je = 0; je < JE; ++je)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) ready = ready && hv[je][hh][1] == tag && hv[je][hh][3] == tag;
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
    for (int je = 0; je < JE; ++je)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int j = w + kDecWaves * je, v0 = hh * 256 + 4 * l;
        if (hn[je][hh]) *reinterpret_cast<u32x2 *>(hs + j * I + v0) = u32x2{hv[je][hh][0], hv[je][hh][2]};
      }
  }
  wave_lds_order();
  if (w == 0) trace_mark(pl, a.ws, 7);
#pragma unroll
  for (int je = 0; je < JE; ++je) {
    const int j = w + kDecWaves * je;
    if (j >= k) break;  // wave-uniform
    // B operand: k-step ks covers blocks 4 ks + q of h (lane group q)
    u32x4 hb[KSD][4];
#pragma unroll
    for (int ks = 0; ks < KSD; ++ks) {
      const int kb = ks * 4 + q;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        hb[ks][kk] = kb < KBd ? *reinterpret_cast<const u32x4 *>(hs + j * I + kb * kBlockK + kk * 8) : u32x4{0, 0, 0, 0};
    }
    const float wt = sh.wts[j];
    // The down scale bytes are taken apart only here, after the h poll
    // (as dn_scale): the compiler would otherwise convert them right where
    // they are loaded and wait there for the loads, which are meant to arrive
    // while h is exchanged.
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KSD; ++ks) {
        uint32_t sc = pf[je][tt].s[ks];
        asm volatile("" : "+v"(sc));
        bf16x8 av[4];
        convert_block_fast(pf[je][tt].w[ks], (sc >> pf[je][tt].sh[ks]) & 0xffu, av);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) acc = mfma16(av[kk], as_bf16x8(hb[ks][kk]), acc);
      }
      if (i == 0) {  // column 0: rows 4q .. 4q + 3 of the tile
#pragma unroll
        for (int vv = 0; vv < 4; ++vv) dacc[(tt * k + j) * 16 + 4 * q + vv] = __fmul_rn(round_bf16(acc[vv]), wt);
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
      for (int jj = 0; jj < k; ++jj) sum = __fadd_rn(sum, dacc[(tt * k + sh.ord[jj]) * 16 + r]);
      a.out[rt * 16 + r] = sum;
      if (lat_out)
        st_dev64(tagr, lat_base + (uint32_t)(K / 2 + pl.lat_S + rt * 16 + r) * 8, u32x2{__float_as_uint(sum), tag});
    }
  }
  trace_mark(pl, a.ws, 8);

  // ------------------------------------------------ O: latent block output --
  // With Plan::lat_out (kimi.py:325-328): out = bf16(bf16(en @ latent_up.T) +
  // bf16(shared_h @ shared_down.T)), en = bf16(bf16(e r) w) the RMS-normalised
  // bf16(expert_sum) (r = 1 / sqrt(mean(e^2) + 1e-5), w = latent_norm).
  // Workgroup b takes output rows b, b + G, .. (wave w: its rows w, w + 8, ..);
  // a lane takes 16-byte chunks l + 64 j of the row's [latent_up | shared_down]
  // (K + S columns) against the same chunks of [en | shared_h] in LDS. The
  // first two rows' weights go out after the gate/up data (the second of them
  // straight into LDS), before the expert sum and shared_h are polled from
  // every workgroup's tagged slots; wave 0 sums e^2 (lane l:
  // chunks of 4 at 4 (l + 64 m), then the wave's butterfly); each lane sums its
  // two parts separately in FP32, the wave's DPP tree sums them, and lane 0
  // rounds each part and their sum.
  if (lat_out) {
    const int G = (int)gridDim.x, b = (int)blockIdx.x, h = pl.h, S = pl.lat_S, KC = K / 8, NC = (K + S) / 8;
    const int nro = h > b ? (h - b + G - 1) / G : 0;
    float *es = reinterpret_cast<float *>(lds + single_lds_base(pl));       // [K] the expert sum
    uint16_t *xo = reinterpret_cast<uint16_t *>(es + K);                    // [K + S] en, then shared_h
    const uint32_t sh_base = lat_base + (uint32_t)(K / 2) * 8, es_base = sh_base + (uint32_t)S * 8;
    using Row = OutRow;
    auto issue = out_issue;  // (rows 0 and 1 went out after the gate/up data)
    // this thread's norm weights (k = tid + 512 m), the expert sum and shared_h from their slots
    uint16_t wn[kLatOutMaxK / kDecThreads];
#pragma unroll
    for (int m = 0; m < kLatOutMaxK / kDecThreads; ++m) {
      const int kk = tid + kDecThreads * m;
      wn[m] = kk < K ? a.lat_norm[kk] : (uint16_t)0;
    }
    {
      // element c = tid + 512 m of [expert sum | shared_h], every load of a round in flight at once
      bool ok = true;
      unsigned spins = 0;
      for (;;) {
        u32x2 v[kLatOutPoll];
#pragma unroll
        for (int m = 0; m < kLatOutPoll; ++m) {
          const int c = tid + kDecThreads * m;
          const uint32_t off = c < K ? es_base + (uint32_t)c * 8 : sh_base + (uint32_t)(c - K) * 8;
          v[m] = c < K + S ? bload8_dev(tagr, off) : u32x2{0u, tag};
        }
        bool ready = true;
#pragma unroll
        for (int m = 0; m < kLatOutPoll; ++m) {
          const int c = tid + kDecThreads * m;
          ready = ready && v[m][1] == tag;
          if (c < K) es[c] = __uint_as_float(v[m][0]);
          else if (c < K + S) xo[c] = (uint16_t)v[m][0];
        }
        if (__syncthreads_or(!ready) == 0) break;
        ++spins;  // (the same in every thread: each exit below is taken by the whole workgroup)
        if ((spins & 63u) == 0u && __syncthreads_or(aborted(ctl, abort0)) != 0) {
          ok = false;
          break;
        }
        if (spins > kSpinLimit) {
          if (tid == 0) raise_timeout(ctl);
          ok = false;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      if (!ok) return leave(true);
    }
    if (w == 0) {  // r = 1 / sqrt(mean(bf16(e)^2) + eps)
      float ss = 0.f;
      f32x4 ec[kLatOutMaxK / 256];  // every chunk read at once
#pragma unroll
      for (int m = 0; m < kLatOutMaxK / 256; ++m)
        ec[m] = 4 * (l + 64 * m) < K ? *reinterpret_cast<const f32x4 *>(es + 4 * (l + 64 * m))
                                      : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < kLatOutMaxK / 256; ++m) {
        if (4 * (l + 64 * m) < K) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float e = round_bf16(ec[m][v]);
            ss += e * e;
          }
        }
      }
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) ss += shfl_xor(ss, m);
      if (l == 0) sh.rred[0] = 1.0f / __fsqrt_rn(ss / (float)K + kLatOutRmsEps);
    }
    __syncthreads();
    const float rn = sh.rred[0];
#pragma unroll
    for (int m = 0; m < kLatOutMaxK / kDecThreads; ++m) {
      const int kk = tid + kDecThreads * m;
      if (kk < K) xo[kk] = f32_to_bf16_bits(round_bf16(round_bf16(es[kk]) * rn) * bf16_bits_to_f32(wn[m]));
    }
    __syncthreads();
    // the rows' values are stored after the loop: a store inside it would be
    // counted by the next row's wait (vmcnt counts stores too)
    uint16_t yv[kLatOutRowsPerWave];
    // row 1 from LDS (its loads, older than the poll's, have landed)
#pragma unroll
    for (int jc = 0; jc < kLatOutChunks; ++jc) r1w.v[jc] = *reinterpret_cast<const u32x4 *>(o_row1 + jc * 1024 + 16 * l);
    auto row_out = [&](int m, const Row &rw) {
      const int ri = w + kDecWaves * m;
      if (ri >= nro) return;  // wave-uniform
      float s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int jc = 0; jc < kLatOutChunks; ++jc) {
        const int c = l + 64 * jc;
        if (c < NC) {
          const u32x4 xv = *reinterpret_cast<const u32x4 *>(xo + c * 8);
          float p = 0.f;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            p = fmaf(bf16_bits_to_f32(rw.v[jc][d] & 0xFFFFu), bf16_bits_to_f32(xv[d] & 0xFFFFu), p);
            p = fmaf(bf16_bits_to_f32(rw.v[jc][d] >> 16), bf16_bits_to_f32(xv[d] >> 16), p);
          }
          if (c < KC) s1 += p;
          else s2 += p;
        }
      }
      s1 = wave_sum_f32(s1);
      s2 = wave_sum_f32(s2);
      yv[m] = f32_to_bf16_bits(round_bf16(s1) + round_bf16(s2));
    };
#pragma unroll
    for (int m = 0; m < kLatOutRowsPerWave; m += 2) {
      wait_vm<kLatOutChunks>();
      row_out(m, r0w);
      issue(m + 2, r0w);
      wait_vm<kLatOutChunks>();
      row_out(m + 1, r1w);
      issue(m + 3, r1w);
    }
    wait_vm<0>();
    if (l == 0) {
#pragma unroll
      for (int m = 0; m < kLatOutRowsPerWave; ++m)
        if (w + kDecWaves * m < nro) a.lat_y[b + G * (w + kDecWaves * m)] = yv[m];
    }
    trace_mark(pl, a.ws, 19);
  }
  if (pl.o_trace && tid == 0)
    reinterpret_cast<uint64_t *>(a.ws + pl.o_trace)[blockIdx.x * kTraceSlots + 55] = kTraceSingle;
  if (blockIdx.x == 0 && tid == 0) {  // this kernel's code range, for the next launch's warm-up
    crange[0] = pc0;
    crange[1] = program_counter();
  }
  if (tag == last_tag_of_cycle()) {
    // the barrier counters, read now: no barrier of this launch completes before this workgroup arrives
    const BarrierBase bb = tid == 0 ? barrier_base(ctl) : BarrierBase{0u, 0u, 0u};
    if (!clear_tag_area(ctl, bb, 1, tagr)) return leave(true);
  }
  leave(false);
  trace_mark(pl, a.ws, kTraceExit);
}

}  // namespace k3moe
