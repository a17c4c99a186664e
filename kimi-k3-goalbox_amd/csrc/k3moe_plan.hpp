// Launch plan and workspace layout of one MoE step (host and device).
//
// Three execution paths share the workspace conventions:
//   single   B = 1 on shapes it fits: one persistent kernel, no grid barrier
//            (k3moe_single.hpp)
//   decode   B <= 64 tokens: one persistent kernel, one 512-thread workgroup
//            per CU, phases handed over through tagged slots and at most two
//            grid barriers (k3moe_decode.hpp)
//   general  any B: a chain of eight to ten kernels (k3moe_general.hpp,
//            k3moe_xgemm.hpp, k3moe_fgemm.hpp)
// The workspace starts with a control block (kCtlBytes): the barrier counters
// of the persistent kernel and a sticky error word. It must be zero before the
// first step; the barrier counters only grow (32-bit, wrapping), and each
// launch takes its barrier targets from their values at its start.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "k3moe.h"

namespace k3moe {

constexpr int kWavesPerBlock = 4;  // general path: 4 independent waves per block
constexpr int kThreads = kWavesPerBlock * 64;
constexpr int kMaxExperts = 1024;
constexpr int kMaxTopk = 32;
constexpr int kGroupChunk = 128;   // tokens per placement chunk in k_group
constexpr int kXMinPairsPerExpert = 16;  // general path: grouped GEMMs from this many token-expert pairs per expert
constexpr int kMaxRouterSplits = 8;      // general path: router k-splits (partials summed by the top-k kernel)

constexpr int kDecWaves = 8;       // decode path: waves per workgroup
constexpr int kDecThreads = kDecWaves * 64;
constexpr int kDecMaxTokens = 64;
constexpr int kDecMaxPairs = 1024;
constexpr int kDecMaxSplits = 10;  // router k-splits across workgroups
constexpr int kDecMaxLds = 160 * 1024;   // gfx950: 160 KiB of LDS per workgroup
constexpr int kDecStaticLds = 1024;  // decode kernel's static LDS (round table, counters), upper bound
constexpr int kDnStage = 128;        // decode down: y rows staged per wave (32 B + a 4-byte tag each)

// LDS of the workgroup top-k (block_topk): group maxima of the 32- and 64-bit keys per wave, up to
// kMaxExperts candidates, two counts
constexpr int kBlockTopkBytes = 12 * kDecWaves * 32 + 8 * kMaxExperts + 16;

constexpr int kRedundantTokens = 1;    // decode: route every token in every workgroup up to this batch
constexpr int kRedundantKeys = 8192;   // ... and up to this many (token, expert) keys

// Control block (uint32 words): the sticky status word, the abort counter and
// the decode kernel's code range (words 4-7) in the first 128-byte line, the
// top barrier counter in the second, then kBarGroups group counters kCtlStride
// words (128 B) apart.
//   status (kCtlErr): OR of kErr* bits of every step since the workspace init
//   abort (kCtlAbort): grows by one whenever a workgroup gives up waiting; a
//     launch reads it at its start and its barriers stop waiting early only
//     when it moves during that launch (a timeout of an earlier launch leaves
//     the status set but does not shorten later launches' waits)
constexpr int kCtlErr = 2;
constexpr int kCtlAbort = 3;
constexpr int kCtlCodeSingle = 8;  // 2 x uint64: the single-token kernel's code range of its last launch
constexpr int kCtlCodeLatent = 12;  // 4 x (2 x uint64): the latent kernels' code ranges (k_latent<0>, <1>, k_latent_sk<0>, <1>)
// Launch counters of the single-token and decode kernels (k3moe_single.hpp,
// k3moe_decode.hpp): each of their workgroups adds one, on counter blockIdx %
// kEpochCounters, when it leaves; the sum, divided by the grid size (the same
// for both), counts their earlier launches on this workspace.
// kCtlEpochStride words (64 bytes) apart.
constexpr int kCtlEpoch = 640, kEpochCounters = 16, kCtlEpochStride = 16;
constexpr int kCtlCode = 4;  // 2 x uint64: the decode kernel's code range (start, end) of its last launch
constexpr int kCtlTop = 32;
constexpr int kBarGroups = 16, kCtlGroup = 64, kCtlStride = 32;
constexpr int kCtlBytes = 4 * (kCtlGroup + kBarGroups * kCtlStride);  // 2304
// A zero area follows the control block: loads of inactive lanes and of k-steps
// past a range read it instead of branching. Zeroed with the control block by
// the workspace init and never written by a step. Holds any row offset used
// (K <= 16384 activations: 32 KiB + lane offsets).
constexpr int kZeroBytes = 64 * 1024;
// Then the latent block's arrival counters (one uint32 per output row tile,
// k3moe_latent.hpp): zero between launches; the launch that completes a tile
// puts its counter back to zero.
constexpr int kLatCntBytes = 16384;
constexpr int kOffLatCnt = 4096 + kZeroBytes;
// Then the persistent kernels' tagged exchange area: 8-byte slots {payload,
// tag}, where the tag identifies the launch that wrote the payload (zero never
// does, so a zeroed area holds no valid slot). Only the single-token and decode
// kernels write it; both number their launches on the same counters, so a slot
// left by any earlier launch never carries the current tag.
constexpr int kTagBytes = 2 * 1024 * 1024;
constexpr int kTagCopies = 8;  // single-token router partials: one copy per XCD (workgroup b reads copy b mod 8)
// The decode kernel's regions: the routed pairs (16-byte slots {id, tag,
// weight, tag}), the gate/up completion slots (slot d + b: active expert d,
// workgroup b; or, pinned, slot gw: the workgroup's wave gw = 8 b + w), then
// the router partials ([B][Srw][Epad] slots).
constexpr int kTagDecPairs = 0;
constexpr int kTagDecDone = kTagDecPairs + kDecMaxPairs * 16;
constexpr int kTagDecPart = kTagDecDone + 8 * 1024 * 8;  // done slots: d + b (staged), or wave gw < 8 x 1024 (pinned)
// With the latent block's output (Plan::lat_out, pinned, at most 512
// workgroups): workgroup b's "expert sum written" slot, the last 512 of the
// done slots (pinned plans of at most 512 workgroups use the first 4096).
constexpr int kLatFlagsMax = 512;
constexpr int kTagDecFlags = kTagDecDone + (8 * 1024 - kLatFlagsMax) * 8;
constexpr int kOffTag = kOffLatCnt + kLatCntBytes;
constexpr int kInitBytes = kOffTag + kTagBytes;  // control block (page-padded), zero area, counters, tags
constexpr int kTraceSlots = 64;    // phase timestamps per workgroup when tracing
constexpr int kTraceEntry = 56, kTraceExit = 57;  // the workgroup's first instruction and its end
constexpr int kErrBarrierTimeout = 1;  // a wait timed out: that step's outputs are invalid
constexpr int kErrRoutes = 2;          // forced routes out of range or repeated in a row: those rows used their own top-k

enum Path { kPathGeneral = 0, kPathDecode = 1 };

struct Plan {
  int B, E, k, h, K, I, gating, act;
  int P;     // token-expert pairs, B*k
  int Dmax;  // upper bound of distinct experts, min(E, P)
  int Epad;  // E rounded up to 16
  int path;
  // general path
  int RTr, TTr, KSr, Sr;
  int RTg, KSg, Sg;
  int RTd, KSd, RPWd, RGd;
  // decode path
  int G;    // persistent workgroups
  int Srw;  // router k-splits across workgroups
  int U8;   // gate/up units per expert: 8 gate + 8 up rows each
  int lds_red, lds_grp, lds_scr, lds_total;  // dynamic LDS layout, bytes
  int NX;      // gate/up: activation rows staged in LDS per round (also the chunk size in tokens)
  int xpitch;  // staged row pitch in elements (K + 8: rows start in different banks)
  int pinned;  // 1: gate/up by whole units per wave, the rows of the workgroup's tokens in LDS (row t at t xpitch)
  int lds_pin;  // bytes of the pinned rows' region, room for every token's row (the last LDS region)
  int dn_cap;   // expert-major down: y rows staged per wave
  int stall;     // test hook (k3moe_debug_stall): > 0 makes the router-logit waits give up after this many polls
  int trace;      // 1: the decode kernel records phase timestamps at o_trace
  int single;     // 1: the single-token kernel runs the step (k3moe_single.hpp)
  int redundant;  // 1: every workgroup routes every token (no barrier before grouping)
  int xgemm;      // general path: 1 = grouped-GEMM expert kernels, 0 = per-16-token streams
  int fgemm;      // grouped GEMMs on the scaled FP4 MFMA with two-term E4M3 activations (k3moe_fgemm.hpp)
  int lat_in;     // single-token or decode kernel: 1 = it also computes the latent block's inputs (latent, shared_h)
  int lat_S;      // ... the shared experts' width S
  int lat_out;    // single-token or decode kernel: 1 = it also computes the latent block's output (lat_in too)
  // workspace byte offsets (o_ebf: the decode kernel's bf16 copy of the expert
  // sum, B x K, which the latent block's output phase reads)
  size_t o_ctl, o_zero, o_logit, o_ids, o_w, o_nact, o_active, o_aoff, o_acnt, o_ptok, o_pw, o_pof, o_gpart, o_gcnt,
      o_gchunk, o_h, o_y, o_xq, o_hq, o_ebf, o_trace, total;
};

__host__ __device__ inline int cdiv(long a, long b) { return (int)((a + b - 1) / b); }

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
__host__ __device__ inline int align16(int v) { return (v + 15) & ~15; }

// Decode-path LDS layout for plan p; returns the total bytes. Regions: red
// (the router's per-wave tiles; the staged gate/up's cut-group tiles), grp
// (the grouping lists), scr (top-k, grouping and down scratch; the staged
// gate/up's activation rows), then, when pinned, room for every token's row.
// Pinned: from 2 tokens up to as many as fit, gate/up gives each wave whole
// units (no staging rounds, no groups cut between waves) of chunks of up to 16
// tokens, and after the grouping each workgroup loads the rows of the tokens
// its units need, under its first weight loads.
inline int decode_lds(Plan &p) {
  const int room_all = kDecMaxLds - kDecStaticLds;
  p.xpitch = p.K + 8;
  p.lds_grp = align16(4 * (4 * p.Dmax + 1 + 4 * p.P));              // active list + chunk offsets + pairs + chunk experts
  p.redundant = p.B * p.E <= kRedundantKeys && p.B <= kRedundantTokens;
  {
    const int nt = p.redundant ? p.B : 1;
    const int topk = 8 * p.P + 4 * (3 * nt * p.E + kDecWaves * kMaxTopk) + 16 + kBlockTopkBytes;
    const int group = 8 * p.P + 4 * (4 * p.E + 32);
    int scr = topk > group ? topk : group;
    int down = (p.B <= 16 ? 2 : 1) * kDecWaves * p.B * 16 * 4;
    if (down < p.P * 16 * 4) down = p.P * 16 * 4;
    if (down > scr) scr = down;
    const int red = cdiv(p.B, 16) * kDecWaves * 256 * 4;
    const int pin = p.B * p.xpitch * 2;
    // the expert-major down's y stage takes what is left, up to kDnStage rows per wave
    int cap = (room_all - red - p.lds_grp - pin - 16) / (kDecWaves * 36);
    if (cap > kDnStage) cap = kDnStage;
    cap &= ~15;
    if (kDecWaves * cap * 36 > scr) scr = kDecWaves * cap * 36;
    p.pinned = p.B >= 2 && p.K % 512 == 0 && cap >= 32 && red + p.lds_grp + align16(scr) + pin <= room_all;
    if (p.pinned) {
      p.lds_red = red;
      p.lds_scr = align16(scr);
      p.lds_pin = pin;
      p.dn_cap = cap;
      p.NX = 16;
      p.lds_total = p.lds_red + p.lds_grp + p.lds_scr + p.lds_pin;
      return p.lds_total;
    }
  }
  p.lds_pin = 0;
  p.dn_cap = kDnStage;
  p.lds_red = kDecWaves * 2 * 2 * 256 * 4;                          // per wave 2 x 2 16x16 fp32 tiles
  const int nt = p.redundant ? p.B : 1;
  const int routed = 8 * p.P;                                       // ids + weights per pair
  const int topk = routed + 4 * (3 * nt * p.E + kDecWaves * kMaxTopk) + 16 + kBlockTopkBytes;  // keys, scores, picks, block_topk
  const int group = routed + 4 * (4 * p.E + 32);                    // counts, offsets, bitmaps, wave sums
  int down = (p.B <= 16 ? 2 : 1) * kDecWaves * p.B * 16 * 4;       // paired down: per-wave accumulators (2 row tiles)
  if (down < kDecWaves * kDnStage * 36) down = kDecWaves * kDnStage * 36;  // expert-major down: per-wave y stages
  if (down < p.P * 16 * 4) down = p.P * 16 * 4;                     // row-tile down: one 16-row slice per pair
  int scr = topk;
  if (group > scr) scr = group;
  if (down > scr) scr = down;
  // gate/up stages activation rows in the same scratch: as many rows as fit, at most 16
  const int room = kDecMaxLds - kDecStaticLds - p.lds_red - p.lds_grp;
  p.NX = room > 0 ? room / (p.xpitch * 2) : 0;
  if (p.NX > 16) p.NX = 16;
  if (p.NX * p.xpitch * 2 > scr) scr = p.NX * p.xpitch * 2;
  p.lds_scr = align16(scr);
  if (p.NX < 1) return 1 << 30;  // no decode path
  p.lds_total = p.lds_red + p.lds_grp + p.lds_scr;
  return p.lds_total;
}

// The single-token kernel (k3moe_single.hpp) takes the step when it fits:
// one token, top-k <= 16 of at most 1024 experts, the expert width K a
// multiple of 512 (whole 512-column gate/up super-steps, at most kSingleMaxSS
// per wave) and at most 8192 (its staged row), I <= 512 (the down
// projection's k-steps, at most 4), at most two 16-row output tiles per
// workgroup, the workgroup's gate/up units times a wave's super-steps at most
// kSingleSlots (all loaded at once), and its tagged partials
// and intermediates fitting the tag area. Its dynamic LDS: the keys (3 E
// words), the staged row (2 K bytes), fixed scratch, the top-k's, the chosen
// experts' h (2 k I bytes) and the down products (2 row tiles x k x 16 fp32).
constexpr int kSingleMaxSS = 2;  // gate/up super-steps of 512 columns per wave: ceil(K / 4096)
constexpr int kSingleMaxK = kSingleMaxSS * 8 * 512;  // 8192: the expert width K
constexpr int kSingleMaxTopk = 16;
constexpr int kSingleRouterRows = 4;  // router rows (experts) per workgroup: E <= 4 G
constexpr int kSingleSlots = 4;  // gate/up register slots per wave: units of the workgroup x super-steps per wave
constexpr int kSingleScratchBytes = 3840;
__host__ __device__ inline int single_lds(const Plan &p) {
  return align16(3 * 4 * p.E) + 2 * p.K + kSingleScratchBytes + kBlockTopkBytes + align16(2 * p.k * p.I) +
         2 * p.k * 16 * 4;
}
// With the latent block's output (Plan::lat_out) the expert sum [K] fp32 and
// [en | shared_h] [K + S] bf16 follow, from this (16-byte aligned) offset.
__host__ __device__ inline int single_lds_base(const Plan &p) { return align16(single_lds(p)); }
inline void single_plan(const k3moe_dims &d, Plan &p) {
  const bool tags_fit = (long)kTagCopies * p.E * 8 + (long)p.k * (p.I / 2) * 8 <= kTagBytes;
  p.single = (d.path == K3MOE_PATH_AUTO || d.path == K3MOE_PATH_SINGLE) && p.B == 1 && p.k <= kSingleMaxTopk &&
             p.E <= kMaxExperts && p.K % 512 == 0 && p.K <= kSingleMaxSS * kDecWaves * 512 && p.I <= 512 &&
             p.I % 32 == 0 && p.h % 128 == 0 && p.h <= 16 * kDecThreads && p.E <= kSingleRouterRows * p.G &&
             p.RTd <= 2 * p.G &&
             cdiv(p.k * (p.I / 8), p.G) * (p.K / 512 > kDecWaves ? 2 : 1) <= kSingleSlots && tags_fit;
}

// The persistent kernels with the latent block's inputs (latent and shared_h,
// the projections of kimi.py:317 and 326). The single-token kernel: workgroup
// b computes a contiguous share of the latent row pairs and of the shared pairs (gate and up row)
// of width h, at most kLatRowsMax rows in all, and publishes the
// latent in tagged slots (one per row pair, after the logits and the h slots)
// that every workgroup polls before its gate/up products. Returns whether one
// of the two kernels takes them for shared width S (setting lat_in, lat_S).
constexpr int kLatRowsMax = 48;  // rows (latent rows + shared gate and up rows) per workgroup
// The decode kernel's latent phases: their reduction area (the first 32 KiB of
// the dynamic LDS: 2 parts x 2 tiles x 8 waves x 256 fp32), then their staged
// token rows. The workgroup's LDS holds nothing else while they run.
constexpr int kLatRedBytes = 32768;
// The single-token kernel's latent block output (Plan::lat_out): a lane's
// 16-byte chunks of a row of [latent_up | shared_down] (K + S <= 64 x 8 x
// kLatOutChunks), output rows per wave, the expert sum's width, its RMS epsilon
// (kimi.py:325) and the slots a thread polls for [expert sum | shared_h].
constexpr int kLatOutChunks = 9, kLatOutRowsPerWave = 4, kLatOutMaxK = 4096;
constexpr int kLatOutRow1Bytes = 8 * kLatOutChunks * 1024;  // the single-token kernel: each wave's second output row
constexpr int kLatOutPoll = (kLatOutMaxK + 512 + 511) / 512;  // K + S <= 64 x 8 x 9 = 4608 < 9 x 512 + 1
constexpr float kLatOutRmsEps = 1e-5f;
inline int lat_rows_max(const Plan &p, int S) { return 2 * cdiv(p.K / 2, p.G) + 2 * cdiv(S, p.G); }
__host__ __device__ inline uint32_t lat_slot_base(const Plan &p) { return (uint32_t)(kTagCopies * p.E * 8 + p.k * (p.I / 2) * 8); }
// The decode kernel takes them too with the pinned gate/up and at most 16
// tokens (one MFMA token tile) whose rows of x fit in LDS after kLatRedBytes
// (row pitch h + 8; at most 8 tokens of h 7168): the G - B workgroups
// that route no token share the rows out in whole pairs, at most 16 pairs
// (two 16-row tiles) each.
inline bool lat_in_plan(Plan &p, int S) {
  const bool single = p.single && S > 0 && lat_rows_max(p, S) <= kLatRowsMax &&
                      (long)lat_slot_base(p) + (long)(p.K / 2) * 8 <= kTagBytes;
  const long lds_x = (long)kLatRedBytes + (long)p.B * (p.h + 8) * 2;
  const bool decode = !p.single && p.path == kPathDecode && p.pinned && !p.redundant && p.B <= 16 && S > 0 &&
                      p.h % 512 == 0 && p.G > p.B && cdiv((p.K + 2 * S) / 2, p.G - p.B) <= 16 &&
                      lds_x <= kDecMaxLds - kDecStaticLds;
  const bool ok = single || decode;
  p.lat_in = ok ? 1 : 0;
  p.lat_S = ok ? S : 0;
  if (ok && decode && lds_x > p.lds_total) p.lds_total = (int)lds_x;
  return ok;
}

// The single-token kernel also takes the block's output (after lat_in_plan):
// K <= kLatOutMaxK, K + S within a lane's chunks, at most kLatOutRowsPerWave
// output rows per wave (h <= 32 G), the expert sum and [en | shared_h] in LDS.
// The decode kernel takes it too with its latent projections and at most 8
// tokens (wave t normalises token t): K and S multiples of 128, K <= 4096, at
// most 32 output rows per workgroup, [en | shared_h] of every token and then
// latent_norm in LDS after kLatRedBytes, the expert sum's bf16 copy at o_ebf.
inline bool lat_out_plan(Plan &p) {
  const int S = p.lat_S;
  if (p.single) {
    const long lds = (long)single_lds_base(p) + align16(4 * p.K) + align16(2 * (p.K + S)) + kLatOutRow1Bytes;
    const bool ok = p.lat_in && p.K <= kLatOutMaxK && p.K % 8 == 0 && S % 8 == 0 &&
                    p.K + S <= 64 * 8 * kLatOutChunks && cdiv(p.h, p.G) <= kDecWaves * kLatOutRowsPerWave &&
                    (long)lat_slot_base(p) + (long)(p.K / 2 + S + p.K) * 8 <= kTagBytes &&
                    lds <= kDecMaxLds - kDecStaticLds;
    p.lat_out = ok ? 1 : 0;
    if (ok) p.lds_total = (int)lds;
    return ok;
  }
  const long lds = (long)kLatRedBytes + align16((long)p.B * (p.K + S + 8) * 2) + 2 * kLatOutMaxK;
  const bool ok = p.lat_in && p.path == kPathDecode && p.B <= kDecWaves && p.G <= kLatFlagsMax && p.o_ebf &&
                  p.K % 128 == 0 && S % 128 == 0 &&
                  p.K <= kLatOutMaxK && cdiv(p.h, p.G) <= 32 && lds <= kDecMaxLds - kDecStaticLds;
  p.lat_out = ok ? 1 : 0;
  if (ok && lds > p.lds_total) p.lds_total = (int)lds;
  return ok;
}

// n_cus: compute units of the device (the persistent grid size); trace: reserve
// a timestamp area (kTraceSlots x 8 bytes per workgroup, up to 1024 groups).
inline void make_plan(const k3moe_dims &d, int n_cus, Plan &p, int trace = 0) {
  p.B = d.tokens; p.E = d.experts; p.k = d.topk; p.h = d.hidden; p.K = d.latent; p.I = d.inter;
  p.gating = d.gating; p.act = d.activation;
  p.P = p.B * p.k;
  p.Dmax = p.E < p.P ? p.E : p.P;
  p.Epad = cdiv(p.E, 16) * 16;
  p.RTr = cdiv(p.E, 16);
  p.TTr = cdiv(p.B, 16);
  p.KSr = cdiv(p.h, 128);
  p.RTg = p.I / 16;
  p.KSg = cdiv(p.K, 128);
  p.RTd = p.K / 16;
  p.KSd = cdiv(p.I, 128);
  p.RPWd = 4;
  p.RGd = cdiv(p.RTd, p.RPWd);
  p.U8 = p.I / 8;

  // decode path when the token count, pair count and LDS layout fit. The
  // choice and the workspace size use the largest router split (srw_cap), so
  // they do not depend on the device's CU count; the split used is smaller
  // when the grid is small.
  // persistent grid: the largest power of two <= the CU count (at most 1024),
  // so that the barrier's group and member counts are powers of two and its
  // wrapping counters stay consistent (MI355X: all 256 CUs)
  p.G = 1;
  while (p.G * 2 <= n_cus && p.G * 2 <= 1024) p.G *= 2;
  long base = (long)p.RTr * p.TTr;
  // (a split of fewer k-steps than waves leaves waves idle, but spreads the
  // router and x reads over more workgroups)
  int srw_cap = kDecMaxSplits;
  if (srw_cap > p.KSr) srw_cap = p.KSr;
  if (srw_cap < 1) srw_cap = 1;
  // the decode kernel's router partials, [B][Srw][Epad] tagged slots, fit the tag area
  const long part_room = kTagBytes - kTagDecPart;
  while (srw_cap > 1 && (long)srw_cap * p.B * p.Epad * 8 > part_room) --srw_cap;
  p.Srw = srw_cap;
  p.path = kPathGeneral;
  if ((d.path == K3MOE_PATH_AUTO || d.path == K3MOE_PATH_DECODE || d.path == K3MOE_PATH_SINGLE) &&
      p.B <= kDecMaxTokens && p.P <= kDecMaxPairs && (long)p.B * p.Epad * 8 <= part_room &&
      decode_lds(p) <= kDecMaxLds - kDecStaticLds)
    p.path = kPathDecode;
  // general path expert kernels: grouped GEMMs when the experts average at
  // least kXMinPairsPerExpert tokens (and the widths allow 128-k steps)
  const bool widths = p.K % 128 == 0 && p.I % 128 == 0;
  p.xgemm = d.path == K3MOE_PATH_GROUPED || d.path == K3MOE_PATH_GROUPED_BF16 ||
            (d.path != K3MOE_PATH_STREAMED && widths && (long)p.P >= (long)kXMinPairsPerExpert * p.E);
  // the FP4-MFMA grouped GEMMs take whole units of output rows: 256 of I for gate/up, 512 of K for down
  // and whole 128-k steps
  p.fgemm = p.xgemm && d.path != K3MOE_PATH_GROUPED_BF16 && p.K % 512 == 0 && p.I % 256 == 0;
  p.Srw = (int)(p.G / p.RTr);  // decode router units: (row tile, split), every token tile
  if (p.Srw > srw_cap) p.Srw = srw_cap;
  if (p.Srw < 1) p.Srw = 1;
  decode_lds(p);

  // general path splits: router tiles of 64 tokens x 384 experts, at least 256 workgroups
  // (at most 8 splits), gate/up about 2048 waves
  p.Sr = cdiv(256, (long)cdiv(p.B, 64) * cdiv(p.E, 384));
  if (p.Sr > kMaxRouterSplits) p.Sr = kMaxRouterSplits;
  if (p.Sr > p.KSr) p.Sr = p.KSr;
  if (p.Sr < 1) p.Sr = 1;
  base = (long)p.Dmax * p.RTg;
  p.Sg = cdiv(2048, base);
  if (p.Sg > p.KSg) p.Sg = p.KSg;
  if (p.Sg < 1) p.Sg = 1;
  const int logit_splits = p.path == kPathDecode ? 0 : p.Sr;  // decode: partials in the tag area
  if (p.path == kPathDecode) p.Sr = p.Srw;

  size_t o = 0;
  auto take = [&](size_t bytes) { size_t at = o; o = align256(o + bytes); return at; };
  p.o_ctl = take(4096);
  p.o_zero = take(kZeroBytes);
  take(kLatCntBytes);  // the latent block's counters, kept by MoE steps on a shared workspace
  take(kTagBytes);     // the persistent kernels' tagged exchange area
  p.o_logit = take((size_t)logit_splits * p.B * p.Epad * 4);
  p.o_ids = take((size_t)p.P * 4);
  p.o_w = take((size_t)p.P * 4);
  p.o_nact = take(4);
  p.o_active = take((size_t)p.E * 4);
  p.o_aoff = take((size_t)p.E * 4);
  p.o_acnt = take((size_t)p.E * 4);
  p.o_ptok = take((size_t)p.P * 4);
  p.o_pw = take((size_t)p.P * 4);
  p.o_pof = take((size_t)p.P * 4);
  const bool general = p.path == kPathGeneral;
  p.o_gpart = take(general && p.Sg > 1 ? (size_t)p.Sg * p.P * 2 * p.I * 4 : 0);
  p.o_gcnt = take(general ? (size_t)p.Dmax * p.RTg * 4 : 0);
  p.o_gchunk = take(general ? (size_t)cdiv(p.B, kGroupChunk) * p.E * 4 : 0);  // grouping: per-chunk counts
  const bool fg = general && p.fgemm;
  p.o_h = take(fg ? 0 : (size_t)p.P * p.I * 2);
  // two-term E4M3 activations of the FP4-MFMA GEMMs: expert inputs [B, K] and h [P, I]
  // (hi, lo, then the hi and lo block scales)
  p.o_xq = take(fg ? (size_t)p.B * p.K * 2 + (size_t)p.B * (p.K / 32) * 2 : 0);
  p.o_hq = take(fg ? (size_t)p.P * p.I * 2 + (size_t)p.P * (p.I / 32) * 2 : 0);
  // pair outputs: the general path, and the decode path's expert-major down (I = 256, 384, 512)
  p.o_y = take((general || p.I == 256 || p.I == 384 || p.I == 512) ? (size_t)p.P * p.K * 2 : 0);
  p.trace = trace && p.path == kPathDecode;
  p.stall = 0;
  p.lat_in = 0;
  p.lat_S = 0;
  p.lat_out = 0;
  p.o_ebf = take(p.path == kPathDecode && p.B <= kDecWaves ? (size_t)p.B * p.K * 2 : 0);
  single_plan(d, p);
  if (p.single) {
    p.path = kPathDecode;
    p.lds_total = single_lds(p);
  }
  p.o_trace = p.trace ? take((size_t)1024 * kTraceSlots * 8) : 0;  // last area of the workspace
  p.total = o;
}

}  // namespace k3moe
