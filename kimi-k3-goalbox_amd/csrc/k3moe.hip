// k3moe: MXFP4 mixture-of-experts step for MI355X (gfx950), C ABI.
//
// Replaces the MoE block of the reference's Kimi K3 decode oracle
// (megabench/tasks/kimi.py:307-324) and its MXFP4 decode
// (megabench/tasks/quantization.py:40-51). Declarations: include/k3moe.h.
//
// Dispatch: B <= 64 tokens (and B*k <= 1024) runs the persistent decode
// kernel (k3moe_decode.hpp); larger batches run the six-kernel general path
// (k3moe_general.hpp). Both are enqueued on the caller's stream with no host
// synchronisation and no device allocation.
#include <hip/hip_runtime.h>
#include <stdarg.h>

#include <atomic>
#include <mutex>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "k3moe.h"
#include "k3moe_codec.hpp"
#include "k3moe_decode.hpp"
#include "k3moe_device.hpp"
#include "k3moe_fgemm.hpp"
#include "k3moe_general.hpp"
#include "k3moe_latent.hpp"
#include "k3moe_plan.hpp"
#include "k3moe_single.hpp"
#include "k3moe_xgemm.hpp"

using namespace k3moe;

// The allocation-free entry point's workspace (k3moe_moe_step_noalloc): one
// copy per GPU the library runs on, held until the process ends. Its address
// on a device comes from hipGetSymbolAddress with that device current (the
// name is only a host-side stand-in); every call on a GPU shares it.
constexpr size_t kScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

namespace {

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
  if (d->path < K3MOE_PATH_AUTO || d->path > K3MOE_PATH_GROUPED_BF16)
    return fail(K3MOE_EINVAL, "unknown path %d", d->path);
  if ((d->path == K3MOE_PATH_GROUPED || d->path == K3MOE_PATH_GROUPED_BF16) && (d->latent % 128 || d->inter % 128))
    return fail(K3MOE_EINVAL, "the grouped GEMM path needs latent (%d) and inter (%d) multiples of 128", d->latent,
                d->inter);
  if ((long)d->tokens * d->topk > (1L << 30)) return fail(K3MOE_EINVAL, "tokens*topk too large");
  return K3MOE_OK;
}

// Compute units of the current device, cached per device ordinal. Without a
// usable device (workspace sizing on a host without a GPU) the MI355X count
// is assumed: the decode-path workspace does not depend on it beyond the
// router split, which is bounded.
constexpr int kDefaultCus = 256;
int g_cus[64];

int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return kDefaultCus;
  }
  if (g_cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
      (void)hipGetLastError();
      return kDefaultCus;
    }
    g_cus[dev] = n;
  }
  return g_cus[dev];
}

// K3MOE_TRACE=1 in the environment makes decode steps record per-workgroup
// phase timestamps (32 x uint64 per workgroup, 100 MHz) in the last 256 KiB
// of the workspace, a profiling aid; the workspace size includes that area.
// Test hook (k3moe_debug_stall): > 0 makes every later step's router-logit
// waits give up after this many polls; 0, the default, leaves them bounded by
// kSpinLimit only.
std::atomic<int> g_stall{0};

int trace_enabled() {
  static int v = -1;
  if (v < 0) {
    const char *e = getenv("K3MOE_TRACE");
    v = (e && e[0] == '1') ? 1 : 0;
  }
  return v;
}

int launch_check(const char *what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(K3MOE_EHIP, "%s launch failed: %s", what, hipGetErrorString(err));
  return K3MOE_OK;
}

// Lets the decode kernel use more than 64 KiB of dynamic LDS (once per process).
// Raises kernel fn's dynamic LDS limit to `limit` bytes (once per kernel and process).
int grant_lds(const void *fn, int limit, int &granted, const char *what) {
  if (granted >= limit) return K3MOE_OK;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, limit) != hipSuccess)
    return fail(K3MOE_EHIP, "setting the %s kernel's LDS limit failed: %s", what, hipGetErrorString(hipGetLastError()));
  granted = limit;
  return K3MOE_OK;
}

// The decode kernel instantiation for a plan: whole gate/up super-steps (K a
// multiple of 512) and the expert-major down variant of its I.
typedef void (*DecodeKernel)(Plan, DecodeArgs);
DecodeKernel decode_kernel(const Plan &p, int &slot) {
  // the latent block's phases (which need whole 512-column gate/up chunks, AL)
  // in their own instantiations: row 2
  static const DecodeKernel table[3][4] = {
      {k_moe_decode<false, 0, false>, k_moe_decode<false, 2, false>, k_moe_decode<false, 3, false>,
       k_moe_decode<false, 4, false>},
      {k_moe_decode<true, 0, false>, k_moe_decode<true, 2, false>, k_moe_decode<true, 3, false>,
       k_moe_decode<true, 4, false>},
      {k_moe_decode<true, 0, true>, k_moe_decode<true, 2, true>, k_moe_decode<true, 3, true>,
       k_moe_decode<true, 4, true>}};
  const int al = (p.K / kBlockK) % 16 == 0 ? 1 : 0;
  const int row = p.lat_in ? 2 : al;  // (lat_in plans are pinned: AL)
  const int v = p.I == 256 ? 1 : p.I == 384 ? 2 : p.I == 512 ? 3 : 0;
  slot = row * 4 + v;
  return table[row][v];
}

// The single-token kernel's instantiation `slot` may use more than 64 KiB of dynamic LDS.
int allow_single_lds(const void *fn, int slot, int bytes) {
  static int granted[8] = {0};
  if (bytes <= 65536) return K3MOE_OK;
  return grant_lds(fn, kDecMaxLds - kDecStaticLds, granted[slot], "single-token");
}

int allow_lds(DecodeKernel fn, int slot, int bytes) {
  static int granted[12] = {0};
  if (bytes <= 65536) return K3MOE_OK;
  // dynamic + static LDS must fit the 160 KiB of a workgroup
  return grant_lds(reinterpret_cast<const void *>(fn), kDecMaxLds - kDecStaticLds, granted[slot], "decode");
}

int allow_xgemm_lds() {
  static int granted_gu = 0, granted_dn = 0;
  int rc = grant_lds(reinterpret_cast<const void *>(&k_xgemm<true>), kXLds, granted_gu, "gate/up GEMM");
  if (!rc) rc = grant_lds(reinterpret_cast<const void *>(&k_xgemm<false>), kXLds, granted_dn, "down GEMM");
  return rc;
}

int allow_fgemm_lds() {
  static int granted_gu = 0, granted_dn = 0;
  int rc = grant_lds(reinterpret_cast<const void *>(&k_fgemm<true>), kFLds, granted_gu, "FP4 gate/up GEMM");
  if (!rc) rc = grant_lds(reinterpret_cast<const void *>(&k_fgemm<false>), kFLds, granted_dn, "FP4 down GEMM");
  return rc;
}

int check_latent_dims(const k3moe_latent_dims *d) {
  if (!d) return fail(K3MOE_EINVAL, "dims is NULL");
  if (d->tokens < 1) return fail(K3MOE_EINVAL, "tokens must be >= 1, got %d", d->tokens);
  if (d->hidden < 128 || d->hidden % 128 || d->latent < 128 || d->latent % 128 || d->shared < 128 ||
      d->shared % 128)
    return fail(K3MOE_EINVAL, "hidden (%d), latent (%d) and shared (%d) must be positive multiples of 128",
                d->hidden, d->latent, d->shared);
  if (d->activation != K3MOE_ACT_SITU && d->activation != K3MOE_ACT_SILU)
    return fail(K3MOE_EINVAL, "unknown activation %d", d->activation);
  return K3MOE_OK;
}

// Plans of both latent kernels for a launch of min(tokens, kLatMaxTokens)
// tokens (larger batches run as consecutive launches of up to that many; the
// workspace covers the larger plan of the full launch, which also covers a
// shorter last one).
int latent_plans(const k3moe_latent_dims *d, int n_cus, LatPlan &pin, LatPlan &pout) {
  int rc = check_latent_dims(d);
  if (rc) return rc;
  k3moe_latent_dims c = *d;
  if (c.tokens > kLatMaxTokens) c.tokens = kLatMaxTokens;
  const char *why = latent_plan(c, n_cus, 0, pin);
  if (!why) why = latent_plan(c, n_cus, 1, pout);
  if (why) return fail(K3MOE_EINVAL, "latent block geometry B=%d h=%d lh=%d S=%d: %s", d->tokens, d->hidden,
                       d->latent, d->shared, why);
  if (trace_enabled()) {  // one trace area for both kernels, the last 1024 x kTraceSlots x 8 bytes
    const long at = pin.total > pout.total ? pin.total : pout.total;
    pin.o_trace = pout.o_trace = at;
    pin.total = pout.total = at + 1024L * kTraceSlots * 8;
  }
  return K3MOE_OK;
}

int allow_latent_lds(int out, int sk, int bytes) {
  static int granted[2][2] = {{0, 0}, {0, 0}};
  if (bytes <= 65536) return K3MOE_OK;
  const void *fn = sk ? (out ? reinterpret_cast<const void *>(&k_latent_sk<1>)
                             : reinterpret_cast<const void *>(&k_latent_sk<0>))
                      : (out ? reinterpret_cast<const void *>(&k_latent<1>)
                             : reinterpret_cast<const void *>(&k_latent<0>));
  return grant_lds(fn, kLatMaxLds, granted[sk][out], "latent block");
}

int latent_launch(const k3moe_latent_dims *dims, int out, const LatArgs &a, size_t workspace_bytes, void *stream) {
  LatPlan pin, pout;
  int rc = latent_plans(dims, device_cus(), pin, pout);
  if (rc) return rc;
  const size_t need = (size_t)(pin.total > pout.total ? pin.total : pout.total);
  if (!a.ws || workspace_bytes < need)
    return fail(K3MOE_EWORKSPACE, "workspace of %zu bytes is smaller than the %zu required", workspace_bytes, need);
  if (reinterpret_cast<uintptr_t>(a.ws) % 256) return fail(K3MOE_EWORKSPACE, "workspace must be 256-byte aligned");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const long h = dims->hidden, lh = dims->latent, S = dims->shared;
  for (int b0 = 0; b0 < dims->tokens; b0 += kLatMaxTokens) {  // token rows b0 .. b0 + nb - 1
    k3moe_latent_dims c = *dims;
    c.tokens = dims->tokens - b0 < kLatMaxTokens ? dims->tokens - b0 : kLatMaxTokens;
    LatPlan p;
    const char *why = latent_plan(c, device_cus(), out, p);
    if (why) return fail(K3MOE_EINVAL, "latent block geometry B=%d h=%d lh=%d S=%d: %s", c.tokens, c.hidden,
                         c.latent, c.shared, why);
    p.o_trace = (out ? pout : pin).o_trace;
    LatArgs ac = a;
    if (!out) {
      ac.x = a.x + b0 * h;
      ac.ya = a.ya + b0 * lh;
      ac.yb = a.yb + b0 * S;
    } else {
      ac.x = a.x + b0 * S;
      ac.esum = a.esum + b0 * lh;
      ac.ya = a.ya + b0 * h;
    }
    if ((rc = allow_latent_lds(out, p.sk, p.lds_total))) return rc;
    if (p.sk && out) hipLaunchKernelGGL(k_latent_sk<1>, dim3(p.G), dim3(kLatThreads), p.lds_total, st, p, ac);
    else if (p.sk) hipLaunchKernelGGL(k_latent_sk<0>, dim3(p.G), dim3(kLatThreads), p.lds_total, st, p, ac);
    else if (out) hipLaunchKernelGGL(k_latent<1>, dim3(p.G), dim3(kLatThreads), p.lds_total, st, p, ac);
    else hipLaunchKernelGGL(k_latent<0>, dim3(p.G), dim3(kLatThreads), p.lds_total, st, p, ac);
    if ((rc = launch_check(out ? "latent_out" : "latent_in"))) return rc;
  }
  return K3MOE_OK;
}

// The expert GEMMs' activation, elementwise (debug entry point k3moe_activation).
__global__ void k_activation(int act, int fast, const float *g, const float *u, float *out, long n) {
  for (long j = (long)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += (long)gridDim.x * blockDim.x)
    out[j] = fast ? fast_act(act, g[j], u[j]) : apply_act(act, g[j], u[j]);
}

__global__ void k_zero_words(uint32_t *p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// The device address of `scratch` on the current device, looked up once per
// device. The first lookup also zeroes its control block, zero area, counters
// and tag area with a kernel on `st` and waits for it (once per device and
// process), so that calls on any stream after it find the array initialised;
// a first call inside a stream capture would record that kernel instead of
// running it, so it is refused with a message.
std::mutex g_scratch_mu;
void *g_scratch[64];

bool scratch_ready() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return g_scratch[dev] != nullptr;
}

int scratch_address(void **out, hipStream_t st) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess)
    return fail(K3MOE_EHIP, "hipGetDevice failed: %s", hipGetErrorString(hipGetLastError()));
  if (dev < 0 || dev >= 64) return fail(K3MOE_EINVAL, "device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cap) != hipSuccess)
      return fail(K3MOE_EHIP, "hipStreamIsCapturing failed: %s", hipGetErrorString(hipGetLastError()));
    if (cap != hipStreamCaptureStatusNone)
      return fail(K3MOE_EINVAL,
                  "the allocation-free scratch of device %d is initialised by the first call on that device, "
                  "which must not be captured: call k3moe_workspace_init(NULL, 0, stream) once before capturing",
                  dev);
    void *ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr)
      return fail(K3MOE_EHIP, "hipGetSymbolAddress(scratch) on device %d failed: %s", dev, hipGetErrorString(err));
    hipLaunchKernelGGL(k_zero_words, dim3(cdiv(kInitBytes / 4, 256)), dim3(256), 0, st, reinterpret_cast<uint32_t *>(ptr),
                       kInitBytes / 4);
    int rc = launch_check("scratch init");
    if (rc) return rc;
    if (hipStreamSynchronize(st) != hipSuccess)
      return fail(K3MOE_EHIP, "waiting for the scratch init on device %d failed: %s", dev,
                  hipGetErrorString(hipGetLastError()));
    g_scratch[dev] = ptr;
  }
  *out = g_scratch[dev];
  return K3MOE_OK;
}

}  // namespace

extern "C" {

const char *k3moe_last_error(void) { return g_err; }

const char *k3moe_version(void) { return "k3moe 0.2 gfx950"; }

int k3moe_workspace_bytes(const k3moe_dims *dims, size_t *bytes) {
  g_err[0] = 0;
  int rc = check_dims(dims);
  if (rc) return rc;
  if (!bytes) return fail(K3MOE_EINVAL, "bytes is NULL");
  Plan p;
  make_plan(*dims, kDefaultCus, p, trace_enabled());
  *bytes = p.total;
  return K3MOE_OK;
}

int k3moe_workspace_layout(const k3moe_dims *dims, k3moe_layout *layout) {
  g_err[0] = 0;
  int rc = check_dims(dims);
  if (rc) return rc;
  if (!layout) return fail(K3MOE_EINVAL, "layout is NULL");
  Plan p;
  make_plan(*dims, device_cus(), p, trace_enabled());
  if (p.path == kPathDecode)
    return fail(K3MOE_EINVAL, "the persistent decode path keeps its grouping in LDS (tokens %d, pairs %d)", p.B, p.P);
  layout->active_count = (int64_t)p.o_nact;
  layout->active = (int64_t)p.o_active;
  layout->offsets = (int64_t)p.o_aoff;
  layout->counts = (int64_t)p.o_acnt;
  layout->pair_token = (int64_t)p.o_ptok;
  layout->pair_weight = (int64_t)p.o_pw;
  layout->pair_of = (int64_t)p.o_pof;
  const bool split = p.fgemm && p.xgemm;
  layout->pair_h = split ? -1 : (int64_t)p.o_h;
  layout->pair_y = (int64_t)p.o_y;
  layout->input_split = split ? (int64_t)p.o_xq : -1;
  layout->h_split = split ? (int64_t)p.o_hq : -1;
  return K3MOE_OK;
}

int k3moe_workspace_init(void *workspace, size_t workspace_bytes, void *stream) {
  g_err[0] = 0;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (!workspace) {  // the current device's allocation-free scratch
    void *ws = nullptr;
    const bool fresh = !scratch_ready();
    int rc = scratch_address(&ws, st);
    if (rc || fresh) return rc;  // a first lookup has just zeroed it
    workspace = ws;
    workspace_bytes = kScratchBytes;
  }
  if (workspace_bytes < (size_t)kInitBytes)
    return fail(K3MOE_EWORKSPACE, "workspace must hold at least %d bytes", kInitBytes);
  if (reinterpret_cast<uintptr_t>(workspace) % 256) return fail(K3MOE_EWORKSPACE, "workspace must be 256-byte aligned");
  hipLaunchKernelGGL(k_zero_words, dim3(cdiv(kInitBytes / 4, 256)), dim3(256), 0, st,
                     reinterpret_cast<uint32_t *>(workspace), kInitBytes / 4);
  return launch_check("workspace_init");
}

int k3moe_workspace_status(const void *workspace, int32_t *status, void *stream) {
  g_err[0] = 0;
  if (!status) return fail(K3MOE_EINVAL, "status is NULL");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (!workspace) {  // the current device's allocation-free scratch
    void *ws = nullptr;
    int rc = scratch_address(&ws, st);
    if (rc) return rc;
    workspace = ws;
  }
  uint32_t word = 0;
  const uint32_t *src = reinterpret_cast<const uint32_t *>(workspace) + kCtlErr;
  if (hipMemcpyAsync(&word, src, 4, hipMemcpyDeviceToHost, st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess)
    return fail(K3MOE_EHIP, "reading the workspace status failed: %s", hipGetErrorString(hipGetLastError()));
  *status = (int32_t)word;
  return K3MOE_OK;
}

// The latent block's input projections for k3moe_latent_moe_step's one-launch
// path: the single-token kernel computes latent (into `latent`) and shared_h.
struct LatInArgs {
  int S;
  const void *latent_down, *shared_gate, *shared_up;
  void *latent, *shared_h;
  // the block's output too when the single-token kernel takes it (out != NULL; *did_out reports it)
  const void *latent_norm, *latent_up, *shared_down;
  void *out;
  bool *did_out;
};
constexpr int kNotFused = -1000;  // moe_step_impl: the plan has no one-launch latent path

static int moe_step_impl(const k3moe_dims *dims, const void *x, const void *latent, const void *router,
                         const float *router_bias, const uint8_t *gate_blocks, const uint8_t *gate_scales,
                         const uint8_t *up_blocks, const uint8_t *up_scales, const uint8_t *down_blocks,
                         const uint8_t *down_scales, const int64_t *routes, float *expert_sum, int64_t *expert_ids,
                         float *route_weights, float *shortfall, void *workspace, size_t workspace_bytes,
                         void *stream, const LatInArgs *lat);

int k3moe_moe_step(const k3moe_dims *dims, const void *x, const void *latent, const void *router,
                   const float *router_bias, const uint8_t *gate_blocks, const uint8_t *gate_scales,
                   const uint8_t *up_blocks, const uint8_t *up_scales, const uint8_t *down_blocks,
                   const uint8_t *down_scales, const int64_t *routes, float *expert_sum, int64_t *expert_ids,
                   float *route_weights, float *shortfall, void *workspace, size_t workspace_bytes,
                   void *stream) {
  g_err[0] = 0;
  return moe_step_impl(dims, x, latent, router, router_bias, gate_blocks, gate_scales, up_blocks, up_scales,
                       down_blocks, down_scales, routes, expert_sum, expert_ids, route_weights, shortfall, workspace,
                       workspace_bytes, stream, nullptr);
}

int k3moe_latent_moe_step(const k3moe_dims *dims, int32_t shared, const void *x, const void *latent_down,
                          const void *shared_gate, const void *shared_up, void *latent, void *shared_h,
                          const void *router, const float *router_bias, const uint8_t *gate_blocks,
                          const uint8_t *gate_scales, const uint8_t *up_blocks, const uint8_t *up_scales,
                          const uint8_t *down_blocks, const uint8_t *down_scales, const int64_t *routes,
                          float *expert_sum, int64_t *expert_ids, float *route_weights, float *shortfall,
                          void *workspace, size_t workspace_bytes, void *stream) {
  g_err[0] = 0;
  if (!latent_down || !shared_gate || !shared_up || !latent || !shared_h)
    return fail(K3MOE_EINVAL, "a required pointer is NULL");
  if (!dims) return fail(K3MOE_EINVAL, "dims is NULL");
  const LatInArgs lat{shared, latent_down, shared_gate, shared_up, latent, shared_h,
                      nullptr, nullptr, nullptr, nullptr, nullptr};
  int rc = moe_step_impl(dims, x, latent, router, router_bias, gate_blocks, gate_scales, up_blocks, up_scales,
                         down_blocks, down_scales, routes, expert_sum, expert_ids, route_weights, shortfall,
                         workspace, workspace_bytes, stream, &lat);
  if (rc != kNotFused) return rc;
  // two launches: the input projections, then the step on their latent
  const k3moe_latent_dims ld{dims->tokens, dims->hidden, dims->latent, shared, dims->activation};
  if ((rc = k3moe_latent_in(&ld, x, latent_down, shared_gate, shared_up, latent, shared_h, workspace,
                            workspace_bytes, stream)))
    return rc;
  return k3moe_moe_step(dims, x, latent, router, router_bias, gate_blocks, gate_scales, up_blocks, up_scales,
                        down_blocks, down_scales, routes, expert_sum, expert_ids, route_weights, shortfall,
                        workspace, workspace_bytes, stream);
}

int k3moe_latent_block(const k3moe_dims *dims, int32_t shared, const void *x, const void *latent_down,
                       const void *shared_gate, const void *shared_up, const void *latent_norm,
                       const void *latent_up, const void *shared_down, const void *router,
                       const float *router_bias, const uint8_t *gate_blocks, const uint8_t *gate_scales,
                       const uint8_t *up_blocks, const uint8_t *up_scales, const uint8_t *down_blocks,
                       const uint8_t *down_scales, const int64_t *routes, void *latent, void *shared_h,
                       float *expert_sum, int64_t *expert_ids, float *route_weights, float *shortfall, void *out,
                       void *workspace, size_t workspace_bytes, void *stream) {
  g_err[0] = 0;
  if (!latent_down || !shared_gate || !shared_up || !latent_norm || !latent_up || !shared_down || !latent ||
      !shared_h || !out)
    return fail(K3MOE_EINVAL, "a required pointer is NULL");
  if (!dims) return fail(K3MOE_EINVAL, "dims is NULL");
  bool did_out = false;
  const LatInArgs lat{shared, latent_down, shared_gate, shared_up, latent, shared_h,
                      latent_norm, latent_up, shared_down, out, &did_out};
  int rc = moe_step_impl(dims, x, latent, router, router_bias, gate_blocks, gate_scales, up_blocks, up_scales,
                         down_blocks, down_scales, routes, expert_sum, expert_ids, route_weights, shortfall,
                         workspace, workspace_bytes, stream, &lat);
  const k3moe_latent_dims ld{dims->tokens, dims->hidden, dims->latent, shared, dims->activation};
  if (rc == kNotFused) {  // the input projections, then the step on their latent
    if ((rc = k3moe_latent_in(&ld, x, latent_down, shared_gate, shared_up, latent, shared_h, workspace,
                              workspace_bytes, stream)))
      return rc;
    rc = k3moe_moe_step(dims, x, latent, router, router_bias, gate_blocks, gate_scales, up_blocks, up_scales,
                        down_blocks, down_scales, routes, expert_sum, expert_ids, route_weights, shortfall,
                        workspace, workspace_bytes, stream);
  }
  if (rc || did_out) return rc;
  return k3moe_latent_out(&ld, expert_sum, latent_norm, latent_up, shared_h, shared_down, out, workspace,
                          workspace_bytes, stream);
}

static int moe_step_impl(const k3moe_dims *dims, const void *x, const void *latent, const void *router,
                         const float *router_bias, const uint8_t *gate_blocks, const uint8_t *gate_scales,
                         const uint8_t *up_blocks, const uint8_t *up_scales, const uint8_t *down_blocks,
                         const uint8_t *down_scales, const int64_t *routes, float *expert_sum, int64_t *expert_ids,
                         float *route_weights, float *shortfall, void *workspace, size_t workspace_bytes,
                         void *stream, const LatInArgs *lat) {
  int rc = check_dims(dims);
  if (rc) return rc;
  if (!x || !router || !gate_blocks || !gate_scales || !up_blocks || !up_scales || !down_blocks ||
      !down_scales || !expert_sum || !expert_ids || !route_weights)
    return fail(K3MOE_EINVAL, "a required pointer is NULL");
  if (!latent && dims->latent != dims->hidden)
    return fail(K3MOE_EINVAL, "latent width %d differs from hidden %d but no latent input was given",
                dims->latent, dims->hidden);
  Plan p;
  make_plan(*dims, device_cus(), p, trace_enabled());
  p.stall = g_stall.load(std::memory_order_relaxed);
  if (lat && !lat_in_plan(p, lat->S)) return kNotFused;
  if (lat && lat->out) *lat->did_out = lat_out_plan(p);
  if (dims->path == K3MOE_PATH_DECODE && p.path != kPathDecode)
    return fail(K3MOE_EINVAL, "the persistent decode path needs tokens <= %d and tokens*topk <= %d", kDecMaxTokens,
                kDecMaxPairs);
  if (dims->path == K3MOE_PATH_SINGLE && !p.single)
    return fail(K3MOE_EINVAL,
                "the single-token kernel needs tokens == 1, topk <= 16, experts <= 1024, latent a multiple of 512 "
                "up to 8192, inter <= 512 (got tokens %d, topk %d, experts %d, latent %d, inter %d)",
                dims->tokens, dims->topk, dims->experts, dims->latent, dims->inter);
  if (!workspace || workspace_bytes < p.total)
    return fail(K3MOE_EWORKSPACE, "workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
                p.total);
  if (reinterpret_cast<uintptr_t>(workspace) % 256)
    return fail(K3MOE_EWORKSPACE, "workspace must be 256-byte aligned");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char *ws = reinterpret_cast<char *>(workspace);
  const uint16_t *xin = reinterpret_cast<const uint16_t *>(latent ? latent : x);

  if (p.path == kPathDecode) {
    DecodeArgs a{};
    a.x = reinterpret_cast<const uint16_t *>(x);
    a.xin = xin;
    a.router = reinterpret_cast<const uint16_t *>(router);
    a.bias = router_bias;
    a.gblk = gate_blocks; a.gscl = gate_scales;
    a.ublk = up_blocks; a.uscl = up_scales;
    a.dblk = down_blocks; a.dscl = down_scales;
    a.routes = routes;
    a.out = expert_sum;
    a.out_ids = expert_ids;
    a.out_w = route_weights;
    a.out_short = shortfall;
    a.ws = ws;
    if (p.lat_in) {  // the kernel computes the latent into `latent` (the expert input) and shared_h
      a.lat_ld = reinterpret_cast<const uint16_t *>(lat->latent_down);
      a.lat_sg = reinterpret_cast<const uint16_t *>(lat->shared_gate);
      a.lat_su = reinterpret_cast<const uint16_t *>(lat->shared_up);
      a.lat_sh = reinterpret_cast<uint16_t *>(lat->shared_h);
      a.xin = reinterpret_cast<const uint16_t *>(lat->latent);
    }
    if (p.lat_out) {  // ... and the block's output
      a.lat_norm = reinterpret_cast<const uint16_t *>(lat->latent_norm);
      a.lat_up = reinterpret_cast<const uint16_t *>(lat->latent_up);
      a.lat_sd = reinterpret_cast<const uint16_t *>(lat->shared_down);
      a.lat_y = reinterpret_cast<uint16_t *>(lat->out);
    }
    if (p.single) {
      // instantiations: chosen experts per wave in the down phase (1: k <= 8, 2: k <= 16) and
      // the down projection's k-steps (2: I <= 256, 4: I <= 512)
      // (and the latent block's phases: a separate instantiation)
      const bool je2 = p.k > kDecWaves, ks4 = p.I > 256, lat = p.lat_in != 0;
      auto launch = [&](auto kernel) -> int {
        int r = allow_single_lds(reinterpret_cast<const void *>(kernel), lat * 4 + je2 * 2 + ks4, p.lds_total);
        if (r) return r;
        hipLaunchKernelGGL(kernel, dim3(p.G), dim3(kDecThreads), p.lds_total, st, p, a);
        return launch_check("single-token step");
      };
      if (lat) {
        if (je2 && ks4) return launch(k_moe_single<2, 4, true>);
        if (je2) return launch(k_moe_single<2, 2, true>);
        if (ks4) return launch(k_moe_single<1, 4, true>);
        return launch(k_moe_single<1, 2, true>);
      }
      if (je2 && ks4) return launch(k_moe_single<2, 4, false>);
      if (je2) return launch(k_moe_single<2, 2, false>);
      if (ks4) return launch(k_moe_single<1, 4, false>);
      return launch(k_moe_single<1, 2, false>);
    }
    int slot = 0;
    const DecodeKernel fn = decode_kernel(p, slot);
    if ((rc = allow_lds(fn, slot, p.lds_total))) return rc;
    hipLaunchKernelGGL(fn, dim3(p.G), dim3(kDecThreads), p.lds_total, st, p, a);
    return launch_check("decode step");
  }

  const int nr = cdiv(p.B, kRM) * cdiv(p.E, kRExperts) * p.Sr;
  hipLaunchKernelGGL(k_router, dim3(nr), dim3(kRWaves * 64), 0, st, p, reinterpret_cast<const uint16_t *>(x),
                     reinterpret_cast<const uint16_t *>(router), ws);
  if ((rc = launch_check("router"))) return rc;
  hipLaunchKernelGGL(k_topk, dim3(cdiv(p.B, kWavesPerBlock)), dim3(kThreads), 0, st, p, router_bias, routes, ws,
                     expert_ids, route_weights, shortfall);
  if ((rc = launch_check("topk"))) return rc;
  const int nch = cdiv(p.B, kGroupChunk);
  hipLaunchKernelGGL(k_group_count, dim3(nch), dim3(256), 0, st, p, ws);
  if ((rc = launch_check("group count"))) return rc;
  hipLaunchKernelGGL(k_group_scan, dim3(1), dim3(1024), 0, st, p, ws);
  if ((rc = launch_check("group scan"))) return rc;
  hipLaunchKernelGGL(k_group_place, dim3(nch), dim3(256), 0, st, p, ws);
  if ((rc = launch_check("group place"))) return rc;
  if (p.fgemm) {  // many tokens per expert: grouped GEMMs on the scaled FP4 MFMA
    if ((rc = allow_fgemm_lds())) return rc;
    uint8_t *xq = reinterpret_cast<uint8_t *>(ws + p.o_xq);
    const long nxb = (long)p.B * (p.K / kBlockK);
    MxAct ax{xq, xq + (size_t)p.B * p.K, xq + (size_t)2 * p.B * p.K, xq + (size_t)2 * p.B * p.K + nxb, p.K};
    long qg = (nxb + 31) / 32;
    if (qg > 8192) qg = 8192;
    hipLaunchKernelGGL(k_quant, dim3((unsigned)qg), dim3(256), 0, st, xin, nxb, const_cast<uint8_t *>(ax.hi),
                       const_cast<uint8_t *>(ax.lo), const_cast<uint8_t *>(ax.shi), const_cast<uint8_t *>(ax.slo));
    if ((rc = launch_check("activation split"))) return rc;
    hipLaunchKernelGGL(k_fgemm<true>, dim3(p.G), dim3(kFThreads), kFLds, st, p, ax, gate_blocks, gate_scales, up_blocks,
                       up_scales, ws);
    if ((rc = launch_check("FP4 gate/up GEMM"))) return rc;
    const uint8_t *hq = reinterpret_cast<const uint8_t *>(ws + p.o_hq);
    const size_t nh = (size_t)p.P * p.I;
    MxAct ah{hq, hq + nh, hq + 2 * nh, hq + 2 * nh + (size_t)p.P * (p.I / kBlockK), p.I};
    hipLaunchKernelGGL(k_fgemm<false>, dim3(p.G), dim3(kFThreads), kFLds, st, p, ah, down_blocks, down_scales, nullptr,
                       nullptr, ws);
    if ((rc = launch_check("FP4 down GEMM"))) return rc;
  } else if (p.xgemm) {  // grouped GEMMs on bf16 MFMA, weights decoded in registers
    if ((rc = allow_xgemm_lds())) return rc;
    hipLaunchKernelGGL(k_xgemm<true>, dim3(p.G), dim3(kXThreads), kXLds, st, p, xin, gate_blocks, gate_scales,
                       up_blocks, up_scales, ws);
    if ((rc = launch_check("gate/up GEMM"))) return rc;
    hipLaunchKernelGGL(k_xgemm<false>, dim3(p.G), dim3(kXThreads), kXLds, st, p,
                       reinterpret_cast<const uint16_t *>(ws + p.o_h), down_blocks, down_scales, nullptr, nullptr, ws);
    if ((rc = launch_check("down GEMM"))) return rc;
  } else {
    const long ng = (long)p.Dmax * p.RTg * p.Sg;
    hipLaunchKernelGGL(k_gateup, dim3(cdiv(ng, kWavesPerBlock)), dim3(kThreads), 0, st, p, xin, gate_blocks,
                       gate_scales, up_blocks, up_scales, ws);
    if ((rc = launch_check("gateup"))) return rc;
    const long nd = (long)p.Dmax * p.RGd;
    hipLaunchKernelGGL(k_down, dim3(cdiv(nd, kWavesPerBlock)), dim3(kThreads), 0, st, p, down_blocks, down_scales,
                       ws);
    if ((rc = launch_check("down"))) return rc;
  }
  const long nc = (long)p.B * (p.K / 8);
  hipLaunchKernelGGL(k_combine, dim3(cdiv(nc, 256)), dim3(256), 0, st, p, ws, expert_sum);
  return launch_check("combine");
}

int k3moe_latent_workspace_bytes(const k3moe_latent_dims *dims, size_t *bytes) {
  g_err[0] = 0;
  LatPlan pin, pout;
  int rc = latent_plans(dims, kDefaultCus, pin, pout);
  if (rc) return rc;
  if (!bytes) return fail(K3MOE_EINVAL, "bytes is NULL");
  *bytes = (size_t)(pin.total > pout.total ? pin.total : pout.total);
  return K3MOE_OK;
}

int k3moe_latent_in(const k3moe_latent_dims *dims, const void *x, const void *latent_down, const void *shared_gate,
                    const void *shared_up, void *latent, void *shared_h, void *workspace, size_t workspace_bytes,
                    void *stream) {
  g_err[0] = 0;
  if (!x || !latent_down || !shared_gate || !shared_up || !latent || !shared_h)
    return fail(K3MOE_EINVAL, "a required pointer is NULL");
  LatArgs a{};
  a.x = reinterpret_cast<const uint16_t *>(x);
  a.wa = reinterpret_cast<const uint16_t *>(latent_down);
  a.wb = reinterpret_cast<const uint16_t *>(shared_gate);
  a.wc = reinterpret_cast<const uint16_t *>(shared_up);
  a.ya = reinterpret_cast<uint16_t *>(latent);
  a.yb = reinterpret_cast<uint16_t *>(shared_h);
  a.ws = reinterpret_cast<char *>(workspace);
  return latent_launch(dims, 0, a, workspace_bytes, stream);
}

int k3moe_latent_out(const k3moe_latent_dims *dims, const float *expert_sum, const void *latent_norm,
                     const void *latent_up, const void *shared_h, const void *shared_down, void *out,
                     void *workspace, size_t workspace_bytes, void *stream) {
  g_err[0] = 0;
  if (!expert_sum || !latent_norm || !latent_up || !shared_h || !shared_down || !out)
    return fail(K3MOE_EINVAL, "a required pointer is NULL");
  LatArgs a{};
  a.x = reinterpret_cast<const uint16_t *>(shared_h);
  a.esum = expert_sum;
  a.norm = reinterpret_cast<const uint16_t *>(latent_norm);
  a.wa = reinterpret_cast<const uint16_t *>(latent_up);
  a.wb = reinterpret_cast<const uint16_t *>(shared_down);
  a.ya = reinterpret_cast<uint16_t *>(out);
  a.ws = reinterpret_cast<char *>(workspace);
  return latent_launch(dims, 1, a, workspace_bytes, stream);
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

int k3moe_activation(int32_t act, int32_t fast, const float *g, const float *u, float *out, int64_t n, void *stream) {
  g_err[0] = 0;
  if (act != K3MOE_ACT_SITU && act != K3MOE_ACT_SILU) return fail(K3MOE_EINVAL, "act must be SITU or SILU, got %d", act);
  if (fast != 0 && fast != 1) return fail(K3MOE_EINVAL, "fast must be 0 or 1, got %d", fast);
  if (n < 0) return fail(K3MOE_EINVAL, "n must be >= 0");
  if (n == 0) return K3MOE_OK;
  if (!g || !u || !out) return fail(K3MOE_EINVAL, "a required pointer is NULL");
  long grid = (long)((n + 255) / 256);
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(k_activation, dim3((unsigned)grid), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), act,
                     fast, g, u, out, n);
  return launch_check("activation");
}

int k3moe_mxfp4_encode(const void *in, int32_t in_dtype, int64_t n_blocks, uint8_t *blocks, uint8_t *scales,
                       void *stream) {
  g_err[0] = 0;
  if (n_blocks < 0) return fail(K3MOE_EINVAL, "n_blocks must be >= 0");
  if (in_dtype != K3MOE_DTYPE_F32 && in_dtype != K3MOE_DTYPE_BF16 && in_dtype != K3MOE_DTYPE_F16)
    return fail(K3MOE_EINVAL, "in_dtype must be f32, bf16 or f16, got %d", in_dtype);
  if (n_blocks == 0) return K3MOE_OK;
  if (!in || !blocks || !scales) return fail(K3MOE_EINVAL, "a required pointer is NULL");
  if (reinterpret_cast<uintptr_t>(in) % 16 || reinterpret_cast<uintptr_t>(blocks) % 4)
    return fail(K3MOE_EINVAL, "in must be 16-byte aligned and blocks 4-byte aligned");
  long grid = (long)((n_blocks + kEncThreads / 4 - 1) / (kEncThreads / 4));
  if (grid > 16384) grid = 16384;
  hipLaunchKernelGGL(k_encode, dim3((unsigned)grid), dim3(kEncThreads), 0, reinterpret_cast<hipStream_t>(stream), in,
                     in_dtype, n_blocks, blocks, scales);
  return launch_check("encode");
}

int k3moe_debug_stall(int32_t polls) {
  g_err[0] = 0;
  if (polls < 0) return fail(K3MOE_EINVAL, "polls must be >= 0 (got %d)", polls);
  g_stall.store(polls, std::memory_order_relaxed);
  return K3MOE_OK;
}

int k3moe_moe_step_noalloc(const k3moe_dims *dims, const void *x, const void *latent, const void *router,
                           const float *router_bias, const uint8_t *gate_blocks, const uint8_t *gate_scales,
                           const uint8_t *up_blocks, const uint8_t *up_scales, const uint8_t *down_blocks,
                           const uint8_t *down_scales, const int64_t *routes, float *expert_sum, int64_t *expert_ids,
                           float *route_weights, float *shortfall, void *stream) {
  g_err[0] = 0;
  int rc = check_dims(dims);
  if (rc) return rc;
  Plan p;
  make_plan(*dims, device_cus(), p, trace_enabled());
  if (p.total > kScratchBytes)
    return fail(K3MOE_EWORKSPACE,
                "this step needs a %zu-byte workspace; the allocation-free entry point's scratch holds %zu "
                "(tokens %d, experts %d, topk %d, latent %d, inter %d): use k3moe_moe_step with a workspace",
                p.total, kScratchBytes, dims->tokens, dims->experts, dims->topk, dims->latent, dims->inter);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  void *ws = nullptr;
  if ((rc = scratch_address(&ws, st))) return rc;
  return k3moe_moe_step(dims, x, latent, router, router_bias, gate_blocks, gate_scales, up_blocks, up_scales,
                        down_blocks, down_scales, routes, expert_sum, expert_ids, route_weights, shortfall, ws,
                        kScratchBytes, stream);
}

}  // extern "C"
