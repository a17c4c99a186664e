/* k3moe: MXFP4 mixture-of-experts step for AMD Instinct MI355X (gfx950).
 *
 * C ABI of the native library libk3moe.so. Plain pointers and sizes only;
 * every pointer argument except `stream` is a device pointer. The library
 * never allocates device memory, never frees caller memory and never writes
 * an input buffer. All work is enqueued asynchronously on `stream` (a
 * hipStream_t passed as void*); no entry point synchronises the host.
 *
 * Return value: 0 on success, a negative K3MOE_E* code on failure, with a
 * thread-local message available from k3moe_last_error().
 *
 * Reference counterpart: the reference has no native code. Its MoE step is
 * inline Python in megabench/tasks/kimi.py:307-324, reached through the
 * candidate plug-in `build(case) -> run(inputs)`
 * (megabench/harness/runner.py:53-69). Each entry point below names the
 * reference lines it replaces.
 */
#ifndef K3MOE_H
#define K3MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define K3MOE_OK 0
#define K3MOE_EINVAL -1      /* bad geometry, dtype code or null pointer */
#define K3MOE_EWORKSPACE -2  /* workspace too small or misaligned */
#define K3MOE_EHIP -3        /* a HIP runtime call failed */

/* Gating rule. */
#define K3MOE_GATING_SIGMOID_BIAS 0 /* kimi.py:308-315: sigmoid, +bias, top-k, renorm */
#define K3MOE_GATING_SOFTMAX 1      /* tasks/distributed.py:174-176: top-k logits, softmax */

/* Gated activation between the gate/up and down projections. */
#define K3MOE_ACT_SITU 0 /* kimi.py:194-196: 4 tanh(g/4) sigmoid(g) 25 tanh(u/25) */
#define K3MOE_ACT_SILU 1 /* tasks/distributed.py:184: silu(g) u */

/* Execution path. AUTO runs the single persistent kernel for decode-sized
 * batches (tokens <= 64, tokens*topk <= 1024) and the multi-kernel path
 * otherwise; the other values force one (DECODE fails with K3MOE_EINVAL when
 * the shape does not fit it). All give the same expert sets. The multi-kernel
 * path (GENERAL) runs the expert projections as grouped GEMMs (weights read
 * once per 128 tokens of an expert) when the experts average at least 16
 * tokens and hidden/latent and inter are multiples of 128, and as per-16-token
 * streams otherwise; GROUPED and STREAMED force one of the two (GROUPED fails
 * with K3MOE_EINVAL when the widths are not multiples of 128). The grouped
 * GEMMs run on the scaled FP4 MFMA (MXFP4 weights as stored, activations as
 * two E4M3 terms with E8M0 block scales, which represent the bf16 values) when
 * latent is a multiple of 512 and inter of 256, and on bf16 MFMA after an
 * in-register decode otherwise; GROUPED_BF16 forces the latter. A single token
 * runs on its own persistent kernel when its shape fits (SINGLE below); AUTO
 * picks it then, DECODE forces the general persistent kernel. */
#define K3MOE_PATH_AUTO 0
#define K3MOE_PATH_GENERAL 1
#define K3MOE_PATH_DECODE 2
#define K3MOE_PATH_GROUPED 3
#define K3MOE_PATH_STREAMED 4
#define K3MOE_PATH_SINGLE 5 /* the single-token kernel (fails with K3MOE_EINVAL when the
                             * shape does not fit it: one token, topk <= 8, experts <= 512,
                             * latent a multiple of 512 up to 8192, inter <= 256) */
#define K3MOE_PATH_GROUPED_BF16 6 /* grouped GEMMs on bf16 MFMA (same conditions as GROUPED) */

/* Element type codes. */
#define K3MOE_DTYPE_BF16 0
#define K3MOE_DTYPE_F32 1
#define K3MOE_DTYPE_F16 2 /* accepted by k3moe_mxfp4_encode only */

/* Geometry and options of one MoE step.
 *   tokens   B: rows of x (and of latent)
 *   experts  E: router rows; leading dim of every expert tensor
 *   topk     k: experts per token, 1 <= k <= 32, k <= E
 *   hidden   h: width of x and of the router rows (the router's K)
 *   latent   K: width of the expert input and of expert_sum (== hidden
 *               unless a separate latent input is given); multiple of 32
 *   inter    I: expert intermediate width; multiple of 32
 * Expert tensor layouts are the reference's (kimi.py:116-119), all u8:
 *   gate_blocks, up_blocks [E, I, K/32, 16]   gate_scales, up_scales [E, I, K/32]
 *   down_blocks            [E, K, I/32, 16]   down_scales            [E, K, I/32]
 * Byte j of a 16-byte block holds element 2j (low nibble) and 2j+1 (high). */
typedef struct k3moe_dims {
    int32_t tokens;
    int32_t experts;
    int32_t topk;
    int32_t hidden;
    int32_t latent;
    int32_t inter;
    int32_t gating;     /* K3MOE_GATING_* */
    int32_t activation; /* K3MOE_ACT_* */
    int32_t x_dtype;    /* K3MOE_DTYPE_BF16 (x, latent and router are bf16) */
    int32_t path;       /* K3MOE_PATH_*: execution path, normally AUTO */
} k3moe_dims;

/* Device workspace bytes the step needs for `dims` (256-byte aligned base,
 * zero-initialised control block, see k3moe_workspace_init).
 * Replaces the temporaries of kimi.py:308-323 (logits, index lists, the
 * per-expert decoded weights, which this library never materialises). */
int k3moe_workspace_bytes(const k3moe_dims *dims, size_t *bytes);

/* One MoE step (kimi.py:307-324 without the TP all-reduce of line 324):
 *   x            [B, h]  bf16   router input (`normalized`, kimi.py:308)
 *   latent       [B, K]  bf16   expert input, or NULL to use x (kimi.py:317,322)
 *   router       [E, h]  bf16   (kimi.py:114)
 *   router_bias  [E]     fp32   or NULL for zero bias (kimi.py:115, 309)
 *   expert tensors as in k3moe_dims
 *   routes       [B, k]  int64  forced expert sets (kimi.py:311-313), or NULL;
 *                               ids must be in range and distinct per row (a row
 *                               that is not keeps its own top-k and sets
 *                               K3MOE_STATUS_ROUTES in the workspace status)
 * Outputs (written, never read):
 *   expert_sum   [B, K]  fp32   routing-weighted sum of expert outputs (kimi.py:318, 323)
 *   expert_ids   [B, k]  int64  chosen experts, ascending per row (kimi.py:316)
 *   route_weights[B, k]  fp32   gating weights aligned with expert_ids (kimi.py:314-315)
 *   shortfall    [B]     fp32   k-th best biased score minus the weakest chosen
 *                               one, clamped at 0 (kimi.py:313); NULL allowed,
 *                               written only when routes != NULL
 * Numerics follow the BF16 serving oracle: FP32 router logits and gating,
 * FP32 accumulation, gate/up outputs, the activation and the down output
 * rounded to bf16 where kimi.py:322 casts, FP32 weighted combine in ascending
 * expert order. */
int k3moe_moe_step(const k3moe_dims *dims,
                   const void *x, const void *latent,
                   const void *router, const float *router_bias,
                   const uint8_t *gate_blocks, const uint8_t *gate_scales,
                   const uint8_t *up_blocks, const uint8_t *up_scales,
                   const uint8_t *down_blocks, const uint8_t *down_scales,
                   const int64_t *routes,
                   float *expert_sum, int64_t *expert_ids, float *route_weights,
                   float *shortfall,
                   void *workspace, size_t workspace_bytes, void *stream);

/* k3moe_moe_step without a workspace argument, for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc. No counterpart in the reference. The
 * workspace is a 16 MiB array in the library's device memory, one per GPU,
 * held until the process ends (every step of the persistent decode path fits:
 * tokens <= 64; a step that needs more, such as a prefill chunk, fails with
 * K3MOE_EWORKSPACE and a message). The first call on a device looks its
 * address up, zeroes its control block with a kernel on `stream` and waits
 * for that kernel (once per device and process, so later calls on any stream
 * find it initialised; that first call must not be under stream capture:
 * call k3moe_workspace_init(NULL, 0, stream) before capturing); no call
 * allocates or frees memory. Its status word is read with
 * k3moe_workspace_status(NULL, ...) and reset, after a K3MOE_STATUS_TIMEOUT
 * too, with k3moe_workspace_init(NULL, ...). All calls on one GPU share the
 * array, so calls that may overlap on one GPU (other streams, other threads)
 * race. Arguments, outputs, numerics and errors are those of k3moe_moe_step. */
int k3moe_moe_step_noalloc(const k3moe_dims *dims,
                           const void *x, const void *latent,
                           const void *router, const float *router_bias,
                           const uint8_t *gate_blocks, const uint8_t *gate_scales,
                           const uint8_t *up_blocks, const uint8_t *up_scales,
                           const uint8_t *down_blocks, const uint8_t *down_scales,
                           const int64_t *routes,
                           float *expert_sum, int64_t *expert_ids, float *route_weights,
                           float *shortfall, void *stream);

/* Where a step of the multi-kernel path leaves its token grouping
 * (kimi.py:319-320: `indices.unique()` and the `(indices == e).nonzero()`
 * lists) in the workspace, as byte offsets from its base. For tests and tools
 * that inspect a step; after a step on the GENERAL, GROUPED or STREAMED path
 * (or AUTO above the decode limits) the workspace holds:
 *   active_count  int32          D, the number of distinct experts chosen
 *   active        int32 [D]      those experts, ascending
 *   offsets       int32 [D]      first pair of each active expert
 *   counts        int32 [D]      pairs of each active expert
 *   pair_token    int32 [B k]    token of each pair: expert-major, tokens ascending
 *   pair_weight   fp32  [B k]    routing weight of each pair
 *   pair_of       int32 [B k]    pair of (token t, slot j), slots in expert_ids order
 *   pair_h        bf16  [B k, I] each pair's activation output, cast(act(gate, up))
 *   pair_y        bf16  [B k, K] each pair's down projection, cast(h @ down.T)
 *   input_split   the FP4-MFMA grouped GEMMs' expert inputs as two E4M3 terms:
 *                 hi u8 [B, K], lo u8 [B, K], then their E8M0 block scales
 *                 hi u8 [B, K/32], lo u8 [B, K/32] (-1 on other paths)
 *   h_split       h in the same form: [B k, I] twice, then [B k, I/32] twice
 *                 (-1 on other paths; pair_h is then -1 too: h is kept only split)
 * The persistent decode path keeps its grouping in LDS; for dims that select
 * it this returns K3MOE_EINVAL. */
typedef struct k3moe_layout {
    int64_t active_count;
    int64_t active;
    int64_t offsets;
    int64_t counts;
    int64_t pair_token;
    int64_t pair_weight;
    int64_t pair_of;
    int64_t pair_h;
    int64_t pair_y;
    int64_t input_split;
    int64_t h_split;
} k3moe_layout;

int k3moe_workspace_layout(const k3moe_dims *dims, k3moe_layout *layout);

/* Zero the workspace's first 2183168 bytes (the control block with the barrier
 * and launch counters and the sticky status word, a zero area the kernels read
 * in place of inactive data, the latent block's row-tile counters and the
 * persistent kernels' tagged exchange area) with a small
 * kernel on `stream`. A workspace must be
 * initialised once before its first step; each step leaves the counters at
 * zero, so one workspace serves any number of consecutive steps on one
 * stream (steps that overlap on one workspace race). workspace == NULL
 * means the current device's allocation-free scratch (k3moe_moe_step_noalloc;
 * workspace_bytes is then ignored): it zeroes the same bytes of it, or, if no
 * call on this device has used the scratch yet, initialises it and waits for
 * that. No reference counterpart: the reference allocates its temporaries per
 * call. */
int k3moe_workspace_init(void *workspace, size_t workspace_bytes, void *stream);

/* Status bits of the workspace's sticky status word (an OR over every step
 * since k3moe_workspace_init). */
#define K3MOE_STATUS_TIMEOUT 1 /* a persistent step's wait timed out (its workgroups
                                * were not all resident): that step's outputs are
                                * invalid, and the workspace's barrier counters must
                                * be re-initialised (k3moe_workspace_init) before
                                * later steps on it are trusted */
#define K3MOE_STATUS_ROUTES 2  /* forced routes held an id out of [0, experts) or a
                                * repeated id in a row: such rows used their own
                                * top-k selection instead (kimi.py:364-367) */

/* Copy the workspace's sticky status word to *status (0 = every step so far
 * completed normally, else K3MOE_STATUS_* bits). Synchronises `stream`.
 * k3moe_moe_step and the latent entry points never synchronise, so a caller
 * that needs the guarantee reads the status after its steps. workspace ==
 * NULL reads the current device's allocation-free scratch (the status of
 * k3moe_moe_step_noalloc calls on this device since its initialisation or
 * the last k3moe_workspace_init(NULL, ...)). No reference counterpart. */
int k3moe_workspace_status(const void *workspace, int32_t *status, void *stream);

/* Geometry of the latent MoE block around the routed experts of a Kimi K3
 * layer (kimi.py:317, 325-328; weight shapes kimi.py:112-121):
 *   tokens      B: rows of x (up to 64 per kernel launch; larger batches run as
 *               consecutive launches of 64 token rows on the same stream)
 *   hidden      h: width of x and of the block's output (7168)
 *   latent      lh: width of the experts' input and of expert_sum (3584)
 *   shared      S: this rank's shared-expert width (intermediate x
 *               shared_experts / tp: 768 on a TP8 rank)
 *   activation  K3MOE_ACT_*: the shared experts' activation (SiTU, kimi.py:326)
 * h, lh and S are multiples of 128. Weights are bf16, row-major:
 *   latent_down [lh, h]   latent_up [h, lh]   latent_norm [lh]
 *   shared_gate, shared_up [S, h]             shared_down [h, S]
 * Both entry points share one workspace (and may share the MoE step's, which
 * is then sized for the larger of the two); it must be initialised by
 * k3moe_workspace_init. */
typedef struct k3moe_latent_dims {
    int32_t tokens;
    int32_t hidden;
    int32_t latent;
    int32_t shared;
    int32_t activation; /* K3MOE_ACT_* */
} k3moe_latent_dims;

/* Device workspace bytes k3moe_latent_in and k3moe_latent_out need for `dims`.
 * Replaces the temporaries of kimi.py:317, 325-327. */
int k3moe_latent_workspace_bytes(const k3moe_latent_dims *dims, size_t *bytes);

/* The block's projections of the normalised layer input, before the experts
 * (kimi.py:317 and the inner part of 326-327, one rank, no all-reduce):
 *   x          [B, h]   bf16   `normalized`
 * Outputs (written, never read):
 *   latent     [B, lh]  bf16   bf16(x @ latent_down.T): the experts' input
 *                              (k3moe_moe_step's `latent`)
 *   shared_h   [B, S]   bf16   bf16(act(bf16(x @ shared_gate.T), bf16(x @ shared_up.T)))
 * FP32 accumulation, rounded where kimi.py:246-247 and 326 cast. */
int k3moe_latent_in(const k3moe_latent_dims *dims, const void *x, const void *latent_down,
                    const void *shared_gate, const void *shared_up, void *latent, void *shared_h,
                    void *workspace, size_t workspace_bytes, void *stream);

/* The block's output from the experts' sum and the shared activation
 * (kimi.py:325-328, one rank, no all-reduce):
 *   expert_sum [B, lh]  fp32   k3moe_moe_step's expert_sum
 *   shared_h   [B, S]   bf16   k3moe_latent_in's shared_h
 * Output (written, never read):
 *   out        [B, h]   bf16   bf16(routed + shared) with
 *                              routed = bf16(rms(bf16(expert_sum), latent_norm, eps 1e-5) @ latent_up.T),
 *                              rms as common.py:13-21 (normalised value cast
 *                              to bf16, then times the bf16 weight),
 *                              shared = bf16(shared_h @ shared_down.T) */
int k3moe_latent_out(const k3moe_latent_dims *dims, const float *expert_sum, const void *latent_norm,
                     const void *latent_up, const void *shared_h, const void *shared_down, void *out,
                     void *workspace, size_t workspace_bytes, void *stream);

/* The block's input projections and its routed MoE step in one call
 * (kimi.py:317 and the inner part of 326-327, then 307-324 on the latent):
 * k3moe_latent_in's outputs and k3moe_moe_step's, the step taking the latent
 * it computes as its expert input (`latent`, written here). `dims` is the
 * step's geometry (dims->latent = lh, dims->activation also the shared
 * experts'); `shared` is S. With one token and the single-token kernel's
 * geometry (and at most 48 latent and shared rows per workgroup: lh/2 + S
 * <= 24 x the CU count) both run in one launch: every workgroup streams its
 * share of the projections' weights while the routing goes on, and the
 * gate/up products wait for the latent through tagged slots. With 2 to 16
 * tokens on the decode kernel's pinned plans (and (lh + 2S)/2 rows at most 16
 * per non-routing workgroup) they also run in one launch: the workgroups that
 * route no token stream the projections while the routing runs and a grid
 * barrier publishes the latent. Otherwise the two run as k3moe_latent_in and
 * k3moe_moe_step launches. The workspace must
 * hold both k3moe_workspace_bytes(dims) and k3moe_latent_workspace_bytes of
 * the block's dims. Arguments, outputs, numerics and errors as those two
 * entry points'. */
int k3moe_latent_moe_step(const k3moe_dims *dims, int32_t shared,
                          const void *x, const void *latent_down,
                          const void *shared_gate, const void *shared_up,
                          void *latent, void *shared_h,
                          const void *router, const float *router_bias,
                          const uint8_t *gate_blocks, const uint8_t *gate_scales,
                          const uint8_t *up_blocks, const uint8_t *up_scales,
                          const uint8_t *down_blocks, const uint8_t *down_scales,
                          const int64_t *routes,
                          float *expert_sum, int64_t *expert_ids, float *route_weights,
                          float *shortfall,
                          void *workspace, size_t workspace_bytes, void *stream);

/* The whole latent MoE block in one call (kimi.py:317-328, one rank, no
 * all-reduce): k3moe_latent_moe_step's outputs and k3moe_latent_out's `out`
 * from its expert sum. With one token and the single-token kernel's geometry
 * (as for k3moe_latent_moe_step, and lh <= 4096, lh + S <= 4608, h <= 32 x
 * the CU count) all of it runs in one launch: after the combine every
 * workgroup polls the expert sum and shared_h from the others' tagged slots,
 * normalises it and streams its share of the output rows (their weights
 * issued before the poll). With 2 to 8 tokens where k3moe_latent_moe_step
 * runs in one launch (and lh, S multiples of 128, lh <= 4096, h <= 32 x the
 * CU count) the decode kernel does the same after a grid barrier over the
 * expert sum (the combine also writes its bf16 rounding to the workspace for
 * the norm). Otherwise it runs as k3moe_latent_moe_step and k3moe_latent_out. Arguments, outputs, numerics and errors as those entry
 * points' (the one-launch path sums the output rows in another FP32 order:
 * within a bf16 step of the other's, mostly equal). */
int k3moe_latent_block(const k3moe_dims *dims, int32_t shared,
                       const void *x, const void *latent_down,
                       const void *shared_gate, const void *shared_up,
                       const void *latent_norm, const void *latent_up, const void *shared_down,
                       const void *router, const float *router_bias,
                       const uint8_t *gate_blocks, const uint8_t *gate_scales,
                       const uint8_t *up_blocks, const uint8_t *up_scales,
                       const uint8_t *down_blocks, const uint8_t *down_scales,
                       const int64_t *routes,
                       void *latent, void *shared_h,
                       float *expert_sum, int64_t *expert_ids, float *route_weights,
                       float *shortfall, void *out,
                       void *workspace, size_t workspace_bytes, void *stream);

/* MXFP4 decode, unpack_mxfp4 (megabench/tasks/quantization.py:40-51) plus the
 * `.to(act)` cast of kimi.py:321: n_blocks blocks of 16 bytes and n_blocks
 * scales -> n_blocks*32 values of out_dtype (K3MOE_DTYPE_F32 or _BF16),
 * bit-exact including -0.0, subnormal results and NaN for scale 255. */
int k3moe_mxfp4_decode(const uint8_t *blocks, const uint8_t *scales, int64_t n_blocks,
                       int32_t out_dtype, void *out, void *stream);

/* Debug: the expert GEMMs' activation act(g, u) (K3MOE_ACT_SITU, kimi.py:194-196,
 * or K3MOE_ACT_SILU, tasks/distributed.py:184) on n fp32 pairs, written to out:
 * fast = 0 is the library-function form the decode kernels use, fast = 1 the
 * exponential-and-reciprocal form of the prefill GEMM's epilogue. For tests
 * that pin both against a float64 reference. No reference counterpart beyond
 * the formulas. */
int k3moe_activation(int32_t act, int32_t fast, const float *g, const float *u, float *out, int64_t n,
                     void *stream);

/* Test hook for the failure path of the persistent kernels (no reference
 * counterpart): with polls > 0, the router-logit waits of every later
 * k3moe_moe_step / k3moe_moe_step_noalloc on the single-token or decode kernel
 * never see their data and give up after `polls` polls, as a wait that timed
 * out does: the step leaves NaN in expert_sum, sets K3MOE_STATUS_TIMEOUT in the
 * workspace status and every workgroup ends normally; k3moe_workspace_init then
 * makes the workspace usable again. polls = 0 (the default) turns it off.
 * Process-wide; returns K3MOE_EINVAL for polls < 0. */
int k3moe_debug_stall(int32_t polls);

/* MXFP4 encode, pack_mxfp4 (megabench/tasks/quantization.py:13-37): n_blocks
 * groups of 32 consecutive values of in_dtype (K3MOE_DTYPE_F32, _BF16 or
 * _F16; in 16-byte aligned) -> n_blocks blocks of 16 bytes (byte j: element
 * 2j in the low nibble, 2j+1 in the high one; blocks 4-byte aligned) and
 * n_blocks E8M0 scale bytes. Bit for bit with the
 * reference's torch CPU chain: block exponent ceil(log2(max|x|/6)) with the
 * fp32 logarithm rounded to nearest (clamped to [-126, 127]), fp32 products
 * x 2^-e, round to nearest with ties to the even code; a block holding a NaN
 * gets scale byte 127, code 7 for its NaN and infinite elements and 0 for
 * the rest (torch's result on x86). */
int k3moe_mxfp4_encode(const void *in, int32_t in_dtype, int64_t n_blocks, uint8_t *blocks,
                       uint8_t *scales, void *stream);

/* Message of the last failing call on this thread ("" if none). */
const char *k3moe_last_error(void);

/* Library version string. */
const char *k3moe_version(void);

#ifdef __cplusplus
}
#endif

#endif /* K3MOE_H */
