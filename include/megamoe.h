/*
 * megamoe.h — C ABI of the MI355X (gfx950) FP8 mixture-of-experts decode layer.
 *
 * One call computes, for T tokens, the MoE block that the reference composes
 * in eager PyTorch:
 *
 *   router logits  = fp32(router) @ fp32(x)                 megabench/tasks/frontier.py:343
 *   routing        = sigmoid + bias, group-limited top-k,   megabench/tasks/frontier.py:229-242
 *                    or softmax over the top-k logits       megabench/tasks/references/moe.py:68-70,
 *                                                           megabench/tasks/distributed.py:174-176
 *   per (token, slot) expert:  W8A8 linear (FP8 E4M3, 128x128 block scales,
 *                    per-token-per-128 activation scales)   megabench/tasks/frontier.py:180-186,
 *                                                           megabench/tasks/quantization.py:87-131
 *                    h = bf16(silu(fp32 g) * fp32 u)        megabench/tasks/frontier.py:337
 *   combine        = slot-order fp32 sum of bf16(d)*w, plus the shared expert,
 *                    one bf16 rounding                      megabench/tasks/frontier.py:349-354
 *
 * The reference has no native code on this path: each entry point below
 * replaces a sequence of eager aten calls inside the case's reference(), and
 * the Python submission that calls it keeps the reference harness contract
 * build(case) -> run(inputs) -> outputs (megabench/README.md:83-104,
 * megabench/harness/runner.py:69-87).
 *
 * Conventions: all pointers are device pointers unless stated otherwise.
 * Every call is asynchronous on `stream` (a hipStream_t passed as void*;
 * NULL is the default stream), allocates nothing and throws nothing. Each
 * returns a megamoe_status code.
 */
#ifndef MEGAMOE_H
#define MEGAMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum megamoe_status {
  MEGAMOE_OK = 0,
  MEGAMOE_ERR_INVALID_ARGUMENT = 1, /* a required pointer is NULL or a count is negative */
  MEGAMOE_ERR_SHAPE = 2,            /* geometry the layer does not define (H or I not a multiple of 128, K > E, ...) */
  MEGAMOE_ERR_WORKSPACE = 3,        /* workspace smaller than megamoe_workspace_bytes() */
  MEGAMOE_ERR_HIP = 4,              /* a HIP runtime call or kernel launch failed */
  MEGAMOE_ERR_UNSUPPORTED = 5,      /* within the layer's definition but beyond this build's limits */
  MEGAMOE_ERR_SCRATCH = 6           /* megamoe_forward_noalloc: the call needs more workspace than
                                       MEGAMOE_SCRATCH_BYTES */
};

/* Size of the fixed device scratch of megamoe_forward_noalloc (32 MiB per GPU, held from the
 * library's first use on that GPU until the process ends). */
#define MEGAMOE_SCRATCH_BYTES (32u << 20)

enum megamoe_gate {
  MEGAMOE_GATE_SOFTMAX = 0, /* ids = top-k logits (stable); w = softmax over the selected logits (renormalize=1)
                               or the full softmax at the selected ids (renormalize=0) */
  MEGAMOE_GATE_SIGMOID = 1  /* p = sigmoid(logits); ids chosen on p + bias (group-limited);
                               w = p[ids] / (sum + 1e-20) when renormalize=1, else p[ids] */
};

/* Geometry and routing rule of one MoE layer. The same struct describes
 * every entry point; fields an entry point does not use are ignored. */
typedef struct megamoe_desc {
  int32_t tokens;         /* T >= 0 */
  int32_t hidden;         /* H, multiple of 128 */
  int32_t experts;        /* E routed experts, 1..1024 */
  int32_t topk;           /* K, 1..min(E, 32) */
  int32_t intermediate;   /* I of one routed expert, multiple of 128 */
  int32_t shared_experts; /* S >= 0; the shared expert is one MLP of intermediate S*I */
  int32_t groups;         /* G, divides E; 1 disables group limiting */
  int32_t top_groups;     /* groups kept, 1..G */
  int32_t gate;           /* enum megamoe_gate */
  int32_t renormalize;    /* see enum megamoe_gate */
  int32_t pow2_scales;    /* 1: activation scales rounded up to a power of two
                             (quantization.py:57-59 power_of_two=True) */
  float routed_scaling;   /* multiplies every routed weight (frontier.py:242) */
} megamoe_desc;

/* Tensors of one forward call. Layouts are row-major and dense, exactly as
 * the case's inputs hold them (frontier.py:157-176 for the expert stacks):
 *   x              bf16 [T, H]
 *   router         fp32 [E, H]
 *   router_bias    fp32 [E] or NULL (treated as zero)
 *   gate, up       e4m3fn [E, I, H];  gate_scale, up_scale fp32 [E, I/128, H/128]
 *   down           e4m3fn [E, H, I];  down_scale          fp32 [E, H/128, I/128]
 *   shared_gate, shared_up  e4m3fn [S*I, H]; scales fp32 [S*I/128, H/128]
 *   shared_down             e4m3fn [H, S*I]; scale  fp32 [H/128, S*I/128]
 *   y              bf16 [T, H]     (output)
 *   expert_ids     int64 [T, K]    (output, selection order)
 *   expert_weights fp32 [T, K]     (output)
 * Inputs are only read. The workspace holds intermediates between the
 * kernels of one call; it needs no initialisation. */
typedef struct megamoe_tensors {
  const void* x;
  const float* router;
  const float* router_bias;
  const uint8_t* gate;
  const float* gate_scale;
  const uint8_t* up;
  const float* up_scale;
  const uint8_t* down;
  const float* down_scale;
  const uint8_t* shared_gate;
  const float* shared_gate_scale;
  const uint8_t* shared_up;
  const float* shared_up_scale;
  const uint8_t* shared_down;
  const float* shared_down_scale;
  void* y;
  int64_t* expert_ids;
  float* expert_weights;
  void* workspace;
  size_t workspace_bytes;
} megamoe_tensors;

/* Bytes of device workspace megamoe_forward (and megamoe_layer_forward) needs for `desc`
 * (host call). No reference counterpart: the reference allocates through PyTorch. */
int megamoe_workspace_bytes(const megamoe_desc* desc, size_t* bytes);

/* The whole layer: router, routing, permute, gate/up + SwiGLU, down, combine.
 * Replaces the MoE block of megabench/tasks/frontier.py:335-354 (sigmoid
 * configs) and megabench/tasks/references/moe.py:66-78 (softmax configs). */
int megamoe_forward(const megamoe_desc* desc, const megamoe_tensors* t, void* stream);

/* megamoe_forward with no workspace argument and no allocation: the workspace is the
 * library's fixed device scratch (MEGAMOE_SCRATCH_BYTES per GPU, a file-scope device array),
 * so the call allocates nothing, in the library or in any routine it calls. For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). No reference counterpart. t->workspace and t->workspace_bytes are
 * ignored. Returns MEGAMOE_ERR_SCRATCH, launching nothing, when megamoe_workspace_bytes(desc)
 * exceeds MEGAMOE_SCRATCH_BYTES (each of the five benchmark configs fits: Kimi-K2 at 128 tokens needs
 * 29 MiB). All calls on one GPU share its scratch: calls that overlap on that GPU (on two
 * streams, or from two threads) race and must be ordered by the caller. */
int megamoe_forward_noalloc(const megamoe_desc* desc, const megamoe_tensors* t, void* stream);

/* megamoe_forward with a device event between its stages; blocks until the
 * call has finished and writes the elapsed ms of each stage to stage_ms[0..4]
 * (router, select + x quantization, permute, experts = gate/up + down,
 * combine). For
 * measurement; the results equal megamoe_forward's. */
int megamoe_forward_timed(const megamoe_desc* desc, const megamoe_tensors* t, void* stream,
                          float* stage_ms);

/* megamoe_forward that also records events[0..5] (hipEvent_t, created by the caller)
 * on `stream` at the stage boundaries: before the router, then after each stage
 * (router, select + x quantization, permute, experts, combine). Asynchronous like
 * megamoe_forward; for measuring a timed loop. No reference counterpart. */
int megamoe_forward_events(const megamoe_desc* desc, const megamoe_tensors* t, void* stream,
                           void* const* events);

/* Router logits only: logits fp32 [T, E] = router @ x, with fp64 accumulation
 * rounded once to fp32. `workspace` as for megamoe_forward.
 * Replaces `values['router'].float() @ normalized.float()` (frontier.py:343). */
int megamoe_router_logits(const megamoe_desc* desc, const void* x, const float* router, float* logits,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Routing from given logits fp32 [T, E]: expert_ids int64 [T, K] and
 * expert_weights fp32 [T, K]. bias may be NULL.
 * Replaces frontier.route (frontier.py:229-242) applied per token and the
 * stable-argsort softmax routing of distributed.py:174-176. */
int megamoe_route(const megamoe_desc* desc, const float* logits, const float* bias, int64_t* expert_ids,
                  float* expert_weights, void* stream);

/* The decoder-block steps either side of the layer (frontier.py:335,354):
 *   normalized = rms(x, norm_weight, eps, weight_in_fp32)   common.py:13-21
 *   y          = x + bf16(layer(normalized))                frontier.py:354 (residual = 1)
 * norm_weight is bf16 [H] (the block's ln2 gamma, frontier.py:87); NULL skips the
 * normalization (the layer reads x). eps is 1e-6 for DeepSeek and 1e-5 otherwise in the
 * reference (frontier.py:258), which also applies the gamma in fp32 for DeepSeek only. */
typedef struct megamoe_block {
  const void* norm_weight; /* bf16 [H] or NULL */
  float eps;               /* >= 0 */
  int32_t weight_in_fp32;  /* 1: bf16(n * w); 0: bf16(bf16(n) * w) */
  int32_t residual;        /* 1: y = bf16(x + bf16(layer output)); 0: y = layer output */
} megamoe_block;

/* megamoe_forward for the block: RMSNorm of x (a sixth kernel, before the router; the
 * router and the experts read the normalized rows), the layer, and the residual add in the
 * combine. x is the block input (the residual stream). `events` is NULL or
 * events[0..5] as for megamoe_forward_events (the normalization counts to the router
 * stage). Workspace: megamoe_workspace_bytes(). Replaces frontier.py:335-354 from the ln2
 * normalization to the residual add. */
int megamoe_block_forward(const megamoe_desc* desc, const megamoe_tensors* t, const megamoe_block* block,
                          void* stream, void* const* events);

/* RMSNorm of bf16 rows [rows, cols] with a bf16 gamma [cols] into bf16 out [rows, cols]
 * (cols a multiple of 8; rows 16-byte aligned): s = sum of x^2 in fp64, r = 1/sqrt(fp32(s/cols)
 * + eps) with correctly rounded fp32 operations, out = bf16(x*r*w) (weight_in_fp32) or
 * bf16(bf16(x*r)*w). Replaces common.rms (megabench/tasks/common.py:13-21). */
int megamoe_rms_norm(int32_t rows, int32_t cols, const void* x, const void* weight, float eps,
                     int32_t weight_in_fp32, void* out, void* stream);

/* Epilogue variants of the FP8 layer's experts (routed and shared alike). With g, u the
 * bf16 gate and up outputs:
 *   swiglu 0: h = bf16(silu(fp32 g) * fp32 u), rounded once (frontier.py:337, DeepSeek/TileRT);
 *   swiglu 1: h = bf16(bf16(silu(g)) * u), silu rounded to bf16 first (F.silu(gate)*up on
 *             bf16, frontier.py:338 and glm53.py:174-175);
 *   swiglu_limit > 0: g = min(g, limit) and u = clamp(u, -limit, limit) before either form
 *             (glm53.py:175, SWIGLU_LIMIT = 10); 0 clamps nothing. */
typedef struct megamoe_epilogue {
  int32_t swiglu;
  float swiglu_limit;
} megamoe_epilogue;

/* megamoe_forward with optional block steps and epilogue variant: `block` NULL runs the
 * layer alone (as megamoe_forward), else as megamoe_block_forward; `epilogue` NULL is
 * {0, 0} (the DeepSeek form). `events` is NULL or events[0..5] as megamoe_forward_events
 * (asynchronous: recorded, not waited for). Replaces the MoE step of the frontier decoders
 * that use these forms: frontier.py:335-354 (sigmoid routing, shared expert) with
 * glm53.py:263-274 for GLM-5.3-Flash. */
int megamoe_forward_ex(const megamoe_desc* desc, const megamoe_tensors* t, const megamoe_block* block,
                       const megamoe_epilogue* epilogue, void* stream, void* const* events);

/* megamoe_forward_ex in the W8A16 form: the expert GEMMs read the bf16 rows (x, or the
 * normalized x of the block form) without quantizing them, and h = bf16(silu(g) * u) stays
 * in bf16 for the down GEMM: g, u = bf16(dequant(W, s) @ fp32(x)), d = bf16(dequant(W_d, s_d)
 * @ fp32(h)). The routing, the combine and the tensors are megamoe_forward_ex's; x_scale
 * work (pow2_scales) does not apply. Replaces frontier.py:180-183 with quantize=False, which
 * the DeepSeek family uses for every expert GEMM (frontier.py:190, 265-270, DEEPSEEK_FP8_
 * ACTIVATIONS), in the MoE step of frontier.py:335-354. Stream-ordered (five launches, six
 * with the block's normalization); `events` as megamoe_forward_ex's; the one-launch form is
 * megamoe_layer_forward_w8a16. */
int megamoe_forward_w8a16(const megamoe_desc* desc, const megamoe_tensors* t, const megamoe_block* block,
                          const megamoe_epilogue* epilogue, void* stream, void* const* events);

/* megamoe_forward_w8a16 as ONE kernel launch (megamoe_layer_forward's persistent kernel with
 * the W8A16 expert units): the arguments, the workspace rule (zeroed before its first use)
 * and the results are megamoe_layer_forward's, and the results equal megamoe_forward_w8a16's
 * bit for bit. `events` NULL or events[0..1]. Replaces what megamoe_forward_w8a16 replaces. */
int megamoe_layer_forward_w8a16(const megamoe_desc* desc, const megamoe_tensors* t, const megamoe_block* block,
                                const megamoe_epilogue* epilogue, void* stream, void* const* events);

/* The layer (block == NULL) or the block, with an optional epilogue variant, as ONE kernel
 * launch: the arguments and results are megamoe_forward_ex's, bit for bit. The reference
 * harness audits each call's kernel launches against the case's budget, one by default
 * (megabench/cases.py:32, megabench/harness/benchmark.py:73-100); the stream-ordered form
 * above takes five (six with the block's normalization). One persistent kernel drains a
 * queue of units in dependency order: RMSNorm rows (block form), router tiles, per-token
 * routing (with the token's activation quantization), the permute (run by the routing unit
 * that finishes last), gate/up and down units, combine units.
 * Workspace: megamoe_workspace_bytes(desc) bytes, ZEROED before its first use with this
 * entry point (e.g. hipMemset once after allocation); each call leaves its control words
 * zero again, so later calls need nothing. Calls sharing a workspace must be ordered (one
 * stream). `events` is NULL or events[0..1] (hipEvent_t, created by the caller), recorded
 * before and after the launch. Replaces frontier.py:335-354 (and glm53.py:263-274 for the
 * clamped-SwiGLU form) as megamoe_forward_ex does. */
int megamoe_layer_forward(const megamoe_desc* desc, const megamoe_tensors* t, const megamoe_block* block,
                          const megamoe_epilogue* epilogue, void* stream, void* const* events);

/* Outcome of the last megamoe_layer_forward (or megamoe_forward / megamoe_forward_ex) call on
 * `workspace`: *gave_up = 1 if one of its bounded waits between workgroups gave up (after
 * 0.2 s; every kernel still ends, and y is NaN), else 0. Synchronizes `stream` (a host call
 * that copies one word). No reference counterpart: the reference's eager layer has no
 * waits. Test hook: with the environment variable MEGAMOE_FORCE_WAIT_TIMEOUT=1,
 * megamoe_layer_forward's combine units wait for a count the down units never reach, for
 * 20 us, so the call reports a wait that gave up. */
int megamoe_layer_status(const megamoe_desc* desc, const void* workspace, size_t workspace_bytes, int32_t* gave_up,
                         void* stream);

/* GPT-OSS's combine (gptoss.py:112-124): per token t, its K expert outputs (bf16
 * expert_out [T*K, H], row t*K + k for slot k) accumulate in ascending expert id order
 * (expert_ids int64 [T*K], distinct within a token; a repeated id counts once), in bf16:
 * o = bf16(o + bf16(p * e)) from o = 0 with the slot's bf16 weight p (weights bf16 [T*K]);
 * y = bf16(residual + o) when residual (bf16 [T, H]) is given, else y = o. */
int megamoe_combine_by_expert_id(int32_t tokens, int32_t hidden, int32_t topk, const void* expert_out,
                                 const int64_t* expert_ids, const void* weights, const void* residual, void* y,
                                 void* stream);

/* Tensors of the MXFP4 form (megabench/tasks/megamoe.py, serial): the routed experts of a
 * DeepSeek-V4-style layer with FP4 weights, routing given.
 *   x            e4m3fn [T, H];  x_scales uint8 [T, H/32] (E8M0: 2^(s-127))
 *   topk_idx     int64 [T, K] (distinct experts per token, each in [0, E));
 *   topk_weights fp32 [T, K] (applied inside the SwiGLU)
 *   l1_blocks    uint8 [E, 2I, H/32, 16] (E2M1 codes, two per byte, even element in the low
 *                nibble; rows 0..I-1 gate, I..2I-1 up);  l1_scales uint8 [E, 2I, H/32]
 *   l2_blocks    uint8 [E, H, I/32, 16];  l2_scales uint8 [E, H, I/32]
 *   y            bf16 [T, H] (output) */
typedef struct megamoe_mx_tensors {
  const uint8_t* x;
  const uint8_t* x_scales;
  const int64_t* topk_idx;
  const float* topk_weights;
  const uint8_t* l1_blocks;
  const uint8_t* l1_scales;
  const uint8_t* l2_blocks;
  const uint8_t* l2_scales;
  void* y;
  void* workspace;
  size_t workspace_bytes;
} megamoe_mx_tensors;

/* Workspace of megamoe_mx_forward and megamoe_mx_layer_forward (host call). desc: tokens, hidden and intermediate
 * (multiples of 256), experts, topk; shared_experts must be 0; the other fields are
 * unused. No reference counterpart. */
int megamoe_mx_workspace_bytes(const megamoe_desc* desc, size_t* bytes);

/* The routed experts in MXFP4 (megamoe.py:116-182, serial mode): per (token, slot) row,
 * l1 = bf16(x @ l1.T) on the scaled MFMA (E2M1 x E4M3 with both E8M0 scales), gate =
 * min(gate, limit), up = clamp(up, +-limit), a = gate*sigmoid(gate)*up*w (fp32), h = E4M3 of a
 * with E8M0 scales per 32 (quantization.py:67-109), d = bf16(h @ l2.T); y = bf16(slot-order
 * fp32 sum of d). Out-of-range or repeated expert ids make every element of y NaN. `events`
 * is NULL or events[0..3] (before the permute, after the permute, the experts and the
 * combine). Replaces megamoe.reference(serial=True), megamoe.py:153-182. */
int megamoe_mx_forward(const megamoe_desc* desc, float swiglu_limit, const megamoe_mx_tensors* t, void* stream,
                       void* const* events);

/* megamoe_mx_forward in one kernel launch (the reference's budget of one launch per call,
 * megabench/cases.py:32): one persistent kernel runs the permute, the expert units and the
 * combine, with the results of megamoe_mx_forward bit for bit. Rows that average 24 or more
 * per expert (the batch-shaped EP share) take megamoe_mx_forward's kernels instead. Workspace:
 * megamoe_mx_workspace_bytes(desc) bytes, ZEROED before its first use with this entry point;
 * each call leaves its control words zero again. Calls sharing a workspace must be ordered.
 * `events` is NULL or events[0..1], recorded before and after the call. Replaces
 * megamoe.reference(serial=True), megamoe.py:153-182. */
int megamoe_mx_layer_forward(const megamoe_desc* desc, float swiglu_limit, const megamoe_mx_tensors* t,
                             void* stream, void* const* events);

/* Outcome of the last megamoe_mx_layer_forward on `workspace`: *failed = 1 if one of its
 * bounded waits gave up or the expert ids were bad (y is NaN), else 0. Synchronizes `stream`.
 * No reference counterpart (test hook as megamoe_layer_status). */
int megamoe_mx_layer_status(const megamoe_desc* desc, const void* workspace, size_t workspace_bytes, int32_t* failed,
                            void* stream);

/* Expert parallelism, one rank's share (megamoe.py:153-182 with ep ranks): expert e belongs
 * to rank e / (E/ep). A rank sends each (token, slot) row to the owner of the slot's expert,
 * runs its local experts over the rows it receives, and sums the outputs that come back.
 * The two exchanges between these calls (all_to_all_single, parallel.py:52-68) are the
 * caller's collectives.
 *
 * The send buffers of megamoe_ep_dispatch, for this rank's T tokens (T*K rows):
 *   rows        uint8 [T*K, H] (E4M3 bytes);  row_scales uint8 [T*K, H/32] (E8M0)
 *   ids         int64 [T*K] (global expert ids);  weights fp32 [T*K]
 *   counts      int64 [ep] rows per destination rank, in rank order
 *   slot_rows   int32 [T*K] send row of (token t, slot k) at t*K + k */
typedef struct megamoe_ep_send {
  uint8_t* rows;
  uint8_t* row_scales;
  int64_t* ids;
  float* weights;
  int64_t* counts;
  int32_t* slot_rows;
} megamoe_ep_send;

/* Dispatch (megamoe.py:160-171, and the send counts of parallel.py:59-68): the rows in a
 * stable order by owner rank, so each destination receives this rank's rows in (token,
 * slot) order. desc: tokens, hidden (a multiple of 256), experts (divisible by ep), topk;
 * t: x, x_scales, topk_idx, topk_weights (16- and 8-byte aligned x and x_scales, as the send
 * rows and row scales). An id outside [0, E) makes every count -1 and every slot row -1, and
 * nothing is packed. Limits: ep <= 256, T*K <= 49152 (MEGAMOE_ERR_UNSUPPORTED beyond). */
int megamoe_ep_dispatch(const megamoe_desc* desc, int32_t ep, const megamoe_mx_tensors* t,
                        const megamoe_ep_send* send, void* stream);

/* The local experts over the received rows (megamoe.py:131-150): desc.tokens = R received
 * rows, desc.topk = 1, desc.experts = E/ep local experts; t->x, x_scales are the received
 * rows and scales, topk_idx their global ids (int64 [R], each in [expert_base, expert_base +
 * E/ep)), topk_weights [R]; l1/l2 hold the local experts only; y = bf16 [R, H], each row's
 * weighted expert output (the returned payload). Rows are computed exactly as in
 * megamoe_mx_forward, whose result for a row depends only on the row, its expert's weights
 * and the layer's down-projection split, so a rank's rows equal the serial layer's bit for
 * bit when the splits agree (they do whenever both have at least 2048 down units of 128
 * rows). Workspace: megamoe_mx_workspace_bytes(desc). Bad ids make every element NaN. */
int megamoe_ep_experts(const megamoe_desc* desc, float swiglu_limit, int64_t expert_base, const megamoe_mx_tensors* t,
                       void* stream, void* const* events);

/* Combine at the source (megamoe.py:176-182): returned = bf16 [T*K, H], the outputs of this
 * rank's send rows in send order; y[t] = bf16(fp32 sum over slots k in order of
 * returned[slot_rows[t*K + k]]). A slot row of -1 makes the token's row NaN. */
int megamoe_ep_combine(int32_t tokens, int32_t hidden, int32_t topk, const void* returned, const int32_t* slot_rows,
                       void* y, void* stream);

/* Dynamic E4M3 quantization of bf16 rows [rows, cols] with one fp32 scale
 * per row per 128 columns (the last block may be partial; padding counts as
 * zero): q e4m3fn [rows, cols], scales fp32 [rows, ceil(cols/128)].
 * Replaces pack_fp8_activation(value, power_of_two=pow2)
 * (megabench/tasks/quantization.py:87-109, scale_format="float"). */
int megamoe_quantize_rows(int32_t rows, int32_t cols, const void* x, uint8_t* q, float* scales,
                          int32_t pow2, void* stream);

/* Self-test of the E4M3 encoder the kernels use (gfx950's v_cvt_pk_fp8_f32, round to nearest
 * even, positive NaN recoded to 0x7f) against the bitwise rule of quantization.py:106,125:
 * for every fp32 bit pattern m in [first, first + count) with the sign bit clear (count may
 * reach 2^31 - first), m and -m, adds the number of codes that differ to *mismatches (a
 * device pointer to a uint64 the caller zeroes). Every clamped value lies in [0, 448.0f =
 * 0x43e00000] in magnitude or is NaN (0x7f800001 and up); infinity is clamped to 448 before
 * any encoding, and the rule is not defined for it. Asynchronous on `stream`. No reference
 * counterpart (test hook). */
int megamoe_e4m3_selftest(uint32_t first, uint32_t count, uint64_t* mismatches, void* stream);

/* Text for a status code (static storage). */
const char* megamoe_status_string(int status);

/* ABI version of this library: 10 (1, plus megamoe_block_forward and megamoe_rms_norm in 2,
 * plus megamoe_mx_workspace_bytes and megamoe_mx_forward in 3, plus megamoe_ep_dispatch,
 * megamoe_ep_experts and megamoe_ep_combine in 4, plus megamoe_forward_ex and
 * megamoe_combine_by_expert_id in 5, plus megamoe_forward_noalloc in 6, plus
 * megamoe_layer_forward in 7, plus megamoe_layer_status in 8, plus megamoe_mx_layer_forward
 * and megamoe_mx_layer_status in 9, plus megamoe_e4m3_selftest in 10, plus
 * megamoe_forward_w8a16 and megamoe_layer_forward_w8a16 in 11). */
int megamoe_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MEGAMOE_H */
