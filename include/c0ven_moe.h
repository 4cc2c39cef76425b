/* The MoE block on one MI355X: a C ABI over HIP.
 *
 * Replaces, for the mixture-of-experts block of the qwen4exp model, the reference's expert executors:
 *   - core/cpu/experts.h:32-60   CpuExperts::compute / compute_many / h_rows (the CPU expert path), and
 *   - the decode and prefill kernel lists of that block, model.cpp:1348-1414 and prompt.cpp:609-655
 *     (mv_xmx_bf16 router rows, router_group, moe_gate_up_g, moe_down_g, moe_combine; p_router, p_moe_count / scan /
 *     fill / scatter, moe_gate_up_t, moe_down_t, p_moe_combine).
 * The conventions are the reference's C ABI's (include/engine_api.h:1-10, :28-34, :384, :414-421):
 *   - every call returns a moe_status with engine_status's values; moe_last_error(ctx) gives the message;
 *   - no exception and no callback crosses the ABI; only plain structs, pointers and sizes do;
 *   - the library owns device memory (it uploads and lays out the weights itself); the caller owns x and y;
 *   - one host thread uses a context at a time; calls are synchronous unless named _async;
 *   - y is overwritten, never accumulated into (core/cpu/experts.cpp:112, :256-258);
 *   - exported symbols carry the moe_ prefix; everything else is hidden.
 * The data contracts are c0ven_quant.h (shared/quant.h) and c0ven_moe_tile.h (shared/moe_tile.h). */
#ifndef C0VEN_MOE_H
#define C0VEN_MOE_H

#include <stddef.h>
#include <stdint.h>

#include "c0ven_moe_tile.h"
#include "c0ven_quant.h"

#ifdef __cplusplus
extern "C" {
#endif

#if defined(C0VEN_MOE_EXPORT)
#define MOE_API __attribute__((visibility("default")))
#else
#define MOE_API
#endif

#define MOE_API_VERSION 1

typedef enum {
  MOE_OK = 0,
  MOE_ERROR = 1, /* see moe_last_error */
  MOE_BAD_ARGUMENT = 2,
  MOE_BUSY = 3,
  MOE_TIMEOUT = 4
} moe_status;

typedef struct moe_ctx moe_ctx;

/* The block's shape and types (ExpertShape, core/cpu/experts.h:24-31, with the router and the shared expert of
 * docs/spec/MODEL_LAYER.md section 4). Zero means the default given here. */
typedef struct {
  uint32_t n_embd;       /* H: K of gate and up, rows of down; a multiple of 512 */
  uint32_t n_ff;         /* F: rows of gate and up, K of down; a multiple of 64 and of down's block */
  uint32_t n_expert;     /* E routed experts, at most 512 */
  uint32_t n_used;       /* k, at most 16 */
  uint32_t n_layer;      /* layers held resident (default 1) */
  uint32_t gate_type;    /* QT_Q8_0, QT_Q4_K, QT_Q5_K, QT_Q6_K, QT_IQ3_S, QT_IQ4_NL, QT_IQ4_XS, QT_Q2_0, QT_IQ3_XXS or
                          * QT_IQ2_S: gate and up of the routed experts (the last two need moe_set_codebooks) */
  uint32_t down_type;    /* the same set: down of the routed experts */
  uint32_t has_shared;   /* 1: one shared expert with a sigmoid gate (the router's row E) */
  uint32_t sh_gate_type; /* the shared expert's gate (and up, unless sh_up_type says otherwise) */
  uint32_t sh_down_type;
  uint32_t max_tokens;   /* the most tokens one forward takes, at most 16384 (default 16) */
  float swiglu_limit;    /* > 0: gate = min(gate, L), up = clamp(up, -L, L) before the SiLU; 0 = off */
  int32_t device;        /* HIP device ordinal */
  uint32_t borrowed_immutable; /* 1: the bytes behind moe_compute_many's expert pointers do not change while the
                                * context lives, so their device copies are kept (keyed by pointer) across calls;
                                * 0: they are uploaded again on every call */
  uint32_t hc_lr;        /* > 0: the layers hold a hyper-connection mix and combine of this low rank (at most 512, a
                          * multiple of 8; the model's is 320) for moe_forward_hc */
  uint32_t sh_up_type;   /* the shared expert's up, when it differs from its gate (0: sh_gate_type). The model file
                          * mixes them per layer (blk.0: gate Q4_K, up IQ4_XS), as the reference runs the shared gate,
                          * up and down as three matvecs of their own types (model.cpp:828-830). Gate and up must take
                          * the same activation type, and may differ only among the types without a codebook. */
  uint32_t flags;        /* MOE_FLAG_* below */
} moe_config;

/* moe_config.flags: the prefill router sums every logit exactly (fp64, k order: the oracle's bits for the weights and
 * y too) instead of on the bf16 matrix cores within a bound, with the top k certified (the same ids; the weights and
 * y within the block's tolerance). */
#define MOE_FLAG_EXACT_ROUTER 1u
/* moe_config.flags: the prefill hyper-connection mix sums every W_down and W_inject product in the decode path's fixed
 * order, not only those its bound leaves open (slow: the check of that fallback). */
#define MOE_FLAG_HC_FIXED_ORDER 2u

/* The routing result of a forward, per token: k expert ids in rank order and their weights. */
typedef struct {
  int32_t *ids; /* ntok x n_used, or null */
  float *w;     /* ntok x n_used, or null */
} moe_route_out;

/* A pre-routed expert job (CpuExperts::Job, core/cpu/experts.h:46-50): the expert (layer, index; n_expert names the
 * shared expert), the token it serves and its weight. */
typedef struct {
  uint32_t layer;
  uint32_t expert;
  uint32_t tok;
  float w;
} moe_job;

/* Opens a context on cfg->device and allocates the resident weights of every layer and the scratch. */
MOE_API moe_status moe_open(const moe_config *cfg, moe_ctx **out);
MOE_API void moe_close(moe_ctx *ctx);
/* The last error's message, valid until the next call on ctx (ctx may be null for moe_open's failures). */
MOE_API const char *moe_last_error(const moe_ctx *ctx);

/* The router of a layer: (n_expert + 1) x n_embd bf16, row-major, the last row the shared expert's gate
 * (blk.N.ffn_gate_inp and ffn_gate_inp_shexp). bias: n_expert fp32 logit biases, or null for none. */
MOE_API moe_status moe_load_router(moe_ctx *ctx, uint32_t layer, const uint16_t *router_bf16, const float *bias);
/* One expert's three matrices in the file's layout (ggml blocks, row-major): gate and up n_ff x n_embd, down
 * n_embd x n_ff, of the context's types (expert == n_expert: the shared expert, of the shared types: gate
 * sh_gate_type, up sh_up_type, down sh_down_type). The library
 * repacks them into its device layout; the caller's buffers are not kept. */
MOE_API moe_status moe_load_expert(moe_ctx *ctx, uint32_t layer, uint32_t expert, const uint8_t *gate,
                                   const uint8_t *up, const uint8_t *down);

/* The block for ntok rows of x (host memory, rows x_stride floats apart) into y (y_stride): router, experts, shared
 * expert, combine. Synchronous. route may be null. Up to 16 tokens run the decode kernel (the decode and verify
 * shapes); more run the prefill kernels (router GEMM, counting-sort dispatch into MoeTiles, grouped MFMA expert GEMMs,
 * combine), up to max_tokens. */
MOE_API moe_status moe_forward(moe_ctx *ctx, uint32_t layer, const float *x, uint32_t ntok, uint64_t x_stride,
                               float *y, uint64_t y_stride, moe_route_out *route);
/* The same on device memory (x and y ntok x n_embd fp32, contiguous, 16-byte aligned; ids and w ntok x n_used or
 * null), enqueued on
 * stream (a hipStream_t; null: the context's stream). Nothing is copied and nothing waits. A context's forwards share
 * its scratch (work counters, hand-off records, intermediate buffers), so they must be ordered: enqueue them on one
 * stream, or make each stream wait for the previous forward's (an event) before enqueueing the next. moe_check
 * reports a forward whose internal waits gave up (MOE_TIMEOUT). */
MOE_API moe_status moe_forward_async(moe_ctx *ctx, uint32_t layer, const float *x_dev, uint32_t ntok, float *y_dev,
                                     int32_t *ids_dev, float *w_dev, void *stream);
/* No counterpart in the reference: moe_forward_async for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). The decode kernel only (ntok at most
 * min(max_tokens, 16)); its scratch lives in one statically sized array per GPU (16 MiB, set up when the first context
 * opens on that GPU) instead of the context's, and the call allocates nothing. A context whose decode scratch would
 * exceed the array is refused with MOE_BAD_ARGUMENT. Every call on a GPU shares that GPU's array, so calls on one GPU
 * must be ordered (one stream, or event waits): calls that overlap on one GPU race. Results equal moe_forward_async's. */
MOE_API moe_status moe_forward_async_noalloc(moe_ctx *ctx, uint32_t layer, const float *x_dev, uint32_t ntok,
                                             float *y_dev, int32_t *ids_dev, float *w_dev, void *stream);
/* An expert's matrices borrowed from the caller in the file's layout (ExpertWeights, core/cpu/experts.h:14-22): gate
 * and up n_ff x n_embd, down n_embd x n_ff, of the context's routed types. down_parts 2 stores down as two regions,
 * the first part of every row's blocks, then the second: with down_blocks {0, 0} the parts are equal and each row is
 * two dots added in order (supported where a part is one 256-value unit or the types have one term a row part), with
 * down_blocks set they are the parts' widths in blocks and the row is joined again (the file row's bits). */
typedef struct {
  const uint8_t *gate, *up, *down;
  uint32_t down_parts;
  uint16_t down_blocks[2];
} moe_expert_weights;

/* A job (CpuExperts::Job, core/cpu/experts.h:40-45): its expert's borrowed weights, the token and the weight. Jobs with
 * the same gate pointer are one expert, read once for all their tokens. */
typedef struct {
  moe_expert_weights expert;
  uint32_t tok;
  float w;
} moe_cm_job;

/* CpuExperts::compute_many (core/cpu/experts.h:40-49, experts.cpp:152-284) on borrowed weights: y (ntok rows, y_stride
 * floats apart; host memory) overwritten with, for each token, its jobs in the order given of w * down(silu(gate x) *
 * (up x)). The distinct experts are repacked and uploaded to the context's device copies (again on every call unless
 * borrowed_immutable), then ntok <= 16 runs the decode kernel and more the prefill kernels (up to max_tokens, which must
 * then exceed 16). A token takes at most n_used + 1 jobs. Synchronous. */
MOE_API moe_status moe_compute_many(moe_ctx *ctx, const moe_cm_job *jobs, uint32_t njobs, uint32_t ntok, const float *x,
                                    uint64_t x_stride, float *y, uint64_t y_stride);
/* CpuExperts::compute_many on resident experts: y[tok] = sum over the jobs with that tok, in the order given, of
 * w * expert(x[tok]); no router, no gate. Synchronous, host buffers. */
MOE_API moe_status moe_forward_experts(moe_ctx *ctx, const moe_job *jobs, uint32_t njobs, uint32_t ntok,
                                       const float *x, uint64_t x_stride, float *y, uint64_t y_stride);
/* CpuExperts::h_rows (core/cpu/experts.h:52-56): the h rows one pass of the down kernels takes, 256 here (one unit;
 * the GPU path has no task split). 0 when n_ff is not a multiple of it. */
MOE_API uint32_t moe_h_rows(const moe_config *cfg);
/* Whether moe_open would accept cfg's shape and types (the checks it makes before it touches a device); the reason
 * of a refusal is moe_last_error(null). No device is needed. No counterpart in the reference, whose loader checks a
 * file's types as it reads them. */
MOE_API moe_status moe_check_config(const moe_config *cfg);

/* The dispatch of the last prefill forward (p_moe_count / scan / fill, prompt.cl:682-738): ntiles receives the number
 * of MoeTiles, tiles (room for cap) the tiles in expert order, perm (ntok x n_used, or null) the assignment
 * (token * n_used + rank) at each row of the expert-ordered activations. Within an expert the rows are in token
 * order (the reference's fill takes atomic order). Synchronous. */
MOE_API moe_status moe_prefill_dispatch(moe_ctx *ctx, MoeTile *tiles, uint32_t cap, uint32_t *ntiles, uint32_t *perm);
/* The number of tokens whose top k the prefill router had to sum exactly (the bound left the winners or their order
 * open) since the last call, then cleared. Synchronous. */
MOE_API moe_status moe_prefill_exact_tokens(moe_ctx *ctx, uint32_t *n);

/* The hyper-connection module before a layer's block (docs/spec/MODEL_LAYER.md 1.1-1.2; the hc_ffn_* tensors of
 * blk.N): gamma 4 n_embd fp32 (hc_ffn_norm, the folded 1 + w), W_down hc_lr x 4 n_embd bf16, W_inject 4 x 4 n_embd
 * bf16, W_up 4 n_embd x hc_lr bf16 (row s n_embd + i), each row-major as the file holds it. Needs hc_lr > 0. */
MOE_API moe_status moe_load_hc(moe_ctx *ctx, uint32_t layer, const float *gamma, const uint16_t *w_down,
                               const uint16_t *w_inject, const uint16_t *w_up);
/* The block with its hyper-connection mix and combine fused into the decode launch (model.cpp:1350-1416: hc_mix, the
 * block, hc_combine): R_dev (device, ntok x 4 x n_embd fp32, the residual streams, 16-byte aligned) gives the
 * block's input x = (1/4) sum_s n_s sigma(a_s) and receives R_s += 2 sigma(inject_s / 4) y. y_dev (ntok x n_embd,
 * 16-byte aligned, may be null), ids_dev and w_dev (may be null) receive y and the routing. 1 <= ntok <= max_tokens:
 * up to 16 tokens the mix and combine are items of the decode launch, above that kernels around the prefill block
 * (prompt.cpp:478-504). No counterpart entry point in the reference, whose kernel list runs the same steps as
 * separate launches. */
MOE_API moe_status moe_forward_hc_async(moe_ctx *ctx, uint32_t layer, float *R_dev, uint32_t ntok, float *y_dev,
                                        int32_t *ids_dev, float *w_dev, void *stream);
/* The same with R (ntok x 4 x n_embd) and y (ntok x n_embd, may be null) in host memory; synchronous. */
MOE_API moe_status moe_forward_hc(moe_ctx *ctx, uint32_t layer, float *R, uint32_t ntok, float *y,
                                  moe_route_out *route);

/* Experts on the CPU (the hybrid of core/models/qwen4exp: layout.h:64-71 MissJob, layer.cl:838-884, model.cpp:1597-
 * 1627). resident (n_expert flags; null: all) says which routed experts of a layer the device holds; a decode forward
 * (up to 16 tokens) computes only those, and for each token publishes its misses in a record in host memory: */
typedef struct {
  uint32_t seq;       /* the forward's step (moe_last_step), stored last, behind a system-scope release */
  uint32_t nmiss;     /* routed experts of the token not resident */
  int32_t ids[16];    /* the misses' ids in rank order, then their weights */
  float w[16];
  int32_t all[16];    /* every routed id in rank order */
  /* followed by float x[n_embd]: the block's input for the token */
} moe_miss_job;
/* The host answers with ans_y[t] = its experts' sum over token t's misses, w in rank order (CpuExperts::compute_many
 * on the misses as jobs: y overwritten, then each job's w * out added in order), for every token with nmiss > 0, then
 * stores *ans_seq = the step (release). The forward's combine for such a token waits for that store (bounded: a
 * forward whose answer does not come within seconds reports MOE_TIMEOUT through moe_check) and adds ans_y[t]'s row
 * after the resident experts' terms and the shared expert's, as layer.cl:869-884 does. Tokens without misses do not
 * wait. The prefill path refuses a layer with non-resident experts. */
MOE_API moe_status moe_set_resident(moe_ctx *ctx, uint32_t layer, const uint8_t *resident);
/* The records and the answer, allocated in pinned host memory on the first call and kept until moe_close: jobs (a
 * moe_miss_job record a token, job_stride bytes apart, room for min(max_tokens, 16) tokens), ans_y (16 x n_embd
 * floats), ans_seq. A layer with misses needs them set up before its forwards. */
MOE_API moe_status moe_miss_buffers(moe_ctx *ctx, void **jobs, uint64_t *job_stride, float **ans_y,
                                    uint32_t **ans_seq);
/* The step number of the last forward enqueued on ctx (what its records' seq and the answer's seq must hold). */
MOE_API uint32_t moe_last_step(const moe_ctx *ctx);

/* Waits for the context's stream. */
MOE_API moe_status moe_sync(moe_ctx *ctx);
/* Waits for stream (null: the context's stream), then reports whether any forward since the last check had a wait
 * inside the decode kernel give up (MOE_TIMEOUT: its y is not to be trusted) and clears that state. Call it after
 * moe_forward_async calls on a stream of the caller's. */
MOE_API moe_status moe_check(moe_ctx *ctx, void *stream);
/* The context's HIP stream (a hipStream_t). */
MOE_API void *moe_stream(moe_ctx *ctx);

/* Per-kernel timing with HIP events recorded on the stream each kernel runs on, around every launch of every forward
 * while on (off by default; turning it on or off clears the record). on = 1 times every kernel; on = 2 only the
 * decode kernel and the prefill gate/up launches (each event pair puts packets between the launches, so fewer pairs
 * disturb a timed run less). moe_kernel_times waits for the recorded forwards, gives each kernel's average duration
 * per launch over them (names and avg_ms have room for cap entries; n receives how many kernels, forwards how many
 * forwards were averaged) and clears the record. */
MOE_API moe_status moe_set_timing(moe_ctx *ctx, int on);
MOE_API moe_status moe_kernel_times(moe_ctx *ctx, const char **names, float *avg_ms, uint32_t cap, uint32_t *n,
                                    uint32_t *forwards);

/* Tracing: while on, the decode kernel stamps every work item (s_memrealtime, a 100 MHz clock) when it starts, when
 * what it waits for is in (its operands staged), when its results are computed and stored, and when it ends (after
 * the hand-off work it does as the last of its kind). moe_trace gives the last forward's stamps as (start, ready,
 * computed, end) quadruples in item order, up to cap of them (a cap past n copies the rest of the 65536-quadruple
 * buffer too); n receives the number of items, bounds (8 entries, or null) where each kind begins: lead (router
 * rows; the hyper-connection mix's items, when moe_forward_hc ran, are the ones before it), top-k, the shared expert's gate/up and down (which run beside the router), the routed gate/up and down, the
 * combine, and the end. Items are dealt to the work-groups in order from one counter, as they ask. */
MOE_API uint32_t moe_grid(const moe_ctx *ctx);
/* Sets the decode kernel's grid, a multiple of 8 (0: back to what the device holds at once, the default). Any such
 * grid completes, whatever part of it the device admits at a time (another stream's kernels holding CUs, or a grid
 * larger than the device holds): the dispatcher deals work-groups to the eight XCDs in turn and each XCD starts its
 * share in index order, and every item's dependencies come earlier in that order, so the precondition is only that
 * each XCD eventually admits work-groups of the kernel. No counterpart in the reference (its kernel list has no
 * persistent kernel). */
MOE_API moe_status moe_set_grid(moe_ctx *ctx, uint32_t grid);
MOE_API moe_status moe_set_trace(moe_ctx *ctx, int on);
MOE_API moe_status moe_trace(moe_ctx *ctx, uint64_t *stamps, uint32_t cap, uint32_t *n, uint32_t *bounds);

/* Copies the resident experts (and shared expert) of src_layer over those of dst_layer, device to device. */
MOE_API moe_status moe_copy_experts(moe_ctx *ctx, uint32_t src_layer, uint32_t dst_layer);
/* Bytes of one resident matrix in the device layout: which = 0 routed gate (up is the same), 1 routed down,
 * 2 shared gate, 3 shared down, 4 shared up. These are the weights' own bytes, the block's algorithmic traffic per matrix. */
MOE_API moe_status moe_expert_bytes(const moe_ctx *ctx, uint32_t which, uint64_t *bytes);

/* Device bytes the context holds: resident weights and scratch. */
MOE_API uint64_t moe_device_bytes(const moe_ctx *ctx);

/* Decodes rows x cols values of a matrix of type in the file's layout through the device layout and the kernels'
 * decoders, into out (host, rows x cols fp32). For checking the layout and the decoders against the format. */
MOE_API moe_status moe_dequantize(moe_ctx *ctx, uint32_t type, const uint8_t *blocks, uint32_t rows, uint32_t cols,
                                  float *out);

/* The codebooks IQ3_XXS and IQ2_S decode through: a buffer in the QGRID layout of c0ven_quant.h, as the reference
 * packs ggml-common.h's tables (core/load/codebooks.cpp:14-33), at least QGRID_KVALUES bytes. iq2s_grid and
 * iq3xxs_grid are taken from it (this build does not carry them); its IQ3_S region must equal ggml's iq3s_grid, the
 * check that the buffer has the layout. A context whose types include IQ3_XXS or IQ2_S refuses forwards and
 * moe_dequantize of those types until this is called. No counterpart call in the reference, whose kernels receive the
 * same buffer at load time. */
MOE_API moe_status moe_set_codebooks(moe_ctx *ctx, const uint8_t *qgrid, uint64_t bytes);

/* Synthetic inputs (seeded, so that every machine draws the same values): counter-based normals, the library's
 * quantisers, the Zipf logit bias of BASELINE's configs. nthreads <= 0: all cores. */
MOE_API void moe_synth_normal(uint64_t seed, uint64_t stream, float sigma, float *out, uint64_t n, int nthreads);
/* rows x cols fp32 (row-major) into blocks of type (Q8_0: ggml's quantize_row_q8_0_ref; the others: this library's
 * own quantisers, which write valid blocks but are not ggml's search). IQ3_XXS and IQ2_S search the codebooks of the
 * last moe_synth_set_codebooks. Returns MOE_OK or BAD_ARGUMENT. */
/* The codebooks the IQ3_XXS and IQ2_S quantisers below search (a QGRID-layout buffer, as for moe_set_codebooks);
 * kept until the process ends. */
MOE_API moe_status moe_synth_set_codebooks(const uint8_t *qgrid, uint64_t bytes);
MOE_API moe_status moe_quantize(uint32_t type, const float *x, uint32_t rows, uint32_t cols, uint8_t *out,
                                int nthreads);
/* A matrix of N(0, sigma) values drawn from (seed, stream), quantised: the same bytes as moe_synth_normal followed by
 * moe_quantize, without the fp32 copy. */
MOE_API moe_status moe_synth_matrix(uint64_t seed, uint64_t stream, float sigma, uint32_t type, uint32_t rows,
                                    uint32_t cols, uint8_t *out, int nthreads);
/* bias[e] = -s ln(1 + pi(e)), pi a seeded permutation of the experts: softmax weights proportional to Zipf(s) ranks. */
MOE_API void moe_zipf_bias(uint64_t seed, uint32_t n_expert, float s, float *out);
/* Bytes of rows x cols values of type in the file's layout. */
MOE_API uint64_t moe_row_bytes(uint32_t type, uint32_t cols);

/* For the ABI test: one row per field of every struct above, "struct.field" with its offset and size, then one row
 * per struct, "struct", offset 0 and its size. Returns the number of rows; table may be null. */
typedef struct {
  const char *name;
  uint32_t offset;
  uint32_t size;
} moe_abi_row;
MOE_API uint32_t moe_abi_layout(moe_abi_row *table, uint32_t cap);

#ifdef __cplusplus
}
#endif

#endif
