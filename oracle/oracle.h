/* TEST INFRASTRUCTURE - the CPU oracle of the MoE block. Not product code: only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load it, as the checker; the product (c0ven_amd/) never links or calls it.
 *
 * A plain-C restatement of the reference's CPU expert path and of the block around it:
 *   - the weight decoders (ggml's dequantize_row_q8_0 / _q4_K / _q5_K / _q6_K / _iq3_s / _iq4_nl / _iq4_xs / _q2_0 /
 *     _iq3_xxs / _iq2_s, as docs/spec/QUANT_FORMATS.md:176-212, :373-400, :401-417, :419-445, :447-466, :234-246,
 *     :213-232, :251-270, :147-168, :115-137 state them;
 *     the last two through codebooks the caller supplies, as ggml-common.h is absent);
 *   - the activation quantisers the CPU path converts x and h with (q8_0, QUANT_FORMATS.md:463-465; q8_K,
 *     :528-535), chosen per weight type as core/cpu/experts.cpp:114-123 does (ggml's vec_dot_type);
 *   - the integer block dot products (vec_dot) of each weight type against its activation type;
 *   - CpuExperts::compute / compute_many (core/cpu/experts.cpp:109-150, :152-284): h = silu(g) * u with the optional
 *     clamp (:21-27), h quantised to the down's activation type, y overwritten with the jobs summed in job order;
 *   - the router (docs/spec/MODEL_LAYER.md:414-425): bf16 logits, softmax with the max subtracted and the sum in
 *     double, the top k with ties to the lower expert (kernels/models/qwen4exp/route.h:33-38), weights renormalised
 *     with max(sum, 6.1035e-5) (layer.cl:781-804); the shared expert and its sigmoid gate (MODEL_LAYER.md:444-449);
 *     the combine y = sum_k w_k y_k (rank order) + gs * s (layer.cl:869-884, llama-graph.cpp:2334-2343).
 *
 * Pinned by tests/test_oracle.py: the IQ3_S grid and kvalues_iq4nl against the sha256s in QUANT_FORMATS.md:546-547,
 * every decoder against
 * its closed form on hand-made blocks, the dot products against float dots of the decoded blocks and against brute
 * force, compute against compute_many, the router against brute-force sorting, and the block against a dense fp64
 * SwiGLU FFN where k = E. What only ggml itself could pin (its SIMD float summation order, see ORACLE ORDER below,
 * its bf16 dot order, and the fp32 steps of its CPU Q2_0 dot, whose source the reference does not hold: the oracle
 * takes the CUDA kernel's one term a 32-value half) is stated as unpinned there. */
#ifndef C0VEN_ORACLE_H
#define C0VEN_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ORACLE ORDER. The integer part of every block dot product is exact, so only the fp32 steps fix the bits. ggml's
 * SIMD kernels sum them in an architecture-dependent order that no source in the reference restates; the oracle uses
 * one canonical order, stated per type in oracle.c, and the GPU kernels reproduce it:
 *   - one fp32 term per 32 values for the q8_0 types (a Q8_0 or IQ4_NL block, half a Q2_0 block, as the CUDA
 *     kernels split Q2_0: QUANT_FORMATS.md:264-268) or per super-block (Q4_K, IQ3_S: 256 values);
 *   - a unit of 256 values (eight 32-value terms, one super-block) sums its terms as a pairwise tree; a row's last,
 *     partial unit (n_ff = 640: half a unit) sums the terms it has the same way:
 *     sum(a[0..n)) = sum(a[0..m)) + sum(a[m..n)), m the largest power of two below n (n = 1: a[0]);
 *   - a row adds its units in sequence, from 0.0f: acc = acc + unit_u, u ascending. */

typedef struct {
  uint32_t gate_type, down_type; /* QT_* of gate (and of up unless up_type says otherwise), and of down */
  uint32_t n_embd;               /* K of gate and up, rows of down */
  uint32_t n_ff;                 /* rows of gate and up, K of down */
  float swiglu_limit;            /* > 0: gate = min(gate, L), up = clamp(up, -L, L) before the SiLU */
  uint32_t up_type;              /* up's type when it is not gate_type (0: gate_type); same activation type */
} orc_shape;

typedef struct {
  const uint8_t *gate, *up, *down; /* the expert's three matrices in the file's layout (row-major blocks) */
  uint32_t tok;
  float w;
} orc_job;

typedef struct {
  uint32_t n_embd, n_ff, n_expert, n_used;
  uint32_t gate_type, down_type;       /* routed experts */
  uint32_t sh_gate_type, sh_down_type; /* the shared expert */
  float swiglu_limit;
  const uint16_t *router;              /* (n_expert + 1) x n_embd bf16: the router rows, then the shared gate */
  const float *bias;                   /* n_expert logit biases, or null */
  const uint8_t *const *gate, *const *up, *const *down; /* n_expert pointers each, file layout */
  const uint8_t *sh_gate, *sh_up, *sh_down;             /* null: no shared expert */
  uint32_t sh_up_type;                 /* the shared up's type when it is not sh_gate_type (0: the same) */
} orc_layer;

/* Scalars. */
uint16_t orc_fp32_to_fp16(float f);
float orc_fp16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_bf16(float f);
void orc_expf(const float *x, float *y, int64_t n); /* libm's expf, element by element */

/* The IQ3_S codebook, 512 x u32. */
void orc_iq3s_grid(uint32_t *out);
void orc_iq4nl_values(int8_t *out); /* kvalues_iq4nl, 16 signed bytes */
/* iq2s_grid and iq3xxs_grid from a QGRID-layout buffer (IQ3_XXS and IQ2_S decode through them). */
void orc_set_codebooks(const uint8_t *qgrid);

/* Returns 0, or -1 for a type it does not know or an n that is no whole number of blocks. */
int orc_dequantize_row(uint32_t type, const void *src, float *dst, int64_t n);
int orc_quantize_act(uint32_t act_type, const float *src, void *dst, int64_t n); /* QT_Q8_0 or QT_Q8_K */
int orc_vec_dot(uint32_t type, int64_t n, const void *w_row, const void *act, float *out);

/* CpuExperts::compute_many: y (ntok rows) overwritten; nthreads <= 0 uses one. Returns 0 or -1. */
int orc_compute_many(const orc_shape *s, const orc_job *jobs, uint32_t njobs, uint32_t ntok, const float *x,
                     uint64_t x_stride, float *y, uint64_t y_stride, int nthreads);
/* CpuExperts::compute: one token, experts in order with weights w. */
int orc_compute(const orc_shape *s, const uint8_t *const *gate, const uint8_t *const *up, const uint8_t *const *down,
                const float *w, uint32_t n, const float *x, float *y);

/* The router for ntok rows of x: logits (ntok x (n_expert + 1), the last the shared gate's pre-sigmoid value, may be
 * null), ids and w (ntok x k). */
int orc_route(const uint16_t *router, const float *bias, uint32_t n_expert, uint32_t n_embd, uint32_t k,
              const float *x, uint32_t ntok, uint64_t x_stride, float *logits, int32_t *ids, float *w);

/* topk_row on given logits (n_expert values): ids and w (k each), as orc_route does after its logits. */
int orc_topk_logits(const float *logits, uint32_t n_expert, uint32_t k, int32_t *ids, float *w);

/* The whole block. ids and w (ntok x n_used) may be null. */
int orc_moe_forward(const orc_layer *L, const float *x, uint32_t ntok, uint64_t x_stride, float *y, uint64_t y_stride,
                    int32_t *ids, float *w, int nthreads);

/* The block with the experts whose resident flag is 0 computed apart (the CPU's answer) and added after the shared
 * expert's term, as the device combines them. */
int orc_moe_forward_resident(const orc_layer *L, const uint8_t *resident, const float *x, uint32_t ntok,
                             uint64_t x_stride, float *y, uint64_t y_stride, int nthreads);

/* The CPU baseline (cpu_fast.c): the same block, the same bits as orc_moe_forward, with SIMD integer dot products
 * (AVX-512BW when the CPU has it, else AVX2), the router's rows as SIMD lanes each summed in k order, and
 * OpenMP over rows. Returns 0 or -1. orc_fast_isa names the instruction set it uses. */
int orc_fast_moe_forward(const orc_layer *L, const float *x, uint32_t ntok, uint64_t x_stride, float *y,
                         uint64_t y_stride, int32_t *ids, float *w, int nthreads);
const char *orc_fast_isa(void);

/* The hyper-connection mix before the block (MODEL_LAYER.md 1.1): R (T x 4 x H) to x (T x H) and the inject logits
 * (T x 4), with gamma (4 H), W_down (lr x 4H bf16), W_inject (4 x 4H bf16), W_up (4H x lr bf16, row s H + i). */
int orc_hc_pre(const float *R, uint32_t T, uint32_t H, uint32_t lr, const float *gamma, const uint16_t *w_down,
               const uint16_t *w_inj, const uint16_t *w_up, float *x, float *inject);
/* The combine after it (1.2): R_s += 2 sigma(inject_s / 4) y. */
void orc_hc_post(float *R, uint32_t T, uint32_t H, const float *inject, const float *y);

#ifdef __cplusplus
}
#endif

#endif
