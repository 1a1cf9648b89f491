/*
 * lb_oracle.h — CPU restatement of LightBridge-Engine's quantized-dot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP product
 * (liblightbridge_hip.so) and the CPU baseline that bench.py times beside it.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it; the product never links, loads or falls back to it.
 *
 * Every function restates the reference Rust (crates/..., cited per function in
 * lb_oracle.c) with the same integer decomposition and the same f32 operation
 * order, built with -ffp-contract=off so no multiply-add is fused.
 *
 * Status codes mirror QuantError (crates/bridge-quant-layout/src/error.rs:6-65)
 * and KernelError (crates/bridge-kernels-reference/src/error.rs:7-59).
 */
#ifndef LB_ORACLE_H
#define LB_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (crates/bridge-core/src/ggml_type.rs:10-30). */
enum {
    LBO_F32 = 0,
    LBO_Q4_K = 12,
    LBO_Q5_K = 13,
    LBO_Q8_K = 15,
    LBO_IQ3_S = 21,
    LBO_IQ2_S = 22,
};

enum {
    LBO_OK = 0,
    /* QuantError */
    LBO_UNSUPPORTED_TYPE = 1,
    LBO_ZERO_LOGICAL_ELEMENTS = 2,
    LBO_LOGICAL_ELEMENTS_NOT_DIVISIBLE = 3,
    LBO_ARITHMETIC_OVERFLOW = 4,
    LBO_ENCODED_LENGTH_MISMATCH = 6,
    LBO_OUTPUT_LENGTH_MISMATCH = 7,
    LBO_NON_FINITE_SCALE = 8,
    LBO_NON_FINITE_ACTIVATION = 9,
    LBO_NON_FINITE_Q8_SCALE = 10,
    /* KernelError */
    LBO_DIMENSION_MISMATCH = 20,
    LBO_SCRATCH_TOO_SMALL = 21,
    LBO_NON_FINITE_VALUE = 22,
    LBO_ROUTED_EXPERT_ORDER = 23,
    LBO_DUPLICATE_ROUTED_EXPERT = 24,
    LBO_INVALID_PARAMETER = 25,
};

typedef struct lbo_error {
    int32_t status;
    int32_t ty;          /* GGML type the error refers to */
    uint64_t index;      /* block_index / lane index / row */
    uint64_t expected;
    uint64_t actual;
    uint32_t bits;       /* offending f16/f32 bits */
    uint32_t field;      /* 0 = d, 1 = dmin (NonFiniteScale) */
} lbo_error;

#define LBO_Q8K_BLOCK_ELEMENTS 256
#define LBO_Q8K_BLOCK_BYTES 292

/* Block layout (crates/bridge-quant-layout/src/k_quants.rs:34-54). */
size_t lbo_block_bytes(int ty);

/* quantize_row_q8_k_into (q8_k.rs:16-76). */
int lbo_quantize_row_q8_k(const float *input, size_t n, uint8_t *encoded, size_t encoded_len,
                          lbo_error *err);

/* vec_dot_q8_k (q8_k.rs:80-89): validated scalar dot of one packed row. */
int lbo_vec_dot_q8_k(int ty, const uint8_t *w, size_t w_len, const uint8_t *q8, size_t q8_len,
                     size_t n, float *out, lbo_error *err);

/* vec_dot_q8_k_cpu (q8_k.rs:103-119) through the AVX2 restatement (q8_k.rs:436-731). */
int lbo_vec_dot_q8_k_avx2(int ty, const uint8_t *w, size_t w_len, const uint8_t *q8, size_t q8_len,
                          size_t n, float *out, lbo_error *err);

/* Unvalidated scalar dot (q8_k.rs:163-170) for callers that validated already. */
float lbo_dot_scalar(int ty, const uint8_t *w, const uint8_t *q8, size_t blocks);
float lbo_dot_avx2(int ty, const uint8_t *w, const uint8_t *q8, size_t blocks);

/* Integer stage of the dots, exported for bit-exact checks of the GPU path:
 * IQ2_S / IQ3_S: one int32 block_sum per block (q8_k.rs:337-364, :380-428);
 * Q4_K / Q5_K:   nine int32 per block: lane_sums[0..8] then minimum_sum (q8_k.rs:295-312). */
int lbo_block_sums(int ty, const uint8_t *w, const uint8_t *q8, size_t blocks, int32_t *out);

/* decode_row_into (k_quants.rs:71-105): exact f32 dequantization. */
int lbo_decode_row(int ty, const uint8_t *w, size_t w_len, size_t n, float *out, size_t out_len,
                   lbo_error *err);

/* Matrices use GGML [input_width=K, output_width=rows] row-major bytes (matrix.rs:102-186). */
typedef struct lbo_matrix {
    int32_t ty;
    uint64_t rows;   /* output_width */
    uint64_t k;      /* input_width */
    const uint8_t *bytes;
} lbo_matrix;

/* Execution modes (crates/bridge-kernels-reference/src/gemv.rs:12-16) plus the
 * thread count / ISA of the CPU backend (crates/bridge-kernels-cpu/src/lib.rs:76-126). */
enum { LBO_MODE_DEQUANT_F32 = 0, LBO_MODE_LLAMA_Q8K = 1, LBO_MODE_CPU_PARALLEL_Q8K = 2 };

typedef struct lbo_exec {
    int32_t mode;
    int32_t threads;   /* row-parallel workers for CPU_PARALLEL_Q8K (>= 1) */
    int32_t avx2;      /* 1: AVX2 dots (vec_dot_q8_k_cpu), 0: scalar */
} lbo_exec;

/* gemv_into (gemv.rs:88-115). q8_scratch must hold (K/256)*292 bytes for quantized types. */
int lbo_gemv(const lbo_exec *ex, const lbo_matrix *m, const float *input, size_t input_len,
             float *output, size_t output_len, uint8_t *q8_scratch, size_t q8_len, lbo_error *err);

/* gemv_accumulate_scaled_into (gemv.rs:117-174). */
int lbo_gemv_accumulate(const lbo_exec *ex, const lbo_matrix *m, const float *input,
                        size_t input_len, float *destination, size_t dest_len, float scale,
                        uint8_t *q8_scratch, size_t q8_len, lbo_error *err);

/* Row matvec over an already-quantized Q8_K vector (the metric's unit): y[r] = dot(row r, q8). */
int lbo_gemv_prequantized(const lbo_exec *ex, const lbo_matrix *m, const uint8_t *q8, float *y);

/* SwiGLU expert (crates/bridge-kernels-reference/src/activation.rs:6-178). */
typedef struct lbo_expert {
    lbo_matrix gate, up, down;
} lbo_expert;

/* apply_swiglu (activation.rs:170-178) on arrays; returns first non-finite index or -1. */
int64_t lbo_apply_swiglu(float *gate, const float *up, size_t n);

/* moe_routed_by_id_into (crates/bridge-kernels-reference/src/moe.rs:64-147).
 * preflight = 1 runs the validation pass over every expert first, as the
 * reference does; 0 runs the single accumulate pass (same output). */
int lbo_moe_routed_by_id(const lbo_exec *ex, const uint32_t *ids, const float *coefs,
                         size_t n_routed, const lbo_expert *experts, size_t n_experts,
                         const lbo_expert *shared, const float *input, float *output, int preflight,
                         lbo_error *err);

/* residual_add_in_place (crates/bridge-kernels-reference/src/norm.rs:83-98), as
 * hy3_block_forward_token ends (layer.rs:464): destination += residual. */
int lbo_residual_add_in_place(float *destination, size_t dest_len, const float *residual, size_t residual_len,
                              lbo_error *err);

/* route_experts_into (crates/bridge-model-hy3/src/routing.rs:25-107). */
int lbo_route_sigmoid_bias(const float *logits, const float *bias, size_t n_experts, size_t top_k,
                           float weight_scale, uint32_t *ids, float *coefs, lbo_error *err);

/* Softmax top-k with renormalised weights (the benchmark configs' router; no
 * reference counterpart).  Spec: order experts by (logit desc, id asc), take
 * the first k, m = max logit, e_i = expf(l_i - m) over the k in that order,
 * s = sum of e_i in that order, coef_i = e_i / s; output sorted by id. */
int lbo_route_softmax_topk(const float *logits, size_t n_experts, size_t top_k, uint32_t *ids,
                           float *coefs, lbo_error *err);

/* F32 router logits as dot_f32_row (gemv.rs:286-303): sequential sum over K. */
void lbo_router_logits_f32(const float *w, size_t n_experts, size_t k, const float *x, float *logits);

/* IEEE binary16 -> binary32 (half 2.7.1 f16::to_f32 semantics). */
float lbo_f16_to_f32(uint16_t h);

/* glibc expf as the reference's f32::exp links it (exposed for the GPU expf check). */
float lbo_expf(float x);
void lbo_expf_array(const float *x, float *out, size_t n);

#ifdef __cplusplus
}
#endif
#endif
