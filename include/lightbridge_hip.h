/*
 * lightbridge_hip.h — C ABI of the MI355X (gfx950) backend for LightBridge's
 * quantized-dot hot path: Q8_K activation quantization, the
 * {IQ2_S, IQ3_S, Q4_K, Q5_K} x Q8_K integer-dot matvecs and the SwiGLU MoE
 * expert FFN built from them.
 *
 * Plain C types only.  Every buffer argument named *_dev is a device pointer
 * (hipMalloc / torch CUDA memory) on the context's device; work is ordered on
 * the context's stream.  Functions return an lbh_status; on error they fill
 * *err (if non-NULL) and leave every output buffer unchanged (the reference's
 * atomicity rule, crates/bridge-quant-layout/src/q8_k.rs:16-33,
 * crates/bridge-kernels-reference/src/gemv.rs:245-272).
 *
 * Functions marked [sync] wait for their stream to report an error the
 * reference reports synchronously.  Functions marked [async] only enqueue.
 *
 * Status codes map 1:1 onto QuantError (crates/bridge-quant-layout/src/error.rs:6-65)
 * and KernelError (crates/bridge-kernels-reference/src/error.rs:7-59).
 */
#ifndef LIGHTBRIDGE_HIP_H
#define LIGHTBRIDGE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (crates/bridge-core/src/ggml_type.rs:10-30). */
enum lbh_ggml_type {
    LBH_F32 = 0,
    LBH_Q4_K = 12,
    LBH_Q5_K = 13,
    LBH_Q8_K = 15,
    LBH_IQ3_S = 21,
    LBH_IQ2_S = 22,
};

typedef enum lbh_status {
    LBH_OK = 0,
    /* QuantError */
    LBH_UNSUPPORTED_TYPE = 1,
    LBH_ZERO_LOGICAL_ELEMENTS = 2,
    LBH_LOGICAL_ELEMENTS_NOT_DIVISIBLE = 3,
    LBH_ARITHMETIC_OVERFLOW = 4,
    LBH_ENCODED_LENGTH_MISMATCH = 6,
    LBH_OUTPUT_LENGTH_MISMATCH = 7,
    LBH_NON_FINITE_SCALE = 8,
    LBH_NON_FINITE_ACTIVATION = 9,
    LBH_NON_FINITE_Q8_SCALE = 10,
    /* KernelError */
    LBH_DIMENSION_MISMATCH = 20,
    LBH_SCRATCH_TOO_SMALL = 21,
    LBH_NON_FINITE_VALUE = 22,
    LBH_ROUTED_EXPERT_ORDER = 23,
    LBH_DUPLICATE_ROUTED_EXPERT = 24,
    LBH_INVALID_PARAMETER = 25,
    /* backend */
    LBH_HIP_ERROR = 100,
    LBH_NULL_ARGUMENT = 101,
    LBH_UNSUPPORTED_SHAPE = 102,
    LBH_DEVICE_TIMEOUT = 103,   /* a bounded in-kernel wait gave up (the result was discarded) */
    LBH_SCRATCH_IN_USE = 104,   /* lbh_gemm_q8_k_noalloc: the GPU's static scratch is still in use by a
                                   call on another stream */
} lbh_status;

/* Error payload: the fields of the corresponding QuantError/KernelError variant. */
typedef struct lbh_error {
    int32_t status;
    int32_t ty;        /* GGML type the error refers to */
    uint64_t index;    /* block_index (NonFiniteScale), lane (NonFiniteActivation/Value), expert id */
    uint64_t expected;
    uint64_t actual;
    uint32_t bits;     /* offending binary16 / binary32 bits */
    uint32_t field;    /* NonFiniteScale: 0 = d, 1 = dmin */
    uint64_t row;      /* matrix row for weight errors */
    int32_t hip_error; /* hipError_t for LBH_HIP_ERROR */
    int32_t reserved;
} lbh_error;

typedef struct lbh_ctx lbh_ctx;
typedef struct lbh_matrix lbh_matrix;
typedef struct lbh_moe lbh_moe;
typedef struct lbh_router lbh_router;

/* Q8_K ABI constants (crates/bridge-quant-layout/src/q8_k.rs:7-12). */
#define LBH_Q8_K_BLOCK_ELEMENTS 256
#define LBH_Q8_K_BLOCK_BYTES 292

/* ---- backend / dispatch surface -------------------------------------------
 * Counterpart of CpuBackend / CpuCapabilities (crates/bridge-kernels-cpu/src/lib.rs:19-126):
 * the hip backend joins cpu_parallel_avx2_q8_k / cpu_parallel_scalar_q8_k. */

/* Backend name reported beside CpuCapabilities::backend_name (lib.rs:50-56): "hip_gfx950_q8_k". */
const char *lbh_backend_name(void);

/* Number of visible HIP devices whose ISA is gfx950 (0 when none: the caller keeps the CPU backend). */
int32_t lbh_device_count(void);

/* CpuBackend::new (lib.rs:76-90): opens `device`; `stream` is a hipStream_t or NULL (null stream). */
lbh_status lbh_ctx_create(int32_t device, void *stream, lbh_ctx **out, lbh_error *err);
lbh_status lbh_ctx_destroy(lbh_ctx *ctx);
lbh_status lbh_ctx_set_stream(lbh_ctx *ctx, void *stream);
/* Launch-shape knobs (no reference counterpart: the CPU backend's only knob is
 * its thread count, CpuBackendConfig, lib.rs:7-17).  value 0 restores the default. */
enum lbh_tuning_key {
    LBH_TUNE_GEMV_LPU = 1,         /* lanes per (row, block) unit: 1, 2 or 4 */
    LBH_TUNE_GEMV_MAX_BLOCKS = 2,  /* workgroup cap of the persistent matvec row loop (0: resident x CUs) */
    LBH_TUNE_GEMM_SHAPE = 3,       /* K-quant GEMM schedule: 0 = default (3 from 97 tokens, else 2);
                                      1 = 2 x 2 tiles of 32 x 32, direct buffer-to-LDS loads one block
                                      ahead; 2 = 2 x 2 tiles staged through registers two blocks ahead;
                                      3 = 3 x 4 tiles, the nine chains in three passes over K */
    LBH_TUNE_GEMV_DEPTH = 4,       /* matvec row steps in flight per wave: 1, 2, 3 or 4; 1 runs the
                                      one-lane-per-unit IQ instances as 1024-thread workgroups with
                                      the activations in LDS (the default for large IQ shapes) */
};
lbh_status lbh_ctx_set_tuning(lbh_ctx *ctx, int32_t key, int32_t value);
/* Compute units of the context's device. */
int32_t lbh_ctx_cu_count(const lbh_ctx *ctx);
/* Waits for the context's stream. */
lbh_status lbh_ctx_synchronize(lbh_ctx *ctx, lbh_error *err);

/* ---- Q8_K quantization ------------------------------------------------------ */

/* [sync] quantize_row_q8_k_into (crates/bridge-quant-layout/src/q8_k.rs:16-76):
 * n f32 (n % 256 == 0) -> (n/256) * 292 bytes, bit-identical to the reference. */
lbh_status lbh_quantize_row_q8_k_into(lbh_ctx *ctx, const float *input_dev, size_t n,
                                      uint8_t *encoded_dev, size_t encoded_len, lbh_error *err);

/* [async] Unchecked form for the hot path: `rows` independent vectors of n floats
 * (row stride n) -> rows * (n/256) * 292 bytes.  Non-finite input is not
 * reported (call the checked form to validate). */
lbh_status lbh_quantize_q8_k_rows(lbh_ctx *ctx, const float *input_dev, size_t rows, size_t n,
                                  uint8_t *encoded_dev);

/* ---- packed matrices ---------------------------------------------------------
 * PackedMatrix (crates/bridge-kernels-reference/src/matrix.rs:102-186): GGML
 * [input_width = k, output_width = rows] row-major block bytes.  Upload checks
 * the exact byte length and the finiteness of every block's f16 d (and dmin),
 * the checks validate_vec_dot_q8_k repeats per call (q8_k.rs:121-161,
 * k_quants.rs:178-208), and stores the bytes in HBM in the backend's lossless
 * device layout.  F32 matrices (ggml_type 0: rows x k floats, k a multiple of
 * 256, else LBH_UNSUPPORTED_SHAPE) serve lbh_gemv_into, lbh_gemv_accumulate_
 * scaled_into and the lbh_gemv_dequant_* forms, which compute dot_f32_row for
 * them in every mode (gemv.rs:88-101, :128-146, :286-303); the Q8_K entry
 * points (lbh_gemv_q8_k, lbh_gemv_f32, lbh_gemv_q8_k_into, lbh_gemv_block_sums,
 * the MoE layers, the GEMM) refuse them with LBH_UNSUPPORTED_TYPE, and
 * lbh_matrix_create_streamed takes the quantized types only. */

/* [sync] `bytes` is host memory when bytes_on_device == 0, device memory otherwise. */
lbh_status lbh_matrix_create(lbh_ctx *ctx, int32_t ggml_type, size_t rows, size_t k, const void *bytes,
                             size_t byte_len, int32_t bytes_on_device, lbh_matrix **out, lbh_error *err);
/* Reader of a tensor's GGML payload: writes `bytes` bytes starting at `offset`
 * (relative to the tensor's first byte) into dst; returns 0 or a reader-specific
 * non-zero code (reported as LBH_SOURCE_READ_FAILED with the code in `actual`). */
typedef int32_t (*lbh_byte_reader)(void *user, uint64_t offset, uint8_t *dst, size_t bytes);
#define LBH_SOURCE_READ_FAILED 36
/* [sync] lbh_matrix_create for a tensor streamed from its source (a GGUF file's
 * payload, crates/bridge-gguf/src/reader.rs:194-341 locates it) straight to HBM:
 * the reader fills 32 MiB pinned chunks, each checked on the host (the
 * validation of lbh_matrix_create, same error payload) and DMA'd and repacked
 * while the next one is read; no host copy of the whole tensor and no device
 * staging of it.  On error nothing is created. */
lbh_status lbh_matrix_create_streamed(lbh_ctx *ctx, int32_t ggml_type, size_t rows, size_t k, lbh_byte_reader reader,
                                      void *user, lbh_matrix **out, lbh_error *err);
lbh_status lbh_matrix_destroy(lbh_matrix *m);
/* [sync] Inverse of the device layout: writes the original GGML bytes to host memory. */
lbh_status lbh_matrix_read_ggml(lbh_ctx *ctx, const lbh_matrix *m, void *host_bytes, size_t byte_len,
                                lbh_error *err);
size_t lbh_matrix_rows(const lbh_matrix *m);
size_t lbh_matrix_k(const lbh_matrix *m);
int32_t lbh_matrix_type(const lbh_matrix *m);
size_t lbh_matrix_bytes(const lbh_matrix *m);

/* ---- matvec ------------------------------------------------------------------ */

/* [sync] gemv_into(CpuParallelQ8K) (crates/bridge-kernels-reference/src/gemv.rs:56-70, :88-115):
 * output[r] = vec_dot_q8_k(row r, Q8_K(input)).  q8_scratch_dev holds >= (k/256)*292 bytes.
 * An F32 matrix takes gemv_cpu_parallel_f32_into (gemv.rs:72-86): output[r] =
 * dot_f32_row(r), bit-identical, after prepare_dequant's checks (dimensions,
 * finite input, finite weights: NonFiniteValue field 1, index 0, `row` and
 * `actual` = the first non-finite weight's row and column); the Q8_K scratch is
 * not used. */
lbh_status lbh_gemv_into(lbh_ctx *ctx, const lbh_matrix *m, const float *input_dev, size_t input_len,
                         float *output_dev, size_t output_len, uint8_t *q8_scratch_dev, size_t q8_len,
                         lbh_error *err);

/* [sync] gemv_accumulate_scaled_into (gemv.rs:117-174): destination[r] += scale * dot(row r). */
lbh_status lbh_gemv_accumulate_scaled_into(lbh_ctx *ctx, const lbh_matrix *m, const float *input_dev,
                                           size_t input_len, float *destination_dev, size_t dest_len,
                                           float scale, uint8_t *q8_scratch_dev, size_t q8_len,
                                           lbh_error *err);

/* [async] The matvec over an already-quantized Q8_K vector (the benchmark unit):
 * accumulate == 0: y[r] = dot(row r, q8);  accumulate != 0: y[r] += coef * dot(row r, q8). */
lbh_status lbh_gemv_q8_k(lbh_ctx *ctx, const lbh_matrix *m, const uint8_t *q8_dev, float *y_dev,
                         float coef, int32_t accumulate);

/* [async] Fused form of gemv_into / gemv_accumulate_scaled_into without the
 * finiteness checks: the kernel quantizes x (k floats) to Q8_K itself (bytes
 * identical to lbh_quantize_row_q8_k_into; written to q8_out when non-NULL)
 * and computes the matvec in the same launch. */
lbh_status lbh_gemv_f32(lbh_ctx *ctx, const lbh_matrix *m, const float *x_dev, uint8_t *q8_out_dev, float *y_dev,
                        float coef, int32_t accumulate);

/* [async] Integer stage for bit-exact verification: per (row, block) the IQ2_S/IQ3_S
 * block_sum (one int32) or the Q4_K/Q5_K lane_sums[8] + minimum_sum (nine int32)
 * of q8_k.rs:295-312, :337-364, :380-428.  out_dev holds rows * (k/256) * {1|9} int32. */
lbh_status lbh_gemv_block_sums(lbh_ctx *ctx, const lbh_matrix *m, const uint8_t *q8_dev, int32_t *out_dev);

/* ---- checked dots over caller-supplied Q8_K ----------------------------------
 * The reference's dot API takes a packed weight row and an already-quantized
 * Q8_K row (crates/bridge-quant-layout/src/lib.rs:16-19): vec_dot_q8_k,
 * validate_vec_dot_q8_k and the typed vec_dot_{q4_k,q5_k,iq2_s,iq3_s}_q8_k
 * (q8_k.rs:80-101, :172-186).  These entry points take `rows` consecutive raw
 * GGML rows (rows = 1 is exactly the reference call) in device memory, no
 * upload needed, any byte alignment.  Checks, in the order of
 * validate_vec_dot_q8_k_inner (q8_k.rs:121-161): type (UnsupportedType),
 * logical_elements (ZeroLogicalElements / LogicalElementsNotDivisible),
 * weights_len == rows * row bytes and q8_len == (n/256) * 292
 * (EncodedLengthMismatch, ty = the weight type / Q8_K), then per row in order
 * the weights' f16 d / dmin (NonFiniteScale: index = block, field, bits, row)
 * and the Q8_K d of every block (NonFiniteQ8Scale: index = block, bits).
 * logical_elements is limited to 64 blocks (UnsupportedShape). */

/* [sync] validate_vec_dot_q8_k (q8_k.rs:91-101). */
lbh_status lbh_validate_vec_dot_q8_k(lbh_ctx *ctx, int32_t ggml_type, const uint8_t *weights_dev, size_t weights_len,
                                     size_t rows, const uint8_t *q8_dev, size_t q8_len, size_t logical_elements,
                                     lbh_error *err);

/* [sync] vec_dot_q8_k (q8_k.rs:80-89) per row: out_dev[r] = dot(row r, q8), bit-identical;
 * out_len must equal rows (OutputLengthMismatch).  On any error out_dev is unchanged. */
lbh_status lbh_vec_dot_q8_k_into(lbh_ctx *ctx, int32_t ggml_type, const uint8_t *weights_dev, size_t weights_len,
                                 size_t rows, const uint8_t *q8_dev, size_t q8_len, size_t logical_elements,
                                 float *out_dev, size_t out_len, lbh_error *err);

/* [sync] Checked lbh_gemv_q8_k over an uploaded matrix (its weight scales were checked
 * at upload): accumulate == 0: y[r] = dot(row r, q8); else y[r] += coef * dot(row r, q8)
 * after the checks of gemv_accumulate_scaled_into (finite coef, finite destination:
 * NonFiniteValue, field 2 / 3).  Then y_len == rows (DimensionMismatch, index 1),
 * q8_len == (k/256) * 292 (EncodedLengthMismatch) and the Q8_K scales
 * (NonFiniteQ8Scale).  On any error y_dev is unchanged. */
lbh_status lbh_gemv_q8_k_into(lbh_ctx *ctx, const lbh_matrix *m, const uint8_t *q8_dev, size_t q8_len, float *y_dev,
                              size_t y_len, float coef, int32_t accumulate, lbh_error *err);

/* ---- DequantF32 execution mode ----------------------------------------------
 * ReferenceExecutionMode::DequantF32 (crates/bridge-kernels-reference/src/gemv.rs:12-16):
 * output[r] = the sequential f32 sum over every element of decode(w[r][i]) * input[i]
 * (dot_dequant_row, gemv.rs:305-328, with the exact decoders of k_quants.rs:242-300,
 * iq2_s.rs:9-39, iq3_s.rs:9-53), bit-identical.  No Q8_K quantization is involved. */

/* [sync] gemv_dequant_f32_into (gemv.rs:33-41): validate_dimensions (DimensionMismatch,
 * NonFiniteValue on the input) as lbh_gemv_into. */
lbh_status lbh_gemv_dequant_into(lbh_ctx *ctx, const lbh_matrix *m, const float *input_dev, size_t input_len,
                                 float *output_dev, size_t output_len, lbh_error *err);

/* [sync] The DequantF32 arm of gemv_accumulate_scaled_into (gemv.rs:117-151):
 * destination[r] += scale * dot_dequant_row(r). */
lbh_status lbh_gemv_dequant_accumulate_scaled_into(lbh_ctx *ctx, const lbh_matrix *m, const float *input_dev,
                                                   size_t input_len, float *destination_dev, size_t dest_len,
                                                   float scale, lbh_error *err);

/* [async] Unchecked form: accumulate == 0: y = dot; else y += coef * dot. */
lbh_status lbh_gemv_dequant_f32(lbh_ctx *ctx, const lbh_matrix *m, const float *x_dev, float *y_dev, float coef,
                                int32_t accumulate);

/* ---- token batches on the matrix cores (prefill) ----------------------------------
 * The reference has no batched path ("grouped prefill unavailable", docs/STATUS.md:29):
 * it evaluates vec_dot_q8_k (q8_k.rs:80-89) row by row for one token at a time.
 * These entry points compute y[t][r] = vec_dot_q8_k(row r, token t) for a batch of
 * tokens with v_mfma_f32_32x32x16_f16 on integer operands, bit-identical to the per-row
 * dot for Q4_K and Q5_K (dot_q4_or_q5_k, q8_k.rs:247-327): the sub-block scales are
 * folded into the weights of an MFMA-ready copy of the matrix (integers <= 1953, exact
 * in f16), every (block, lane residue) sum is an exact integer below 2^24, and the
 * nine f32 chains per block run in the reference order. */

/* [sync] Builds the matrix's MFMA-ready copy (Q4_K / Q5_K only; 3.9x (Q4_K) or 3.2x
 * (Q5_K) the packed bytes, allocated once and freed with the matrix). */
lbh_status lbh_matrix_prepare_gemm(lbh_ctx *ctx, lbh_matrix *m, lbh_error *err);
/* HBM bytes the matrix holds: the packed planes (lbh_matrix_bytes) plus the MFMA-ready
 * copy once prepared (no reference counterpart: the reference's PackedMatrix is its bytes). */
size_t lbh_matrix_device_bytes(const lbh_matrix *m);

/* Device workspace bytes of lbh_gemm_q8_k for n_tokens tokens of k elements (0 if k % 256). */
size_t lbh_gemm_workspace_bytes(size_t n_tokens, size_t k);

/* [async] y_dev[t * rows + r] = vec_dot_q8_k(row r, token t) for t < n_tokens: q8_dev holds
 * n_tokens consecutive Q8_K rows of k/256 blocks (quantize_row_q8_k_into layout).  The matrix
 * must be prepared (lbh_matrix_prepare_gemm); workspace_dev holds lbh_gemm_workspace_bytes. */
lbh_status lbh_gemm_q8_k(lbh_ctx *ctx, const lbh_matrix *m, const uint8_t *q8_dev, size_t n_tokens, float *y_dev,
                         void *workspace_dev, size_t workspace_len);

/* Bytes of the per-GPU static scratch that lbh_gemm_q8_k_noalloc stages its
 * activation tiles in: lbh_gemm_workspace_bytes(n_tokens, k) must not exceed it,
 * which admits up to 928 tokens at k = 4096 and 544 tokens at k = 7168. */
#define LBH_NOALLOC_SCRATCH_BYTES (8u << 20)

/* [async] lbh_gemm_q8_k without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc); no counterpart in the reference.  Same results as lbh_gemm_q8_k.
 * It allocates nothing: the activation tiles go to a static device array of
 * LBH_NOALLOC_SCRATCH_BYTES that each GPU holds from library load to process
 * end.  Calls whose tiles exceed it fail with LBH_SCRATCH_TOO_SMALL (expected =
 * bytes needed, actual = the limit).  Every call on one GPU uses that GPU's one
 * array.  An eager call on a stream other than the last eager call's, while
 * that call has not finished, is refused with LBH_SCRATCH_IN_USE (nothing is
 * launched; actual = n_tokens); calls on one stream are ordered by it.  Calls
 * recorded under stream capture are not checked: replays of graphs that hold
 * this call must not overlap other uses of the array on the same GPU. */
lbh_status lbh_gemm_q8_k_noalloc(lbh_ctx *ctx, const lbh_matrix *m, const uint8_t *q8_dev, size_t n_tokens,
                                 float *y_dev, lbh_error *err);

/* ---- SwiGLU mixture-of-experts block ---------------------------------------------
 * A resident MoE layer: routed experts (SwiGluExpert, crates/bridge-kernels-reference/
 * src/activation.rs:6-60: gate/up [ffn, hidden], down [hidden, ffn]) and an optional
 * always-on shared expert, plus the scratch of one call (allocated once here, as the
 * reference's SwiGluScratch is: no allocation per call).  Supported type sets: routed
 * gate/up IQ2_S; routed down IQ3_S or IQ2_S; shared gate/up Q4_K or IQ2_S; shared down
 * Q5_K, IQ3_S or IQ2_S.  At most 16 routed experts per token. */

/* [sync] */
lbh_status lbh_moe_create(lbh_ctx *ctx, const lbh_matrix *const *gate, const lbh_matrix *const *up,
                          const lbh_matrix *const *down, size_t n_experts, const lbh_matrix *shared_gate,
                          const lbh_matrix *shared_up, const lbh_matrix *shared_down, lbh_moe **out,
                          lbh_error *err);
lbh_status lbh_moe_destroy(lbh_moe *moe);
/* Launch-shape knob: workgroups of the routed and shared gate/up streams
 * (1..65536 each) and output rows per down workgroup (1..256).  Defaults:
 * two routed workgroups per CU; for the shared stream its byte share of two
 * per CU beside the router chains, and in the routing-given and selecting
 * gate/up launches whatever fills one round of resident workgroups.  A set
 * value applies to every launch. */
lbh_status lbh_moe_set_tiles(lbh_moe *moe, int32_t wg_routed, int32_t wg_shared, int32_t tile_d);
/* Schedule of the asynchronous single-token forwards of a layer with a shared
 * expert: 1 runs the shared expert's gate/up and down on a second stream of
 * the layer beside the routed experts (and beside the router chains of
 * lbh_moe_block_forward), forked from and joined back to the context's stream;
 * 0 (default) runs the routed and shared experts in the same two launches on
 * the context's stream, which measured faster on MI355X (38.7 vs 50.9 us per
 * token at the configs[2] shapes in HIP-graph replay).  Same bits either way.
 * The layer's second stream and shared-output buffer are per layer: forwards
 * on one layer must be ordered (one caller stream). */
lbh_status lbh_moe_set_streams(lbh_moe *moe, int32_t two_streams);

/* [sync] moe_routed_by_id_into (crates/bridge-kernels-reference/src/moe.rs:64-147):
 * ids ascending with no duplicates, coefs finite (host arrays); output[hidden] =
 * sum over routed experts in id order of coef * down(SwiGLU(gate x, up x)), then
 * + 1.0 * shared, accumulated in the reference's order; bit-identical results.
 * Errors follow the reference's precedence and leave the output unchanged, except
 * NonFiniteValue on an accumulated destination (index = row), where, as in the
 * reference, the output holds the accumulation up to the step that overflowed. */
lbh_status lbh_moe_routed_by_id_into(lbh_ctx *ctx, lbh_moe *moe, const uint32_t *ids, const float *coefs,
                                     size_t n_routed, const float *input_dev, size_t input_len, float *output_dev,
                                     size_t output_len, lbh_error *err);

/* [sync] moe_routed_by_id_into in the DequantF32 execution mode (the same
 * moe.rs:64-147 with ReferenceExecutionMode::DequantF32; the CLI's --backend
 * dequant-f32): every matvec decodes the weights to f32 and runs the sequential f32
 * dot on the f32 input (dot_dequant_row, gemv.rs:33-41), no Q8_K step.  Same
 * arguments, order of the sums and error precedence as lbh_moe_routed_by_id_into;
 * bit-identical to the reference in that mode.  A checking path (one device
 * round trip per expert), not a decode loop's. */
lbh_status lbh_moe_routed_by_id_dequant_f32_into(lbh_ctx *ctx, lbh_moe *moe, const uint32_t *ids, const float *coefs,
                                                 size_t n_routed, const float *input_dev, size_t input_len,
                                                 float *output_dev, size_t output_len, lbh_error *err);

/* [async] The same computation without validation or status readback (graph
 * capturable): ids must be ascending, distinct and < n_experts (the last is checked),
 * coefs and x finite. */
lbh_status lbh_moe_forward(lbh_ctx *ctx, lbh_moe *moe, const uint32_t *ids, const float *coefs, size_t n_routed,
                           const float *x_dev, float *y_dev);

/* ---- batched MoE decode ----------------------------------------------------------
 * The reference decodes one token at a time: Hy3ScalarModel::evaluate_inner
 * (crates/bridge-runtime/src/hy3_scalar.rs:504-650) calls moe_routed_by_id_into
 * (crates/bridge-kernels-reference/src/moe.rs:64-147) per token.  These entry points
 * take a batch of tokens in one call; token t's output is bit-identical to that
 * call on token t.  The batch's (token, routed expert) pairs are sorted by expert
 * on the device, so each selected expert's weights stream from HBM once per chunk
 * of its tokens. */

/* [sync] Allocates the scratch of batched calls of up to max_tokens tokens (<= 256)
 * with up to top_k routed experts each (the reference allocates its SwiGluScratch
 * once, activation.rs:146-168; no allocation happens per call). */
lbh_status lbh_moe_reserve_batch(lbh_moe *moe, size_t max_tokens, size_t top_k, lbh_error *err);

/* Launch-shape knob of the batched kernels: tokens per chunk (1..16) and rows per
 * workgroup of the VALU routed/shared gate-up and down streams (the matrix-core
 * streams' tiles are set by lbh_moe_set_batch_engine). */
lbh_status lbh_moe_set_batch_tiles(lbh_moe *moe, int32_t tokens_per_chunk, int32_t rows_gate_up_routed,
                                   int32_t rows_gate_up_shared, int32_t rows_down_routed, int32_t rows_down_shared);

/* Engine of the batched IQ2_S / IQ3_S streams (no counterpart in the reference,
 * whose batch is a loop over tokens).  Chunks of at least mx_min_tokens tokens
 * (1..16; default 4) run on the f16 matrix cores, one 16-row x 16-token product
 * per codebook step, with mx_rows_gate_up / mx_rows_down rows per workgroup
 * (16, 32 or 64; 0: the defaults 16 and 32); smaller chunks run on the VALU
 * integer dots; mx_min_tokens = 0
 * keeps every chunk on the VALU.  Every choice gives the same bits.  Resets the
 * tokens per chunk (16 with the matrix cores, 8 without) and the VALU row tiles
 * to their defaults. */
lbh_status lbh_moe_set_batch_engine(lbh_moe *moe, int32_t mx_min_tokens, int32_t mx_rows_gate_up,
                                    int32_t mx_rows_down);

/* [sync] Tile copies for the batched matrix-core streams (no counterpart in the
 * reference, whose batch is a loop over tokens).  Those streams read a 16-row x
 * one-block tile per step; in the matrix layout the 16 rows of a block lie a row
 * apart, so each step reads 16 pieces of 16 cache lines whose other pieces come
 * back in later steps.  This call gives the IQ2_S / IQ3_S gate, up and down
 * matrices (rows a multiple of 16) of the listed routed experts a second copy,
 * owned by the layer, with the 16 rows of every block adjacent.  The
 * matrix-core streams then read those copies; every other kernel keeps reading
 * the caller's matrices.  The results are the same bits.  The cost is a second
 * copy of those bytes in HBM (lbh_moe_batch_tile_copy_bytes).
 *   experts = NULL: every routed expert.  n_experts = 0 with a list: drop the
 *   copies.  Each call replaces the previous copies.  It waits for the device's
 *   work in flight before releasing them.  Graphs that captured batched calls
 *   before it hold the released copies' addresses: capture them again. The
 *   same holds after lbh_moe_reserve_batch.
 * The copies are taken at this call: call it again after an expert's bytes
 * change.  Until lbh_moe_set_batch_engine is called, the layer's engine follows
 * the copies.  With copies, chunks of 2+ tokens run on the matrix cores, one wave
 * per 16-row tile.  Without, chunks of 4+ tokens run on the split tiles.  Each
 * measured fastest in its case.  Layers over an expert cache have no static
 * expert table and return LBH_INVALID_PARAMETER. */
lbh_status lbh_moe_make_batch_tile_copies(lbh_ctx *ctx, lbh_moe *moe, const uint32_t *experts, size_t n_experts,
                                          lbh_error *err);

/* HBM bytes of the layer's tile copies (0 when none). */
size_t lbh_moe_batch_tile_copy_bytes(const lbh_moe *moe);

/* [async] Batched form of lbh_moe_forward: ids_dev / coefs_dev are device arrays
 * [n_tokens][top_k] (each token's ids ascending and distinct), x_dev [n_tokens][hidden],
 * y_dev [n_tokens][hidden].  Unchecked; a routing with an id >= n_experts or a token
 * naming an expert twice leaves y unchanged.  The layer's batch scratch and its second
 * stream (independent launches run there, joined back to ctx's stream before the
 * call's work ends) are per layer: batched calls on one layer must not overlap. */
lbh_status lbh_moe_forward_batch(lbh_ctx *ctx, lbh_moe *moe, const uint32_t *ids_dev, const float *coefs_dev,
                                 size_t n_tokens, size_t top_k, const float *x_dev, float *y_dev);

/* [async] lbh_moe_forward_batch with the residual add of each token's block fused
 * into the combine: hidden_dev[t][i] += ffn_delta[t][i] (layer.rs:464, norm.rs:83-98). */
lbh_status lbh_moe_forward_batch_residual(lbh_ctx *ctx, lbh_moe *moe, const uint32_t *ids_dev, const float *coefs_dev,
                                          size_t n_tokens, size_t top_k, const float *x_dev, float *hidden_dev);

/* [sync] Checked form with host routing: every token's ids/coefs are validated with
 * the rules and error variants of moe_routed_by_id_into (moe.rs:73-129; err->row =
 * the token), then x must be finite (NonFiniteValue, index = lane, row = token); on
 * any error y is unchanged.  Non-finite intermediate values (SwiGLU, accumulation)
 * are not reported by the batched form: they propagate into y. */
lbh_status lbh_moe_routed_by_id_batch_into(lbh_ctx *ctx, lbh_moe *moe, const uint32_t *ids, const float *coefs,
                                           size_t n_tokens, size_t top_k, const float *input_dev, size_t input_len,
                                           float *output_dev, size_t output_len, lbh_error *err);

/* [async] route_experts_into over a batch of finished router logits
 * (crates/bridge-model-hy3/src/routing.rs:25-107 for mode 1; mode 0 is the
 * softmax top-k of lbh_router_route_into): logits_dev [n_tokens][n_experts]
 * (n_experts <= 256) -> ids_dev / coefs_dev [n_tokens][top_k], ids ascending.
 * bias_dev (mode 1) is the selection bias [n_experts].  Unchecked: logits finite. */
lbh_status lbh_route_experts_batch(lbh_ctx *ctx, const float *logits_dev, size_t n_tokens, size_t n_experts,
                                   size_t top_k, int32_t mode, float weight_scale, const float *bias_dev,
                                   uint32_t *ids_dev, float *coefs_dev);

/* ---- router -------------------------------------------------------------------
 * F32 router [hidden, n_experts] (GGML; n_experts rows of `hidden` floats) resident
 * in HBM, n_experts <= 256.  bias (optional) is the selection bias exp_probs_b. */

/* [sync] `weights`/`bias` are host memory when on_device == 0, device memory otherwise. */
lbh_status lbh_router_create(lbh_ctx *ctx, const float *weights, size_t n_experts, size_t hidden, const float *bias,
                             int32_t on_device, lbh_router **out, lbh_error *err);
lbh_status lbh_router_destroy(lbh_router *router);

/* [sync] Router logits (gemv_into of the F32 router, gemv.rs:286-303: bit-identical
 * sequential sums) and top_k selection into host ids/coefs (ascending ids):
 *   mode 0: softmax over the top k by (logit desc, id asc), renormalised (the
 *           benchmark configuration; no reference counterpart);
 *   mode 1: route_experts_into (crates/bridge-model-hy3/src/routing.rs:25-107).
 * logits_host (optional) receives the n_experts logits. */
lbh_status lbh_router_route_into(lbh_ctx *ctx, lbh_router *router, const float *x_dev, size_t x_len, size_t top_k,
                                 int32_t mode, float weight_scale, uint32_t *ids, float *coefs, float *logits_host,
                                 lbh_error *err);

/* [async] One MoE block decode step entirely on the device: router + top-k, then the
 * routed and shared experts (lbh_moe_forward semantics) reading the device routing.
 * Unchecked: x must be finite.  A routing the selection rejects (a non-finite logit,
 * or a router chain whose bounded wait gave up) leaves y unchanged and is recorded
 * on the router for lbh_router_take_status, where route_experts_into returns the
 * error (crates/bridge-model-hy3/src/routing.rs:72-77). */
lbh_status lbh_moe_block_forward(lbh_ctx *ctx, lbh_moe *moe, lbh_router *router, const float *x_dev, size_t top_k,
                                 int32_t mode, float weight_scale, float *y_dev);

/* [async] lbh_moe_block_forward ending as hy3_block_forward_token does
 * (crates/bridge-kernels-reference/src/layer.rs:429-464): the block's output is
 * added to the hidden state in place, hidden[i] = hidden[i] + ffn_delta[i]
 * (residual_add_in_place, norm.rs:83-98, fused into the combine; its finiteness
 * checks are not made: unchecked like the forward).  x_dev is the normalized
 * FFN input, hidden_dev the residual stream [hidden]. */
lbh_status lbh_moe_block_forward_residual(lbh_ctx *ctx, lbh_moe *moe, lbh_router *router, const float *x_dev,
                                          size_t top_k, int32_t mode, float weight_scale, float *hidden_dev);

/* [sync] What the block decodes on this router rejected since the last call, then
 * cleared: waits for the context's stream.  *rejected (optional) receives the number
 * of rejected steps.  Returns LBH_DEVICE_TIMEOUT if a router chain's bounded wait
 * gave up, else LBH_NON_FINITE_VALUE for the first rejected step with
 * route_experts_into's payload (expert index, value bits, field 8 logit / 9 bias /
 * 10 selection score), else LBH_OK.  No counterpart in the reference, whose
 * synchronous routing returns that error from the step itself (routing.rs:72-77). */
lbh_status lbh_router_take_status(lbh_ctx *ctx, lbh_router *router, uint64_t *rejected, lbh_error *err);

/* ---- HBM expert cache ---------------------------------------------------------
 * Counterpart of CompressedCache<ExpertKey> (crates/bridge-cache/src/lib.rs:32-595)
 * as the runtime uses it for routed experts (crates/bridge-runtime/src/hy3_scalar.rs:
 * 456-459, 575-604): a fixed byte ceiling, pins held by leases, LRU eviction of
 * unpinned entries, admission after `admit_after_requests` misses of a key
 * (below it an entry is ephemeral: dropped when its last lease is released),
 * concurrent misses of one key deduplicated.  Entries live in HBM in the device
 * layout, one fixed-size slot per expert.  A miss calls the caller's loader,
 * which writes the expert's tight record (gate | up | down GGML bytes: the
 * record of an expert-major sidecar, crates/bridge-format/src/lib.rs:63-100, read
 * by Sidecar::read_expert :309-329) straight into pinned staging; the record is
 * DMA'd and repacked on the cache's copy stream.  Thread-safe. */
typedef struct lbh_expert_cache lbh_expert_cache;

/* CacheConfig (lib.rs:13-30). */
typedef struct lbh_expert_cache_config {
    uint64_t capacity_bytes;
    uint64_t admit_after_requests;
} lbh_expert_cache_config;

/* CacheStats (lib.rs:480-494), plus the slot geometry and bytes DMA'd. */
typedef struct lbh_cache_stats {
    uint64_t capacity_bytes, used_bytes, reserved_bytes;
    uint64_t resident_entries, pinned_entries, loading_entries, heat_entries;
    uint64_t hits, misses, loads, waits, evictions;
    uint64_t entry_bytes, slots, bytes_uploaded;
} lbh_cache_stats;

/* A pinned entry (CacheLease, lib.rs:396-443): release it exactly once. */
typedef struct lbh_expert_lease {
    uint32_t layer, expert;
    int32_t slot;
    int32_t reserved;
} lbh_expert_lease;

/* Loader of one tight record (the closure given to get_or_try_insert, lib.rs:129-265):
 * writes the record into dst (capacity `bytes`), sets *written to the length
 * written, returns 0 on success or a loader-specific non-zero code. */
typedef int32_t (*lbh_expert_loader)(void *user, uint32_t layer, uint32_t expert, uint8_t *dst, size_t bytes,
                                     size_t *written);

/* CacheError status codes (lib.rs:496-516) and LoadError::Loader (lib.rs:518-524). */
#define LBH_CACHE_ZERO_CAPACITY 30            /* ZeroCapacity */
#define LBH_CACHE_ZERO_ADMISSION_THRESHOLD 31 /* ZeroAdmissionThreshold */
#define LBH_CACHE_ENTRY_TOO_LARGE 32          /* EntryTooLarge { requested = expected, capacity = actual } */
#define LBH_CACHE_CAPACITY_PINNED 33          /* CapacityPinned { requested = expected } */
#define LBH_CACHE_LOADED_SIZE_MISMATCH 34     /* LoadedSizeMismatch { expected, actual } */
#define LBH_CACHE_LOADER_FAILED 35            /* LoadError::Loader: the loader's code in `actual` */

/* CompressedCache::new (lib.rs:75-99) for the routed experts of one shape:
 * gate/up [ffn x hidden] of gate_up_type, down [hidden x ffn] of down_type.
 * Allocates capacity_bytes / entry_bytes slots in HBM (entry_bytes = the tight
 * record length) and two pinned staging buffers. */
lbh_status lbh_expert_cache_create(lbh_ctx *ctx, const lbh_expert_cache_config *config, uint32_t hidden, uint32_t ffn,
                                   int32_t gate_up_type, int32_t down_type, lbh_expert_cache **out, lbh_error *err);
lbh_status lbh_expert_cache_destroy(lbh_expert_cache *cache);
/* Tight record length of one expert: the `expected_bytes` of every load. */
uint64_t lbh_expert_cache_entry_bytes(const lbh_expert_cache *cache);

/* get_or_try_insert (lib.rs:129-265): a hit pins the entry; a miss reserves a slot
 * (evicting least recently used unpinned entries; LBH_CACHE_CAPACITY_PINNED when
 * pins block it, before the loader runs), calls the loader, checks the length and
 * every f16 d / dmin (LBH_NON_FINITE_SCALE with the block, field, bits and row,
 * `expected` = 0 gate / 1 up / 2 down), then uploads on the copy stream.  A
 * concurrent miss of the same key waits for the first one.  On any error the
 * reservation is released and nothing is inserted.  Work that reads the entry is
 * ordered after its upload by lbh_moe_forward_leased. */
lbh_status lbh_expert_cache_get_or_load(lbh_expert_cache *cache, uint32_t layer, uint32_t expert,
                                        lbh_expert_loader loader, void *user, lbh_expert_lease *out,
                                        lbh_error *err);
/* get (lib.rs:101-127): pins a ready entry (*found = 1) or counts a miss (*found = 0). */
lbh_status lbh_expert_cache_get(lbh_expert_cache *cache, uint32_t layer, uint32_t expert, lbh_expert_lease *out,
                                int32_t *found);
/* Drop of CacheLease (lib.rs:419-443): unpins; an ephemeral entry whose last pin
 * goes is removed.  The slot is not reused before the work the context's stream
 * holds at this call has finished. */
lbh_status lbh_expert_cache_release(lbh_expert_cache *cache, lbh_expert_lease *lease);
/* stats (lib.rs:267-299) and clear_unpinned (lib.rs:301-322). */
lbh_status lbh_expert_cache_stats(lbh_expert_cache *cache, lbh_cache_stats *out);
lbh_status lbh_expert_cache_clear_unpinned(lbh_expert_cache *cache, uint64_t *removed);
/* [sync] The leased entry's tight record read back from HBM (inverse of the repack):
 * byte-identical to what the loader wrote. */
lbh_status lbh_expert_cache_read_record(lbh_expert_cache *cache, const lbh_expert_lease *lease, void *host_out,
                                        size_t bytes, lbh_error *err);

/* A MoE layer whose routed experts come from `cache` (same hidden / ffn / types)
 * and whose shared expert (optional) is resident: the runtime's streaming MoE
 * (hy3_scalar.rs:561-626).  Only lbh_moe_forward_leased computes with it. */
lbh_status lbh_moe_create_cached(lbh_ctx *ctx, lbh_expert_cache *cache, const lbh_matrix *shared_gate,
                                 const lbh_matrix *shared_up, const lbh_matrix *shared_down, lbh_moe **out,
                                 lbh_error *err);
/* [async] lbh_moe_forward over leased experts: leases[i] is routed expert i (ascending
 * expert ids, distinct, n_routed <= 16) with coefficient coefs[i]; the computation
 * waits on the copy stream for each entry's upload. */
lbh_status lbh_moe_forward_leased(lbh_ctx *ctx, lbh_moe *moe, const lbh_expert_lease *leases, const float *coefs,
                                  size_t n_routed, const float *x_dev, float *y_dev);

/* ---- diagnostics ------------------------------------------------------------- */

/* Polls of the router chains' bounded LDS-ring waits before they give up (0: the
 * default, 2^22; negative: every wait gives up at once, which lets a test drive
 * the give-up path deterministically: lbh_router_route_into then returns
 * LBH_DEVICE_TIMEOUT and lbh_moe_block_forward leaves y unchanged). */
lbh_status lbh_router_set_spin_limit(lbh_router *router, int64_t limit);

/* [sync] The device expf used by SwiGLU and the routers (swiglu == 0), or the
 * SwiGLU element gate / (1 + exp(-gate)) * up (swiglu != 0, up_dev required). */
lbh_status lbh_debug_expf(lbh_ctx *ctx, const float *in_dev, float *out_dev, size_t n, int32_t swiglu,
                          const float *up_dev, lbh_error *err);
/* The same function compiled for the host CPU (no device needed), for checking
 * the device arithmetic against the C library on any machine. */
void lbh_debug_expf_host(const float *in, float *out, size_t n, int32_t swiglu, const float *up);

/* [async] Floor references for the matvec rooflines (no counterpart in the
 * reference): an empty kernel (the launch floor), and a plain read of a
 * matrix's device bytes with 16-byte non-temporal loads (the memory floor of a
 * matvec over it) in one of several launch shapes: `grid` workgroups of 256
 * lanes (1..LBH_DEBUG_READ_MAX_GRID), `unroll` loads in flight per lane (1, 2,
 * 4 or 8), grid-strided (slab == 0) or one contiguous slab per workgroup.
 * One word per wave is XOR-folded into sink_dev, which holds 4 * grid words. */
#define LBH_DEBUG_READ_MAX_GRID 65536
lbh_status lbh_debug_empty_kernel(lbh_ctx *ctx);
lbh_status lbh_debug_read_matrix(lbh_ctx *ctx, const lbh_matrix *m, uint32_t *sink_dev, int32_t grid, int32_t unroll,
                                 int32_t slab);

/* [sync] Converts n binary16 values with the device conversion the kernels use. */
lbh_status lbh_debug_f16_to_f32(lbh_ctx *ctx, const uint16_t *in_dev, float *out_dev, size_t n,
                                lbh_error *err);

#ifdef __cplusplus
}
#endif
#endif
