// lbh_internal.h — declarations shared by the kernel and C-ABI translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "lbh_layout.h"

namespace lbh {

// Per-context device status words written by validation kernels and read by
// compute kernels, which skip all writes when a word is set (atomicity).
struct DevStatus {
    unsigned long long first_bad_input;   // first non-finite input lane, ~0ull when none
    unsigned long long first_bad_dest;    // first non-finite destination lane
    unsigned long long first_bad_scale;   // weight upload: 2 * unit + field
    unsigned long long pad;
};

enum : int32_t { MAT_ROW_MAJOR = 0, MAT_TILE16 = 1 };

// Unit of (row r, block b) of a matrix with nb blocks per row stored in unit
// order `order` (MAT_TILE16 needs rows % 16 == 0).
__host__ __device__ inline uint32_t unit_index(int32_t order, uint32_t r, uint32_t b, uint32_t nb) {
    return order == MAT_TILE16 ? (((r >> 4) * nb + b) << 4) + (r & 15u) : r * nb + b;
}

// A matrix in the device layout (lbh_layout.h).
struct MatView {
    const uint8_t *planes;
    int32_t type;
    int32_t nb;        // 256-element blocks per row
    int32_t rows;
    // Unit order of the planes: MAT_ROW_MAJOR (u = r * nb + b) everywhere
    // except the batched matrix-core streams' tile copies, MAT_TILE16
    // (u = ((r / 16) * nb + b) * 16 + r % 16: the 16 rows of a block adjacent).
    int32_t order;
    long long units;   // rows * nb
    long long bytes;   // size of the planes allocation
};

struct GemvArgs {
    MatView m;
    const uint8_t *q8;            // (nb) Q8_K blocks, or NULL when x is given
    const float *x;               // f32 input quantized inside the kernel (q8 == NULL)
    uint8_t *q8_out;              // optional: the Q8_K bytes of x, written by workgroup 0
    float *y;                     // NULL: row values not stored (integer-stage export only)
    float coef;
    int32_t accumulate;
    int32_t *block_sums;          // optional integer-stage export
    const DevStatus *status;      // optional: skip when any validation word is set
};

// Launch-shape knobs of the matvec kernels (0 = built-in default).
struct GemvTuning {
    int lpu;          // lanes per (row, block) unit: 1, 2 or 4
    int max_blocks;   // cap on workgroups of the persistent row loop (0: resident occupancy x CUs)
    int depth;        // row steps in flight per wave (2..4)
    int cu_count;     // compute units of the device (sizes the default grid)
};

// ---------------------------------------------------------------- MoE block

constexpr int MOE_MAX_ROUTED = 16;
constexpr int MOE_SHARED_SLOT = MOE_MAX_ROUTED;   // scratch slot of the shared expert

// Routing of one token: routed expert ids (ascending) and coefficients.
struct MoeRoute {
    int32_t n;
    int32_t pad;
    uint32_t ids[MOE_MAX_ROUTED];
    float coefs[MOE_MAX_ROUTED];
};

struct ExpertDev {
    MatView gate, up, down;
};

struct RouterArgs {
    const float *w;             // transposed, interleaved by four: w[(j * n_experts + e) * 4 + c] = row e, input 4j + c
    const float *bias;          // selection bias [n_experts] (mode 1)
    const float *x;             // [hidden]
    float *logits;              // [n_experts]
    MoeRoute *route;            // selection output
    unsigned long long *status; // optional: (first bad expert << 2) | field
    int32_t n_experts, hidden, top_k, mode;
    float weight_scale;
    // F32 matvec use of the chains (lbh_gemv_* on an F32 matrix): accumulate
    // != 0 stores logits[e] + coef * sum (gemv_accumulate_scaled_into), and
    // skip_if (optional) suppresses the stores when a validation scan fired.
    int32_t accumulate;
    float coef;
    const DevStatus *skip_if;
    // Bounded waits of the router chains' LDS ring: polls before giving up
    // (0: the default 2^22; < 0: give up at once, a host-forced test of that
    // path).  A chain that gives up stores a NaN logit (the selection then
    // rejects the route) and sets *timeout to 1 (sticky; optional).
    long long spin_limit;
    unsigned long long *timeout;
    // Optional record of the selections a block decode rejected (the routed
    // gate/up kernel writes it): [0] rejected selections, [1] the first one's
    // code (as `bad` of select_route), [2] its logit bits | bias bits << 32.
    unsigned long long *reject;
};

// Device status of one MoE call (~0 when clean).
struct MoeStatus {
    unsigned long long first_bad_swiglu;   // (expert order << 32) | lane; order n = shared
    unsigned long long first_bad_fold;     // (accumulate step << 32) | row
    unsigned long long first_bad_input;    // first non-finite input lane
    unsigned long long pad;
};

struct MoeArgs {
    const ExpertDev *experts;   // device table [n_experts]
    ExpertDev shared;
    int32_t has_shared;
    int32_t hidden;             // input / output width
    int32_t ffn_r, ffn_s;       // hidden widths of the routed / shared experts
    MoeRoute route;             // routing, unless route_dev is set
    const MoeRoute *route_dev;  // routing written by the device router
    const float *x;             // [hidden]
    float *h;                   // SwiGLU outputs: slot * h_stride
    int32_t h_stride;
    float *y;                   // [hidden]
    MoeStatus *status;
    int32_t tile_r, tile_s;     // gate/up rows per workgroup (routed, shared)
    int32_t tiles_r, tiles_s;   // workgroups per routed expert / for the shared expert
    int32_t tile_d;             // output rows per down workgroup
    int32_t stop_step;          // combine steps 0..stop_step only (error fix-up); large = all
    int32_t check;              // record non-finite SwiGLU lanes / accumulations
    int32_t n_launch;           // routed experts covered by this launch
    int32_t type_gate_r;        // GGML type of every routed gate/up matrix
    int32_t type_down_r;        // GGML type of every routed down matrix
    // Block decode: the gate/up kernel selects the routing from finished router
    // logits (router.logits) and publishes it to route_dev for the down kernel;
    // the shared expert's gate/up ran beside the router chains.
    int32_t select_in_kernel;
    int32_t skip_shared_gate_up;
    RouterArgs router;
    // Host-given routing: the routed experts' plane pointers per routing slot
    // travel in the arguments (no dependent load of the expert table before
    // the first weight loads); every routed expert has routed_shape's views.
    int32_t routed_given;
    // residual != 0: the combine adds the block's output to y in place,
    // y[r] = y[r] + delta[r] (residual_add_in_place, crates/bridge-kernels-
    // reference/src/norm.rs:83-98, as hy3_block_forward_token ends, layer.rs:464).
    int32_t residual;
    // Two-stream decode: the shared expert's FFN on a second stream beside the
    // routed experts.  gate_part: 0 both streams in one launch, 1 routed only,
    // 2 shared only.  down_part: 0 both and the combine, 1 routed downs and the
    // combine adding d_shared (written by part 2) last, 2 the shared down only,
    // its raw rows to d_shared.
    int32_t gate_part, down_part;
    float *d_shared;            // [hidden]
    ExpertDev routed_shape;
    const uint8_t *routed_planes[MOE_MAX_ROUTED][3];   // gate, up, down
};

// ------------------------------------------------ K-quant GEMM on f16 MFMA

constexpr int GEMM_MAX_MATS = 3;

// One matrix of a GEMM launch: its MFMA-ready copy and output.
struct MatGemm {
    const uint8_t *a;      // [ceil(rows / 32)][nb] A tiles (operands, then (d, dmin) per row)
    float *y;              // y[t * ldy + r]
    int32_t rows;
    int32_t ldy;
};

struct GemmArgs {
    MatGemm mat[GEMM_MAX_MATS];   // matrices sharing K and the activations
    const uint8_t *b;             // [ceil(n_tokens / 32)][nb] B tiles (operands, then d8 per token)
    int32_t n_mat, nb, n_tokens, shape;
};

// ------------------------------------------------------ batched MoE decode

constexpr int BATCH_MAX_TOKENS = 256;
constexpr int BATCH_MAX_EXPERTS = 1024;
constexpr int BATCH_MAX_TC = 16;      // tokens staged per chunk

// Scratch and shape of one batched call (all pointers device memory).
struct BatchArgs {
    const ExpertDev *experts;   // device table [n_experts]
    ExpertDev shared;
    int32_t has_shared;
    int32_t hidden, ffn_r, ffn_s, n_experts;
    int32_t n_tokens, top_k;
    const uint32_t *ids;        // [n_tokens][top_k]
    const float *coefs;         // [n_tokens][top_k]
    const float *x;             // [n_tokens][hidden]
    float *y;                   // [n_tokens][hidden]
    // plan written by the sort: plan[0] = routed chunks (0 when the routing is
    // invalid), plan[1] = invalid-routing flags (1: id out of range, 2: repeated id)
    int32_t *plan;
    int32_t *chunk_expert, *chunk_p0, *chunk_n;   // [max_chunks]
    int32_t *pair_token;        // sorted pair -> token
    int32_t *pair_of;           // token * top_k + slot -> sorted pair
    uint8_t *q8x;               // [n_tokens][hidden / 256] Q8_K blocks of x
    uint8_t *q8x_rm;            // the same with residue-major qs (K-quant consumers)
    float *g_r, *u_r;           // [pairs][ffn_r] gate / up outputs, sorted pair order
    uint8_t *q8h_r;             // [pairs][ffn_r / 256] Q8_K of h_r
    uint8_t *q8h_s;             // [n_tokens][ffn_s / 256] Q8_K of h_s (residue-major for K-quants)
    float *d_r;                 // [pairs][hidden] routed down outputs
    float *d_s;                 // [n_tokens][hidden] shared down outputs
    int32_t max_chunks;         // routed chunks the launches cover
    int32_t tc;                 // tokens per chunk (1..BATCH_MAX_TC)
    int32_t rt_gu_r, rt_gu_s;   // VALU streams: gate/up rows per workgroup (routed, shared)
    int32_t rt_d_r, rt_d_s;     // VALU streams: down rows per workgroup (routed, shared)
    int32_t type_gate_r, type_down_r;
    // The shared expert's gate / up outputs (every stream type; SwiGLU is
    // formed in the h quantization, as for the routed pairs); on the K-quant
    // types its gate/up and down run on the matrix cores (-> d_s).
    int32_t shared_gemm, gemm_shape;
    MatGemm sg, su, sd;         // MFMA-ready copies of the shared gate / up / down
    float *g_s, *u_s;           // [n_tokens][ffn_s]
    uint8_t *bx, *bh;           // GEMM activation tiles of x and of the shared h
    // mx = 1: chunks of at least mx_min tokens of the IQ2_S / IQ3_S streams run
    // on the f16 matrix cores (mx_split_* waves share each 16-row tile) and read the
    // operand copies of the Q8_K rows (quants XOR 0x80 at 256 bytes a block,
    // scales apart) of x and of the routed and shared h; the VALU streams take the smaller chunks
    // and stage vc = min(tc, mx_min - 1) tokens (tc when mx = 0).
    int32_t mx, mx_min, mx_split_gu, mx_split_d, vc;
    int32_t residual;           // y[t][r] += delta (as MoeArgs::residual)
    // The matrix-core streams' routed views [n_experts]: an expert's 16-row
    // tile copies where lbh_moe_make_batch_tile_copies made them, else its
    // views in `experts`.
    const ExpertDev *experts_mx;
    uint8_t *xq_mx, *hq_mx_r, *hq_mx_s;
    float *xd_mx, *hd_mx_r, *hd_mx_s;
};

// Batch selection: top-k of each token's finished logits (select_route).
struct RouteBatchArgs {
    RouterArgs r;               // n_experts, top_k, mode, weight_scale, bias
    const float *logits;        // [n_tokens][n_experts]
    uint32_t *ids;              // [n_tokens][top_k]
    float *coefs;
    unsigned long long *status; // optional: (token << 32 | expert << 2 | field), min over the batch
    int32_t n_tokens;
    int32_t pad;
};

size_t gemm_a_bytes(int rows, int nb);
size_t gemm_b_bytes(int n_tokens, int nb);
hipError_t launch_prep_a(const MatView &m, uint8_t *a, hipStream_t s);
hipError_t launch_prep_b(const uint8_t *q8, int n_tokens, int nb, uint8_t *b, hipStream_t s);
hipError_t launch_kq_gemm(const GemmArgs &g, hipStream_t s);

hipError_t launch_route_batch(const RouteBatchArgs &a, hipStream_t s);
// A second stream and fork/join events for a batched call: the launches that
// do not depend on each other (the shared expert's GEMMs, the matrix-core
// chunks) run on `side` beside the main stream's VALU chunks, and the main
// stream waits for them before the next stage.  NULL: all on the main stream.
struct BatchStreams {
    hipStream_t side;
    hipEvent_t fork[2], join[2];
};
hipError_t launch_moe_batch(const BatchArgs &a, hipStream_t s, const BatchStreams *bs);
int batch_lds_bytes(const BatchArgs &a, int stage);
bool batch_types_supported(int gate_r, int down_r, int gate_s, int down_s);

hipError_t launch_router(const RouterArgs &a, hipStream_t s);
hipError_t launch_router_logits(const RouterArgs &a, hipStream_t s);
// The router chains over any number of rows: output[r] = dot_f32_row(r, x)
// of an F32 matrix in the router layout (rows <= 2^31 - 8, k % 256 == 0).
hipError_t launch_f32_chains(const RouterArgs &a, hipStream_t s);
// F32 matrix [rows, k] between GGML row-major order and the router layout
// (w[(j * rows + r) * 4 + c] = row r, input 4j + c); to_device selects the
// direction.  k % 4 == 0.
hipError_t launch_f32_layout(const float *src, float *dst, long long rows, long long k, int to_device, hipStream_t s);
// First non-finite weight of an F32 matrix in the router layout, as the
// row-major index r * k + i (atomicMin into *first).
hipError_t launch_find_nonfinite_f32w(const float *w, long long rows, long long k, unsigned long long *first,
                                      hipStream_t s);
hipError_t launch_moe_router_shared(const MoeArgs &a, hipStream_t s);
hipError_t launch_moe_gate_up(const MoeArgs &a, hipStream_t s);
hipError_t launch_moe_down(const MoeArgs &a, hipStream_t s);
hipError_t launch_moe_reset_status(MoeStatus *st, hipStream_t s);
// LDS of one single-token MoE down launch (gfx950 gives a workgroup at most MOE_MAX_LDS).
constexpr int MOE_MAX_LDS = 160 * 1024;
// Gate/up workgroups of the (routed, shared) type pair resident on one CU at once.
int moe_gate_up_resident_per_cu(int type_gate_r, int type_gate_s, int hidden);
int moe_down_lds_bytes(int type_down_r, int type_down_s, int n_routed, int has_shared, int ffn_r, int ffn_s,
                       int tile_d);
hipError_t launch_expf(const float *in, float *out, long long n, int swiglu, const float *up, hipStream_t s);

hipError_t launch_quantize_q8k(const float *x, uint8_t *out, long long nblocks, const DevStatus *st,
                               hipStream_t s);
hipError_t launch_find_nonfinite(const float *x, long long n, unsigned long long *first, hipStream_t s);
hipError_t launch_reset_status(DevStatus *st, hipStream_t s);
hipError_t launch_gemv(const GemvArgs &a, const GemvTuning &t, hipStream_t s);
hipError_t launch_repack(int ty, const uint8_t *ggml, uint8_t *planes, long long units, int to_device,
                         hipStream_t s);
hipError_t launch_repack_range(int ty, const uint8_t *src, uint8_t *dst, long long U, long long u0, long long n,
                               hipStream_t s);
// Copy of an IQ2_S / IQ3_S matrix (rows % 16 == 0) with its units in
// MAT_TILE16 order at dst (m.bytes bytes).
hipError_t launch_units_to_tiles(const MatView &m, uint8_t *dst, hipStream_t s);
hipError_t launch_validate_scales(int ty, const uint8_t *ggml, long long units,
                                  unsigned long long *first, hipStream_t s);
hipError_t launch_f16_to_f32(const uint16_t *in, float *out, long long n, hipStream_t s);
hipError_t launch_empty(hipStream_t s);
// sink holds grid * 4 words (one per wave).
hipError_t launch_stream_read(const void *src, long long bytes, uint32_t *sink, int grid, int unroll, int slab,
                              hipStream_t s);

// Raw GGML row dots (vec_dot_q8_k per row; 1 <= nb <= 64), the Q8_K scale scan
// and the DequantF32 matvec (lbh_dot.hip).  `st` words set -> no writes.
hipError_t launch_dot_ggml(int ty, const uint8_t *w, long long rows, int nb, const uint8_t *q8, float *y,
                           const DevStatus *st, hipStream_t s);
hipError_t launch_find_nonfinite_q8(const uint8_t *q8, long long nblocks, unsigned long long *first, hipStream_t s);
hipError_t launch_gemv_dequant(const MatView &m, const float *x, float *y, float coef, int accumulate,
                               const DevStatus *st, hipStream_t s);

}  // namespace lbh
