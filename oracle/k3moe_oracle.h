/*
 * k3moe_oracle — CPU restatement of Moonshine's routed-MoE layer.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP
 * implementation in moonshine_amd/: only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it. The product path never links,
 * loads or calls it.
 *
 * Every function states the reference behaviour it restates (file:line into
 * outerreaches/moonshine) and the reduction order it uses. Two orders exist:
 *
 *   - "w64" orders: the fixed wave64 orders the HIP kernels implement. They
 *     use explicit fmaf() and separately rounded adds, so a conforming GPU
 *     result is bit-identical to the oracle's.
 *   - "ref" orders: the reference kernels' own lane orders (256-lane router
 *     GEMV, 128-lane MXFP4 GEMV), for tolerance checks against the reference
 *     built from its sources (oracle/_ref).
 *
 * Pinning (what each function is checked against in tests/):
 *   k3o_expf / k3o_tanhf   glibc expf/tanhf over dense sweeps (ulp bound)
 *   k3o_e2m1 / k3o_e8m0    closed-form tables, exhaustive
 *   k3o_bf16 conversions   exhaustive bf16->f32->bf16 round trip, RNE ties
 *   logits                 fp64 dot product (error bound), single-nonzero KAT
 *   top-k                  all-equal logits, bias-dominated argsort, brute
 *                          force sort, sum of weights == scale
 *   plan                   brute-force stable sort, every route exactly once
 *   mxfp4 GEMV             fp64 (reference envelope bars), power-of-two KATs
 *   combine / add          sequential fp32 definition + hand-computed cases
 *   layer                  composition of the above; fp64 layer bound
 *   E4M3 / MXFP8 quant     exhaustive decode vs the OCP closed form; every
 *                          code round-trips; RNE at every midpoint;
 *                          torch.float8_e4m3fn conversion on a dense sweep;
 *                          block-scale invariants (max in [256, 512));
 *                          split: hi + lo == x for in-range elements
 *   prefill ledger         the reference's locked constants
 *                          (tests/test_k3_prefill_plan.c:15-26)
 */
#ifndef K3MOE_ORACLE_H
#define K3MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar helpers ---------------------------------------------------- */
float    k3o_bf16_to_f32(uint16_t v);
uint16_t k3o_f32_to_bf16(float f);
float    k3o_e2m1(uint8_t nibble);
float    k3o_e8m0(uint8_t exponent);
float    k3o_expf(float x);
float    k3o_tanhf(float x);
float    k3o_sigmoid(float x, int use_libm);
float    k3o_router_sigmoid(float x);

/* ---- activations (k3_rocm_ops.cu:66-83 SiTU; SwiGLU = limit form) ------ */
void k3o_situ(uint16_t *out, const uint16_t *gate, const uint16_t *up,
              uint64_t n, float beta, float linear_beta, int use_libm);
void k3o_swiglu(uint16_t *out, const uint16_t *gate, const uint16_t *up,
                uint64_t n, int use_libm);

/* ---- router logits (k3_rocm_ops.cu:359-425, 512-661) ------------------- */
/* order: 0 = w64 (HIP kernels), 1 = reference 256-lane, 2 = fp64 */
void k3o_router_logits(float *logits, const uint16_t *weights,
                       const uint16_t *input, uint32_t tokens,
                       uint32_t experts, uint32_t hidden, int order);

/* ---- router top-k (k3_rocm_ops.cu:1361-1450) ---------------------------- */
int k3o_router_topk(uint32_t *ids, float *weights, const float *logits,
                    const float *bias, uint32_t tokens, uint32_t experts,
                    uint32_t top_k, float scale, int use_libm);

/* ---- routing plan (k3_engine_prefill.inc:1006-1018, 1175-1194) -------- */
int k3o_route_plan(uint32_t *counts, uint32_t *offsets, uint32_t *unique,
                   uint32_t *unique_count, uint32_t *token_index,
                   uint32_t *route_index, const uint32_t *ids,
                   uint32_t tokens, uint32_t top_k, uint32_t experts);

/* ---- MXFP4 GEMV/GEMM (k3_rocm_ops.cu:179-357) -------------------------- */
/* order: 0 = w64, 1 = reference 128-lane, 2 = fp64 (output f32 via out_f32) */
void k3o_mxfp4_gemm(uint16_t *out, float *out_f32, const uint8_t *packed,
                    const uint8_t *scales, const uint16_t *input,
                    uint32_t vectors, uint32_t rows, uint32_t columns,
                    int order);
void k3o_bf16_gemm_f32(float *out, const uint16_t *weights,
                       const uint16_t *input, uint32_t vectors,
                       uint32_t rows, uint32_t columns, int order);

/* ---- static projections of the K3-native tail (k3_rocm_ops.cu:662-867) - */
/* Q8-128: int8 codes [rows, cols], f32 scales [rows, cols / 128]. */
void k3o_q8_quantize(int8_t *q, float *scales, const uint16_t *w,
                     uint32_t rows, uint32_t cols);
void k3o_q8_dequantize(uint16_t *w, const int8_t *q, const float *scales,
                       uint32_t rows, uint32_t cols);
/* order: 0 = w64, 1 = reference 256-thread, 2 = fp64 (out_f32) */
void k3o_q8_gemm(uint16_t *out, float *out_f32, const int8_t *q,
                 const float *scales, const uint16_t *input, uint32_t vectors,
                 uint32_t rows, uint32_t cols, int order);
/* order: 0 = the library's (thread t of 256 owns 8-element chunks t,
 * t + 256, ... with fmaf(v, v, s); per-wave butterfly; (w0 + w1) + (w2 +
 * w3); IEEE 1/sqrt), 1 = reference 256-thread tree, 2 = fp64 */
void k3o_rms_norm(uint16_t *out, const uint16_t *in, const uint16_t *weight,
                  uint32_t vectors, uint32_t hidden, float eps, int order);

/* ---- combine (k3_rocm_ops.cu:1452-1510) -------------------------------- */
void k3o_weighted_sum(uint16_t *out, const uint16_t *vectors,
                      const float *weights, uint32_t tokens,
                      uint32_t vector_count, uint32_t hidden);
void k3o_add(uint16_t *out, const uint16_t *left, const uint16_t *right,
             uint64_t n);
void k3o_copy_rows(uint16_t *out, const uint16_t *in, const uint32_t *row_ids,
                   uint32_t row_count, uint32_t row_size, int scatter);

/* ---- whole routed-MoE layer --------------------------------------------- */
typedef struct {
    const uint8_t *w1_packed, *w1_scales; /* gate [F, H] */
    const uint8_t *w2_packed, *w2_scales; /* down [H, F] */
    const uint8_t *w3_packed, *w3_scales; /* up   [F, H] */
} k3o_expert;

typedef struct {
    uint32_t hidden, experts, top_k, ffn;
    float    scale;
    uint32_t activation;       /* 0 = SiTU(beta, linear_beta), 1 = SwiGLU */
    float    beta, linear_beta;
} k3o_shape;

/*
 * Computes output[t] for the listed tokens (all when token_list == NULL).
 * When ids_in/weights_in are given, routing is taken from them instead of
 * the router (lets a test check the expert stage on the GPU's own routes).
 * experts[e] may be NULL for experts that are never selected.
 * expert_out (optional) receives [tokens, top_k, hidden] bf16 slot outputs.
 * The router's logits are always in the reference's lane order.
 * gemv_order (the expert GEMVs): 0 = w64, 1 = reference lane order, 2 =
 * fp64, 3 = MX8 (the
 * expert inputs -- x for gate/up, the activation for down -- quantized to
 * MXFP8, products accumulated in fp64; same bf16 rounding points as the
 * other orders), 4 = split MX8 (inputs as the two-term hi + lo
 * reconstruction, fp64 accumulation). x is encoded with one scale per
 * token row (k3o_mx8_quantize_rows / k3o_mx8_split_rows), the activation
 * with one per 32 columns (k3o_mx8_quantize / k3o_mx8_split).
 * Returns 0 on success, -1 when a selected expert has no weights.
 */
int k3o_layer(const k3o_shape *shape, uint32_t tokens,
              const uint16_t *hidden_in, const uint16_t *residual,
              const uint16_t *router_weight, const float *router_bias,
              const k3o_expert *experts,
              const uint32_t *ids_in, const float *weights_in,
              const uint32_t *token_list, uint32_t token_list_count,
              uint16_t *output, uint32_t *ids_out, float *weights_out,
              float *logits_out, uint16_t *expert_out, int gemv_order,
              int threads);

/* ---- MX8 activations (precision mode of the MFMA prefill path) ---------- */
float   k3o_e4m3(uint8_t code);
uint8_t k3o_f32_to_e4m3(float v);
void    k3o_mx8_quantize(uint8_t *q, uint8_t *scales, const uint16_t *src, uint64_t n);
void    k3o_mx8_split(uint8_t *hi_q, uint8_t *hi_s, uint8_t *lo_q, uint8_t *lo_s,
                      const uint16_t *src, uint64_t n);
/* the same encodings with one scale per row of a [rows, cols] matrix */
void    k3o_mx8_quantize_rows(uint8_t *q, uint8_t *scales, const uint16_t *src, uint64_t rows,
                              uint64_t cols);
void    k3o_mx8_split_rows(uint8_t *hi_q, uint8_t *hi_s, uint8_t *lo_q, uint8_t *lo_s,
                           const uint16_t *src, uint64_t rows, uint64_t cols);

/* ---- prefill byte ledger (k3_prefill.c:136-234, 236-446) ---------------- */
typedef struct {
    uint64_t hidden_row_bytes, attn_res_row_bytes, main_scratch_bytes;
    uint64_t moe_scratch_bytes, mla_scratch_bytes, route_bytes;
    uint64_t expert_index_bytes, batch_workspace_bytes;
    uint64_t incremental_workspace_bytes, mla_append_bytes;
} k3o_workspace;
int k3o_prefill_workspace(uint32_t chunk_tokens, k3o_workspace *out);

#ifdef __cplusplus
}
#endif
#endif
