#ifndef K3_MOE_H
#define K3_MOE_H

/*
 * Routed-MoE layer entry points that have no single counterpart in
 * Moonshine's k3_rocm_ops.h: they fuse what the engine sequences on the
 * host in decode_routed_layer (k3_engine.cu:1425-1939) and
 * prefill_routed_layer / prefill_stream_routed_layer
 * (k3_engine_prefill.inc:999-1285, 1287-1627), with the routing plan built
 * on the device instead of by the host loop at
 * k3_engine_prefill.inc:1175-1194.
 *
 * Conventions are those of k3_rocm_ops.h: device pointers, a hipStream_t
 * passed as void *, arguments validated before any launch (false without
 * launching), launch errors reported synchronously, execution asynchronous.
 * Nothing here allocates: the caller passes a workspace of at least
 * k3_moe_workspace_bytes(). Calls that share a workspace must be ordered on
 * one stream.
 */

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * One routed expert in the checkpoint-native MXFP4 layout: packed
 * [rows, columns / 2] (low nibble = even column) and E8M0 scales
 * [rows, columns / 32]. Fields follow the six-tensor span order of
 * k3_prefill.c:71-75 (w1 = gate, w2 = down, w3 = up). Tensors must start
 * 8-byte aligned; the 8-mod-16 starts of real checkpoint spans
 * (k3_rocm_ops.cu:207-223) are read as 8-byte pairs by the exact kernels
 * and as 16-byte direct-to-LDS pieces (which take 8-byte aligned sources
 * on gfx950) by the MFMA kernels, with the same results as aligned
 * tensors.
 */
typedef struct {
    const void *gate_packed;  /* w1.weight_packed [ffn, hidden / 2]  */
    const void *gate_scales;  /* w1.weight_scale  [ffn, hidden / 32] */
    const void *down_packed;  /* w2.weight_packed [hidden, ffn / 2]  */
    const void *down_scales;  /* w2.weight_scale  [hidden, ffn / 32] */
    const void *up_packed;    /* w3.weight_packed [ffn, hidden / 2]  */
    const void *up_scales;    /* w3.weight_scale  [ffn, hidden / 32] */
} k3_moe_expert;

typedef enum {
    /* beta*tanh(g/beta) * sigmoid(g) * lb*tanh(u/lb): K3's SiTU
     * (k3_rocm_ops.cu:66-83, beta = 4, lb = 25 at k3_engine.cu:1056). */
    K3_MOE_ACT_SITU = 0,
    /* g * sigmoid(g) * u: SiTU's beta, lb -> infinity limit. */
    K3_MOE_ACT_SWIGLU = 1,
} k3_moe_activation;

typedef enum {
    /* Fixed wave64 fp32 orders on the vector ALUs: bit-identical to the
     * CPU oracle, to the per-matrix k3_rocm_mxfp4_* entry points and
     * between decode and any batch size. */
    K3_MOE_EXACT = 0,
    /* Grouped GEMM on CDNA4 scaled MFMA for token_count > 1: weights stay
     * MXFP4; each bf16 activation enters as two E4M3 terms hi + lo, each
     * with E8M0 scales (one per token row for the gate/up input, one per
     * 32 values for the activation that feeds down), which reproduce it
     * exactly except for elements more than 2^6 below the maximum of their
     * scale run (error <= 2^-22 of it). Products are those of the bf16 inputs; accumulation
     * is fp32 in MFMA order, so results match EXACT within bf16 tolerance,
     * not bit for bit. One token runs the EXACT decode path. */
    K3_MOE_MFMA = 1,
    /* As K3_MOE_MFMA with one E4M3 term (half the MFMA work). Activation
     * quantisation error is ~4% per element and survives the dot products
     * (~5% relative on expert outputs): an approximate mode, not a
     * drop-in for the reference's numerics. */
    K3_MOE_MFMA_FP8 = 2,
} k3_moe_precision;

typedef struct {
    uint32_t hidden;          /* H: router columns, expert input/output width */
    uint32_t expert_count;    /* E <= 1024 */
    uint32_t top_k;           /* k <= 32 */
    uint32_t ffn;             /* F: expert intermediate width */
    float    scaling_factor;  /* routed scale (> 0) */
    uint32_t activation;      /* k3_moe_activation */
    float    beta;            /* SiTU gate bound (ignored for SwiGLU) */
    float    linear_beta;     /* SiTU up bound (ignored for SwiGLU) */
} k3_moe_shape;

/* Bytes of workspace k3_moe_forward_bf16 needs for token_count rows. */
size_t k3_moe_workspace_bytes(const k3_moe_shape *shape, uint32_t token_count);

/*
 * Prepares a freshly allocated workspace. The current kernels keep no state
 * in the workspace between calls, so this only validates the arguments; it
 * is part of the contract so later versions may keep counters there.
 */
bool k3_moe_workspace_init(void *workspace, size_t workspace_bytes, void *stream);

/*
 * Device routing plan (replaces the host loop at
 * k3_engine_prefill.inc:1175-1194). For every selected expert in
 * ascending id, rows in (token asc, rank asc) order: a stable sort of the
 * flattened routes by expert id.
 *   counts[E], offsets[E + 1], unique[E]      per-expert row counts, their
 *                                             exclusive scan, selected ids
 *   summary[4] = {unique count, routes dropped as invalid ids,
 *                 max rows of one expert, 0}
 *   token_index[T*k], route_index[T*k]        row -> token, row -> token*k+rank
 * scratch: at least k3_moe_plan_scratch_bytes(T, E) bytes.
 */
size_t k3_moe_plan_scratch_bytes(uint32_t token_count, uint32_t expert_count);
bool k3_moe_route_plan(uint32_t *counts, uint32_t *offsets, uint32_t *unique,
                       uint32_t *summary, uint32_t *token_index,
                       uint32_t *route_index, const uint32_t *expert_ids,
                       uint32_t token_count, uint32_t top_k,
                       uint32_t expert_count, void *scratch,
                       size_t scratch_bytes, void *stream);

/*
 * The router's choice values, the quantity the top-k orders experts by:
 * choices[t, e] = sigmoid(logits[t, e]) + bias[e] for t < token_count, e <
 * expert_count, with the sigmoid evaluated exactly as the reference's
 * router kernel evaluates it (k3_rocm_ops.cu:1386 under its fast-math
 * build); bias may be NULL (the choice is then the sigmoid itself). For
 * inspecting routing margins (how close a token is to swapping experts).
 * token_count * expert_count must fit the grid (< 2^40).
 */
bool k3_moe_router_choices_f32(float *choices, const float *logits, const float *bias,
                               uint32_t token_count, uint32_t expert_count, void *stream);

/*
 * Routes of a token batch, replacing the prefill router pair
 * k3_rocm_bf16_gemm_f32 + k3_rocm_router_topk_f32_batch
 * (k3_engine_prefill.inc:1448-1460) with the same ids and weights, bit for
 * bit. From 32 tokens on (hidden % 64 == 0, hidden <= 8192, expert_count
 * <= 1024, 16-byte aligned hidden and router_weight) the logits run on bf16
 * MFMA and each token recomputes in the exact order only the experts that a
 * rigorous error bound cannot rule out of its top-k; otherwise the exact
 * logits and top-k kernels run. expert_ids / expert_weights: [T, k] (may be
 * host-mapped). scratch: k3_moe_router_scratch_bytes(T, E) bytes of device
 * memory (256-byte aligned). token_count <= 65535.
 */
size_t k3_moe_router_scratch_bytes(uint32_t token_count, uint32_t expert_count);
bool k3_moe_router_bf16(uint32_t *expert_ids, float *expert_weights, const void *hidden,
                        const void *router_weight, const void *router_bias,
                        uint32_t token_count, uint32_t expert_count, uint32_t hidden_size,
                        uint32_t top_k, float scaling_factor, void *scratch,
                        size_t scratch_bytes, void *stream);

/*
 * The whole routed-MoE layer for token_count rows:
 *   logits = router_weight[E, H] . hidden[t]        (f32)
 *   ids, weights = top-k(sigmoid(logits) + bias)    (k3_rocm_router_topk)
 *   y[t, r] = down_e(act(gate_e . hidden[t], up_e . hidden[t]))
 *   output[t] = bf16(residual[t] + bf16(sum_r weights[t, r] * y[t, r]))
 * residual may be NULL (output is then the combine alone). experts is a
 * DEVICE array of expert_count descriptors. expert_ids / expert_weights
 * ([T, k] u32 / f32) are optional extra copies of the routes and may be
 * host-mapped memory. token_count <= 65535. output, hidden and residual
 * rows are read and written 16 bytes at a time: the three pointers must
 * be 16-byte aligned (false otherwise).
 */
bool k3_moe_forward_bf16(void *output, const void *hidden, const void *residual,
                         const void *router_weight, const void *router_bias,
                         const k3_moe_expert *experts,
                         const k3_moe_shape *shape, uint32_t token_count,
                         uint32_t precision, void *expert_ids,
                         void *expert_weights, void *workspace,
                         size_t workspace_bytes, void *stream);

/*
 * k3_moe_forward_bf16 for a layer whose router reads another input than its
 * experts: the K3 engine's form, where the router runs on the post-norm
 * hidden state [T, router_columns] (k3_engine.cu:1554-1557,
 * k3_engine_prefill.inc:1448-1453) and the experts on the latent [T,
 * shape->hidden] produced by routed_expert_down_proj (k3_engine.cu:1668-1672).
 * output [T, shape->hidden] = bf16(residual + bf16(sum_r w_r y_r)), or the
 * combine alone when residual is NULL (the engine's routed_up projection
 * follows it). No reference counterpart: it replaces the router, top-k,
 * host sync, expert loop and weighted sum of decode_routed_layer and
 * prefill_routed_layer. router_columns % 8 == 0 (one token runs the decode
 * kernels up to 8192 router columns, the batched router above that);
 * router_input and router_weight 16-byte aligned; workspace
 * k3_moe_workspace_bytes(shape, T) (the router's width does not change it).
 * Routes, workspace and alignment otherwise as k3_moe_forward_bf16.
 */
bool k3_moe_routed_bf16(void *output, const void *router_input, uint32_t router_columns,
                        const void *expert_input, const void *residual,
                        const void *router_weight, const void *router_bias,
                        const k3_moe_expert *experts, const k3_moe_shape *shape,
                        uint32_t token_count, uint32_t precision, void *expert_ids,
                        void *expert_weights, void *workspace, size_t workspace_bytes,
                        void *stream);

/*
 * k3_moe_forward_bf16 without a caller workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. The workspace is a static device array of
 * K3_MOE_STATIC_WORKSPACE_BYTES per GPU, held until the process ends;
 * its address is looked up once per device on the first call there. A
 * shape / token count whose k3_moe_workspace_bytes() exceeds it is
 * rejected (false, with a message on stderr): at the K3 config (H 7168,
 * E 896, k 16, F 2048) up to 64 tokens fit. The call allocates nothing.
 * Every call on one GPU shares that GPU's array: calls that may overlap
 * on one GPU (two streams, two host threads) race and must be serialised
 * by the caller. The array belongs to the library's code object, so each
 * GPU where the library is loaded holds it even if this entry point is
 * never called; its address is cached per device, so a process that calls
 * this entry point must not hipDeviceReset that device afterwards.
 * Arguments otherwise as k3_moe_forward_bf16.
 */
#define K3_MOE_STATIC_WORKSPACE_BYTES (32u << 20)
bool k3_moe_forward_static_bf16(void *output, const void *hidden, const void *residual,
                                const void *router_weight, const void *router_bias,
                                const k3_moe_expert *experts,
                                const k3_moe_shape *shape, uint32_t token_count,
                                uint32_t precision, void *expert_ids,
                                void *expert_weights, void *stream);

/*
 * Stage boundaries of k3_moe_forward_profiled_bf16. stage_events[i] (a
 * hipEvent_t, or NULL) is recorded on the stream just before stage i is
 * launched; stage_events[K3_MOE_STAGE_END] after the last one. Stages a
 * call does not run record their event at the same point as the next one.
 * This is the device-side counterpart of the reference's phase ledger
 * (k3_engine.h:69-99).
 */
enum {
    K3_MOE_STAGE_ROUTER = 0,   /* router logits */
    K3_MOE_STAGE_TOPK = 1,     /* top-k + route weights */
    K3_MOE_STAGE_PLAN = 2,     /* routing plan (T > 1) */
    K3_MOE_STAGE_GATE_UP = 3,  /* gate/up products + activation */
    K3_MOE_STAGE_DOWN = 4,     /* down products, one bf16 row per route */
    K3_MOE_STAGE_COMBINE = 5,  /* weighted combine + residual */
    K3_MOE_STAGE_END = 6,
    K3_MOE_STAGE_COUNT = 7,
};

typedef struct {
    void *stage_events[K3_MOE_STAGE_COUNT];
} k3_moe_profile;

bool k3_moe_forward_profiled_bf16(void *output, const void *hidden,
                                  const void *residual,
                                  const void *router_weight,
                                  const void *router_bias,
                                  const k3_moe_expert *experts,
                                  const k3_moe_shape *shape,
                                  uint32_t token_count, uint32_t precision,
                                  void *expert_ids, void *expert_weights,
                                  void *workspace, size_t workspace_bytes,
                                  const k3_moe_profile *profile, void *stream);

/*
 * Expert stage only, on routes computed elsewhere (ids/weights [T, k] on
 * the device): lets the engine keep its own router, and lets tests check
 * the expert products on identical routes. Alignment as for
 * k3_moe_forward_bf16.
 */
bool k3_moe_experts_bf16(void *output, const void *hidden, const void *residual,
                         const void *expert_ids, const void *expert_weights,
                         const k3_moe_expert *experts,
                         const k3_moe_shape *shape, uint32_t token_count,
                         uint32_t precision, void *workspace,
                         size_t workspace_bytes, void *stream);

/*
 * MXFP8 quantisation of `count` bf16 values (count % 32 == 0; src and the
 * code arrays 16-byte aligned) as the MFMA precisions feed the gate/up
 * activation to the down products: per block of 32, X = floor(log2(max
 * |x|)) - 8 (+1 if the maximum would exceed 448 after scaling; >= -127),
 * scale byte X + 127, codes E4M3(x * 2^-X) rounded to nearest even. With
 * lo_codes/lo_scales non-NULL the residual x - hi is quantised the same
 * way (the two-term split of K3_MOE_MFMA). No reference counterpart:
 * exported so callers and tests can check the activation encoding on its
 * own.
 */
bool k3_moe_mx8_quantize_bf16(uint8_t *hi_codes, uint8_t *hi_scales, uint8_t *lo_codes,
                              uint8_t *lo_scales, const void *src, uint64_t count,
                              void *stream);

/*
 * The same encoding with one scale per row (and term) of a [rows, cols]
 * bf16 matrix (cols % 8 == 0; src 16-byte and the code arrays 8-byte
 * aligned; scale arrays of `rows` bytes): how the MFMA precisions feed the
 * token rows to the gate/up products. No reference counterpart.
 */
bool k3_moe_mx8_quantize_rows_bf16(uint8_t *hi_codes, uint8_t *hi_scales, uint8_t *lo_codes,
                                   uint8_t *lo_scales, const void *src, uint32_t rows,
                                   uint32_t cols, void *stream);

/*
 * K3-native MoE layer: the routed experts run on a latent of width D (the
 * `routed` shape's hidden) between two static projections, beside a dense
 * shared expert (k3_engine.cu:1549-1563, 1668-1689, 1851-1897):
 *
 *   ids, w   = top-k(router(x))                      router on H columns
 *   latent   = routed_down . x                       [D]
 *   routed   = bf16(sum_r w_r * expert_r(latent))    rank order, no residual
 *   full     = routed_up . rms_norm(routed, routed_norm, eps)     [H]
 *   shared   = shared_down . act(shared_gate . x, shared_up . x)  [H]
 *   output   = bf16(residual + bf16(full + shared))  (residual nullable)
 *
 * x is the post-attention-norm hidden state [T, H]; the shared expert uses
 * the routed shape's activation. Static weights are bf16 or Q8-128
 * (k3_static_store.h's two kinds). Each step is the library's own entry
 * point of the same operation, so every intermediate is bit-identical to
 * calling them in this order. No reference counterpart as one call: the
 * reference engine issues these launches itself.
 */
typedef enum {
    K3_MOE_STATIC_BF16 = 0,   /* data bf16 [rows, columns] */
    K3_MOE_STATIC_Q8_128 = 1  /* data int8 [rows, columns], scales f32 [rows, columns / 128] */
} k3_moe_static_kind;

typedef struct {
    uint32_t    kind;     /* k3_moe_static_kind */
    uint32_t    rows;
    uint32_t    columns;
    const void *data;
    const void *scales;   /* Q8-128 only */
} k3_moe_static_weight;

typedef struct {
    k3_moe_shape routed;         /* hidden = latent D; experts, top-k, F, scale, activation */
    uint32_t     model_hidden;   /* H: router columns, layer input/output width */
    uint32_t     shared_hidden;  /* shared expert intermediate width */
    float        norm_epsilon;   /* routed RMSNorm epsilon (1e-5 in K3) */
} k3_moe_native_shape;

typedef struct {
    const void           *router_weight;  /* bf16 [E, H] */
    const void           *router_bias;    /* f32 [E] */
    k3_moe_static_weight  routed_down;    /* [D, H] */
    const void           *routed_norm;    /* bf16 [D] */
    k3_moe_static_weight  routed_up;      /* [H, D] */
    k3_moe_static_weight  shared_gate;    /* [shared_hidden, H] */
    k3_moe_static_weight  shared_up;      /* [shared_hidden, H] */
    k3_moe_static_weight  shared_down;    /* [H, shared_hidden] */
    const k3_moe_expert  *experts;        /* [E], on the latent */
} k3_moe_native_weights;

/* Bytes of workspace k3_moe_native_forward_bf16 needs for token_count rows. */
size_t k3_moe_native_workspace_bytes(const k3_moe_native_shape *shape, uint32_t token_count);

/* The layer above; expert_ids/expert_weights (nullable, [T, k]) receive
 * the routes. output, x and residual rows 16-byte aligned; precision as
 * for k3_moe_forward_bf16: it selects the expert products' arithmetic, and
 * under the MXFP8 precisions batches of 32 or more tokens also run the
 * static projections on bf16 MFMA (exact products, fp32 sums in another
 * order than K3_MOE_EXACT's rows kernels).
 * shared_stream (nullable, like the reference engine's shared_stream,
 * k3_engine.cu:1668-1689) takes the latent projection and the shared
 * expert's gate/up while `stream` routes; the call joins it back with events before the shared
 * down projection, so the result and its completion on `stream` are the
 * same as without it. The fork/join events are created once per host
 * thread and device (no device memory). The event calls cost host time
 * (tens of microseconds per call on ROCm 7): at one token the layer is
 * then host-bound, so an eager caller is faster without it and a caller
 * that captures the call in a graph faster with it. */
bool k3_moe_native_forward_bf16(void *output, const void *hidden, const void *residual,
                                const k3_moe_native_weights *weights,
                                const k3_moe_native_shape *shape, uint32_t token_count,
                                uint32_t precision, void *expert_ids, void *expert_weights,
                                void *workspace, size_t workspace_bytes, void *stream,
                                void *shared_stream);

/*
 * The K3-native block's token-batch projection at the MXFP8 precisions, on
 * bf16 MFMA. No counterpart in the reference (its projections are the VALU
 * row kernels behind k3_rocm_q8_128_gemm_bf16 / k3_rocm_bf16_gemm_bf16);
 * exposed for callers that want the MFMA form directly and for its tests.
 *   q8:  output[t, r] = bf16(sum_b scales[r, b] sum_{k in block b} q[r, k] input[t, k])
 *   bf16 weights: output[t, r] = bf16(sum_k w[r, k] input[t, k])
 * Every product is exact (int8 codes are exact in bf16); only the fp32
 * summation order differs from the row kernels. columns % 128 == 0 (q8) or
 * % 64 == 0, input 16-byte and weights 8-byte (q8) or 16-byte aligned,
 * both operands under 2 GiB; false otherwise.
 */
bool k3_moe_proj_mfma_bf16(void *output, const void *weights, const float *scales,
                           const void *input, uint32_t vector_count, uint32_t rows,
                           uint32_t columns, bool q8, void *stream);

/*
 * Synthetic resident expert store for benchmarks and tests: fills `bytes`
 * of device memory at `base` with the counter-based generator
 * k3_moe_synth_byte(seed, stream, index) below. Packed tensors use uniform
 * bytes (two uniform e2m1 codes); scale tensors use 121 + (value % 5), i.e.
 * E8M0 exponents 2^-6 .. 2^-2.
 */
bool k3_moe_synth_fill(void *base, uint64_t bytes, uint64_t seed,
                       uint64_t stream_id, uint32_t kind, void *stream);
/* Host evaluation of the same generator (kind 0 = packed, 1 = scales). */
void k3_moe_synth_fill_host(void *base, uint64_t bytes, uint64_t seed,
                            uint64_t stream_id, uint32_t kind);

#ifdef __cplusplus
}
#endif

#endif
