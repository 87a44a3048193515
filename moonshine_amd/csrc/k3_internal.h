/* Launch helpers shared between the translation units of libk3moe. */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace k3 {

struct RouterRows; /* k3_topk.h */

/* f32 [tokens, rows] = bf16 weights [rows, cols] . bf16 input [tokens, cols]
 * in the w64 order. */
bool launch_bf16_rows_f32_any(float *out, const void *weights, const void *input,
                              uint32_t tokens, uint32_t rows, uint32_t cols,
                              hipStream_t stream);

/* The same order with bf16 [tokens, rows] output (rounded once). */
bool launch_bf16_rows_bf16_any(uint16_t *out, const void *weights, const void *input,
                               uint32_t tokens, uint32_t rows, uint32_t cols,
                               hipStream_t stream);

/* Single-vector Q8-128 projection for cols <= 8192 (bit-identical to the
 * one-wave-per-row kernel); out = bf16(v), or bf16(add2 + bf16(add1 +
 * bf16(v))) with the nullable addends. */
bool q8_gemv_fits(uint32_t cols, const void *codes, const void *x);
bool launch_q8_gemv(uint16_t *out, const void *codes, const void *scales, const void *x,
                    uint32_t rows, uint32_t cols, const uint16_t *add1, const uint16_t *add2,
                    hipStream_t stream);
/* launch_q8_gemv on rms_norm(x, norm_weight, eps) (the RMSNorm entry
 * point's bits), without the normalised vector ever leaving the kernel.
 * norm_weight 16-byte aligned. */
bool launch_q8_gemv_norm(uint16_t *out, const void *codes, const void *scales, const void *x,
                         const void *norm_weight, float eps, uint32_t rows, uint32_t cols,
                         hipStream_t stream);
/* act = bf16(act(bf16(gate . x), bf16(up . x))) for two Q8-128 matrices. */
bool launch_q8_gateup(uint16_t *act, const void *gate_codes, const void *gate_scales,
                      const void *up_codes, const void *up_scales, const void *x, uint32_t rows,
                      uint32_t cols, uint32_t kind, float beta, float lb, hipStream_t stream);

/* Certified MFMA router for token batches (k3_router.hip): the exact
 * router's routes and weights, with the logit GEMM on bf16 MFMA. approx
 * holds router_slice_cap(T, E) x T x E floats, norms E floats. mark (nullable) is called with the
 * top-k stage between the logits and the selection. */
struct StageMarker;
constexpr uint32_t kRouterMaxSlices = 16;
constexpr uint32_t kCertifiedMinTokens = 32; /* below: the exact logits + top-k kernels */
uint32_t router_slice_cap(uint32_t T, uint32_t E);              /* for sizing approx */
uint32_t router_slices(uint32_t T, uint32_t E, uint32_t H);     /* <= the cap */
bool router_certified_supported(uint32_t tokens, uint32_t experts, uint32_t hidden,
                                uint32_t top_k, const void *router_weight, const void *x);
bool launch_router_certified(uint32_t *ids, float *weights, uint32_t *ids2, float *w2,
                             float *approx, float *norms, const void *router_weight,
                             const void *router_bias, const void *x, uint32_t T, uint32_t E,
                             uint32_t H, uint32_t k, float scale, hipStream_t stream,
                             const StageMarker *mark);

/* launch_q8_gateup (rows x cols) and launch_q8_gemv (out_rows x cols, no
 * addends) on the same x as one launch; the same bits as the two calls.
 * With `router` (its x and cols those of the projections), the same launch
 * also writes the router's logits, scores and keys (router_rows_wave). */
bool launch_q8_gateup_and_gemv(uint16_t *act, const void *gate_codes, const void *gate_scales,
                               const void *up_codes, const void *up_scales, const void *x,
                               uint32_t rows, uint32_t cols, uint32_t kind, float beta, float lb,
                               uint16_t *out, const void *codes, const void *scales,
                               uint32_t out_rows, const RouterRows *router, hipStream_t stream);

/* Static projection of a token batch on bf16 MFMA (k3_proj.hip), for the
 * MXFP8 precisions: out [T, N] bf16 = w [N, K] . x [T, K], w Q8-128 codes
 * with [N, K / 128] scales (q8) or bf16. Products exact; fp32 summation
 * order differs from the exact rows kernels. */
bool proj_mfma_supported(uint32_t tokens, uint32_t rows, uint32_t cols, bool q8,
                         const void *weights, const void *x);
bool launch_proj_mfma(uint16_t *out, const void *x, const void *weights, const float *scales,
                      uint32_t T, uint32_t N, uint32_t K, bool q8, hipStream_t stream);

/* Router top-k; ids2/w2 (nullable) receive extra copies (e.g. mapped host
 * memory) while ids/w stay in device memory for later kernels. */
bool launch_router_topk(uint32_t *ids, float *w, uint32_t *ids2, float *w2,
                        const float *logits, const float *bias, uint32_t tokens,
                        uint32_t experts, uint32_t top_k, float scale,
                        hipStream_t stream);

/* Counter-based generator of the synthetic expert store. */
__host__ __device__ inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
__host__ __device__ inline uint64_t synth_key(uint64_t seed, uint64_t stream_id) {
    return mix64(seed ^ mix64(stream_id + 0x632be59bd9b4e019ull));
}
__host__ __device__ inline uint64_t synth_word(uint64_t key, uint64_t w) {
    return mix64(key + (w + 1u) * 0x9e3779b97f4a7c15ull);
}
__host__ __device__ inline uint8_t synth_byte(uint64_t key, uint64_t i, uint32_t kind) {
    if (kind == 0u) return (uint8_t)(synth_word(key, i >> 3) >> (8u * (i & 7u)));
    return (uint8_t)(121u + (uint32_t)((synth_word(key, i) >> 32) % 5u));
}

}  // namespace k3
