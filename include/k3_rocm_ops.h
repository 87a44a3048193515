#ifndef K3_ROCM_OPS_H
#define K3_ROCM_OPS_H

/*
 * The routed-MoE subset of Moonshine's k3_rocm_ops.h, with unchanged
 * signatures, implemented by libk3moe for gfx950. Each declaration cites
 * the reference declaration it replaces (k3_rocm_ops.h:line) and its
 * reference launcher (k3_rocm_ops.cu:line).
 *
 * Conventions (k3_rocm_ops.h:14-19 of the reference): tensor pointers are
 * contiguous device pointers (router outputs may be HIP-mapped host
 * memory); `stream` is a hipStream_t passed as void *, NULL = default
 * stream; invalid arguments return false before any launch; launch errors
 * are returned synchronously while execution stays asynchronous. Nothing
 * allocates.
 */

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* k3_rocm_ops.h:20-26 / k3_rocm_ops.cu:1566-1590. SiTU on bf16 gate/up. */
bool k3_rocm_situ_bf16(void       *output,
                       const void *gate,
                       const void *up,
                       uint64_t    element_count,
                       float       beta,
                       float       linear_beta,
                       void       *stream);

/* No reference counterpart: SwiGLU g*sigmoid(g)*u, the activation of the
 * benchmark configurations (SiTU's beta, linear_beta -> infinity limit). */
bool k3_rocm_swiglu_bf16(void       *output,
                         const void *gate,
                         const void *up,
                         uint64_t    element_count,
                         void       *stream);

/* k3_rocm_ops.h:40-51 / k3_rocm_ops.cu:1592-1602. packed [rows, columns/2]
 * (low nibble = even column), scales [rows, columns/32] E8M0. */
bool k3_rocm_mxfp4_gemv_bf16(void       *output,
                             const void *packed,
                             const void *scales,
                             const void *input,
                             uint32_t    rows,
                             uint32_t    columns,
                             void       *stream);

/* k3_rocm_ops.h:53-66 / k3_rocm_ops.cu:1661-1692. Per-row order identical
 * to the GEMV. */
bool k3_rocm_mxfp4_gemm_bf16(void       *output,
                             const void *packed,
                             const void *scales,
                             const void *input,
                             uint32_t    vector_count,
                             uint32_t    rows,
                             uint32_t    columns,
                             void       *stream);

/* k3_rocm_ops.h:67-80 / k3_rocm_ops.cu:1604-1659. batch_tile 16/32/64. */
bool k3_rocm_mxfp4_gemm_tiled_bf16(void       *output,
                                   const void *packed,
                                   const void *scales,
                                   const void *input,
                                   uint32_t    vector_count,
                                   uint32_t    rows,
                                   uint32_t    columns,
                                   uint32_t    batch_tile,
                                   void       *stream);

/* k3_rocm_ops.h:107-112 / k3_rocm_ops.cu:1792-1801. Router logits. */
bool k3_rocm_bf16_gemv_f32(void       *output,
                           const void *weights,
                           const void *input,
                           uint32_t    rows,
                           uint32_t    columns,
                           void       *stream);

/* k3_rocm_ops.h:114-120 / k3_rocm_ops.cu:1858-1885. */
bool k3_rocm_bf16_gemm_f32(void       *output,
                           const void *weights,
                           const void *input,
                           uint32_t    vector_count,
                           uint32_t    rows,
                           uint32_t    columns,
                           void       *stream);

/* k3_rocm_ops.h:122-130 / k3_rocm_ops.cu:1803-1856. */
bool k3_rocm_bf16_gemm_tiled_f32(void       *output,
                                 const void *weights,
                                 const void *input,
                                 uint32_t    vector_count,
                                 uint32_t    rows,
                                 uint32_t    columns,
                                 uint32_t    batch_tile,
                                 void       *stream);

/* k3_rocm_ops.h:82-87 / k3_rocm_ops.cu:1694-1703. bf16 [rows, columns]
 * weights x bf16 input -> bf16: the bf16_gemv_f32 order rounded once. */
bool k3_rocm_bf16_gemv_bf16(void       *output,
                            const void *weights,
                            const void *input,
                            uint32_t    rows,
                            uint32_t    columns,
                            void       *stream);

/* k3_rocm_ops.h:99-105 / k3_rocm_ops.cu:1760-1789. Per-row order identical
 * to the GEMV for every vector. */
bool k3_rocm_bf16_gemm_bf16(void       *output,
                            const void *weights,
                            const void *input,
                            uint32_t    vector_count,
                            uint32_t    rows,
                            uint32_t    columns,
                            void       *stream);

/* k3_rocm_ops.h:89-97 / k3_rocm_ops.cu:1727-1758. batch_tile in {16, 32,
 * 64}, otherwise false; results do not depend on it. */
bool k3_rocm_bf16_gemm_tiled_bf16(void       *output,
                                  const void *weights,
                                  const void *input,
                                  uint32_t    vector_count,
                                  uint32_t    rows,
                                  uint32_t    columns,
                                  uint32_t    batch_tile,
                                  void       *stream);

/* k3_rocm_ops.h:138-144 / k3_rocm_ops.cu:1887-1908. Symmetric int8 in
 * 128-element blocks: scale = max|w| / 127 (1 for an all-zero block), code
 * = clamp(rint(w / scale), -127, 127), IEEE division, NaN codes as 0.
 * quantized [rows, columns] int8, scales [rows, columns / 128] f32;
 * columns % 128 == 0, weights 4-byte and quantized 2-byte aligned. */
bool k3_rocm_bf16_quantize_q8_128(void       *quantized,
                                  void       *scales,
                                  const void *weights,
                                  uint32_t    rows,
                                  uint32_t    columns,
                                  void       *stream);

/* k3_rocm_ops.h:146-152 / k3_rocm_ops.cu:1910-1934. w = bf16(q * scale). */
bool k3_rocm_q8_128_dequantize_bf16(void       *weights,
                                    const void *quantized,
                                    const void *scales,
                                    uint32_t    rows,
                                    uint32_t    columns,
                                    void       *stream);

/* k3_rocm_ops.h:154-161 / k3_rocm_ops.cu:1936-1946. Row order: lane l owns
 * 32-column groups l, l + 64, ...; gs = fmaf(q, x, gs) over a group, acc =
 * fmaf(gs, scale, acc); wave64 butterfly; bf16 round. columns % 128 == 0,
 * quantized 8-byte, input 16-byte and scales 4-byte aligned. */
bool k3_rocm_q8_128_gemv_bf16(void       *output,
                              const void *quantized,
                              const void *scales,
                              const void *input,
                              uint32_t    rows,
                              uint32_t    columns,
                              void       *stream);

/* k3_rocm_ops.h:163-171 / k3_rocm_ops.cu:2007-2039. Per-row order identical
 * to the GEMV for every vector. */
bool k3_rocm_q8_128_gemm_bf16(void       *output,
                              const void *quantized,
                              const void *scales,
                              const void *input,
                              uint32_t    vector_count,
                              uint32_t    rows,
                              uint32_t    columns,
                              void       *stream);

/* k3_rocm_ops.h:173-182 / k3_rocm_ops.cu:1972-2005. batch_tile in {16, 32,
 * 64}, otherwise false; results do not depend on it. */
bool k3_rocm_q8_128_gemm_tiled_bf16(void       *output,
                                    const void *quantized,
                                    const void *scales,
                                    const void *input,
                                    uint32_t    vector_count,
                                    uint32_t    rows,
                                    uint32_t    columns,
                                    uint32_t    batch_tile,
                                    void       *stream);

/* k3_rocm_ops.h:301-307 / k3_rocm_ops.cu:2399-2418. Latent RMSNorm of the
 * K3-native MoE tail. */
bool k3_rocm_rms_norm_bf16(void       *output,
                           const void *input,
                           const void *weight,
                           uint32_t    vector_count,
                           uint32_t    hidden_size,
                           float       epsilon,
                           void       *stream);

/* k3_rocm_ops.h:377-390 / k3_rocm_ops.cu:2532-2543. ids in (choice desc,
 * id asc) order; weights = score / (1e-20 + sum of selected scores) * scale. */
bool k3_rocm_router_topk_f32(void       *expert_ids,
                             void       *expert_weights,
                             const void *logits,
                             const void *correction_bias,
                             uint32_t    expert_count,
                             uint32_t    top_k,
                             float       scaling_factor,
                             void       *stream);

/* k3_rocm_ops.h:392-401 / k3_rocm_ops.cu:2545-2571. */
bool k3_rocm_router_topk_f32_batch(void       *expert_ids,
                                   void       *expert_weights,
                                   const void *logits,
                                   const void *correction_bias,
                                   uint32_t    vector_count,
                                   uint32_t    expert_count,
                                   uint32_t    top_k,
                                   float       scaling_factor,
                                   void       *stream);

/* k3_rocm_ops.h:403-408 / k3_rocm_ops.cu:2573-2582. */
bool k3_rocm_weighted_sum_bf16(void       *output,
                               const void *vectors,
                               const void *weights,
                               uint32_t    vector_count,
                               uint32_t    hidden_size,
                               void       *stream);

/* k3_rocm_ops.h:410-417 / k3_rocm_ops.cu:2584-2608. */
bool k3_rocm_weighted_sum_bf16_batch(void       *output,
                                     const void *vectors,
                                     const void *weights,
                                     uint32_t    token_count,
                                     uint32_t    vector_count,
                                     uint32_t    hidden_size,
                                     void       *stream);

/* k3_rocm_ops.h:419-425 / k3_rocm_ops.cu:2610-2637. */
bool k3_rocm_gather_rows_bf16(void       *output,
                              const void *input,
                              const void *row_ids,
                              uint32_t    row_count,
                              uint32_t    row_size,
                              void       *stream);

/* k3_rocm_ops.h:427-433 / k3_rocm_ops.cu:2639-2666. */
bool k3_rocm_scatter_rows_bf16(void       *output,
                               const void *input,
                               const void *row_ids,
                               uint32_t    row_count,
                               uint32_t    row_size,
                               void       *stream);

/* k3_rocm_ops.h:435-439 / k3_rocm_ops.cu:2668-2686. */
bool k3_rocm_add_bf16(void       *output,
                      const void *left,
                      const void *right,
                      uint64_t    element_count,
                      void       *stream);

#ifdef __cplusplus
}
#endif

#endif
