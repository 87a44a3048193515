/*
 * K3-native MoE layer (k3_engine.cu:1549-1563 router, 1668-1689 latent
 * projection and shared expert, 1851-1897 routed tail and residual): a
 * host-side composition of the library's entry points on one stream, into
 * a caller-provided workspace. Every step is the entry point of the same
 * operation, so intermediates are bit-identical to calling them in order.
 */
#include "../../include/k3_moe.h"
#include "../../include/k3_rocm_ops.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr size_t kAlign = 256;

size_t up256(size_t n) { return (n + kAlign - 1u) & ~(kAlign - 1u); }

struct NativeWorkspace {
    float *logits;
    uint32_t *ids;
    float *weights;
    uint16_t *latent, *routed, *normed, *full, *gate, *up, *act, *shared, *sum;
    void *experts;
    size_t expert_bytes, bytes;
};

NativeWorkspace carve(void *base, const k3_moe_native_shape &s, uint32_t T) {
    NativeWorkspace w{};
    uint8_t *p = (uint8_t *)base;
    size_t off = 0;
    auto take = [&](size_t n) {
        uint8_t *q = p ? p + off : nullptr;
        off += up256(n);
        return q;
    };
    const size_t D = s.routed.hidden, H = s.model_hidden, S = s.shared_hidden;
    const size_t E = s.routed.expert_count, k = s.routed.top_k;
    w.logits = (float *)take(4u * T * E);
    w.ids = (uint32_t *)take(4u * T * k);
    w.weights = (float *)take(4u * T * k);
    w.latent = (uint16_t *)take(2u * T * D);
    w.routed = (uint16_t *)take(2u * T * D);
    w.normed = (uint16_t *)take(2u * T * D);
    w.full = (uint16_t *)take(2u * T * H);
    w.gate = (uint16_t *)take(2u * T * S);
    w.up = (uint16_t *)take(2u * T * S);
    w.act = (uint16_t *)take(2u * T * S);
    w.shared = (uint16_t *)take(2u * T * H);
    w.sum = (uint16_t *)take(2u * T * H);
    w.expert_bytes = k3_moe_workspace_bytes(&s.routed, T);
    w.experts = take(w.expert_bytes);
    w.bytes = off;
    return w;
}

bool static_ok(const k3_moe_static_weight &w, uint32_t rows, uint32_t cols) {
    if (!w.data || w.rows != rows || w.columns != cols) return false;
    if (w.kind == K3_MOE_STATIC_BF16) return true;
    return w.kind == K3_MOE_STATIC_Q8_128 && w.scales && cols % 128u == 0u;
}

/* out [T, rows] = w . in [T, columns] with the static weight's own kernel */
bool project(const k3_moe_static_weight &w, void *out, const void *in, uint32_t T,
             hipStream_t st) {
    if (w.kind == K3_MOE_STATIC_BF16)
        return k3_rocm_bf16_gemm_bf16(out, w.data, in, T, w.rows, w.columns, st);
    return k3_rocm_q8_128_gemm_bf16(out, w.data, w.scales, in, T, w.rows, w.columns, st);
}

bool shape_ok(const k3_moe_native_shape *s) {
    return s && s->model_hidden != 0u && s->shared_hidden != 0u && s->routed.hidden != 0u &&
           s->routed.hidden % 8u == 0u && s->model_hidden % 8u == 0u &&
           s->shared_hidden % 8u == 0u && s->norm_epsilon >= 0.0f &&
           k3_moe_workspace_bytes(&s->routed, 1u) != 0u;
}

}  // namespace

extern "C" size_t k3_moe_native_workspace_bytes(const k3_moe_native_shape *shape,
                                                uint32_t token_count) {
    if (!shape_ok(shape) || token_count == 0u || token_count > 65535u) return 0u;
    if (k3_moe_workspace_bytes(&shape->routed, token_count) == 0u) return 0u;
    return carve(nullptr, *shape, token_count).bytes;
}

extern "C" bool k3_moe_native_forward_bf16(void *output, const void *hidden, const void *residual,
                                           const k3_moe_native_weights *weights,
                                           const k3_moe_native_shape *shape,
                                           uint32_t token_count, uint32_t precision,
                                           void *expert_ids, void *expert_weights,
                                           void *workspace, size_t workspace_bytes,
                                           void *stream) {
    if (!output || !hidden || !weights || !workspace || !shape_ok(shape) || token_count == 0u ||
        token_count > 65535u)
        return false;
    const k3_moe_native_weights &W = *weights;
    const k3_moe_native_shape &s = *shape;
    const uint32_t T = token_count, H = s.model_hidden, D = s.routed.hidden;
    const uint32_t S = s.shared_hidden, E = s.routed.expert_count, k = s.routed.top_k;
    if (!W.router_weight || !W.router_bias || !W.routed_norm || !W.experts ||
        !static_ok(W.routed_down, D, H) || !static_ok(W.routed_up, H, D) ||
        !static_ok(W.shared_gate, S, H) || !static_ok(W.shared_up, S, H) ||
        !static_ok(W.shared_down, H, S))
        return false;
    if ((((uintptr_t)output | (uintptr_t)hidden | (uintptr_t)residual) % 16u) != 0u) return false;
    const NativeWorkspace ws = carve(workspace, s, T);
    if (workspace_bytes < ws.bytes || ((uintptr_t)workspace % kAlign) != 0u) return false;
    const hipStream_t st = (hipStream_t)stream;
    const uint64_t n = (uint64_t)T * H;
    /* router on the post-norm hidden state */
    bool ok = k3_rocm_bf16_gemm_f32(ws.logits, W.router_weight, hidden, T, E, H, st) &&
              k3_rocm_router_topk_f32_batch(ws.ids, ws.weights, ws.logits, W.router_bias, T, E,
                                            k, s.routed.scaling_factor, st);
    /* routed experts on the latent, combined in rank order */
    ok = ok && project(W.routed_down, ws.latent, hidden, T, st) &&
         k3_moe_experts_bf16(ws.routed, ws.latent, nullptr, ws.ids, ws.weights, W.experts,
                             &s.routed, T, precision, ws.experts, ws.expert_bytes, st) &&
         k3_rocm_rms_norm_bf16(ws.normed, ws.routed, W.routed_norm, T, D, s.norm_epsilon, st) &&
         project(W.routed_up, ws.full, ws.normed, T, st);
    /* shared expert */
    const uint64_t sn = (uint64_t)T * S;
    ok = ok && project(W.shared_gate, ws.gate, hidden, T, st) &&
         project(W.shared_up, ws.up, hidden, T, st) &&
         (s.routed.activation == K3_MOE_ACT_SWIGLU
              ? k3_rocm_swiglu_bf16(ws.act, ws.gate, ws.up, sn, st)
              : k3_rocm_situ_bf16(ws.act, ws.gate, ws.up, sn, s.routed.beta,
                                  s.routed.linear_beta, st)) &&
         project(W.shared_down, ws.shared, ws.act, T, st);
    /* output = bf16(residual + bf16(full + shared)) */
    if (residual)
        ok = ok && k3_rocm_add_bf16(ws.sum, ws.full, ws.shared, n, st) &&
             k3_rocm_add_bf16(output, residual, ws.sum, n, st);
    else
        ok = ok && k3_rocm_add_bf16(output, ws.full, ws.shared, n, st);
    const size_t rb = (size_t)T * k * 4u;
    if (ok && expert_ids)
        ok = hipMemcpyAsync(expert_ids, ws.ids, rb, hipMemcpyDeviceToDevice, st) == hipSuccess;
    if (ok && expert_weights)
        ok = hipMemcpyAsync(expert_weights, ws.weights, rb, hipMemcpyDeviceToDevice, st) ==
             hipSuccess;
    return ok;
}
