/*
 * K3-native MoE layer (k3_engine.cu:1549-1563 router, 1668-1689 latent
 * projection and shared expert, 1851-1897 routed tail and residual): a
 * host-side composition of the library's kernels on one stream (or two:
 * the latent projection and the shared expert's gate/up on a second one),
 * into a caller-provided workspace. Every step computes the same bits as
 * the entry point of the same operation; at one token the norm runs inside
 * the up projection and the adds inside the shared down projection's
 * epilogue.
 */
#include "../../include/k3_moe.h"
#include "../../include/k3_rocm_ops.h"
#include "k3_decode.h"
#include "k3_internal.h"
#include "k3_topk.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr size_t kAlign = 256;

size_t up256(size_t n) { return (n + kAlign - 1u) & ~(kAlign - 1u); }

struct NativeWorkspace {
    float *logits, *norms;
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
    w.logits = (float *)take(4u * T * E * (T > 1u ? k3::router_slice_cap(T, (uint32_t)E) : 1u));
    w.norms = (float *)take(4u * E);
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
/* Token batches (T >= 32) under the MXFP8 precisions: bf16 MFMA with the
 * exact products and fp32 sums (k3_proj.hip); otherwise the exact rows
 * kernels of the reference entry points. */
constexpr uint32_t kProjMfmaMinTokens = 32;

bool project(const k3_moe_static_weight &w, void *out, const void *in, uint32_t T,
             uint32_t precision, hipStream_t st) {
    const bool q8 = w.kind == K3_MOE_STATIC_Q8_128;
    if (precision != K3_MOE_EXACT && T >= kProjMfmaMinTokens &&
        k3::proj_mfma_supported(T, w.rows, w.columns, q8, w.data, in))
        return k3::launch_proj_mfma((uint16_t *)out, in, w.data, q8 ? (const float *)w.scales : nullptr, T,
                                    w.rows, w.columns, q8, st);
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

/* Fork/join events of the shared-stream form: created once per host thread
 * and device (no device memory), reused by every call. A wait captures the
 * event's latest record when it is enqueued, so re-recording for the next
 * call cannot release an earlier wait. */
namespace {

struct StreamEvents {
    int device = -1;
    hipEvent_t fork = nullptr, latent = nullptr, act = nullptr;
};

bool stream_events(StreamEvents *&out) {
    static thread_local StreamEvents cache[16];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return false;
    StreamEvents &e = cache[dev];
    if (e.device != dev) {
        if (hipEventCreateWithFlags(&e.fork, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&e.latent, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&e.act, hipEventDisableTiming) != hipSuccess)
            return false;
        e.device = dev;
    }
    out = &e;
    return true;
}

}  // namespace

extern "C" bool k3_moe_native_forward_bf16(void *output, const void *hidden, const void *residual,
                                           const k3_moe_native_weights *weights,
                                           const k3_moe_native_shape *shape,
                                           uint32_t token_count, uint32_t precision,
                                           void *expert_ids, void *expert_weights,
                                           void *workspace, size_t workspace_bytes,
                                           void *stream, void *shared_stream) {
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
    /* the side stream takes the latent projection and the shared expert's
     * gate/up (both need only x); the main stream routes meanwhile */
    StreamEvents *ev = nullptr;
    const hipStream_t side = shared_stream && shared_stream != stream ? (hipStream_t)shared_stream
                                                                      : st;
    if (side != st && !stream_events(ev)) return false;
    const float beta = s.routed.activation == K3_MOE_ACT_SWIGLU ? 1.0f : s.routed.beta;
    const float lb = s.routed.activation == K3_MOE_ACT_SWIGLU ? 1.0f : s.routed.linear_beta;
    const bool q8 = W.shared_gate.kind == K3_MOE_STATIC_Q8_128 &&
                    W.shared_up.kind == K3_MOE_STATIC_Q8_128 &&
                    W.shared_down.kind == K3_MOE_STATIC_Q8_128;
    /* one token with Q8-128 weights: gate, up and the activation in one
     * pass, and the down projection's epilogue forms bf16(residual +
     * bf16(full + bf16(shared))) */
    const bool fused = T == 1u && q8 && k3::q8_gemv_fits(H, W.shared_gate.data, hidden) &&
                       k3::q8_gemv_fits(H, W.shared_up.data, hidden) &&
                       k3::q8_gemv_fits(S, W.shared_down.data, ws.act);
    const uint64_t sn = (uint64_t)T * S;
    bool ok = true;
    if (ev) {
        ok = hipEventRecord(ev->fork, st) == hipSuccess &&
             hipStreamWaitEvent(side, ev->fork, 0) == hipSuccess;
    }
    /* one stream, one token, Q8-128 latent: the latent projection and the
     * shared gate/up read the same x, so they run as one grid */
    const bool pair = fused && !ev && W.routed_down.kind == K3_MOE_STATIC_Q8_128 &&
                      k3::q8_gemv_fits(H, W.routed_down.data, hidden);
    const bool decode = T == 1u && k3::decode_supported(s.routed) && H % 8u == 0u &&
                        H <= 8192u &&
                        (((uintptr_t)hidden | (uintptr_t)W.router_weight) % 16u) == 0u;
    /* one-token routes with the pair grid: the router rows join that
     * launch (they read the same x) and only top-k runs after it */
    k3::RouterRows router{};
    const bool router_in_pair =
        pair && decode &&
        k3::native_decode_router_rows(&router, hidden, H, W.router_weight, W.router_bias,
                                      s.routed, ws.experts, ws.expert_bytes);
    /* side stream (or the main one): latent, then the shared activation */
    if (pair) {
        ok = ok && k3::launch_q8_gateup_and_gemv(ws.act, W.shared_gate.data,
                                                 W.shared_gate.scales, W.shared_up.data,
                                                 W.shared_up.scales, hidden, S, H,
                                                 s.routed.activation, beta, lb, ws.latent,
                                                 W.routed_down.data, W.routed_down.scales, D,
                                                 router_in_pair ? &router : nullptr, st);
    } else {
        ok = ok && project(W.routed_down, ws.latent, hidden, T, precision, side);
    }
    if (ev) ok = ok && hipEventRecord(ev->latent, side) == hipSuccess;
    if (pair) {
    } else if (fused) {
        ok = ok && k3::launch_q8_gateup(ws.act, W.shared_gate.data, W.shared_gate.scales,
                                        W.shared_up.data, W.shared_up.scales, hidden, S, H,
                                        s.routed.activation, beta, lb, side);
    } else {
        ok = ok && project(W.shared_gate, ws.gate, hidden, T, precision, side) &&
             project(W.shared_up, ws.up, hidden, T, precision, side) &&
             (s.routed.activation == K3_MOE_ACT_SWIGLU
                  ? k3_rocm_swiglu_bf16(ws.act, ws.gate, ws.up, sn, side)
                  : k3_rocm_situ_bf16(ws.act, ws.gate, ws.up, sn, s.routed.beta,
                                      s.routed.linear_beta, side));
    }
    if (ev) ok = ok && hipEventRecord(ev->act, side) == hipSuccess;
    /* main stream: routes, experts on the latent, norm, up projection */
    bool routes_copied = false;
    if (decode) {
        ok = ok && k3::native_decode_experts(ws.routed, hidden, H, ws.latent, W.router_weight,
                                             W.router_bias, W.experts, s.routed, expert_ids,
                                             expert_weights, ws.experts, ws.expert_bytes,
                                             ev ? ev->latent : nullptr, router_in_pair, st);
        routes_copied = true;
    } else {
        /* token batches: the certified MFMA router (same routes) */
        const bool cert = T >= k3::kCertifiedMinTokens && k3::router_certified_supported(T, E, H, k,
                                                                       W.router_weight, hidden);
        ok = ok &&
             (cert ? k3::launch_router_certified(ws.ids, ws.weights, nullptr, nullptr, ws.logits,
                                                 ws.norms, W.router_weight, W.router_bias,
                                                 hidden, T, E, H, k, s.routed.scaling_factor,
                                                 st, nullptr)
                   : k3_rocm_bf16_gemm_f32(ws.logits, W.router_weight, hidden, T, E, H, st) &&
                         k3_rocm_router_topk_f32_batch(ws.ids, ws.weights, ws.logits,
                                                       W.router_bias, T, E, k,
                                                       s.routed.scaling_factor, st)) &&
             (!ev || hipStreamWaitEvent(st, ev->latent, 0) == hipSuccess) &&
             k3_moe_experts_bf16(ws.routed, ws.latent, nullptr, ws.ids, ws.weights, W.experts,
                                 &s.routed, T, precision, ws.experts, ws.expert_bytes, st);
    }
    /* one token with Q8-128 up weights: the norm runs inside the up
     * projection (same bits as the separate norm) */
    if (T == 1u && W.routed_up.kind == K3_MOE_STATIC_Q8_128 &&
        k3::q8_gemv_fits(D, W.routed_up.data, ws.routed) &&
        ((uintptr_t)W.routed_norm % 16u) == 0u) {
        ok = ok && k3::launch_q8_gemv_norm(ws.full, W.routed_up.data, W.routed_up.scales,
                                           ws.routed, W.routed_norm, s.norm_epsilon, H, D, st);
    } else {
        ok = ok &&
             k3_rocm_rms_norm_bf16(ws.normed, ws.routed, W.routed_norm, T, D, s.norm_epsilon,
                                   st) &&
             project(W.routed_up, ws.full, ws.normed, T, precision, st);
    }
    if (ev) ok = ok && hipStreamWaitEvent(st, ev->act, 0) == hipSuccess;
    if (fused) {
        ok = ok && k3::launch_q8_gemv((uint16_t *)output, W.shared_down.data,
                                      W.shared_down.scales, ws.act, H, S, ws.full,
                                      (const uint16_t *)residual, st);
    } else {
        ok = ok && project(W.shared_down, ws.shared, ws.act, T, precision, st);
        const uint64_t n = (uint64_t)T * H;
        if (residual) /* output = bf16(residual + bf16(full + shared)) */
            ok = ok && k3_rocm_add_bf16(ws.sum, ws.full, ws.shared, n, st) &&
                 k3_rocm_add_bf16(output, residual, ws.sum, n, st);
        else
            ok = ok && k3_rocm_add_bf16(output, ws.full, ws.shared, n, st);
    }
    if (!routes_copied) {
        const size_t rb = (size_t)T * k * 4u;
        if (ok && expert_ids)
            ok = hipMemcpyAsync(expert_ids, ws.ids, rb, hipMemcpyDeviceToDevice, st) == hipSuccess;
        if (ok && expert_weights)
            ok = hipMemcpyAsync(expert_weights, ws.weights, rb, hipMemcpyDeviceToDevice, st) ==
                 hipSuccess;
    }
    return ok;
}
