/* Single-token decode path of libk3moe (see k3_decode.hip). */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/k3_moe.h"

namespace k3 {

struct RouterRows; /* k3_topk.h */

struct DecodeParams {
    uint16_t *output;
    const uint16_t *residual;
    const uint16_t *hidden_in;
    const uint16_t *router_in;  /* router input rows (the layer's hidden_in unless set) */
    const uint16_t *router_weight;
    const float *router_bias;
    const k3_moe_expert *experts;
    float *logits;
    float *scores;
    uint32_t *keys;
    uint32_t *ids;
    float *weights;
    uint32_t *ids_copy;
    float *weights_copy;
    uint16_t *act;          /* [k, ffn] bf16 activations */
    k3_moe_expert *sel;     /* [k] descriptors of the selected experts */
    uint16_t *y;            /* [k, hidden] bf16 per-slot expert outputs */
    uint32_t *slot_mask;    /* bit s: slot s has an expert */
    uint32_t hidden, ffn, expert_count, top_k;
    uint32_t router_cols;       /* router input width (hidden unless set) */
    float scale;
    uint32_t activation;
    float beta, linear_beta;
};

struct StageMarker {
    const k3_moe_profile *profile;
    hipStream_t stream;
    void operator()(int stage) const {
        if (profile && profile->stage_events[stage])
            (void)hipEventRecord((hipEvent_t)profile->stage_events[stage], stream);
    }
};

bool decode_supported(const k3_moe_shape &s);
/* router, top-k, gate/up, down, combine */
bool decode_launch(const DecodeParams &p, hipStream_t stream, const StageMarker &mark);
/* router and top-k only (decode_launch's first half) */
bool decode_launch_route(const DecodeParams &p, hipStream_t stream, const StageMarker &mark);
/* top-k only, on router outputs already in p.logits / p.scores / p.keys */
bool decode_launch_topk(const DecodeParams &p, hipStream_t stream, const StageMarker &mark);
/* gate/up, down, combine on routes in p.ids / p.weights (resolve: look the
 * expert descriptors up first, for routes that did not come from
 * decode_launch's top-k) */
bool decode_launch_experts(const DecodeParams &p, hipStream_t stream, const StageMarker &mark,
                           bool resolve);

/* One-token routed experts of the K3-native layer: router and top-k on x
 * (router_cols wide), experts on `latent` (shape.hidden wide), output =
 * bf16 rank-order combine with no residual. Uses the decode kernels; the
 * workspace is the routed layer's (k3_moe_workspace_bytes(shape, 1)).
 * With latent_ready, the experts wait for that event (the latent may be
 * produced on another stream) while router and top-k do not. */
/* With `routed`, the router outputs are already in the workspace (filled
 * through native_decode_router_rows) and only top-k runs before the
 * experts. */
bool native_decode_experts(void *routed_out, const void *x, uint32_t router_cols,
                           const void *latent, const void *router_weight,
                           const void *router_bias, const k3_moe_expert *experts,
                           const k3_moe_shape &shape, void *ids_copy, void *w_copy,
                           void *workspace, size_t workspace_bytes, hipEvent_t latent_ready,
                           bool routed, hipStream_t stream);

/* The router rows native_decode_experts computes (x, weights and where in
 * the workspace the logits, scores and keys go), for a caller that fuses
 * them into another launch. False when native_decode_experts would reject
 * the arguments. */
bool native_decode_router_rows(RouterRows *out, const void *x, uint32_t router_cols,
                               const void *router_weight, const void *router_bias,
                               const k3_moe_shape &shape, void *workspace,
                               size_t workspace_bytes);

}  // namespace k3
