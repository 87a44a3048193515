/* Single-token decode path of libk3moe (see k3_decode.hip). */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/k3_moe.h"

namespace k3 {

/* Arrival counters of the decode kernels: zero between calls
 * (k3_moe_workspace_init zeroes them once; the last block to arrive at each
 * counter resets it). */
constexpr uint32_t kMaxDownRowBlocks = 16384; /* hidden / 8 */
struct DecodeSync {
    uint32_t arrive_router;
    uint32_t pad[63];
    uint32_t down_arrive[kMaxDownRowBlocks];
};

struct DecodeParams {
    uint16_t *output;
    const uint16_t *residual;
    const uint16_t *hidden_in;
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
    uint16_t *act;
    uint16_t *slot_out;     /* [k, hidden] bf16 down outputs */
    uint32_t *down_arrive;  /* = sync->down_arrive */
    DecodeSync *sync;
    uint32_t hidden, ffn, expert_count, top_k;
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
bool decode_init_sync(DecodeSync *sync, hipStream_t stream);
/* router + top-k, gate/up, down + combine */
bool decode_launch(const DecodeParams &p, hipStream_t stream, const StageMarker &mark);
/* gate/up, down + combine on routes already in p.ids / p.weights */
bool decode_launch_experts(const DecodeParams &p, hipStream_t stream, const StageMarker &mark);

}  // namespace k3
