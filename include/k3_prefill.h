#ifndef K3_PREFILL_H
#define K3_PREFILL_H

/*
 * Layer-major prefill planner of Moonshine's k3_prefill.h, same types and
 * entry points (k3_prefill.h:14-107 there), implemented by libk3moe
 * (moonshine_amd/csrc/k3_prefill_plan.cpp). The plan is payload-free
 * bookkeeping: per-token workspace bytes, the routed-expert read ledger of
 * the checkpoint's physical layout (every expert's six tensors validated as
 * one contiguous 17,547,264-byte U8 span), sweep counts and the decode-cache
 * lease. Conventions (k3_prefill.c:37-46, 247-248): bool result, *plan
 * zeroed on entry, a message in error[0 .. error_size) on failure.
 */

#include "k3_safetensors.h"

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* k3_prefill.h:14-35 */
typedef enum {
    K3_PREFILL_CACHE_RETAIN = 0,                /* keep every decode-cache byte */
    K3_PREFILL_CACHE_BORROW_COLD_WORKSPACE = 1, /* lend the batch workspace from an empty cache */
    K3_PREFILL_CACHE_BORROW_WARM_WORKSPACE = 2, /* lend a slot-aligned tail of a warm cache */
} k3_prefill_cache_lease;

/* k3_prefill.h:37-71 */
typedef struct {
    uint32_t chunk_tokens;
    uint32_t context_remaining;
    uint32_t routed_layers;
    uint32_t routed_layer_sweeps;
    uint32_t expert_read_requests;
    uint32_t shard_segments;

    uint64_t hidden_row_bytes;
    uint64_t attn_res_row_bytes;
    uint64_t main_scratch_bytes;
    uint64_t moe_scratch_bytes;
    uint64_t mla_scratch_bytes;
    uint64_t route_bytes;
    uint64_t expert_index_bytes;
    uint64_t auxiliary_workspace_bytes;
    uint64_t batch_workspace_bytes;
    uint64_t incremental_workspace_bytes;
    uint64_t mla_append_bytes;

    uint64_t routed_layer_payload_bytes;
    uint64_t routed_store_payload_bytes;
    uint64_t routed_store_requested_read_bytes;
    uint64_t routed_store_physical_read_bytes;
    uint64_t staging_window_bytes;
    uint64_t registered_staging_bytes;

    uint64_t decode_cache_bytes;
    uint64_t retained_cache_bytes;
    uint64_t borrowed_cache_bytes;
    uint64_t new_layer_buffer_bytes;
    uint64_t new_device_bytes;
} k3_prefill_plan;

/* k3_prefill.h:82-91 / k3_prefill.c:449-462 */
bool k3_prefill_plan_build(const k3_st_model *model, uint32_t chunk_tokens,
                           uint32_t context_remaining, uint16_t experts_per_layer,
                           uint16_t staging_slots, k3_prefill_cache_lease lease,
                           k3_prefill_plan *plan, char *error, size_t error_size);

/* k3_prefill.h:97-107 / k3_prefill.c:236-447 */
bool k3_prefill_plan_build_with_aux_workspace(const k3_st_model *model, uint32_t chunk_tokens,
                                              uint32_t context_remaining,
                                              uint16_t experts_per_layer, uint16_t staging_slots,
                                              k3_prefill_cache_lease lease,
                                              uint64_t auxiliary_workspace_bytes,
                                              k3_prefill_plan *plan, char *error,
                                              size_t error_size);

#ifdef __cplusplus
}
#endif

#endif
