/*
 * k3_prefill_plan_build(_with_aux_workspace): the payload-free memory and
 * I/O plan of one layer-major K3 prefill chunk (k3_prefill.c:236-462).
 *
 * Host code only. The plan is integer bookkeeping over the K3 geometry
 * and the checkpoint's tensor directory:
 *   - per-token workspace regions times chunk_tokens (k3_prefill.c:136-234);
 *   - for each of the 92 routed layers and 896 experts, the six expert
 *     tensors (w1/w2/w3 packed + scale) must be one contiguous U8 span of
 *     17,547,264 bytes in one shard; the read ledger counts each span's
 *     4 KiB-aligned request (clipped to the shard file for the physical
 *     count), and the layer's spans in (shard, offset) order give the number
 *     of contiguous physical segments;
 *   - staging window, registered staging and the decode-cache lease.
 */
#include "../../include/k3_prefill.h"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>

namespace {

/* K3 geometry the ledger is defined on (k3_prefill.c:8-29). */
namespace k3g {
constexpr uint64_t kContext = 1048576;
constexpr uint64_t kHidden = 7168, kKdaInner = 12288, kKdaHeadDim = 128;
constexpr uint64_t kDense = 33792, kLatent = 3584, kExpertHidden = 3072, kShared = 6144;
constexpr uint64_t kTopK = 16, kExperts = 896, kRoutedLayers = 92, kHeads = 96;
constexpr uint64_t kMlaQLora = 1536, kMlaQ = 96 * 192, kMlaCacheDim = 576, kMlaLayers = 24;
constexpr uint64_t kStagingSlotBytes = 17551360;
constexpr uint64_t kExpertSpanBytes = 17547264;
constexpr uint64_t kPage = 4096;
constexpr uint64_t kBf16 = 2;
}  // namespace k3g

/* Bytes per token of each workspace region. */
struct TokenRegion {
    uint64_t k3_prefill_plan::*field;
    uint64_t per_token;
};

constexpr TokenRegion kRegions[] = {
    {&k3_prefill_plan::hidden_row_bytes, 2 * k3g::kHidden * k3g::kBf16},
    {&k3_prefill_plan::attn_res_row_bytes, 8 * k3g::kHidden * k3g::kBf16},
    {&k3_prefill_plan::main_scratch_bytes,
     (5 * k3g::kHidden + 10 * k3g::kKdaInner + k3g::kKdaHeadDim + k3g::kHeads + 3 * k3g::kDense) *
         k3g::kBf16},
    {&k3_prefill_plan::moe_scratch_bytes,
     k3g::kExperts * 4 + (k3g::kLatent + 3 * k3g::kExpertHidden + k3g::kTopK * k3g::kLatent +
                          2 * k3g::kLatent + k3g::kHidden + 3 * k3g::kShared + k3g::kHidden) *
                             k3g::kBf16},
    {&k3_prefill_plan::mla_scratch_bytes,
     (2 * k3g::kMlaQLora + k3g::kMlaQ + k3g::kMlaCacheDim + k3g::kHeads * k3g::kMlaCacheDim +
      3 * k3g::kKdaInner) *
         k3g::kBf16},
    {&k3_prefill_plan::route_bytes, k3g::kTopK * (4 + 4)},
    {&k3_prefill_plan::expert_index_bytes, 2 * 4},
};

constexpr uint64_t one_token_workspace() {
    uint64_t s = 0;
    for (const TokenRegion &r : kRegions) s += r.per_token;
    return s;
}
static_assert(one_token_workspace() == 1116360, "K3 per-token prefill workspace");

bool add_to(uint64_t &acc, uint64_t v) { return !__builtin_add_overflow(acc, v, &acc); }
bool product(uint64_t a, uint64_t b, uint64_t &out) { return !__builtin_mul_overflow(a, b, &out); }

class Errors {
  public:
    Errors(char *buf, size_t n) : buf_(buf), n_(n) {
        if (buf_ && n_) buf_[0] = '\0';
    }
    __attribute__((format(printf, 2, 3))) bool fail(const char *fmt, ...) const {
        if (buf_ && n_) {
            va_list ap;
            va_start(ap, fmt);
            vsnprintf(buf_, n_, fmt, ap);
            va_end(ap);
        }
        return false;
    }

  private:
    char *buf_;
    size_t n_;
};

/* Binary search of the strcmp-sorted directory (the k3_st_find contract,
 * k3_safetensors.c:539-551). */
const k3_st_tensor *find_tensor(const k3_st_model &m, const char *name) {
    const k3_st_tensor *lo = m.tensors, *hi = m.tensors + m.tensor_count;
    const k3_st_tensor *it = std::lower_bound(
        lo, hi, name, [](const k3_st_tensor &t, const char *n) { return strcmp(t.name, n) < 0; });
    return (it != hi && strcmp(it->name, name) == 0) ? it : nullptr;
}

struct Span {
    uint16_t shard;
    uint64_t start, end;
};

/* The expert's six tensors, in the engine's layout order (w1 packed,
 * w1 scale, w2 packed, w2 scale, w3 packed, w3 scale), must tile one U8
 * span of exactly kExpertSpanBytes in one shard (k3_prefill.c:62-122). */
bool expert_span(const k3_st_model &m, uint32_t layer, uint32_t expert, Span &out,
                 const Errors &err) {
    static const char *const kParts[6] = {"w1.weight_packed", "w1.weight_scale",
                                          "w2.weight_packed", "w2.weight_scale",
                                          "w3.weight_packed", "w3.weight_scale"};
    const k3_st_tensor *prev = nullptr, *first = nullptr;
    for (const char *part : kParts) {
        char name[256];
        const int n = snprintf(name, sizeof name,
                               "language_model.model.layers.%u.block_sparse_moe.experts.%u.%s",
                               layer, expert, part);
        if (n < 0 || (size_t)n >= sizeof name)
            return err.fail("layer-%u expert-%u tensor name overflow", layer, expert);
        const k3_st_tensor *t = find_tensor(m, name);
        if (!t) return err.fail("missing layer-%u expert-%u tensor %s", layer, expert, part);
        const bool joined = !prev || (t->shard == first->shard &&
                                      prev->physical_offset + prev->byte_length == t->physical_offset);
        if (t->dtype != K3_ST_DTYPE_U8 || !joined)
            return err.fail("layer-%u expert-%u tensors are not one contiguous U8 span", layer,
                            expert);
        if (!first) first = t;
        prev = t;
    }
    out.shard = first->shard;
    out.start = first->physical_offset;
    out.end = prev->physical_offset + prev->byte_length;
    if (out.end < out.start || out.end - out.start != k3g::kExpertSpanBytes)
        return err.fail("layer-%u expert-%u physical span is invalid", layer, expert);
    return true;
}

bool plan_layers(const k3_st_model &m, k3_prefill_plan &p, const Errors &err) {
    Span spans[k3g::kExperts];
    for (uint32_t layer = 1; layer <= k3g::kRoutedLayers; layer++) {
        uint64_t layer_bytes = 0;
        for (uint32_t e = 0; e < k3g::kExperts; e++) {
            Span s;
            if (!expert_span(m, layer, e, s, err)) return false;
            if (s.shard >= m.shard_count)
                return err.fail("layer-%u expert-%u has invalid shard %u", layer, e, s.shard);
            const uint64_t a0 = s.start & ~(k3g::kPage - 1);
            const uint64_t a1 = (s.end + k3g::kPage - 1) & ~(k3g::kPage - 1);
            const uint64_t file_end = std::min(a1, m.shards[s.shard].file_bytes);
            if (a1 < a0 || file_end < s.end || a1 - a0 > k3g::kStagingSlotBytes ||
                !add_to(p.routed_store_requested_read_bytes, a1 - a0) ||
                !add_to(p.routed_store_physical_read_bytes, file_end - a0) ||
                !add_to(layer_bytes, s.end - s.start))
                return err.fail("layer-%u expert-%u read ledger overflow", layer, e);
            p.expert_read_requests++;
            spans[e] = s;
        }
        std::sort(spans, spans + k3g::kExperts, [](const Span &a, const Span &b) {
            return a.shard != b.shard ? a.shard < b.shard : a.start < b.start;
        });
        /* contiguous runs in (shard, offset) order = physical segments */
        for (uint32_t i = 0; i < k3g::kExperts; i++) {
            const bool same_shard = i > 0 && spans[i].shard == spans[i - 1].shard;
            if (same_shard && spans[i].start < spans[i - 1].end)
                return err.fail("layer-%u routed expert spans overlap in shard %u", layer,
                                spans[i].shard);
            if (!same_shard || spans[i].start != spans[i - 1].end) p.shard_segments++;
        }
        if (layer == 1)
            p.routed_layer_payload_bytes = layer_bytes;
        else if (layer_bytes != p.routed_layer_payload_bytes)
            return err.fail("layer-%u routed payload differs from layer 1", layer);
        if (!add_to(p.routed_store_payload_bytes, layer_bytes))
            return err.fail("K3 routed-store byte count overflow");
    }
    return true;
}

/* Decode-cache ownership for the lease (k3_prefill.c:383-437): a cold lease
 * lends exactly the batch workspace, a warm lease whole expert slots. */
bool plan_lease(k3_prefill_plan &p, k3_prefill_cache_lease lease, const Errors &err) {
    if (lease == K3_PREFILL_CACHE_RETAIN) {
        p.retained_cache_bytes = p.decode_cache_bytes;
        p.new_device_bytes = p.batch_workspace_bytes;
        return true;
    }
    const bool warm = lease == K3_PREFILL_CACHE_BORROW_WARM_WORKSPACE;
    if (p.decode_cache_bytes < p.batch_workspace_bytes)
        return err.fail("%s K3 prefill cache %.3f GiB cannot lend %.3f GiB batch workspace",
                        warm ? "warm" : "cold", (double)p.decode_cache_bytes / 1073741824.0,
                        (double)p.batch_workspace_bytes / 1073741824.0);
    uint64_t lent = p.batch_workspace_bytes;
    if (warm) {
        uint64_t rounded = p.batch_workspace_bytes;
        if (!add_to(rounded, k3g::kExpertSpanBytes - 1) ||
            !product(rounded / k3g::kExpertSpanBytes, k3g::kExpertSpanBytes, lent) ||
            lent > p.decode_cache_bytes)
            return err.fail("warm K3 prefill cache slot rounding overflow");
    }
    p.borrowed_cache_bytes = lent;
    p.retained_cache_bytes = p.decode_cache_bytes - lent;
    p.new_device_bytes = 0;
    return true;
}

}  // namespace

extern "C" bool k3_prefill_plan_build_with_aux_workspace(
        const k3_st_model *model, uint32_t chunk_tokens, uint32_t context_remaining,
        uint16_t experts_per_layer, uint16_t staging_slots, k3_prefill_cache_lease lease,
        uint64_t auxiliary_workspace_bytes, k3_prefill_plan *plan, char *error,
        size_t error_size) {
    const Errors err(error, error_size);
    if (plan) memset(plan, 0, sizeof *plan);
    const bool lease_ok = lease == K3_PREFILL_CACHE_RETAIN ||
                          lease == K3_PREFILL_CACHE_BORROW_COLD_WORKSPACE ||
                          lease == K3_PREFILL_CACHE_BORROW_WARM_WORKSPACE;
    if (!model || !plan || model->shard_count == 0 || chunk_tokens == 0 ||
        chunk_tokens > context_remaining || context_remaining > k3g::kContext ||
        experts_per_layer == 0 || staging_slots < 2 || !lease_ok)
        return err.fail("invalid K3 prefill-plan arguments");
    k3_prefill_plan &p = *plan;
    p.chunk_tokens = chunk_tokens;
    p.context_remaining = context_remaining;
    p.routed_layers = (uint32_t)k3g::kRoutedLayers;
    p.routed_layer_sweeps = (uint32_t)k3g::kRoutedLayers; /* one sweep per routed layer */

    bool ok = true;
    for (const TokenRegion &r : kRegions) {
        ok = ok && product(r.per_token, chunk_tokens, p.*r.field) &&
             add_to(p.batch_workspace_bytes, p.*r.field);
    }
    if (!ok) return err.fail("K3 prefill workspace byte count overflow");
    p.incremental_workspace_bytes = p.batch_workspace_bytes > one_token_workspace()
                                        ? p.batch_workspace_bytes - one_token_workspace()
                                        : 0;
    if (!product((uint64_t)chunk_tokens * k3g::kMlaLayers, k3g::kMlaCacheDim * k3g::kBf16,
                 p.mla_append_bytes))
        return err.fail("K3 prefill workspace byte count overflow");
    p.auxiliary_workspace_bytes = auxiliary_workspace_bytes;
    if (!add_to(p.batch_workspace_bytes, auxiliary_workspace_bytes))
        return err.fail("K3 auxiliary workspace byte count overflow");

    if (!plan_layers(*model, p, err)) return false;

    if (!product(k3g::kStagingSlotBytes, 2, p.staging_window_bytes) ||
        !product(k3g::kStagingSlotBytes, staging_slots, p.registered_staging_bytes) ||
        !product(k3g::kRoutedLayers * experts_per_layer, k3g::kExpertSpanBytes,
                 p.decode_cache_bytes))
        return err.fail("K3 prefill cache byte count overflow");
    if (!plan_lease(p, lease, err)) return false;
    p.new_layer_buffer_bytes = 0; /* every mode executes from the fixed staging window */
    return true;
}

extern "C" bool k3_prefill_plan_build(const k3_st_model *model, uint32_t chunk_tokens,
                                      uint32_t context_remaining, uint16_t experts_per_layer,
                                      uint16_t staging_slots, k3_prefill_cache_lease lease,
                                      k3_prefill_plan *plan, char *error, size_t error_size) {
    return k3_prefill_plan_build_with_aux_workspace(model, chunk_tokens, context_remaining,
                                                    experts_per_layer, staging_slots, lease, 0,
                                                    plan, error, error_size);
}
