/*
 * C caller of libk3moe (test code): what an engine does through the C ABI
 * (include/k3_moe.h), with no Python. Builds the reduced routed-MoE layer
 * of BASELINE config 0 (H 2048, 64 experts, top-4, F 512, SwiGLU, scale
 * 2.5) in device memory, runs k3_moe_forward_bf16 for one token (decode
 * kernels) and for 8 tokens (grouped kernels), with the routes copied into
 * hipHostMalloc-mapped host memory as the reference engine reads them
 * (k3_engine.cu:623-640), and checks every output bit, id and weight
 * against the C oracle (oracle/k3moe_oracle.h). Then, as an engine's token
 * loop does: a decode token through a chain of layers enqueued back to
 * back on one stream (each layer's output is the next layer's input and
 * residual; routes on the device, one synchronisation at the end, no host
 * round trip between layers -- the sync at k3_engine.cu:1569 is not
 * needed), and the prefill router entry point (k3_moe_router_bf16) on a
 * 40-token batch. Exit status 0 = match.
 */
#include <hip/hip_runtime_api.h>

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/k3_moe.h"
#include "../../oracle/k3moe_oracle.h"

#define H 2048u
#define E 64u
#define K 4u
#define F 512u
#define SEED 4242u

#define CHECK(c)                                                              \
    do {                                                                      \
        if (!(c)) {                                                           \
            fprintf(stderr, "harness: %s failed at line %d\n", #c, __LINE__); \
            exit(1);                                                          \
        }                                                                     \
    } while (0)

static uint64_t rng_state = 0x9e3779b97f4a7c15ull;
static float uniform(void) { /* xorshift64*, [-1, 1) */
    rng_state ^= rng_state >> 12;
    rng_state ^= rng_state << 25;
    rng_state ^= rng_state >> 27;
    const uint64_t v = rng_state * 0x2545f4914f6cdd1dull;
    return (float)((v >> 40) * (1.0 / 8388608.0)) - 1.0f;
}

static uint16_t *bf16_array(size_t n, float scale) {
    uint16_t *a = malloc(2 * n);
    for (size_t i = 0; i < n; i++) a[i] = k3o_f32_to_bf16(uniform() * scale);
    return a;
}

static void *dev_copy(const void *host, size_t bytes) {
    void *d = NULL;
    CHECK(hipMalloc(&d, bytes) == hipSuccess);
    CHECK(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice) == hipSuccess);
    return d;
}

int main(void) {
    const size_t sizes[6] = {F * H / 2, F * H / 32, H * F / 2, H * F / 32, F * H / 2, F * H / 32};
    size_t span = 0, offs[6];
    for (int j = 0; j < 6; j++) {
        offs[j] = span;
        span += (sizes[j] + 255) & ~(size_t)255;
    }
    /* resident experts: device span per expert, filled by the library's
     * counter-based generator; the host copy for the oracle from the same
     * generator */
    uint8_t *store = NULL;
    CHECK(hipMalloc((void **)&store, span * E) == hipSuccess);
    k3_moe_expert table[E];
    k3o_expert host_table[E];
    uint8_t *host_store = malloc(span * E);
    for (uint32_t e = 0; e < E; e++) {
        const void *p[6];
        for (int j = 0; j < 6; j++) {
            uint8_t *d = store + e * span + offs[j];
            CHECK(k3_moe_synth_fill(d, sizes[j], SEED, e * 8u + (uint32_t)j, (uint32_t)(j & 1),
                                    NULL));
            k3_moe_synth_fill_host(host_store + e * span + offs[j], sizes[j], SEED,
                                   e * 8u + (uint32_t)j, (uint32_t)(j & 1));
            p[j] = d;
        }
        table[e] = (k3_moe_expert){p[0], p[1], p[2], p[3], p[4], p[5]};
        const uint8_t *h = host_store + e * span;
        host_table[e] = (k3o_expert){h + offs[0], h + offs[1], h + offs[2],
                                     h + offs[3], h + offs[4], h + offs[5]};
    }
    k3_moe_expert *d_table = dev_copy(table, sizeof table);

    const uint32_t tokens_max = 8u;
    uint16_t *router_w = bf16_array((size_t)E * H, 0.03f);
    float bias[E];
    for (uint32_t e = 0; e < E; e++) bias[e] = uniform() * 0.01f;
    uint16_t *x = bf16_array((size_t)tokens_max * H, 1.7f);
    uint16_t *res = bf16_array((size_t)tokens_max * H, 1.7f);
    void *d_w = dev_copy(router_w, 2 * (size_t)E * H), *d_b = dev_copy(bias, sizeof bias);
    void *d_x = dev_copy(x, 2 * (size_t)tokens_max * H);
    void *d_r = dev_copy(res, 2 * (size_t)tokens_max * H);
    void *d_out = NULL;
    CHECK(hipMalloc(&d_out, 2 * (size_t)tokens_max * H) == hipSuccess);

    const k3_moe_shape shape = {H, E, K, F, 2.5f, K3_MOE_ACT_SWIGLU, 1.0f, 1.0f};
    const size_t ws_bytes = k3_moe_workspace_bytes(&shape, tokens_max);
    CHECK(ws_bytes != 0);
    void *ws = NULL;
    CHECK(hipMalloc(&ws, ws_bytes) == hipSuccess);
    CHECK(k3_moe_workspace_init(ws, ws_bytes, NULL));
    uint32_t *ids_map = NULL;
    float *w_map = NULL;
    CHECK(hipHostMalloc((void **)&ids_map, 4 * tokens_max * K, hipHostMallocMapped) == hipSuccess);
    CHECK(hipHostMalloc((void **)&w_map, 4 * tokens_max * K, hipHostMallocMapped) == hipSuccess);
    void *d_ids = NULL, *d_wts = NULL;
    CHECK(hipHostGetDevicePointer(&d_ids, ids_map, 0) == hipSuccess);
    CHECK(hipHostGetDevicePointer(&d_wts, w_map, 0) == hipSuccess);

    const k3o_shape oshape = {H, E, K, F, 2.5f, 1u, 1.0f, 1.0f};
    int bad = 0;
    const uint32_t runs[2] = {1u, tokens_max};
    for (int run = 0; run < 2; run++) {
        const uint32_t T = runs[run];
        memset(ids_map, 0xff, 4 * T * K);
        CHECK(k3_moe_forward_bf16(d_out, d_x, d_r, d_w, d_b, d_table, &shape, T, K3_MOE_EXACT,
                                  d_ids, d_wts, ws, ws_bytes, NULL));
        CHECK(hipDeviceSynchronize() == hipSuccess);
        uint16_t *got = malloc(2 * (size_t)T * H), *want = malloc(2 * (size_t)T * H);
        uint32_t want_ids[tokens_max * K];
        float want_w[tokens_max * K];
        CHECK(hipMemcpy(got, d_out, 2 * (size_t)T * H, hipMemcpyDeviceToHost) == hipSuccess);
        CHECK(k3o_layer(&oshape, T, x, res, router_w, bias, host_table, NULL, NULL, NULL, 0, want,
                        want_ids, want_w, NULL, NULL, 0, 0) == 0);
        const int d_out_bits = memcmp(got, want, 2 * (size_t)T * H) != 0;
        const int d_ids_bits = memcmp(ids_map, want_ids, 4 * T * K) != 0;
        const int d_w_bits = memcmp(w_map, want_w, 4 * T * K) != 0;
        printf("harness: T=%u output %s, ids %s, weights %s\n", T, d_out_bits ? "DIFFER" : "match",
               d_ids_bits ? "DIFFER" : "match", d_w_bits ? "DIFFER" : "match");
        bad |= d_out_bits | d_ids_bits | d_w_bits;
        free(got);
        free(want);
    }

    /* a decode token through kLayers layers, no host sync in between */
    enum { kLayers = 4 };
    void *d_act[kLayers + 1];
    uint32_t *layer_ids = NULL;
    float *layer_w = NULL;
    CHECK(hipHostMalloc((void **)&layer_ids, 4 * kLayers * K, hipHostMallocMapped) == hipSuccess);
    CHECK(hipHostMalloc((void **)&layer_w, 4 * kLayers * K, hipHostMallocMapped) == hipSuccess);
    memset(layer_ids, 0xff, 4 * kLayers * K);
    d_act[0] = d_x;
    for (int l = 0; l < kLayers; l++) {
        CHECK(hipMalloc(&d_act[l + 1], 2 * (size_t)H) == hipSuccess);
        void *ids_dev = NULL, *w_dev = NULL;
        CHECK(hipHostGetDevicePointer(&ids_dev, layer_ids + l * K, 0) == hipSuccess);
        CHECK(hipHostGetDevicePointer(&w_dev, layer_w + l * K, 0) == hipSuccess);
        CHECK(k3_moe_forward_bf16(d_act[l + 1], d_act[l], d_act[l], d_w, d_b, d_table, &shape,
                                  1u, K3_MOE_EXACT, ids_dev, w_dev, ws, ws_bytes, NULL));
    }
    CHECK(hipDeviceSynchronize() == hipSuccess);
    {
        uint16_t cur[H], nxt[H], got[H];
        uint32_t want_ids[K];
        float want_w[K];
        memcpy(cur, x, sizeof cur);
        int chain_bad = 0;
        for (int l = 0; l < kLayers; l++) {
            CHECK(k3o_layer(&oshape, 1u, cur, cur, router_w, bias, host_table, NULL, NULL, NULL,
                            0, nxt, want_ids, want_w, NULL, NULL, 0, 0) == 0);
            chain_bad |= memcmp(layer_ids + l * K, want_ids, sizeof want_ids) != 0;
            chain_bad |= memcmp(layer_w + l * K, want_w, sizeof want_w) != 0;
            memcpy(cur, nxt, sizeof cur);
        }
        CHECK(hipMemcpy(got, d_act[kLayers], sizeof got, hipMemcpyDeviceToHost) == hipSuccess);
        chain_bad |= memcmp(got, cur, sizeof got) != 0;
        printf("harness: %d-layer decode chain (one stream, one sync) %s\n", kLayers,
               chain_bad ? "DIFFER" : "match");
        bad |= chain_bad;
    }
    for (int l = 1; l <= kLayers; l++) hipFree(d_act[l]);
    hipHostFree(layer_ids);
    hipHostFree(layer_w);

    /* the prefill router entry point on a token batch (the certified MFMA
     * form from 32 tokens on) against the oracle's logits and top-k */
    {
        const uint32_t T = 40u;
        uint16_t *xb = bf16_array((size_t)T * H, 1.3f);
        void *d_xb = dev_copy(xb, 2 * (size_t)T * H);
        const size_t rs = k3_moe_router_scratch_bytes(T, E);
        CHECK(rs != 0);
        void *d_scratch = NULL, *d_rids = NULL, *d_rw = NULL;
        CHECK(hipMalloc(&d_scratch, rs) == hipSuccess);
        CHECK(hipMalloc(&d_rids, 4 * T * K) == hipSuccess);
        CHECK(hipMalloc(&d_rw, 4 * T * K) == hipSuccess);
        CHECK(k3_moe_router_bf16(d_rids, d_rw, d_xb, d_w, d_b, T, E, H, K, 2.5f, d_scratch, rs,
                                 NULL));
        uint32_t got_ids[40 * K], want_ids[40 * K];
        float got_w[40 * K], want_w[40 * K];
        float *logits = malloc(4 * (size_t)T * E);
        CHECK(hipMemcpy(got_ids, d_rids, sizeof got_ids, hipMemcpyDeviceToHost) == hipSuccess);
        CHECK(hipMemcpy(got_w, d_rw, sizeof got_w, hipMemcpyDeviceToHost) == hipSuccess);
        k3o_router_logits(logits, router_w, xb, T, E, H, 1); /* the reference order */
        CHECK(k3o_router_topk(want_ids, want_w, logits, bias, T, E, K, 2.5f, 0) == 0);
        const int rb = memcmp(got_ids, want_ids, sizeof got_ids) != 0 ||
                       memcmp(got_w, want_w, sizeof got_w) != 0;
        printf("harness: router entry point, %u tokens: ids and weights %s\n", T,
               rb ? "DIFFER" : "match");
        bad |= rb;
        free(logits);
        free(xb);
        hipFree(d_xb);
        hipFree(d_scratch);
        hipFree(d_rids);
        hipFree(d_rw);
    }

    hipHostFree(ids_map);
    hipHostFree(w_map);
    hipFree(ws);
    hipFree(d_out);
    hipFree(d_x);
    hipFree(d_r);
    hipFree(d_w);
    hipFree(d_b);
    hipFree(d_table);
    hipFree(store);
    free(host_store);
    free(router_w);
    free(x);
    free(res);
    return bad;
}
