/*
 * C caller of libk3moe (test code): what an engine does through the C ABI
 * (include/k3_moe.h), with no Python. Builds the reduced routed-MoE layer
 * of BASELINE config 0 (H 2048, 64 experts, top-4, F 512, SwiGLU, scale
 * 2.5) in device memory, runs k3_moe_forward_bf16 for one token (decode
 * kernels) and for 8 tokens (grouped kernels), with the routes copied into
 * hipHostMalloc-mapped host memory as the reference engine reads them
 * (k3_engine.cu:623-640), and checks every output bit, id and weight
 * against the C oracle (oracle/k3moe_oracle.h). Exit status 0 = match.
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
