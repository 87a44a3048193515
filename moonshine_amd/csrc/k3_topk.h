/*
 * Router top-k selection by one wavefront.
 *
 * Semantics (k3_rocm_ops.cu:1361-1450): score = sigmoid(logit), choice =
 * score + bias; experts are ordered by (choice desc, id asc) -- the order of
 * the reference's bitonic sort read from its end -- and the first top_k are
 * returned in that order with weight_r = score_r / (1e-20 + sum of the
 * selected scores in rank order) * scale. NaN choices are never selected;
 * missing slots (fewer than top_k selectable experts) get id UINT32_MAX and
 * weight 0.
 *
 * Method: choices are mapped to order-preserving 32-bit keys (0 = not
 * selectable). The top_k-th largest per-lane maximum is a lower bound on
 * the top_k-th largest key, so only keys at or above it (a few dozen for
 * real router outputs) are ranked, by counting with early exit. This is
 * wave-synchronous (no block barrier) and free of LDS atomics; a radix
 * histogram serialised on atomics because one token's keys cluster in a
 * few high-order bins, and a bitwise ballot search paid a VALU-to-scalar
 * round trip per count.
 *
 * Lane l holds experts e = l + 64 j, j < kTopkSlots (E <= 1024).
 */
#pragma once

#include "k3_device.h"

namespace k3 {

constexpr int kTopkSlots = 16;

struct TopkWaveSmem {
    uint32_t lmax[64];
    uint32_t cand_key[1024];
    uint32_t cand_id[1024];
    float cand_score[1024];
    uint32_t out_id[32];
    float out_score[32];
};

__device__ __forceinline__ uint32_t choice_key(float score, float bias) {
    float c = __fadd_rn(score, bias);
    if (c != c) return 0u;
    if (c == 0.0f) c = 0.0f; /* -0 and +0 compare equal */
    const uint32_t u = __float_as_uint(c);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* Orders this wave's LDS accesses (waits for them to complete). */
__device__ __forceinline__ void wave_fence() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
}

/* key[j]/score[j] for expert lane + 64 j. Writes ids/weights[0..top_k) (and
 * the optional copies, which may be host-mapped). Must be called by all 64
 * lanes of the wave; top_k <= 32. With `publish`, ids/weights are written
 * with write-through agent-scope stores (for readers in the same kernel).
 * Returns the rank-`lane` id to lanes < top_k (UINT32_MAX elsewhere). */
__device__ __forceinline__ uint32_t topk_select_wave(const uint32_t (&key)[kTopkSlots],
                                                 const float (&score)[kTopkSlots],
                                                 uint32_t top_k, float scale, uint32_t *ids,
                                                 float *weights, uint32_t *ids_copy,
                                                 float *w_copy, TopkWaveSmem &sm,
                                                 bool publish = false) {
    const uint32_t lane = threadIdx.x & 63u;
    const unsigned long long below = (1ull << lane) - 1ull;
    /* Threshold: the top_k-th largest lane maximum M. The top_k lanes with
     * the largest maxima hold top_k keys >= M, so every key of the true
     * top_k is >= M: only keys >= M need ranking. */
    uint32_t lmax = 0u;
#pragma unroll
    for (int j = 0; j < kTopkSlots; j++) lmax = key[j] > lmax ? key[j] : lmax;
    sm.lmax[lane] = lmax;
    wave_fence();
    uint32_t r = 0u;
#pragma unroll
    for (uint32_t i = 0; i < 64u; i++) {
        const uint32_t v = sm.lmax[i];
        r += (v > lmax || (v == lmax && i < lane)) ? 1u : 0u;
    }
    const unsigned long long pm = __ballot(r == top_k - 1u);
    uint32_t thr = (uint32_t)__shfl((int)lmax, pm ? __ffsll((long long)pm) - 1 : 0, 64);
    if (thr == 0u) thr = 1u; /* key 0 = not selectable */
    /* candidates in id order (j asc, lane asc) */
    uint32_t ncand = 0u;
#pragma unroll
    for (int j = 0; j < kTopkSlots; j++) {
        const bool take = key[j] >= thr;
        const unsigned long long m = __ballot(take);
        if (take) {
            const uint32_t pos = ncand + (uint32_t)__popcll(m & below);
            sm.cand_key[pos] = key[j];
            sm.cand_id[pos] = lane + 64u * j;
            sm.cand_score[pos] = score[j];
        }
        ncand += (uint32_t)__popcll(m);
    }
    wave_fence();
    /* rank = number of candidates ordered before (key desc, id asc); a
     * candidate stops counting once it cannot be selected */
    for (uint32_t base = 0; base < ncand; base += 64u) {
        const uint32_t c = base + lane;
        const bool live = c < ncand;
        const uint32_t mk = live ? sm.cand_key[c] : 0u, mi = live ? sm.cand_id[c] : 0u;
        uint32_t cnt = live ? 0u : top_k;
        for (uint32_t i0 = 0; i0 < ncand; i0 += 16u) {
#pragma unroll
            for (uint32_t i = i0; i < i0 + 16u; i++) {
                const uint32_t ok = i < ncand ? sm.cand_key[i] : 0u;
                const uint32_t oi = sm.cand_id[i < ncand ? i : 0u];
                cnt += (i < ncand && (ok > mk || (ok == mk && oi < mi))) ? 1u : 0u;
            }
            if (__ballot(cnt < top_k) == 0ull) break;
        }
        if (cnt < top_k) {
            sm.out_id[cnt] = mi;
            sm.out_score[cnt] = sm.cand_score[c];
        }
    }
    wave_fence();
    const uint32_t nsel = ncand < top_k ? ncand : top_k;
    /* lane r holds the rank-r score; the denominator adds them in rank
     * order (a sequential chain over lane reads) */
    const float my_score = lane < nsel ? sm.out_score[lane] : 0.0f;
    float den = 1e-20f;
    for (uint32_t q = 0; q < top_k; q++)
        den = __fadd_rn(den, __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                 __builtin_bit_cast(int, my_score), (int)q)));
    uint32_t id = UINT32_MAX;
    if (lane < top_k) {
        id = lane < nsel ? sm.out_id[lane] : UINT32_MAX;
        const float wr = __fmul_rn(__fdiv_rn(my_score, den), scale);
        if (publish) {
            __hip_atomic_store(ids + lane, id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(weights + lane, wr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            ids[lane] = id;
            weights[lane] = wr;
        }
        if (ids_copy) ids_copy[lane] = id;
        if (w_copy) w_copy[lane] = wr;
    }
    return id;
}

}  // namespace k3
