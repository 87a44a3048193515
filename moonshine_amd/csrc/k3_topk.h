/*
 * Router top-k selection by one wavefront.
 *
 * Semantics (k3_rocm_ops.cu:1361-1450): choice = sigmoid(logit) + bias,
 * with the sigmoid evaluated as the reference kernel evaluates it
 * (router_sigmoid, k3_device.h); experts are ordered by (choice desc, id
 * asc) -- the order of the reference's bitonic sort read from its end --
 * and the first top_k are returned in that order with weight_r = score_r /
 * (1e-20 + sum of the selected scores in rank order) * scale, where score
 * is the deterministic sigmoid det_sigmoid (callers pass keys and scores). NaN choices are never selected;
 * missing slots (fewer than top_k selectable experts) get id UINT32_MAX and
 * weight 0.
 *
 * Method (one wave, no block barrier, no atomics): choices are mapped to
 * order-preserving 32-bit keys (0 = not selectable). The top_k-th largest
 * per-lane maximum M is a lower bound on the top_k-th largest key (the
 * top_k lanes with the largest maxima hold top_k keys >= M), so only keys
 * >= M are ranked -- a few dozen for real router outputs. M is found by a
 * 32-step bitwise search over the lane maxima (one ballot per bit). The
 * candidates are compacted to one per lane (positions from a ballot-based
 * prefix sum of the per-lane counts) and ranked from registers with
 * readlane broadcasts, so the only LDS round trips are the compaction and
 * the hand-over of the selected routes to their rank lanes. More than 64
 * candidates (heavy ties) are ranked in 64-candidate passes from LDS.
 *
 * Lane l holds experts e = l + 64 j, j < kTopkSlots (E <= 1024).
 */
#pragma once

#include "k3_device.h"

namespace k3 {

constexpr int kTopkSlots = 16;

struct TopkWaveSmem {
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

/* Per-candidate hooks of topk_select_wave; the default does nothing.
 * candidate(id): called by each lane holding a candidate before ranking
 * (e.g. to start loads keyed by the id); selected(rank): called by that
 * lane when its candidate takes rank `rank` < top_k. */
struct TopkNoHooks {
    __device__ __forceinline__ void candidate(uint32_t) {}
    __device__ __forceinline__ void selected(uint32_t) {}
};

/* Rank of candidate (mk, mi) among the candidates held one per lane
 * (lanes without one hold key 0): the number ordered before it by (key
 * desc, id asc). */
__device__ __forceinline__ uint32_t topk_rank_lanes(uint32_t mk, uint32_t mi, uint32_t ncand) {
    uint32_t cnt = 0u;
    for (uint32_t i0 = 0; i0 < ncand; i0 += 8u) {
#pragma unroll
        for (uint32_t i = 0; i < 8u; i++) {
            const uint32_t ok = (uint32_t)__builtin_amdgcn_readlane((int)mk, (int)(i0 + i));
            const uint32_t oi = (uint32_t)__builtin_amdgcn_readlane((int)mi, (int)(i0 + i));
            cnt += (ok > mk || (ok == mk && oi < mi)) ? 1u : 0u;
        }
    }
    return cnt;
}

template <class Hooks>
__device__ __forceinline__ uint32_t topk_rank_write(uint32_t ncand, uint32_t top_k, float scale,
                                                    uint32_t *ids, float *weights,
                                                    uint32_t *ids_copy, float *w_copy,
                                                    TopkWaveSmem &sm, Hooks &&hooks);

/* key[j]/score[j] for expert lane + 64 j. Writes ids/weights[0..top_k) (and
 * the optional copies, which may be host-mapped). Must be called by all 64
 * lanes of the wave; 1 <= top_k <= 32. Returns the rank-`lane` id to lanes
 * < top_k (UINT32_MAX elsewhere). */
template <class Hooks = TopkNoHooks>
__device__ __forceinline__ uint32_t topk_select_wave(const uint32_t (&key)[kTopkSlots],
                                                     const float (&score)[kTopkSlots],
                                                     uint32_t top_k, float scale, uint32_t *ids,
                                                     float *weights, uint32_t *ids_copy,
                                                     float *w_copy, TopkWaveSmem &sm,
                                                     Hooks &&hooks = Hooks{}) {
    const uint32_t lane = threadIdx.x & 63u;
    const unsigned long long below = (1ull << lane) - 1ull;
    /* threshold: the largest M with at least top_k lane maxima >= M, i.e.
     * the top_k-th largest lane maximum */
    uint32_t lmax = 0u;
#pragma unroll
    for (int j = 0; j < kTopkSlots; j++) lmax = key[j] > lmax ? key[j] : lmax;
    uint32_t thr = 0u;
#pragma unroll
    for (int b = 31; b >= 0; b--) {
        const uint32_t t = thr | (1u << b);
        if ((uint32_t)__popcll(__ballot(lmax >= t)) >= top_k) thr = t;
    }
    if (thr == 0u) thr = 1u; /* key 0 = not selectable */
    /* candidate positions: exclusive prefix sum of the per-lane counts */
    uint32_t mine = 0u;
#pragma unroll
    for (int j = 0; j < kTopkSlots; j++) mine += key[j] >= thr ? 1u : 0u;
    uint32_t pos = 0u, ncand = 0u;
#pragma unroll
    for (int b = 0; b < 5; b++) { /* mine <= 16 */
        const unsigned long long m = __ballot((mine >> b) & 1u);
        pos += (uint32_t)__popcll(m & below) << b;
        ncand += (uint32_t)__popcll(m) << b;
    }
#pragma unroll
    for (int j = 0; j < kTopkSlots; j++) {
        if (key[j] >= thr) {
            sm.cand_key[pos] = key[j];
            sm.cand_id[pos] = lane + 64u * j;
            sm.cand_score[pos] = score[j];
            pos++;
        }
    }
    wave_fence();
    return topk_rank_write(ncand, top_k, scale, ids, weights, ids_copy, w_copy, sm, hooks);
}

/* Second half of topk_select_wave: ranks the ncand candidates in
 * sm.cand_key / cand_id / cand_score (keys >= 1) by (key desc, id asc) and
 * writes the first top_k as topk_select_wave does. Must be called by all
 * 64 lanes after the candidates' LDS writes have completed. */
template <class Hooks>
__device__ __forceinline__ uint32_t topk_rank_write(uint32_t ncand, uint32_t top_k, float scale,
                                                    uint32_t *ids, float *weights,
                                                    uint32_t *ids_copy, float *w_copy,
                                                    TopkWaveSmem &sm, Hooks &&hooks) {
    const uint32_t lane = threadIdx.x & 63u;
    if (ncand <= 64u) {
        const bool live = lane < ncand;
        const uint32_t mk = live ? sm.cand_key[lane] : 0u, mi = live ? sm.cand_id[lane] : 0u;
        if (live) hooks.candidate(mi);
        const uint32_t cnt = topk_rank_lanes(mk, mi, ncand);
        if (live && cnt < top_k) {
            sm.out_id[cnt] = mi;
            sm.out_score[cnt] = sm.cand_score[lane];
            hooks.selected(cnt);
        }
    } else {
        /* rank = number of candidates ordered before (key desc, id asc); a
         * candidate stops counting once it cannot be selected */
        for (uint32_t base = 0; base < ncand; base += 64u) {
            const uint32_t c = base + lane;
            const bool live = c < ncand;
            const uint32_t mk = live ? sm.cand_key[c] : 0u, mi = live ? sm.cand_id[c] : 0u;
            if (live) hooks.candidate(mi);
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
                hooks.selected(cnt);
            }
        }
    }
    wave_fence();
    const uint32_t nsel = ncand < top_k ? ncand : top_k;
    /* lane r holds the rank-r score; the denominator adds them in rank
     * order (1e-20 first). Ranks >= nsel hold +0, which leaves the sum
     * unchanged, so the chain runs over a fixed 16 or 32 lanes. */
    const float my_score = lane < nsel ? sm.out_score[lane] : 0.0f;
    float sv[32];
#pragma unroll
    for (int q = 0; q < 32; q++)
        sv[q] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                              __builtin_bit_cast(int, my_score), q));
    float den = 1e-20f;
#pragma unroll
    for (int q = 0; q < 16; q++) den = __fadd_rn(den, sv[q]);
    if (top_k > 16u) {
#pragma unroll
        for (int q = 16; q < 32; q++) den = __fadd_rn(den, sv[q]);
    }
    uint32_t id = UINT32_MAX;
    if (lane < top_k) {
        id = lane < nsel ? sm.out_id[lane] : UINT32_MAX;
        const float wr = __fmul_rn(__fdiv_rn(my_score, den), scale);
        ids[lane] = id;
        weights[lane] = wr;
        if (ids_copy) ids_copy[lane] = id;
        if (w_copy) w_copy[lane] = wr;
    }
    return id;
}

/* One token's router outputs for the top-k: per expert row, the logit
 * (bf16 weight row . bf16 x in the reference's order, ref_chunk /
 * ref_logit_finish), the score det_sigmoid(logit) and the order key
 * choice_key(router_sigmoid(logit), bias) (k3_rocm_ops.cu:1361-1450). */
struct RouterRows {
    const uint16_t *weight; /* [rows, cols] bf16 */
    const float *bias;      /* [rows] */
    const uint16_t *x;      /* [cols] bf16, 16-byte aligned */
    float *logits, *scores;
    uint32_t *keys;
    uint32_t rows, cols;    /* cols % 8 == 0, cols <= 8192 */
};

constexpr int kRouterMaxChunks = 16; /* cols <= 8192 */

/* Rows row0 .. row0 + N - 1 (those below R.rows) on one wave. Every weight
 * chunk and the hidden state are loaded in one batch (one memory round
 * trip), and x is read once for the N rows. */
template <int N>
__device__ __forceinline__ void router_rows_wave(const RouterRows &R, uint32_t row0) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t chunks = R.cols / 8u;
    const uint4 *x4 = (const uint4 *)R.x;
    const uint4 *w[N];
#pragma unroll
    for (int r = 0; r < N; r++) /* rows past the end reread row0 (not stored) */
        w[r] = (const uint4 *)(R.weight + (uint64_t)(row0 + r < R.rows ? row0 + r : row0) * R.cols);
    uint4 wv[N][kRouterMaxChunks], xv[kRouterMaxChunks];
#pragma unroll
    for (int j = 0; j < kRouterMaxChunks; j++) {
        /* out-of-range chunks load chunk 0 and are skipped below */
        const uint32_t c = lane + 64u * j < chunks ? lane + 64u * j : 0u;
#pragma unroll
        for (int r = 0; r < N; r++) wv[r][j] = gload_nt(w[r] + c);
        xv[j] = x4[c];
    }
    float acc[N][4];
#pragma unroll
    for (int r = 0; r < N; r++) acc[r][0] = acc[r][1] = acc[r][2] = acc[r][3] = 0.0f;
#pragma unroll
    for (int j = 0; j < kRouterMaxChunks; j++) {
        if (lane + 64u * j < chunks) {
#pragma unroll
            for (int r = 0; r < N; r++) ref_chunk(acc[r], j, wv[r][j], xv[j]);
        }
    }
    float v = 0.0f;
#pragma unroll
    for (int r = 0; r < N; r++) {
        const float l = ref_logit_finish(acc[r]);
        if (lane == (uint32_t)r) v = l;
    }
    const uint32_t row = row0 + lane;
    if (lane < (uint32_t)N && row < R.rows) {
        R.logits[row] = v;
        R.scores[row] = det_sigmoid(v);
        R.keys[row] = choice_key(router_sigmoid(v), R.bias[row]);
    }
}

}  // namespace k3
