/*
 * Certified MFMA router for token batches (prefill). The routes and weights
 * are those of the exact router -- logits in the reference's own order
 * (ref_quad / ref_chunk: k3_bf16_gemv_kernel<float> and the tiled GEMM,
 * k3_rocm_ops.cu:359-425, 512-661) followed by router_topk_kernel (k3_rocm_ops.cu:1361-1450) -- bit
 * for bit, while the logit GEMM runs on bf16 MFMA:
 *
 *   router_norms_kernel    n_e >= ||w_e|| for every router row
 *   router_mfma_kernel     approximate logits a_te = x_t . w_e (bf16 MFMA,
 *                          fp32 accumulate, any summation order; with few
 *                          tiles, K is split over blocks and
 *                          router_slices_sum_kernel adds the slices)
 *   router_certify_kernel  one block per token: candidates from the
 *                          approximate logits and a rigorous error bound,
 *                          exact reference-order logits for the candidates only,
 *                          then the exact router's top-k on exact keys
 *   router_certify_wave_kernel  the same with one wave per token, for
 *                          batches of 1024 tokens and more
 *
 * Why the routes are exact. Let p_i = w_i x_i (exact in fp32: bf16 x bf16
 * products have 16 significant bits), u = 2^-24. Each MFMA instruction sums
 * a fresh block of 32 products (its C operand is zero); whatever order and
 * rounding the unit uses inside, its result is taken to be within 4 u per
 * term, 128 u sum|p_block|, of the block's real sum (a truncating or
 * block-aligned adder of fp32 width stays within 2 u per term; the worst
 * case measured over adversarial blocks is 8 u sum|p_block|). The H / 32
 * block results are added in fp32 (H / 32 - 1 roundings in any order),
 * and in the exact reference-order sum a product passes at most 3
 * roundings inside its quad, H / 1024 partial adds and an 8-level tree
 * (fewer than the 128 + 6 the bound has room for up to H = 131072). The kernel uses err_e = (H / 32 + 270) u (1 + 2^-10)
 * n_e ||x_t||, which covers both sums' errors together, since sum|p_i| <=
 * ||w_e|| ||x_t|| (Cauchy-Schwarz).
 *
 * The choice is sigmoid(l) + bias. The real sigmoid's slope on [a - err,
 * a + err] is at most s'(max(0, |a| - err)) (the slope falls away from 0),
 * the router sigmoid (router_sigmoid, the hardware exp2/reciprocal sequence)
 * is within 3e-7 of the real one and the bias add rounds once, so the
 * approximate and exact choices differ by at most ce_e = s'(..) err_e + 2e-6
 * + 2^-21 |c_e|, with s'(m) bounded from above by sigmoid_slope_bound.
 * If T_k is the k-th largest approximate choice and E_k the largest ce
 * among the experts at or above it, those k experts have exact choices >=
 * T_k - E_k, so every expert of the exact top-k (ties included) has
 * approximate choice + ce_e >= T_k - E_k. Those are the candidates; every
 * other expert gets key 0 (never selected) and the candidates get their
 * exact keys, so the selection returns what it returns on all exact keys.
 * A token with any non-finite input, approximate logit, norm or bias, or
 * an error bound above 1e30, takes every expert as a candidate (the exact
 * router on that token).
 */
#include "k3_decode.h"
#include "k3_device.h"
#include "k3_internal.h"
#include "k3_lds.h"
#include "k3_topk.h"

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

namespace k3 {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

/* inflation that makes a computed fp32 norm an upper bound of the real one
 * (chains of <= 134 roundings: relative error < 2^-16) */
constexpr float kNormInflate = 1.0f + 1.0f / 4096.0f;

/* ---------------------------------------------------------------------- */
/* row norms                                                               */
/* ---------------------------------------------------------------------- */

/* One wave per router row: n_e = sqrt(sum w^2) * kNormInflate. */
__global__ __launch_bounds__(256) void router_norms_kernel(float *__restrict__ norms,
                                                           const uint16_t *__restrict__ w,
                                                           uint32_t E, uint32_t H) {
    const uint32_t lane = threadIdx.x & 63u, e = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (e >= E) return;
    const uint4 *row = (const uint4 *)(w + (uint64_t)e * H);
    float s = 0.0f;
    for (uint32_t c = lane; c < H / 8u; c += 64u) {
        const uint4 v = row[c];
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            s = fmaf(bf16_lo(u[q]), bf16_lo(u[q]), s);
            s = fmaf(bf16_hi(u[q]), bf16_hi(u[q]), s);
        }
    }
    s = wave_sum(s);
    if (lane == 0u) norms[e] = __fmul_rn(__fsqrt_rn(s), kNormInflate);
}

/* ---------------------------------------------------------------------- */
/* approximate logits on MFMA                                              */
/* ---------------------------------------------------------------------- */

/*
 * out[t, e] ~= x_t . w_e, summed as described above (C = 0 MFMAs, fp32
 * adds of the 32-product blocks). Block tile 128 tokens x 128 experts, 8
 * waves of 32 x 64 (2 x 4 V_MFMA_F32_16X16X32_BF16 tiles), two blocks per
 * CU, K steps of 64 (one 128-byte line per row) staged by direct-to-LDS
 * loads in two buffers: 16 KB of token rows and 16 KB of expert rows per
 * step, eight whole lines per 1 KB chunk with the XOR swizzle of a_slot,
 * so the 16 lanes of each fragment read pass fall on 16 different 16-byte
 * bank groups. Lane l = 16 g + c supplies row c of a fragment with the 8
 * bf16 at K offset 8 g (A: tokens, B: experts; the same K assignment on
 * both operands, which is all a dot product needs); it receives tokens 4 g
 * .. 4 g + 3 of expert column c. Rows past T or E load the last valid row
 * and are not stored. Tiles are dealt to the XCDs in contiguous ranges, a
 * token tile's expert tiles together, so one XCD's L2 serves a token tile
 * to all of its expert tiles. Measured at cfg4 (8192 x 896 x 7168): 0.15
 * ms; staging through registers ran at ~16 bytes per clock per CU (0.23
 * ms), and 128 x 224 tiles with three buffers and one block per CU (one
 * tile per CU) at 0.17 ms.
 */
constexpr uint32_t kRT = 128, kRK = 64;
constexpr uint32_t kRStage = 2u * kRT * 128u; /* [token rows | expert rows] */

/* Step loads of one wave into `stage`: chunks wave and wave + 8 of each
 * region (chunk q holds rows 16 (q / 2) + 8 (q % 2) + lane / 8); src[] are
 * the lane's byte offsets (token rows, then expert rows), kb the step's K
 * byte offset. */
__device__ __forceinline__ void rt_issue(uint8_t *stage, const uint8_t *xb, const uint8_t *wb,
                                         const uint32_t (&src)[4], uint32_t kb, uint32_t wave) {
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const uint32_t q = wave + 8u * (uint32_t)u;
        dma<16>(xb + src[u] + kb, stage + 1024u * q);
        dma<16>(wb + src[2 + u] + kb, stage + kRT * 128u + 1024u * q);
    }
}

/* 8 waves: wave w covers tokens 32 (w / 2) .. + 32 and experts 64 (w % 2)
 * .. + 64 of the block's 128 x 128 tile. */
__global__ __launch_bounds__(512, 4) void router_mfma_kernel(float *__restrict__ out,
                                                             const uint16_t *__restrict__ x,
                                                             const uint16_t *__restrict__ w,
                                                             uint32_t T, uint32_t E, uint32_t H,
                                                             uint32_t S) {
    __shared__ __attribute__((aligned(16))) uint8_t st0[kRStage], st1[kRStage];
    const uint32_t ntt = (T + kRT - 1u) / kRT, net = (E + kRT - 1u) / kRT;
    const uint32_t works = ntt * net * S, per = (works + 7u) / 8u;
    const uint32_t L = blockIdx.x, j8 = L >> 3, wk0 = (L & 7u) * per + j8;
    if (j8 >= per || wk0 >= works) return;
    /* work = (tile, K slice), the slices of a tile together */
    const uint32_t slice = wk0 % S, wk = wk0 / S;
    const uint32_t t0 = (wk / net) * kRT, e0 = (wk % net) * kRT;
    out += (uint64_t)slice * T * E;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1u, g = lane >> 4, c = lane & 15u;
    /* the lane's source byte offsets: chunk q = wave + 8 u holds rows 16 (q
     * / 2) + a_dma_row(lane, q % 2), piece a_dma_piece(lane, q % 2); rows
     * past T or E clamp to the last one (their results are not stored) */
    uint32_t src[4];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const uint32_t q = wave + 8u * (uint32_t)u, h = q & 1u;
        const uint32_t r = 16u * (q >> 1) + a_dma_row(lane, h), pc = a_dma_piece(lane, h);
        const uint32_t ta = t0 + r, eb = e0 + r;
        src[u] = ((ta < T ? ta : T - 1u) * H + 8u * pc) * 2u;
        src[2 + u] = ((eb < E ? eb : E - 1u) * H + 8u * pc) * 2u;
    }
    const uint8_t *xb = (const uint8_t *)x, *wb = (const uint8_t *)w;
    f32x4_t acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    /* this slice's K steps [s0, s0 + nsteps) */
    const uint32_t ksteps = H / kRK;
    const uint32_t s0 = ksteps * slice / S, nsteps = ksteps * (slice + 1u) / S - s0;
    xb += 2u * kRK * s0;
    wb += 2u * kRK * s0;
    /* fragment addresses: A rows 32 wm + 16 i + c, B rows 64 wn + 16 j + c
     * (chunk pair = 16 rows = 2 KB) */
    auto step = [&](const uint8_t *cur) __attribute__((always_inline)) {
        const uint32_t base = lds_addr(cur);
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            const uint32_t a0 = base + 2048u * (2u * wm) + a_slot(c, 4u * (uint32_t)ks + g);
            const uint32_t b0 = base + kRT * 128u + 2048u * (4u * wn) + a_slot(c, 4u * (uint32_t)ks + g);
            u32x4_t af[2], bf[4];
            af[0] = ds_read16<0>(a0);
            af[1] = ds_read16<2048>(a0);
            bf[0] = ds_read16<0>(b0);
            bf[1] = ds_read16<2048>(b0);
            bf[2] = ds_read16<4096>(b0);
            bf[3] = ds_read16<6144>(b0);
            wait_lgkm<0>();
#pragma unroll
            for (int i = 0; i < 2; i++) after_wait(af[i]);
#pragma unroll
            for (int j = 0; j < 4; j++) after_wait(bf[j]);
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    /* a fresh 32-term dot product per instruction (C = 0),
                     * accumulated with one fp32 add per K block */
                    const f32x4_t d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8_t, af[i]), __builtin_bit_cast(bf16x8_t, bf[j]),
                        f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[i][j][r] = __fadd_rn(acc[i][j][r], d[r]);
                }
        }
    };
    /* step s: wait for this wave's loads of s, barrier (all of s landed;
     * every wave is done with the other buffer), issue s + 1 into it,
     * compute s */
    rt_issue(st0, xb, wb, src, 0u, wave);
    for (uint32_t s = 0; s < nsteps; s += 2u) {
        wait_vm<0>();
        __builtin_amdgcn_s_barrier();
        if (s + 1u < nsteps) rt_issue(st1, xb, wb, src, 2u * kRK * (s + 1u), wave);
        step(st0);
        if (s + 1u >= nsteps) break;
        wait_vm<0>();
        __builtin_amdgcn_s_barrier();
        if (s + 2u < nsteps) rt_issue(st0, xb, wb, src, 2u * kRK * (s + 2u), wave);
        step(st1);
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t e = e0 + 64u * wn + 16u * (uint32_t)j + c;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t t = t0 + 32u * wm + 16u * (uint32_t)i + 4u * g + (uint32_t)r;
                if (t < T && e < E) out[(uint64_t)t * E + e] = acc[i][j][r];
            }
        }
}

/* ---------------------------------------------------------------------- */
/* certification and selection                                             */
/* ---------------------------------------------------------------------- */

struct CertArgs {
    uint32_t *ids;
    float *weights;
    uint32_t *ids2;
    float *w2;
    const float *approx;
    const float *norms;
    const float *bias;
    const uint16_t *x;
    const uint16_t *w;
    uint32_t T, E, H, k;
    float scale, err_coef;
};

/* approx[i] = sum of the S K-slice partials approx[q n + i] (fp32 adds,
 * which the error bound counts like the adds inside a slice). */
__global__ __launch_bounds__(256) void router_slices_sum_kernel(float *__restrict__ approx,
                                                                uint32_t S, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * 256u) {
        float v[kRouterMaxSlices];
#pragma unroll
        for (uint32_t q = 0; q < kRouterMaxSlices; q++) v[q] = q < S ? approx[q * n + i] : 0.0f;
        float a = v[0];
#pragma unroll
        for (uint32_t q = 1; q < kRouterMaxSlices; q++)
            if (q < S) a = __fadd_rn(a, v[q]);
        approx[i] = a;
    }
}

/* Sum over the wave of a per-lane count < 32. */
__device__ __forceinline__ uint32_t wave_count(uint32_t v) {
    uint32_t n = 0u;
#pragma unroll
    for (int b = 0; b < 5; b++) n += (uint32_t)__popcll(__ballot((v >> b) & 1u)) << b;
    return n;
}

/* The float whose choice_key is `key` (key != 0). */
__device__ __forceinline__ float key_value(uint32_t key) {
    return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

constexpr uint32_t kNanBits = 0x7fc00000u;

/* batches of at least this many tokens certify with one wave per token
 * (cfg4, 8192 tokens: 365 -> 191 us; at 64 and 512 tokens the block per
 * token is faster: 34 vs 41 us, 39 vs 43 us) */
constexpr uint32_t kCertWaveMinTokens = 1024;

/* Slope bound of the real sigmoid at m >= 0: s(m) (1 - s(m)) = e / (1 +
 * e)^2 with e = exp(-m), formed from e with the hardware exp2 and
 * reciprocal (each within 1 ulp) and products only, so every step is
 * accurate to a small relative error (the argument's rounding moves 2^t
 * by < 2^-16 relative for m < 88) and 1 - s never cancels; the factor 1 +
 * 2^-10 covers all of it. 0 for m >= 88 (the real slope is below 2^-126
 * there; callers take tokens with err > 1e30 down the exact path). */
__device__ __forceinline__ float sigmoid_slope_bound(float m) {
    const float e = __builtin_amdgcn_exp2f(__fmul_rn(fminf(m, 88.0f), -1.44269502162933349609375f));
    const float r = __builtin_amdgcn_rcpf(__fadd_rn(1.0f, e));
    return __fmul_rn(__fmul_rn(__fmul_rn(e, r), r), 1.0f + 1.0f / 1024.0f);
}

/* The k-th largest (with multiplicity) of the wave's keys, key[j] of lane l
 * for expert l + 64 j; 0 when fewer than k keys are nonzero. The k-th
 * largest lane maximum M is a lower bound (the k lanes with the largest
 * maxima hold k keys >= M), so only the keys >= M -- a few dozen -- are
 * ranked, one per lane from `scratch` (64 words); more than 64 of them
 * (heavy ties) take a 32-step bitwise search over every key. */
__device__ __forceinline__ uint32_t kth_largest_key(const uint32_t (&key)[kTopkSlots], uint32_t k,
                                                    uint32_t *scratch) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t lmax = 0u;
#pragma unroll
    for (int j = 0; j < kTopkSlots; j++) lmax = key[j] > lmax ? key[j] : lmax;
    uint32_t m = 0u;
#pragma unroll
    for (int b = 31; b >= 0; b--) {
        const uint32_t t = m | (1u << b);
        if ((uint32_t)__popcll(__ballot(lmax >= t)) >= k) m = t;
    }
    uint32_t mine = 0u;
#pragma unroll
    for (int j = 0; j < kTopkSlots; j++) mine += (m != 0u && key[j] >= m) ? 1u : 0u;
    const uint32_t total = wave_count(mine);
    if (m != 0u && total <= 64u) {
        const unsigned long long below = (1ull << lane) - 1ull;
        uint32_t pos = 0u;
#pragma unroll
        for (int b = 0; b < 5; b++)
            pos += (uint32_t)__popcll(__ballot((mine >> b) & 1u) & below) << b;
#pragma unroll
        for (int j = 0; j < kTopkSlots; j++)
            if (key[j] >= m) scratch[pos++] = key[j];
        wave_fence();
        const uint32_t ck = lane < total ? scratch[lane] : 0u;
        uint32_t gt = 0u, ge = 0u;
        for (uint32_t i = 0; i < total; i++) {
            const uint32_t o = (uint32_t)__builtin_amdgcn_readlane((int)ck, (int)i);
            gt += o > ck ? 1u : 0u;
            ge += o >= ck ? 1u : 0u;
        }
        wave_fence(); /* scratch is reused by the caller */
        const unsigned long long hit = __ballot(lane < total && gt < k && k <= ge);
        return (uint32_t)__builtin_amdgcn_readlane((int)ck, (int)(__ffsll((long long)hit) - 1));
    }
    uint32_t thr = 0u;
    for (int b = 31; b >= 0; b--) {
        const uint32_t tt = thr | (1u << b);
        uint32_t cnt = 0u;
#pragma unroll
        for (int j = 0; j < kTopkSlots; j++) cnt += key[j] >= tt ? 1u : 0u;
        if (wave_count(cnt) >= k) thr = tt;
    }
    return thr;
}

/* The selection of both certification kernels, by one wave: the ncand
 * candidates in sm.cand_id / cand_score (bias) / cand_key (exact logit
 * bits) get their exact keys (router_sigmoid + bias) and weight scores
 * (det_sigmoid), are compacted to keys != 0 (a NaN choice is never
 * selected) and ranked by topk_rank_write: the exact router's top-k over
 * keys that are 0 off the candidate list. */
__device__ __forceinline__ void certify_select(const CertArgs &A, uint32_t t, uint32_t ncand,
                                               TopkWaveSmem &sm) {
    const uint32_t lane = threadIdx.x & 63u;
    const unsigned long long below = (1ull << lane) - 1ull;
    uint32_t nlive = 0u;
    for (uint32_t base = 0; base < ncand; base += 64u) {
        const uint32_t p = base + lane;
        const bool live = p < ncand;
        const float l = live ? __uint_as_float(sm.cand_key[p]) : 0.0f;
        const uint32_t e = live ? sm.cand_id[p] : 0u;
        const float b = live ? sm.cand_score[p] : 0.0f;
        const uint32_t kk = live ? choice_key(router_sigmoid(l), b) : 0u;
        const float sc = det_sigmoid(l);
        const unsigned long long okm = __ballot(kk != 0u);
        const uint32_t q = nlive + (uint32_t)__popcll(okm & below);
        if (kk != 0u) {
            sm.cand_key[q] = kk;
            sm.cand_id[q] = e;
            sm.cand_score[q] = sc;
        }
        nlive += (uint32_t)__popcll(okm);
    }
    wave_fence();
    const uint64_t o = (uint64_t)t * A.k;
    topk_rank_write(nlive, A.k, A.scale, A.ids + o, A.weights + o, A.ids2 ? A.ids2 + o : nullptr,
                    A.w2 ? A.w2 + o : nullptr, sm, TopkNoHooks{});
}

/* Scratch of one certify block (one token). The candidates live in
 * topk.cand_id (ids), cand_score (biases until the selection) and cand_key
 * (exact logit bits until the selection), in candidate order. */
struct CertSmem {
    uint4 x[64 * kTopkSlots]; /* the token's row, 8-element chunks */
    uint32_t ncand;
    TopkWaveSmem topk;
};

/*
 * One block of 4 waves per token. Wave 0 derives the candidate list from
 * the approximate logits; then every wave computes the exact reference-order
 * logits of candidates wave, wave + 4, ... (lane l takes x chunks l, l +
 * 64, ... -- the chunks it owns in that order -- from the block's copy of
 * the row in LDS, and the next candidate row's loads are issued before the
 * current row's FMAs, so two rows are in flight); wave 0 turns them into
 * keys and ranks them (certify_select; every other expert has key 0).
 * Used for batches below kCertWaveMinTokens.
 */
__global__ __launch_bounds__(256, 3) void router_certify_kernel(CertArgs A) {
    __shared__ CertSmem sm;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t t = blockIdx.x;
    const uint32_t E = A.E, H = A.H, chunks = H / 8u;
    const uint4 *xr = (const uint4 *)(A.x + (uint64_t)t * H);
    for (uint32_t c = threadIdx.x; c < chunks; c += 256u) sm.x[c] = xr[c];
    __syncthreads();
    if (wave == 0u) {
        float la[kTopkSlots], nb[kTopkSlots], bs[kTopkSlots];
        const float *ar = A.approx + (uint64_t)t * E;
#pragma unroll
        for (int j = 0; j < kTopkSlots; j++) {
            const uint32_t e = lane + 64u * (uint32_t)j;
            const bool v = e < E;
            la[j] = v ? ar[e] : 0.0f;
            nb[j] = v ? A.norms[e] : 0.0f;
            bs[j] = v ? A.bias[e] : 0.0f;
        }
        /* ||x_t|| (upper bound) */
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < kTopkSlots; j++) {
            const uint32_t c = lane + 64u * (uint32_t)j;
            const uint4 v = c < chunks ? sm.x[c] : make_uint4(0u, 0u, 0u, 0u);
            const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                ss = fmaf(bf16_lo(u[q]), bf16_lo(u[q]), ss);
                ss = fmaf(bf16_hi(u[q]), bf16_hi(u[q]), ss);
            }
        }
        const float nx = __fmul_rn(__fsqrt_rn(wave_sum(ss)), kNormInflate);
        bool fin = isfinite(nx);
#pragma unroll
        for (int j = 0; j < kTopkSlots; j++)
            fin = fin && isfinite(la[j]) && isfinite(nb[j]) && isfinite(bs[j]);
        /* approximate choices and keys; the choice error bound uses the
         * largest sigmoid slope over [a - err, a + err] */
        uint32_t key[kTopkSlots];
        float ch[kTopkSlots], ce[kTopkSlots];
#pragma unroll
        for (int j = 0; j < kTopkSlots; j++) {
            const uint32_t e = lane + 64u * (uint32_t)j;
            key[j] = 0u;
            ch[j] = 0.0f;
            ce[j] = 0.0f;
            if (e < E) {
                const float s = router_sigmoid(la[j]);
                key[j] = choice_key(s, bs[j]);
                ch[j] = __fadd_rn(s, bs[j]);
                const float err = fmaf(__fmul_rn(A.err_coef, nb[j]), nx, 1e-30f);
                const float m = fmaxf(0.0f, __fsub_rn(fabsf(la[j]), err));
                fin = fin && err <= 1e30f;
                ce[j] = fmaf(sigmoid_slope_bound(m), err,
                             fmaf(4.76837158203125e-7f, fabsf(ch[j]), 2e-6f));
            }
        }
        /* the k-th largest approximate key */
        const uint32_t thr = kth_largest_key(key, A.k, sm.topk.cand_key);
        /* E_k: the largest error bound among the experts at or above it */
        float ek = 0.0f;
#pragma unroll
        for (int j = 0; j < kTopkSlots; j++)
            if (thr != 0u && key[j] >= thr) ek = fmaxf(ek, ce[j]);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) ek = fmaxf(ek, __shfl_xor(ek, o, 64));
        const bool exact_all = __ballot(!fin) != 0ull || thr == 0u;
        float lim = 0.0f;
        if (!exact_all) {
            lim = __fsub_rn(key_value(thr), ek);
            lim = __fsub_rn(lim, __fmul_rn(fabsf(lim), 2.384185791015625e-7f));
        }
        uint32_t mine = 0u;
        bool cand[kTopkSlots];
#pragma unroll
        for (int j = 0; j < kTopkSlots; j++) {
            const uint32_t e = lane + 64u * (uint32_t)j;
            cand[j] = e < E && (exact_all || __fadd_rn(ch[j], ce[j]) >= lim);
            mine += cand[j] ? 1u : 0u;
        }
        const unsigned long long below = (1ull << lane) - 1ull;
        uint32_t pos = 0u, ncand = 0u;
#pragma unroll
        for (int b = 0; b < 5; b++) {
            const unsigned long long m = __ballot((mine >> b) & 1u);
            pos += (uint32_t)__popcll(m & below) << b;
            ncand += (uint32_t)__popcll(m) << b;
        }
#pragma unroll
        for (int j = 0; j < kTopkSlots; j++) {
            if (cand[j]) {
                sm.topk.cand_id[pos] = lane + 64u * (uint32_t)j;
                sm.topk.cand_score[pos] = bs[j];
                pos++;
            }
        }
        if (lane == 0u) sm.ncand = ncand;
    }
    __syncthreads();
    /* exact reference-order logits of this wave's candidates, two rows in flight */
    const uint32_t ncand = sm.ncand;
    auto load_row = [&](uint32_t e, uint4 (&v)[kTopkSlots]) __attribute__((always_inline)) {
        const uint32_t eu = (uint32_t)__builtin_amdgcn_readfirstlane((int)e); /* wave-uniform */
        const uint4 *wr = (const uint4 *)(A.w + (uint64_t)eu * H);
#pragma unroll
        for (int j = 0; j < kTopkSlots; j++) {
            const uint32_t c = lane + 64u * (uint32_t)j;
            v[j] = wr[c < chunks ? c : chunks - 1u];
        }
    };
    auto dot_row = [&](const uint4 (&v)[kTopkSlots]) __attribute__((always_inline)) -> float {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < kTopkSlots; j++)
            if (lane + 64u * (uint32_t)j < chunks)
                ref_chunk(acc, j, v[j], sm.x[lane + 64u * (uint32_t)j]);
        return ref_logit_finish(acc);
    };
    uint4 wa[kTopkSlots], wb[kTopkSlots];
    const uint32_t *cid = sm.topk.cand_id;
    if (wave < ncand) load_row(cid[wave], wa);
    for (uint32_t p = wave; p < ncand; p += 8u) {
        /* rows p (in wa) and p + 4 (into wb, issued before p's FMAs) */
        const bool second = p + 4u < ncand;
        if (second) load_row(cid[p + 4u], wb);
        const float l1 = dot_row(wa);
        if (lane == 0u) sm.topk.cand_key[p] = __float_as_uint(l1);
        if (!second) break;
        if (p + 8u < ncand) load_row(cid[p + 8u], wa);
        const float l2 = dot_row(wb);
        if (lane == 0u) sm.topk.cand_key[p + 4u] = __float_as_uint(l2);
    }
    __syncthreads();
    if (wave != 0u) return;
    certify_select(A, t, ncand, sm.topk);
}

/*
 * The certification of router_certify_kernel with one wave per token (4
 * tokens per block, no block barriers), for large batches: the phases a
 * block runs with one busy wave (candidate list, selection) no longer
 * idle three others, and twice as many tokens are in flight per CU. The
 * token's row stays in registers (lane l holds chunks l, l + 64, ..., the
 * chunks the reference order's ref_chunk takes), the candidate rows are
 * computed two in flight, and the
 * selection runs on the candidates only:
 *   candidates  approximate keys, T_k by kth_largest_key, E_k, the bound
 *               lim; candidate ids and biases go to the wave's
 *               cand_id / cand_score (positions in expert order);
 *   exact       reference-order logits of the candidates (into cand_key);
 *   select      each candidate's exact key (router_sigmoid + bias) and
 *               weight score (det_sigmoid), compacted to keys != 0, then
 *               topk_rank_write: the exact router's ranking and weights.
 * Same bound, same candidates' keys and the same ranking as the block
 * kernel, so the same routes.
 */
__global__ __launch_bounds__(256, 2) void router_certify_wave_kernel(CertArgs A) {
    __shared__ TopkWaveSmem smem[4];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t t = 4u * blockIdx.x + wave;
    if (t >= A.T) return; /* wave-uniform; the waves share no barrier */
    TopkWaveSmem &sm = smem[wave];
    const uint32_t E = A.E, H = A.H, chunks = H / 8u;
    const unsigned long long below = (1ull << lane) - 1ull;
    /* one batch of loads: the row's chunks, approximate logits, norms,
     * biases */
    const uint4 *xr = (const uint4 *)(A.x + (uint64_t)t * H);
    const float *ar = A.approx + (uint64_t)t * E;
    float la[kTopkSlots], nb[kTopkSlots], bs[kTopkSlots];
    float ss = 0.0f;
    {
        /* the row for its norm only: it is read again (from L2) for the
         * exact logits rather than held through the candidate phase */
        uint4 xn[kTopkSlots];
#pragma unroll
        for (int j = 0; j < kTopkSlots; j++) {
            const uint32_t c = lane + 64u * (uint32_t)j, e = c;
            xn[j] = c < chunks ? xr[c] : make_uint4(0u, 0u, 0u, 0u);
            la[j] = e < E ? ar[e] : 0.0f;
            nb[j] = e < E ? A.norms[e] : 0.0f;
            bs[j] = e < E ? A.bias[e] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < kTopkSlots; j++) {
            const uint32_t u[4] = {xn[j].x, xn[j].y, xn[j].z, xn[j].w};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                ss = fmaf(bf16_lo(u[q]), bf16_lo(u[q]), ss);
                ss = fmaf(bf16_hi(u[q]), bf16_hi(u[q]), ss);
            }
        }
    }
    const float nx = __fmul_rn(__fsqrt_rn(wave_sum(ss)), kNormInflate);
    bool fin = isfinite(nx);
    uint32_t key[kTopkSlots];
    float ch[kTopkSlots], ce[kTopkSlots];
#pragma unroll
    for (int j = 0; j < kTopkSlots; j++) {
        const uint32_t e = lane + 64u * (uint32_t)j;
        key[j] = 0u;
        ch[j] = 0.0f;
        ce[j] = 0.0f;
        if (e < E) {
            fin = fin && isfinite(la[j]) && isfinite(nb[j]) && isfinite(bs[j]);
            const float s = router_sigmoid(la[j]);
            key[j] = choice_key(s, bs[j]);
            ch[j] = __fadd_rn(s, bs[j]);
            const float err = fmaf(__fmul_rn(A.err_coef, nb[j]), nx, 1e-30f);
            fin = fin && err <= 1e30f;
            const float m = fmaxf(0.0f, __fsub_rn(fabsf(la[j]), err));
            ce[j] = fmaf(sigmoid_slope_bound(m), err,
                         fmaf(4.76837158203125e-7f, fabsf(ch[j]), 2e-6f));
        }
    }
    const bool exact_all = __ballot(!fin) != 0ull;
    uint32_t thr = exact_all ? 0u : kth_largest_key(key, A.k, sm.cand_key);
    float lim = 0.0f;
    const bool every = exact_all || thr == 0u;
    if (!every) {
        float ek = 0.0f;
#pragma unroll
        for (int j = 0; j < kTopkSlots; j++)
            if (key[j] >= thr) ek = fmaxf(ek, ce[j]);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) ek = fmaxf(ek, __shfl_xor(ek, o, 64));
        lim = __fsub_rn(key_value(thr), ek);
        lim = __fsub_rn(lim, __fmul_rn(fabsf(lim), 2.384185791015625e-7f));
    }
    uint32_t mine = 0u;
    bool cand[kTopkSlots];
#pragma unroll
    for (int j = 0; j < kTopkSlots; j++) {
        const uint32_t e = lane + 64u * (uint32_t)j;
        cand[j] = e < E && (every || __fadd_rn(ch[j], ce[j]) >= lim);
        mine += cand[j] ? 1u : 0u;
    }
    uint32_t pos = 0u, ncand = 0u;
#pragma unroll
    for (int b = 0; b < 5; b++) {
        const unsigned long long m = __ballot((mine >> b) & 1u);
        pos += (uint32_t)__popcll(m & below) << b;
        ncand += (uint32_t)__popcll(m) << b;
    }
#pragma unroll
    for (int j = 0; j < kTopkSlots; j++) {
        if (cand[j]) {
            sm.cand_id[pos] = lane + 64u * (uint32_t)j;
            sm.cand_score[pos] = bs[j]; /* the bias until the selection */
            pos++;
        }
    }
    wave_fence();
    uint4 xv[kTopkSlots];
#pragma unroll
    for (int j = 0; j < kTopkSlots; j++) {
        const uint32_t c = lane + 64u * (uint32_t)j;
        xv[j] = c < chunks ? xr[c] : make_uint4(0u, 0u, 0u, 0u);
    }
    /* exact reference-order logits, two candidate rows in flight */
    auto load_row = [&](uint32_t p, uint4 (&v)[kTopkSlots]) __attribute__((always_inline)) {
        const uint32_t eu = (uint32_t)__builtin_amdgcn_readfirstlane((int)sm.cand_id[p]);
        const uint4 *wr = (const uint4 *)(A.w + (uint64_t)eu * H);
#pragma unroll
        for (int j = 0; j < kTopkSlots; j++) {
            const uint32_t c = lane + 64u * (uint32_t)j;
            v[j] = wr[c < chunks ? c : chunks - 1u];
        }
    };
    auto dot_row = [&](const uint4 (&v)[kTopkSlots]) __attribute__((always_inline)) -> float {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < kTopkSlots; j++) {
            if (lane + 64u * (uint32_t)j < chunks) {
                /* opaque copy: keeps the row's fp32 conversions inside the
                 * loop over candidates (hoisted, they would take 128
                 * registers) */
                uint4 xu = xv[j];
                asm volatile("" : "+v"(xu.x), "+v"(xu.y), "+v"(xu.z), "+v"(xu.w));
                ref_chunk(acc, j, v[j], xu);
            }
        }
        return ref_logit_finish(acc);
    };
    uint4 wa[kTopkSlots], wb[kTopkSlots];
    if (ncand > 0u) load_row(0u, wa);
    for (uint32_t p = 0; p < ncand; p += 2u) {
        const bool second = p + 1u < ncand;
        if (second) load_row(p + 1u, wb);
        const float l1 = dot_row(wa);
        if (lane == 0u) sm.cand_key[p] = __float_as_uint(l1);
        if (!second) break;
        if (p + 2u < ncand) load_row(p + 2u, wa);
        const float l2 = dot_row(wb);
        if (lane == 0u) sm.cand_key[p + 1u] = __float_as_uint(l2);
    }
    wave_fence();
    certify_select(A, t, ncand, sm);
}

}  // namespace

/* K slices of the MFMA logits: enough (tile, slice) works to spread over
 * the CUs when there are few tiles (about 512 works: two blocks per CU),
 * at most kRouterMaxSlices; the approximate logits take slices x T x E
 * floats. */
uint32_t router_slice_cap(uint32_t T, uint32_t E) {
    const uint32_t tiles = ((T + kRT - 1u) / kRT) * ((E + kRT - 1u) / kRT);
    const uint32_t S = tiles ? 512u / tiles : 1u;
    return S < 1u ? 1u : (S > kRouterMaxSlices ? kRouterMaxSlices : S);
}

/* ... and at most the K steps. */
uint32_t router_slices(uint32_t T, uint32_t E, uint32_t H) {
    const uint32_t S = router_slice_cap(T, E), ks = H / kRK;
    return ks == 0u ? 1u : (S < ks ? S : ks);
}

/* The certified bound assumes the MFMA unit's per-instruction error measured
 * on gfx950 (4 u per term allowed, 8 u sum|p| worst seen): on any other
 * part the exact router runs. The answer is cached per device (benign race:
 * every writer stores the same value). */
static bool device_is_gfx950() {
    static signed char cache[64];
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
    if (cache[dev] == 0) {
        hipDeviceProp_t prop;
        const bool ok = hipGetDeviceProperties(&prop, dev) == hipSuccess &&
                        strncmp(prop.gcnArchName, "gfx950", 6) == 0;
        cache[dev] = ok ? 1 : -1;
    }
    return cache[dev] > 0;
}

bool router_certified_supported(uint32_t tokens, uint32_t experts, uint32_t hidden,
                                uint32_t top_k, const void *router_weight, const void *x) {
    return device_is_gfx950() && tokens > 0u && experts >= top_k && experts <= 64u * (uint32_t)kTopkSlots &&
           top_k >= 1u && top_k <= 32u && hidden > 0u && hidden % kRK == 0u &&
           hidden <= 8u * 64u * (uint32_t)kTopkSlots &&
           (((uintptr_t)router_weight | (uintptr_t)x) % 16u) == 0u;
}

bool launch_router_certified(uint32_t *ids, float *weights, uint32_t *ids2, float *w2,
                             float *approx, float *norms, const void *router_weight,
                             const void *router_bias, const void *x, uint32_t T, uint32_t E,
                             uint32_t H, uint32_t k, float scale, hipStream_t st,
                             const StageMarker *mark) {
    if (!router_certified_supported(T, E, H, k, router_weight, x)) return false;
    const uint16_t *w = (const uint16_t *)router_weight;
    hipLaunchKernelGGL(router_norms_kernel, dim3((E + 3u) / 4u), dim3(256), 0, st, norms, w, E, H);
    const uint32_t tiles = ((T + kRT - 1u) / kRT) * ((E + kRT - 1u) / kRT);
    const uint32_t S = router_slices(T, E, H), works = tiles * S;
    hipLaunchKernelGGL(router_mfma_kernel, dim3(8u * ((works + 7u) / 8u)), dim3(512), 0, st,
                       approx, (const uint16_t *)x, w, T, E, H, S);
    if (S > 1u) {
        const uint64_t n = (uint64_t)T * E;
        const uint64_t blocks = (n + 255u) / 256u;
        hipLaunchKernelGGL(router_slices_sum_kernel, dim3((uint32_t)(blocks < 4096u ? blocks : 4096u)),
                           dim3(256), 0, st, approx, S, n);
    }
    if (mark) (*mark)(K3_MOE_STAGE_TOPK);
    CertArgs A{ids, weights, ids2, w2, approx, norms, (const float *)router_bias,
               (const uint16_t *)x, w, T, E, H, k, scale,
               (float)(H / 32u + 270u) * 5.9604644775390625e-8f * (1.0f + 1.0f / 1024.0f)};
    if (T >= kCertWaveMinTokens)
        hipLaunchKernelGGL(router_certify_wave_kernel, dim3((T + 3u) / 4u), dim3(256), 0, st, A);
    else
        hipLaunchKernelGGL(router_certify_kernel, dim3(T), dim3(256), 0, st, A);
    return hipGetLastError() == hipSuccess;
}

}  // namespace k3

/* ---------------------------------------------------------------------- */
/* C ABI                                                                   */
/* ---------------------------------------------------------------------- */

namespace {
size_t up256(size_t n) { return (n + 255u) & ~(size_t)255u; }
}  // namespace

extern "C" size_t k3_moe_router_scratch_bytes(uint32_t token_count, uint32_t expert_count) {
    if (token_count == 0u || token_count > 65535u || expert_count == 0u ||
        expert_count > 64u * (uint32_t)k3::kTopkSlots)
        return 0u;
    return up256(4ull * k3::router_slice_cap(token_count, expert_count) * token_count *
                 expert_count) +
           up256(4ull * expert_count);
}

extern "C" bool k3_moe_router_bf16(uint32_t *expert_ids, float *expert_weights,
                                   const void *hidden, const void *router_weight,
                                   const void *router_bias, uint32_t token_count,
                                   uint32_t expert_count, uint32_t hidden_size, uint32_t top_k,
                                   float scaling_factor, void *scratch, size_t scratch_bytes,
                                   void *stream) {
    const size_t need = k3_moe_router_scratch_bytes(token_count, expert_count);
    if (!expert_ids || !expert_weights || !hidden || !router_weight || !router_bias ||
        !scratch || need == 0u || scratch_bytes < need || ((uintptr_t)scratch % 256u) != 0u ||
        hidden_size == 0u || top_k == 0u || top_k > 32u || top_k > expert_count)
        return false;
    const hipStream_t st = (hipStream_t)stream;
    float *logits = (float *)scratch;
    float *norms = (float *)((uint8_t *)scratch +
                             up256(4ull * k3::router_slice_cap(token_count, expert_count) *
                                   token_count * expert_count));
    if (token_count >= k3::kCertifiedMinTokens &&
        k3::router_certified_supported(token_count, expert_count, hidden_size, top_k,
                                       router_weight, hidden))
        return k3::launch_router_certified(expert_ids, expert_weights, nullptr, nullptr, logits,
                                           norms, router_weight, router_bias, hidden,
                                           token_count, expert_count, hidden_size, top_k,
                                           scaling_factor, st, nullptr);
    return k3::launch_bf16_rows_f32_any(logits, router_weight, hidden, token_count, expert_count,
                                        hidden_size, st) &&
           k3::launch_router_topk(expert_ids, expert_weights, nullptr, nullptr, logits,
                                  (const float *)router_bias, token_count, expert_count, top_k,
                                  scaling_factor, st);
}

/* choices[t, e] = router_sigmoid(logits[t, e]) + bias[e] (bias may be NULL). */
__global__ __launch_bounds__(256) void router_choices_kernel(float *__restrict__ out,
                                                             const float *__restrict__ logits,
                                                             const float *__restrict__ bias,
                                                             uint64_t n, uint32_t experts) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const float s = k3::router_sigmoid(logits[i]);
    out[i] = bias ? __fadd_rn(s, bias[i % experts]) : s;
}

extern "C" bool k3_moe_router_choices_f32(float *choices, const float *logits, const float *bias,
                                          uint32_t token_count, uint32_t expert_count,
                                          void *stream) {
    if (!choices || !logits || token_count == 0u || expert_count == 0u) return false;
    const uint64_t n = (uint64_t)token_count * expert_count;
    if ((n + 255u) / 256u > 0xffffffffull) return false;
    hipLaunchKernelGGL(router_choices_kernel, dim3((unsigned)((n + 255u) / 256u)), dim3(256), 0,
                       (hipStream_t)stream, choices, logits, bias, n, expert_count);
    return hipGetLastError() == hipSuccess;
}
