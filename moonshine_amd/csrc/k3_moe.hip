/*
 * libk3moe — the fused routed-MoE layer for gfx950.
 *
 * Dataflow (replacing decode_routed_layer, k3_engine.cu:1554-1897, and
 * prefill_routed_layer, k3_engine_prefill.inc:1448-1614, for the
 * HBM-resident expert store):
 *
 *   router logits (bf16 -> f32, w64 order)        k3_rocm_bf16_gemm_f32
 *   top-k (sigmoid + bias, lowest-id ties)        k3_rocm_router_topk_f32_batch
 *   T == 1: the three decode kernels of k3_decode.hip (router + top-k,
 *           gate/up + activation, down + combine + residual)
 *   T  > 1: device routing plan (count -> scan -> stable scatter), then
 *           grouped gate/up and down over the selected experts only (each
 *           expert's weights are read once per row block for all its
 *           tokens), then the slotted combine. K3_MOE_EXACT runs the w64
 *           VALU kernels below; K3_MOE_MFMA / _FP8 the scaled-MFMA tiles
 *           of k3_mfma.hip.
 *
 * No host synchronisation anywhere: the expert ids never leave the device.
 * Every product uses the per-row w64 order of k3_ops.hip, so the decode and
 * grouped paths give the same bits for the same token.
 */
#include "k3_device.h"
#include "k3_internal.h"
#include "k3_decode.h"
#include "k3_mfma.h"
#include "k3_topk.h"
#include "../../include/k3_moe.h"
#include "../../include/k3_rocm_ops.h"

#include <hip/hip_runtime.h>
#include <mutex>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

using namespace k3;

namespace {

constexpr uint32_t kPlanChunk = 256;  /* tokens per plan block */

inline size_t align256(size_t v) { return (v + 255u) & ~(size_t)255u; }

/* ------------------------------------------------------------------------ */
/* workspace                                                                 */
/* ------------------------------------------------------------------------ */

struct Workspace {
    float *logits;
    float *scores;
    uint32_t *keys;
    uint32_t *ids;
    float *weights;
    uint32_t *counts, *offsets, *unique, *summary;
    uint32_t *token_index, *route_index;
    uint32_t *chunk_base;
    uint16_t *act;
    k3_moe_expert *sel;
    uint16_t *y;
    MfmaBuffers mfma;
    size_t bytes;
};

size_t plan_scratch(uint32_t T, uint32_t E) {
    return align256((size_t)4u * E * ((T + kPlanChunk - 1u) / kPlanChunk));
}

Workspace carve(void *base, const k3_moe_shape &s, uint32_t T) {
    Workspace w{};
    uint8_t *p = (uint8_t *)base;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        uint8_t *r = p ? p + off : nullptr;
        off += align256(bytes);
        return r;
    };
    const uint64_t routes = (uint64_t)T * s.top_k;
    /* router logits; T > 1: the certified router's K-sliced approximations */
    w.logits = (float *)take(4ull * T * s.expert_count *
                             (T > 1u ? router_slice_cap(T, s.expert_count) : 1u));
    w.scores = (float *)take(4ull * s.expert_count);
    w.keys = (uint32_t *)take(4ull * s.expert_count);
    w.ids = (uint32_t *)take(4ull * routes);
    w.weights = (float *)take(4ull * routes);
    w.counts = (uint32_t *)take(4ull * s.expert_count);
    w.offsets = (uint32_t *)take(4ull * (s.expert_count + 1u));
    w.unique = (uint32_t *)take(4ull * s.expert_count);
    w.summary = (uint32_t *)take(16); /* [0..2] plan summary, [3] decode slot mask */
    w.token_index = (uint32_t *)take(4ull * routes);
    w.route_index = (uint32_t *)take(4ull * routes);
    w.chunk_base = (uint32_t *)take(plan_scratch(T, s.expert_count));
    w.act = (uint16_t *)take(2ull * routes * s.ffn);
    w.sel = (k3_moe_expert *)take(T == 1u ? sizeof(k3_moe_expert) * s.top_k : 0u);
    /* grouped path: every T > 1, and T == 1 when the decode kernels do not
     * cover the shape */
    const bool grouped = T > 1u || !decode_supported(s);
    w.y = (uint16_t *)take(2ull * routes * s.hidden); /* per-slot expert outputs */
    if (grouped) {
        /* MFMA path: activation codes reuse `act` (two byte planes of the
         * bf16 activation's size) */
        MfmaBuffers &m = w.mfma;
        for (int t = 0; t < 2; t++) {
            m.xq[t] = take(1ull * T * s.hidden);
            m.xs[t] = take(1ull * T);
            m.aq[t] = w.act ? (uint8_t *)w.act + (uint64_t)t * routes * s.ffn : nullptr;
            m.as[t] = take(1ull * routes * s.ffn / 32u);
        }
        m.routes = (uint32_t)routes;
        mfma_tile_caps(T, s.top_k, s.expert_count, m.tile_cap);
        uint64_t ntiles = 0u;
        for (int c = 0; c < kTileClasses; c++) ntiles += m.tile_cap[c];
        m.tiles = (uint32_t *)take(12ull * ntiles);
        m.tile_count = (uint32_t *)take(4u * kTileClasses);
        m.unaligned = (uint32_t *)take(4ull * (s.expert_count + 1u));
    }
    w.bytes = off;
    return w;
}

/* ------------------------------------------------------------------------ */
/* routing plan                                                              */
/* ------------------------------------------------------------------------ */

/* Route (t, r) is valid when its id is < E and no earlier rank of token t
 * chose the same expert (the router never does; external ids might). The
 * token's k <= K ids are read once into registers (all loads issued
 * together); invalid routes come back as E. A later duplicate matches the
 * first occurrence, which stays, so invalidating in place keeps the rule. */
template <int K>
__device__ __forceinline__ void token_routes(const uint32_t *ids, uint32_t t, uint32_t k,
                                             uint32_t E, uint32_t (&e)[K]) {
#pragma unroll
    for (int r = 0; r < K; r++) e[r] = (uint32_t)r < k ? ids[(uint64_t)t * k + r] : E;
#pragma unroll
    for (int r = 0; r < K; r++) {
        if (e[r] >= E) e[r] = E;
#pragma unroll
        for (int q = 0; q < r; q++)
            if (e[q] == e[r]) e[r] = E;
    }
}

template <int K>
__global__ __launch_bounds__(256) void plan_count_kernel(uint32_t *__restrict__ chunk_counts,
                                                         const uint32_t *__restrict__ ids,
                                                         uint32_t T, uint32_t k, uint32_t E) {
    __shared__ uint32_t hist[1024];
    for (uint32_t e = threadIdx.x; e < E; e += blockDim.x) hist[e] = 0u;
    __syncthreads();
    const uint32_t t = blockIdx.x * kPlanChunk + threadIdx.x;
    if (t < T) {
        uint32_t e[K];
        token_routes<K>(ids, t, k, E, e);
#pragma unroll
        for (int r = 0; r < K; r++)
            if (e[r] < E) atomicAdd(&hist[e[r]], 1u);
    }
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < E; e += blockDim.x)
        chunk_counts[(uint64_t)blockIdx.x * E + e] = hist[e];
}

/* One block of 1024 threads: per-expert scan over chunks, exclusive scan
 * over experts, compaction of the selected ids. */
__global__ __launch_bounds__(1024) void plan_scan_kernel(
        uint32_t *__restrict__ chunk_base, uint32_t *__restrict__ counts,
        uint32_t *__restrict__ offsets, uint32_t *__restrict__ unique,
        uint32_t *__restrict__ summary, uint32_t chunks, uint32_t E, uint32_t routes) {
    __shared__ uint32_t wave_tot[16];
    __shared__ uint32_t wave_sel[16];
    __shared__ uint32_t wave_max[16];
    const uint32_t e = threadIdx.x, lane = e & 63u, wave = e >> 6;
    uint32_t count = 0u;
    if (e < E) {
        for (uint32_t b = 0; b < chunks; b++) {
            const uint32_t c = chunk_base[(uint64_t)b * E + e];
            chunk_base[(uint64_t)b * E + e] = count;
            count += c;
        }
    }
    /* inclusive wave scans of count and of the selected flag */
    uint32_t inc = count, sel = count ? 1u : 0u, mx = count;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t a = __shfl_up(inc, o, 64), b = __shfl_up(sel, o, 64);
        if ((int)lane >= o) { inc += a; sel += b; }
        mx = max(mx, __shfl_xor(mx, o, 64));
    }
    if (lane == 63u) { wave_tot[wave] = inc; wave_sel[wave] = sel; }
    if (lane == 0u) wave_max[wave] = mx;
    __syncthreads();
    uint32_t base = 0u, sbase = 0u;
    for (uint32_t w = 0; w < wave; w++) { base += wave_tot[w]; sbase += wave_sel[w]; }
    const uint32_t excl = base + inc - count;
    if (e < E) {
        counts[e] = count;
        offsets[e] = excl;
        if (count) unique[sbase + sel - 1u] = e;
        for (uint32_t b = 0; b < chunks; b++) chunk_base[(uint64_t)b * E + e] += excl;
    }
    if (e == blockDim.x - 1u) {
        uint32_t total = 0u, nsel = 0u, m = 0u;
        for (uint32_t w = 0; w < blockDim.x / 64u; w++) {
            total += wave_tot[w]; nsel += wave_sel[w]; m = max(m, wave_max[w]);
        }
        offsets[E] = total;
        summary[0] = nsel;
        summary[1] = routes - total;
        summary[2] = m;
        summary[3] = 0u;
    }
}

template <int K>
__global__ __launch_bounds__(256) void plan_scatter_kernel(
        uint32_t *__restrict__ token_index, uint32_t *__restrict__ route_index,
        const uint32_t *__restrict__ chunk_base, const uint32_t *__restrict__ ids, uint32_t T,
        uint32_t k, uint32_t E) {
    __shared__ unsigned long long masks[4][1024];
    for (uint32_t i = threadIdx.x; i < 4u * 1024u; i += blockDim.x) (&masks[0][0])[i] = 0ull;
    __syncthreads();
    const uint32_t t = blockIdx.x * kPlanChunk + threadIdx.x;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    uint32_t e[K];
    if (t < T) {
        token_routes<K>(ids, t, k, E, e);
#pragma unroll
        for (int r = 0; r < K; r++)
            if (e[r] < E) atomicOr(&masks[wave][e[r]], 1ull << lane);
    }
    __syncthreads();
    if (t >= T) return;
    const unsigned long long below = (1ull << lane) - 1ull;
#pragma unroll
    for (int r = 0; r < K; r++) {
        if (e[r] >= E) continue;
        uint32_t before = (uint32_t)__popcll(masks[wave][e[r]] & below);
        for (uint32_t w = 0; w < wave; w++) before += (uint32_t)__popcll(masks[w][e[r]]);
        const uint32_t pos = chunk_base[(uint64_t)blockIdx.x * E + e[r]] + before;
        token_index[pos] = t;
        route_index[pos] = t * k + (uint32_t)r;
    }
}

bool launch_plan(uint32_t *counts, uint32_t *offsets, uint32_t *unique, uint32_t *summary,
                 uint32_t *token_index, uint32_t *route_index, uint32_t *chunk_base,
                 const uint32_t *ids, uint32_t T, uint32_t k, uint32_t E, hipStream_t s) {
    const uint32_t chunks = (T + kPlanChunk - 1u) / kPlanChunk;
    if (k <= 16u)
        hipLaunchKernelGGL(plan_count_kernel<16>, dim3(chunks), dim3(kPlanChunk), 0, s, chunk_base,
                           ids, T, k, E);
    else
        hipLaunchKernelGGL(plan_count_kernel<32>, dim3(chunks), dim3(kPlanChunk), 0, s, chunk_base,
                           ids, T, k, E);
    hipLaunchKernelGGL(plan_scan_kernel, dim3(1), dim3(1024), 0, s, chunk_base, counts, offsets,
                       unique, summary, chunks, E, T * k);
    if (k <= 16u)
        hipLaunchKernelGGL(plan_scatter_kernel<16>, dim3(chunks), dim3(kPlanChunk), 0, s,
                           token_index, route_index, chunk_base, ids, T, k, E);
    else
        hipLaunchKernelGGL(plan_scatter_kernel<32>, dim3(chunks), dim3(kPlanChunk), 0, s,
                           token_index, route_index, chunk_base, ids, T, k, E);
    return hipGetLastError() == hipSuccess;
}

__device__ __forceinline__ float bf16_round(float v) { return bf16_to_f32(f32_to_bf16(v)); }

/* ------------------------------------------------------------------------ */
/* grouped (many tokens), exact order                                        */
/* ------------------------------------------------------------------------ */

/*
 * Work of a grouped exact workgroup: runs of plan rows [base, base + n) of
 * an expert e. Tile mode (list == nullptr): the tiles of the per-class
 * lists (at most 128 rows each, every selected expert; build_tiles_all),
 * walked with stride gridDim.y, so a heavy expert's rows spread over many
 * workgroups and no workgroup is launched past the tile count. List mode:
 * list = (count, expert ids), walked the same way, each expert's rows
 * whole (the MFMA path's fallback for experts whose tensors are not
 * 8-byte aligned).
 */
struct ExactWork {
    const uint32_t *tiles, *tile_count;
    uint32_t cap[kTileClasses];
    const uint32_t *list;       /* list mode: expert ids */
    const uint32_t *list_count; /* their count */
    const uint32_t *counts, *offsets;
};

/* Tile q of the tile lists (classes in order, tile_count[c] of class c
 * stored from the class's segment start); false past the last. */
__device__ __forceinline__ bool exact_tile(const ExactWork &W, uint32_t q, uint32_t &e,
                                           uint32_t &base, uint32_t &n) {
    uint32_t first = 0u;
#pragma unroll
    for (int c = 0; c < kTileClasses; c++) {
        const uint32_t tc = W.tile_count[c];
        if (q < tc) {
            const uint32_t *t = W.tiles + 3u * (first + q);
            e = t[0];
            base = t[1];
            n = t[2];
            return true;
        }
        q -= tc;
        first += W.cap[c];
    }
    return false;
}

/* Gate/up of plan rows [base, base + n) of expert e, weight rows row0 ..
 * row0 + RW of this wave: rows are processed TT tokens at a time, and the
 * weight group loaded for them is reused by all TT. */
template <int RW, int TT>
__device__ __forceinline__ void gateup_rows(uint16_t *__restrict__ act,
                                            const uint16_t *__restrict__ x,
                                            const uint32_t *__restrict__ token_index,
                                            const k3_moe_expert &ex, uint32_t base, uint32_t n,
                                            uint32_t row0, uint32_t H, uint32_t F, uint32_t kind,
                                            float beta, float lb) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t G = H / 32u;
    const uint8_t *gp = (const uint8_t *)ex.gate_packed + (uint64_t)row0 * (H / 2u);
    const uint8_t *up = (const uint8_t *)ex.up_packed + (uint64_t)row0 * (H / 2u);
    const bool a16 = (((uintptr_t)gp | (uintptr_t)up) % 16u) == 0u;
    const uint8_t *gsc = (const uint8_t *)ex.gate_scales + (uint64_t)row0 * G;
    const uint8_t *usc = (const uint8_t *)ex.up_scales + (uint64_t)row0 * G;
    for (uint32_t p0 = 0; p0 < n; p0 += TT) {
        const uint32_t active = n - p0 < (uint32_t)TT ? n - p0 : (uint32_t)TT;
        uint32_t tok[TT];
#pragma unroll
        for (int t = 0; t < TT; t++)
            tok[t] = token_index[base + p0 + ((uint32_t)t < active ? (uint32_t)t : 0u)];
        float acc[TT][2 * RW];
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int i = 0; i < 2 * RW; i++) acc[t][i] = 0.0f;
        for (uint32_t g = lane; g < G; g += 64u) {
            uint4 w[2 * RW];
            float sc[2 * RW];
#pragma unroll
            for (int i = 0; i < RW; i++) {
                w[i] = gload16(gp + (uint64_t)i * (H / 2u) + 16u * g, a16);
                w[RW + i] = gload16(up + (uint64_t)i * (H / 2u) + 16u * g, a16);
                sc[i] = e8m0_to_f32(gsc[(uint64_t)i * G + g]);
                sc[RW + i] = e8m0_to_f32(usc[(uint64_t)i * G + g]);
            }
#pragma unroll
            for (int t = 0; t < TT; t++) {
                if ((uint32_t)t < active) {
                    float xf[32];
                    bf16x32_to_f32((const uint4 *)(x + (uint64_t)tok[t] * H) + 4u * g, xf);
#pragma unroll
                    for (int i = 0; i < 2 * RW; i++)
                        acc[t][i] = fmaf(fp4_group(w[i], xf), sc[i], acc[t][i]);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const float v = wave_sum_rows<2 * RW>(acc[t]);
            const float uu = __shfl_xor(v, 32, 64);
            const int owner = wave_rows_owner<2 * RW>();
            if ((uint32_t)t < active && lane < 32u && (lane & (64u / (2u * RW) - 1u)) == 0u)
                act[(uint64_t)(base + p0 + t) * F + row0 + owner] =
                    f32_to_bf16(gated_act(bf16_round(v), bf16_round(uu), kind, beta, lb));
        }
    }
}

/* grid (up to F / (4 * RW), walk), block 256 (ExactWork); column blocks
 * past the grid's x extent are walked (the hand-off list, usually empty,
 * runs on a small grid). */
template <int RW, int TT>
__global__ __launch_bounds__(256, 2) void grouped_gateup_kernel(
        uint16_t *__restrict__ act, const uint16_t *__restrict__ x, ExactWork W,
        const uint32_t *__restrict__ token_index, const k3_moe_expert *__restrict__ experts,
        uint32_t H, uint32_t F, uint32_t kind, float beta, float lb) {
    const uint32_t nbx = F / (4u * RW);
    const uint32_t listed = W.list ? *W.list_count : 0u;
    if (W.list && blockIdx.y >= listed) return;
    for (uint32_t bx = blockIdx.x; bx < nbx; bx += gridDim.x) {
        const uint32_t row0 = (bx * 4u + (threadIdx.x >> 6)) * RW;
        if (!W.list) {
            uint32_t e, base, n;
            for (uint32_t q = blockIdx.y; exact_tile(W, q, e, base, n); q += gridDim.y)
                gateup_rows<RW, TT>(act, x, token_index, experts[e], base, n, row0, H, F, kind,
                                    beta, lb);
            continue;
        }
        for (uint32_t q = blockIdx.y; q < listed; q += gridDim.y) {
            const uint32_t e = W.list[q];
            gateup_rows<RW, TT>(act, x, token_index, experts[e], W.offsets[e], W.counts[e], row0,
                                H, F, kind, beta, lb);
        }
    }
}

/* Down of plan rows [base, base + n) of expert e into their route slots of
 * y, weight rows row0 .. row0 + RB of this wave, TT tokens at a time. */
template <int RB, int TT>
__device__ __forceinline__ void down_rows(uint16_t *__restrict__ y,
                                          const uint16_t *__restrict__ act,
                                          const uint32_t *__restrict__ route_index,
                                          const k3_moe_expert &ex, uint32_t base, uint32_t n,
                                          uint32_t row0, uint32_t H, uint32_t F) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t G = F / 32u;
    const uint8_t *dp = (const uint8_t *)ex.down_packed + (uint64_t)row0 * (F / 2u);
    const bool a16 = ((uintptr_t)dp % 16u) == 0u;
    const uint8_t *ds = (const uint8_t *)ex.down_scales + (uint64_t)row0 * G;
    for (uint32_t p0 = 0; p0 < n; p0 += TT) {
        const uint32_t active = n - p0 < (uint32_t)TT ? n - p0 : (uint32_t)TT;
        float acc[TT][RB];
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int i = 0; i < RB; i++) acc[t][i] = 0.0f;
        for (uint32_t g = lane; g < G; g += 64u) {
            uint4 w[RB];
            float sc[RB];
#pragma unroll
            for (int i = 0; i < RB; i++) {
                w[i] = gload16(dp + (uint64_t)i * (F / 2u) + 16u * g, a16);
                sc[i] = e8m0_to_f32(ds[(uint64_t)i * G + g]);
            }
#pragma unroll
            for (int t = 0; t < TT; t++) {
                if ((uint32_t)t < active) {
                    float xf[32];
                    bf16x32_to_f32((const uint4 *)(act + (uint64_t)(base + p0 + t) * F) + 4u * g, xf);
#pragma unroll
                    for (int i = 0; i < RB; i++)
                        acc[t][i] = fmaf(fp4_group(w[i], xf), sc[i], acc[t][i]);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const float v = wave_sum_rows<RB>(acc[t]);
            const int owner = wave_rows_owner<RB>();
            if ((uint32_t)t < active && (lane & (64u / RB - 1u)) == 0u)
                y[(uint64_t)route_index[base + p0 + t] * H + row0 + owner] = f32_to_bf16(v);
        }
    }
}

/* grid (up to H / (4 * RB), walk), block 256: y[route] = down_e . act[row]
 * (column blocks walked as in grouped_gateup_kernel). Two
 * waves per SIMD (at most 256 VGPRs): at one wave per SIMD (269 VGPRs) the
 * kernel took 15.0 against 8.7 ms at cfg3. */
template <int RB, int TT>
__global__ __launch_bounds__(256, 2) void grouped_down_kernel(
        uint16_t *__restrict__ y, const uint16_t *__restrict__ act, ExactWork W,
        const uint32_t *__restrict__ route_index, const k3_moe_expert *__restrict__ experts,
        uint32_t H, uint32_t F) {
    const uint32_t nbx = H / (4u * RB);
    const uint32_t listed = W.list ? *W.list_count : 0u;
    if (W.list && blockIdx.y >= listed) return;
    for (uint32_t bx = blockIdx.x; bx < nbx; bx += gridDim.x) {
        const uint32_t row0 = (bx * 4u + (threadIdx.x >> 6)) * RB;
        if (!W.list) {
            uint32_t e, base, n;
            for (uint32_t q = blockIdx.y; exact_tile(W, q, e, base, n); q += gridDim.y)
                down_rows<RB, TT>(y, act, route_index, experts[e], base, n, row0, H, F);
            continue;
        }
        for (uint32_t q = blockIdx.y; q < listed; q += gridDim.y) {
            const uint32_t e = W.list[q];
            down_rows<RB, TT>(y, act, route_index, experts[e], W.offsets[e], W.counts[e], row0,
                              H, F);
        }
    }
}

/* out[t, d] = bf16(residual + bf16(sum_r w[t, r] * y[t*k + r, d])), rank
 * order, invalid routes skipped (k3_rocm_ops.cu:1452-1510). grid
 * (ceil(H / (8 * 128)), T), block 128: a thread owns 8 consecutive d (one
 * 16-byte load per route); every load is issued before the first use, so
 * a token costs one memory round trip. H % 8 == 0, rows 16-byte aligned. */
constexpr uint32_t kCombineThreads = 128;

__global__ __launch_bounds__(128) void combine_kernel(
        uint16_t *__restrict__ out, const uint16_t *__restrict__ y,
        const uint16_t *__restrict__ residual, const uint32_t *__restrict__ ids,
        const float *__restrict__ wts, uint32_t H, uint32_t k, uint32_t E) {
    const uint32_t t = blockIdx.y;
    const uint32_t d = 8u * (blockIdx.x * kCombineThreads + threadIdx.x);
    if (d >= H) return;
    const uint64_t r0 = (uint64_t)t * k;
    uint4 yv[32];
    float w[32];
    bool live[32];
#pragma unroll
    for (int r = 0; r < 32; r++) { /* route 0 stands in for r >= k */
        const uint64_t route = r0 + ((uint32_t)r < k ? (uint32_t)r : 0u);
        yv[r] = *(const uint4 *)(y + route * H + d);
        w[r] = wts[route];
        live[r] = ((uint32_t)r < k) & (ids[route] < E);
    }
    const uint64_t o = (uint64_t)t * H + d;
    const uint4 rv = residual ? *(const uint4 *)(residual + o) : make_uint4(0u, 0u, 0u, 0u);
    float c[8];
#pragma unroll
    for (int i = 0; i < 8; i++) c[i] = 0.0f;
#pragma unroll
    for (int r = 0; r < 32; r++) {
        if (!live[r]) continue;
        const uint32_t u[4] = {yv[r].x, yv[r].y, yv[r].z, yv[r].w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            c[2 * q] = __fadd_rn(c[2 * q], __fmul_rn(w[r], bf16_lo(u[q])));
            c[2 * q + 1] = __fadd_rn(c[2 * q + 1], __fmul_rn(w[r], bf16_hi(u[q])));
        }
    }
    const uint32_t ru[4] = {rv.x, rv.y, rv.z, rv.w};
    uint32_t ov[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        uint32_t lo = f32_to_bf16(bf16_round(c[2 * q])), hi = f32_to_bf16(bf16_round(c[2 * q + 1]));
        if (residual) {
            lo = f32_to_bf16(__fadd_rn(bf16_lo(ru[q]), bf16_round(c[2 * q])));
            hi = f32_to_bf16(__fadd_rn(bf16_hi(ru[q]), bf16_round(c[2 * q + 1])));
        }
        ov[q] = lo | (hi << 16);
    }
    *(uint4 *)(out + o) = make_uint4(ov[0], ov[1], ov[2], ov[3]);
}

/* ------------------------------------------------------------------------ */
/* synthetic store                                                           */
/* ------------------------------------------------------------------------ */

__global__ void synth_fill_kernel(uint8_t *__restrict__ base, uint64_t bytes, uint64_t key,
                                  uint32_t kind) {
    const uint64_t stride = (uint64_t)blockDim.x * gridDim.x;
    if (kind == 0u) {
        const uint64_t words = bytes / 8u;
        for (uint64_t w = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; w < words; w += stride)
            ((uint64_t *)base)[w] = synth_word(key, w);
        for (uint64_t i = words * 8u + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < bytes;
             i += stride)
            base[i] = synth_byte(key, i, 0u);
    } else {
        for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < bytes; i += stride)
            base[i] = synth_byte(key, i, 1u);
    }
}

/* output, hidden and residual (nullable) rows move in 16-byte pieces. */
bool rows_aligned(const void *output, const void *hidden, const void *residual) {
    return (((uintptr_t)output | (uintptr_t)hidden | (uintptr_t)residual) % 16u) == 0u;
}

bool shape_ok(const k3_moe_shape *s) {
    return s && s->hidden && s->hidden % 32u == 0u && s->ffn && s->ffn % 32u == 0u &&
           s->expert_count && s->expert_count <= 1024u && s->top_k && s->top_k <= 32u &&
           s->top_k <= s->expert_count && s->scaling_factor > 0.0f && s->activation <= 1u &&
           (s->activation == 1u || (s->beta > 0.0f && s->linear_beta > 0.0f));
}

/* precision and shape checks shared by the layer entry points; the MFMA
 * precisions need H % 256 == 0 and F % 128 == 0 when T > 1 */
bool precision_ok(const k3_moe_shape *s, uint32_t T, uint32_t precision) {
    if (!shape_ok(s) || T == 0u || T > 65535u || precision > K3_MOE_MFMA_FP8) return false;
    if (precision != K3_MOE_EXACT && T > 1u && !mfma_supported(*s)) return false;
    return true;
}

DecodeParams decode_params(const Workspace &ws, void *output, const void *hidden,
                           const void *residual, const void *router_weight,
                           const void *router_bias, const k3_moe_expert *experts,
                           const k3_moe_shape &s, void *ids_copy, void *w_copy) {
    DecodeParams P{};
    P.output = (uint16_t *)output;
    P.residual = (const uint16_t *)residual;
    P.hidden_in = (const uint16_t *)hidden;
    P.router_in = (const uint16_t *)hidden;
    P.router_cols = s.hidden;
    P.router_weight = (const uint16_t *)router_weight;
    P.router_bias = (const float *)router_bias;
    P.experts = experts;
    P.logits = ws.logits;
    P.scores = ws.scores;
    P.keys = ws.keys;
    P.ids = ws.ids;
    P.weights = ws.weights;
    P.ids_copy = (uint32_t *)ids_copy;
    P.weights_copy = (float *)w_copy;
    P.act = ws.act;
    P.sel = ws.sel;
    P.y = ws.y;
    P.slot_mask = ws.summary + 3;
    P.hidden = s.hidden;
    P.ffn = s.ffn;
    P.expert_count = s.expert_count;
    P.top_k = s.top_k;
    P.scale = s.scaling_factor;
    P.activation = s.activation;
    P.beta = s.activation == 1u ? 1.0f : s.beta;
    P.linear_beta = s.activation == 1u ? 1.0f : s.linear_beta;
    return P;
}

/* Experts the MFMA path hands to the exact kernels (tensors not 8-byte
 * aligned) are walked by a grid of this many expert rows: with none, the
 * blocks exit at once. */
constexpr uint32_t kFallbackExperts = 8;
/* column blocks of the hand-off grid (each walks the rest): an empty list
 * then costs a launch of 8 x 32 blocks, not thousands */
constexpr uint32_t kFallbackCols = 32;

/* Expert stage on routes already in ws.ids / ws.weights. */
bool run_experts(const Workspace &ws, void *output, const void *hidden, const void *residual,
                 const k3_moe_expert *experts, const k3_moe_shape &s, uint32_t T,
                 uint32_t precision, hipStream_t st, const StageMarker &mark) {
    const uint32_t H = s.hidden, F = s.ffn, E = s.expert_count, k = s.top_k;
    const float beta = s.activation == 1u ? 1.0f : s.beta;
    const float lb = s.activation == 1u ? 1.0f : s.linear_beta;
    if (T == 1u && decode_supported(s)) { /* every precision: exact decode */
        const DecodeParams P = decode_params(ws, output, hidden, residual, nullptr, nullptr,
                                             experts, s, nullptr, nullptr);
        return decode_launch_experts(P, st, mark, true);
    }
    mark(K3_MOE_STAGE_PLAN);
    if (!launch_plan(ws.counts, ws.offsets, ws.unique, ws.summary, ws.token_index,
                     ws.route_index, ws.chunk_base, ws.ids, T, k, E, st))
        return false;
    const uint32_t upper = (uint64_t)T * k < E ? T * k : E;
    /* weight rows per wave and tokens per weight load: gate/up 2 x 2
     * (255 VGPRs), down 4 x 4 (two waves per SIMD). Measured against 4 x 4
     * / 2 x 2 / 2 x 1 / 1 x 2 shapes on cfg3 and cfg4: 26.5 and 387 ms per
     * layer, the next best 29.2 and 419 ms. */
    constexpr int RW = 2, TT = 2, RB = 4, TD = 4;
    if (precision != K3_MOE_EXACT) {
        if (!mfma_launch_experts(ws.mfma, ws.y, (const uint16_t *)hidden, ws.counts, ws.offsets,
                                 ws.token_index, ws.route_index, experts, s, T,
                                 precision == K3_MOE_MFMA ? 2u : 1u, st, mark))
            return false;
        /* experts with a tensor that is not 8-byte aligned (no MFMA tiles):
         * the exact kernels, after the MFMA down kernel has consumed the
         * activation codes that share `act` */
        const uint32_t walk = upper < kFallbackExperts ? upper : kFallbackExperts;
        const uint32_t gx = F / (4u * RW) < kFallbackCols ? F / (4u * RW) : kFallbackCols;
        const uint32_t dx = H / (4u * RB) < kFallbackCols ? H / (4u * RB) : kFallbackCols;
        ExactWork W{};
        W.list_count = ws.mfma.unaligned;
        W.list = ws.mfma.unaligned + 1;
        W.counts = ws.counts;
        W.offsets = ws.offsets;
        hipLaunchKernelGGL(HIP_KERNEL_NAME(grouped_gateup_kernel<RW, TT>),
                           dim3(gx, walk), dim3(256), 0, st, ws.act,
                           (const uint16_t *)hidden, W, ws.token_index, experts, H, F,
                           s.activation, beta, lb);
        hipLaunchKernelGGL(HIP_KERNEL_NAME(grouped_down_kernel<RB, TD>), dim3(dx, walk),
                           dim3(256), 0, st, ws.y, ws.act, W, ws.route_index, experts, H, F);
        mark(K3_MOE_STAGE_COMBINE);
        hipLaunchKernelGGL(combine_kernel, dim3((H / 8u + kCombineThreads - 1u) / kCombineThreads, T),
                           dim3(kCombineThreads), 0, st, (uint16_t *)output, ws.y,
                           (const uint16_t *)residual, ws.ids, ws.weights, H, k, E);
        mark(K3_MOE_STAGE_END);
        return hipGetLastError() == hipSuccess;
    }
    mark(K3_MOE_STAGE_GATE_UP);
    /* exact: workgroups over the tile lists of every selected expert */
    if (!build_tiles_all(ws.mfma, ws.counts, ws.offsets, experts, E, st)) return false;
    ExactWork W{};
    W.tiles = ws.mfma.tiles;
    W.tile_count = ws.mfma.tile_count;
    for (int c = 0; c < kTileClasses; c++) W.cap[c] = ws.mfma.tile_cap[c];
    W.counts = ws.counts;
    W.offsets = ws.offsets;
    hipLaunchKernelGGL(HIP_KERNEL_NAME(grouped_gateup_kernel<RW, TT>), dim3(F / (4u * RW), upper),
                       dim3(256), 0, st, ws.act, (const uint16_t *)hidden, W, ws.token_index,
                       experts, H, F, s.activation, beta, lb);
    mark(K3_MOE_STAGE_DOWN);
    hipLaunchKernelGGL(HIP_KERNEL_NAME(grouped_down_kernel<RB, TD>), dim3(H / (4u * RB), upper),
                       dim3(256), 0, st, ws.y, ws.act, W, ws.route_index, experts, H, F);
    mark(K3_MOE_STAGE_COMBINE);
    hipLaunchKernelGGL(combine_kernel, dim3((H / 8u + kCombineThreads - 1u) / kCombineThreads, T),
                       dim3(kCombineThreads), 0, st, (uint16_t *)output, ws.y,
                       (const uint16_t *)residual, ws.ids, ws.weights, H, k, E);
    mark(K3_MOE_STAGE_END);
    return hipGetLastError() == hipSuccess;
}

}  // namespace

/* ======================================================================== */
/* C ABI                                                                     */
/* ======================================================================== */

extern "C" size_t k3_moe_workspace_bytes(const k3_moe_shape *shape, uint32_t token_count) {
    if (!shape_ok(shape) || token_count == 0u || token_count > 65535u) return 0u;
    return carve(nullptr, *shape, token_count).bytes;
}

extern "C" bool k3_moe_workspace_init(void *workspace, size_t workspace_bytes, void *stream) {
    if (!workspace || workspace_bytes == 0u) return false;
    (void)stream;
    return true;
}

extern "C" size_t k3_moe_plan_scratch_bytes(uint32_t token_count, uint32_t expert_count) {
    return plan_scratch(token_count, expert_count);
}

extern "C" bool k3_moe_route_plan(uint32_t *counts, uint32_t *offsets, uint32_t *unique,
                                  uint32_t *summary, uint32_t *token_index,
                                  uint32_t *route_index, const uint32_t *expert_ids,
                                  uint32_t token_count, uint32_t top_k, uint32_t expert_count,
                                  void *scratch, size_t scratch_bytes, void *stream) {
    if (!counts || !offsets || !unique || !summary || !token_index || !route_index ||
        !expert_ids || !scratch || token_count == 0u || token_count > 65535u || top_k == 0u ||
        top_k > 32u || expert_count == 0u || expert_count > 1024u ||
        scratch_bytes < plan_scratch(token_count, expert_count))
        return false;
    return launch_plan(counts, offsets, unique, summary, token_index, route_index,
                       (uint32_t *)scratch, expert_ids, token_count, top_k, expert_count,
                       (hipStream_t)stream);
}

extern "C" bool k3_moe_experts_bf16(void *output, const void *hidden, const void *residual,
                                    const void *expert_ids, const void *expert_weights,
                                    const k3_moe_expert *experts, const k3_moe_shape *shape,
                                    uint32_t token_count, uint32_t precision, void *workspace,
                                    size_t workspace_bytes, void *stream) {
    if (!output || !hidden || !expert_ids || !expert_weights || !experts || !workspace ||
        !precision_ok(shape, token_count, precision) || !rows_aligned(output, hidden, residual))
        return false;
    Workspace ws = carve(workspace, *shape, token_count);
    if (workspace_bytes < ws.bytes) return false;
    const hipStream_t st = (hipStream_t)stream;
    const size_t route_bytes = (size_t)token_count * shape->top_k * 4u;
    if (hipMemcpyAsync(ws.ids, expert_ids, route_bytes, hipMemcpyDeviceToDevice, st) != hipSuccess ||
        hipMemcpyAsync(ws.weights, expert_weights, route_bytes, hipMemcpyDeviceToDevice, st) !=
            hipSuccess)
        return false;
    return run_experts(ws, output, hidden, residual, experts, *shape, token_count, precision, st,
                       StageMarker{nullptr, st});
}

/* Routes of a token batch into ws.ids / ws.weights (and the caller's
 * copies): the certified MFMA router from kCertifiedMinTokens tokens on,
 * the exact w64 logits + top-k below that; both give the same bits. */

static bool route_batch(const Workspace &ws, const void *hidden, const void *router_weight,
                 const void *router_bias, const k3_moe_shape &s, uint32_t T, void *expert_ids,
                 void *expert_weights, hipStream_t st, const StageMarker *mark) {
    const uint32_t E = s.expert_count, H = s.hidden, k = s.top_k;
    if (T >= kCertifiedMinTokens && router_certified_supported(T, E, H, k, router_weight, hidden))
        return launch_router_certified(ws.ids, ws.weights, (uint32_t *)expert_ids,
                                       (float *)expert_weights, ws.logits, ws.scores,
                                       router_weight, router_bias, hidden, T, E, H, k,
                                       s.scaling_factor, st, mark);
    if (!launch_bf16_rows_f32_any(ws.logits, router_weight, hidden, T, E, H, st)) return false;
    if (mark) (*mark)(K3_MOE_STAGE_TOPK);
    return launch_router_topk(ws.ids, ws.weights, (uint32_t *)expert_ids, (float *)expert_weights,
                              ws.logits, (const float *)router_bias, T, E, k, s.scaling_factor,
                              st);
}

extern "C" bool k3_moe_forward_profiled_bf16(void *output, const void *hidden, const void *residual,
                                    const void *router_weight, const void *router_bias,
                                    const k3_moe_expert *experts, const k3_moe_shape *shape,
                                    uint32_t token_count, uint32_t precision, void *expert_ids,
                                    void *expert_weights, void *workspace,
                                    size_t workspace_bytes, const k3_moe_profile *profile,
                                    void *stream) {
    if (!output || !hidden || !router_weight || !router_bias || !experts || !workspace ||
        !precision_ok(shape, token_count, precision) || !rows_aligned(output, hidden, residual))
        return false;
    Workspace ws = carve(workspace, *shape, token_count);
    if (workspace_bytes < ws.bytes) return false;
    const hipStream_t st = (hipStream_t)stream;
    const StageMarker mark{profile, st};
    if (token_count == 1u && decode_supported(*shape) && ((uintptr_t)router_weight % 16u) == 0u) {
        const DecodeParams P = decode_params(ws, output, hidden, residual, router_weight,
                                             router_bias, experts, *shape, expert_ids,
                                             expert_weights);
        return decode_launch(P, st, mark);
    }
    mark(K3_MOE_STAGE_ROUTER);
    if (!route_batch(ws, hidden, router_weight, router_bias, *shape, token_count, expert_ids,
                     expert_weights, st, &mark))
        return false;
    return run_experts(ws, output, hidden, residual, experts, *shape, token_count, precision, st,
                       mark);
}

extern "C" bool k3_moe_routed_bf16(void *output, const void *router_input,
                                   uint32_t router_columns, const void *expert_input,
                                   const void *residual, const void *router_weight,
                                   const void *router_bias, const k3_moe_expert *experts,
                                   const k3_moe_shape *shape, uint32_t token_count,
                                   uint32_t precision, void *expert_ids, void *expert_weights,
                                   void *workspace, size_t workspace_bytes, void *stream) {
    if (!output || !router_input || !expert_input || !router_weight || !router_bias ||
        !experts || !workspace || router_columns == 0u ||
        !precision_ok(shape, token_count, precision) ||
        !rows_aligned(output, expert_input, residual) ||
        (((uintptr_t)router_input | (uintptr_t)router_weight) % 16u) != 0u ||
        router_columns % 8u != 0u)
        return false;
    Workspace ws = carve(workspace, *shape, token_count);
    if (workspace_bytes < ws.bytes) return false;
    const hipStream_t st = (hipStream_t)stream;
    const StageMarker mark{nullptr, st};
    if (token_count == 1u && decode_supported(*shape) && router_columns <= 8192u) {
        DecodeParams P = decode_params(ws, output, expert_input, residual, router_weight,
                                       router_bias, experts, *shape, expert_ids, expert_weights);
        P.router_in = (const uint16_t *)router_input;
        P.router_cols = router_columns;
        return decode_launch(P, st, mark);
    }
    k3_moe_shape rs = *shape; /* the router's width */
    rs.hidden = router_columns;
    if (!route_batch(ws, router_input, router_weight, router_bias, rs, token_count, expert_ids,
                     expert_weights, st, &mark))
        return false;
    return run_experts(ws, output, expert_input, residual, experts, *shape, token_count,
                       precision, st, mark);
}

namespace {

bool native_decode_args_ok(const void *x, uint32_t router_cols, const void *router_weight,
                           const k3_moe_shape &shape) {
    return k3::decode_supported(shape) && router_cols != 0u && router_cols % 8u == 0u &&
           router_cols <= 8192u && (((uintptr_t)x | (uintptr_t)router_weight) % 16u) == 0u;
}

}  // namespace

bool k3::native_decode_router_rows(RouterRows *out, const void *x, uint32_t router_cols,
                                   const void *router_weight, const void *router_bias,
                                   const k3_moe_shape &shape, void *workspace,
                                   size_t workspace_bytes) {
    if (!native_decode_args_ok(x, router_cols, router_weight, shape)) return false;
    const Workspace ws = carve(workspace, shape, 1u);
    if (workspace_bytes < ws.bytes) return false;
    *out = RouterRows{(const uint16_t *)router_weight, (const float *)router_bias,
                      (const uint16_t *)x, ws.logits, ws.scores, ws.keys, shape.expert_count,
                      router_cols};
    return true;
}

bool k3::native_decode_experts(void *routed_out, const void *x, uint32_t router_cols,
                               const void *latent, const void *router_weight,
                               const void *router_bias, const k3_moe_expert *experts,
                               const k3_moe_shape &shape, void *ids_copy, void *w_copy,
                               void *workspace, size_t workspace_bytes, hipEvent_t latent_ready,
                               bool routed, hipStream_t st) {
    if (!native_decode_args_ok(x, router_cols, router_weight, shape)) return false;
    Workspace ws = carve(workspace, shape, 1u);
    if (workspace_bytes < ws.bytes) return false;
    DecodeParams P = decode_params(ws, routed_out, latent, nullptr, router_weight, router_bias,
                                   experts, shape, ids_copy, w_copy);
    P.router_in = (const uint16_t *)x;
    P.router_cols = router_cols;
    const StageMarker mark{nullptr, st};
    if (!(routed ? decode_launch_topk(P, st, mark) : decode_launch_route(P, st, mark)))
        return false;
    if (latent_ready && hipStreamWaitEvent(st, latent_ready, 0) != hipSuccess) return false;
    return decode_launch_experts(P, st, mark, false);
}

extern "C" bool k3_moe_forward_bf16(void *output, const void *hidden, const void *residual,
                                    const void *router_weight, const void *router_bias,
                                    const k3_moe_expert *experts, const k3_moe_shape *shape,
                                    uint32_t token_count, uint32_t precision, void *expert_ids,
                                    void *expert_weights, void *workspace,
                                    size_t workspace_bytes, void *stream) {
    return k3_moe_forward_profiled_bf16(output, hidden, residual, router_weight, router_bias,
                                        experts, shape, token_count, precision, expert_ids,
                                        expert_weights, workspace, workspace_bytes, nullptr,
                                        stream);
}

/* ======================================================================== */
/* Workspace-free entry point                                                */
/* ======================================================================== */

/*
 * The workspace of k3_moe_forward_static_bf16: one array per GPU, held
 * until the process ends. Host code never uses the array's name as an
 * address (on the host it is only a stand-in for the symbol): the device
 * address of the current GPU's copy comes from hipGetSymbolAddress, once
 * per device, and only that pointer is passed to kernels.
 */
static __device__ __align__(256) uint8_t scratch[K3_MOE_STATIC_WORKSPACE_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices];

/* Device address of the current GPU's scratch array, or nullptr. */
void *static_workspace() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) {
            fprintf(stderr, "k3_moe_forward_static_bf16: hipGetSymbolAddress failed on device %d\n",
                    dev);
            return nullptr;
        }
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
}

}  // namespace

extern "C" bool k3_moe_forward_static_bf16(void *output, const void *hidden, const void *residual,
                                           const void *router_weight, const void *router_bias,
                                           const k3_moe_expert *experts,
                                           const k3_moe_shape *shape, uint32_t token_count,
                                           uint32_t precision, void *expert_ids,
                                           void *expert_weights, void *stream) {
    const size_t need = k3_moe_workspace_bytes(shape, token_count);
    if (need == 0u) return false;
    if (need > (size_t)K3_MOE_STATIC_WORKSPACE_BYTES) {
        fprintf(stderr,
                "k3_moe_forward_static_bf16: %u tokens need %zu bytes of workspace, above the "
                "static maximum of %u bytes; use k3_moe_forward_bf16 with a caller workspace\n",
                token_count, need, (unsigned)K3_MOE_STATIC_WORKSPACE_BYTES);
        return false;
    }
    void *ws = static_workspace();
    if (!ws) return false;
    /* The layer keeps no state in its workspace between calls (every
     * buffer is written before it is read), so nothing is cleared here. */
    return k3_moe_forward_profiled_bf16(output, hidden, residual, router_weight, router_bias,
                                        experts, shape, token_count, precision, expert_ids,
                                        expert_weights, ws, need, nullptr, stream);
}

extern "C" bool k3_moe_synth_fill(void *base, uint64_t bytes, uint64_t seed, uint64_t stream_id,
                                  uint32_t kind, void *stream) {
    if (!base || bytes == 0u || kind > 1u || ((uintptr_t)base % 8u) != 0u) return false;
    hipLaunchKernelGGL(synth_fill_kernel, dim3(2048), dim3(256), 0, (hipStream_t)stream,
                       (uint8_t *)base, bytes, synth_key(seed, stream_id), kind);
    return hipGetLastError() == hipSuccess;
}

extern "C" void k3_moe_synth_fill_host(void *base, uint64_t bytes, uint64_t seed,
                                       uint64_t stream_id, uint32_t kind) {
    const uint64_t key = synth_key(seed, stream_id);
    uint8_t *p = (uint8_t *)base;
    uint64_t i = 0;
    if (kind == 0u)
        for (; i + 8u <= bytes; i += 8u) {
            const uint64_t w = synth_word(key, i >> 3);
            memcpy(p + i, &w, 8);
        }
    for (; i < bytes; i++) p[i] = synth_byte(key, i, kind);
}
