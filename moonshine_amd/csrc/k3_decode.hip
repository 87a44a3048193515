/*
 * Single-token decode of the routed-MoE layer on gfx950: five kernels.
 *
 *   router_kernel   4 expert rows per block (one wave each): logit,
 *                   sigmoid score and order key per expert.
 *   topk_kernel     one wave selects the routes (k3_topk.h) and resolves
 *                   the k selected expert descriptors once, so the expert
 *                   kernels reach their weights through a single load.
 *   gateup_kernel   one block per (slot, 8 F-rows): each of its four waves
 *                   streams one 64-group K-stripe of the 8 gate and 8 up
 *                   rows (a coalesced 1 KB row-stripe per load), group sums
 *                   meet in LDS and are combined in the w64 lane order, then
 *                   the activation. 4096 blocks keep ~64 MB of loads in
 *                   flight.
 *   down_kernel     one block per (slot, 4 x 16 rows): each wave streams a
 *                   contiguous 16-row stripe of the slot's down matrix
 *                   (16 KB in flight per wave) and writes bf16 y[slot].
 *   combine_kernel  rank-order weighted sum of the k slot rows plus the
 *                   residual.
 *
 * Every hand-off is a kernel boundary, so all loads and stores are plain
 * (cached). Fusing the stages into one launch was measured and dropped on
 * this part: a cooperative launch alone cost ~18 us, an agent-scope release
 * fence is an L2 write-back (~100 us across a few hundred blocks), and the
 * device-coherent loads/stores that replace it each cost a ~4 us memory
 * round trip under streaming load, which stretched block lifetimes more
 * than the removed kernel boundaries saved (back-to-back kernels here show
 * no gap in the trace).
 */
#include "k3_device.h"
#include "k3_internal.h"
#include "k3_decode.h"
#include "k3_topk.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace k3 {
namespace {

constexpr int kRouterMaxChunks = 16;  /* hidden <= 8192 */
constexpr int kGU = 8;                /* gate (and up) rows per gate/up block */
constexpr int kDownRows = 16;         /* rows per down wave (F <= 2048) */

/* ---------------------------------------------------------------------- */
/* router                                                                  */
/* ---------------------------------------------------------------------- */

/* Rows 4b..4b+3, w64 order (elements in chunks of 8; lane l owns chunks
 * l, l+64, ...; fmaf in column order; wave64 butterfly). Each wave loads
 * its weight row and the hidden state (cache hits after the first wave)
 * in one batch, so the whole row costs a single memory round trip. */
__global__ __launch_bounds__(256) void router_kernel(DecodeParams P) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t chunks = P.hidden / 8u;
    const uint32_t row = 4u * blockIdx.x + (threadIdx.x >> 6);
    if (row >= P.expert_count) return;
    const uint4 *w4 = (const uint4 *)(P.router_weight + (uint64_t)row * P.hidden);
    const uint4 *x4 = (const uint4 *)P.hidden_in;
    uint4 wv[kRouterMaxChunks], xv[kRouterMaxChunks];
#pragma unroll
    for (int j = 0; j < kRouterMaxChunks; j++) {
        /* out-of-range chunks load chunk 0 and are skipped below */
        const uint32_t c = lane + 64u * j < chunks ? lane + 64u * j : 0u;
        wv[j] = w4[c];
        xv[j] = x4[c];
    }
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < kRouterMaxChunks; j++) {
        if (lane + 64u * j < chunks) {
            a = fmaf(bf16_lo(wv[j].x), bf16_lo(xv[j].x), a); a = fmaf(bf16_hi(wv[j].x), bf16_hi(xv[j].x), a);
            a = fmaf(bf16_lo(wv[j].y), bf16_lo(xv[j].y), a); a = fmaf(bf16_hi(wv[j].y), bf16_hi(xv[j].y), a);
            a = fmaf(bf16_lo(wv[j].z), bf16_lo(xv[j].z), a); a = fmaf(bf16_hi(wv[j].z), bf16_hi(xv[j].z), a);
            a = fmaf(bf16_lo(wv[j].w), bf16_lo(xv[j].w), a); a = fmaf(bf16_hi(wv[j].w), bf16_hi(xv[j].w), a);
        }
    }
    const float v = wave_sum(a);
    if (lane == 0u) {
        const float score = det_sigmoid(v);
        P.logits[row] = v;
        P.scores[row] = score;
        P.keys[row] = choice_key(score, P.router_bias[row]);
    }
}

/* ---------------------------------------------------------------------- */
/* top-k + expert descriptors                                              */
/* ---------------------------------------------------------------------- */

/* Lane s < top_k stores the descriptor of route s (id `e`) and the wave
 * publishes the mask of slots that have an expert. One wave. */
__device__ __forceinline__ void resolve_slot(const DecodeParams &P, uint32_t e) {
    const uint32_t s = threadIdx.x;
    k3_moe_expert d{};
    if (s < P.top_k && e < P.expert_count) d = P.experts[e];
    if (s < P.top_k) P.sel[s] = d;
    const uint64_t live = __ballot(s < P.top_k && d.down_packed != nullptr);
    if (s == 0u) *P.slot_mask = (uint32_t)live;
}

/* One wave: select, then resolve the selected descriptors straight from
 * the ids the selection leaves in registers. */
__global__ __launch_bounds__(64) void topk_kernel(DecodeParams P) {
    __shared__ TopkWaveSmem sm;
    const uint32_t lane = threadIdx.x;
    uint32_t key[kTopkSlots];
    float score[kTopkSlots];
#pragma unroll
    for (int j = 0; j < kTopkSlots; j++) {
        const uint32_t e = lane + 64u * j;
        key[j] = e < P.expert_count ? P.keys[e] : 0u;
        score[j] = e < P.expert_count ? P.scores[e] : 0.0f;
    }
    const uint32_t id = topk_select_wave(key, score, P.top_k, P.scale, P.ids, P.weights,
                                         P.ids_copy, P.weights_copy, sm);
    resolve_slot(P, id);
}

/* descriptors for routes given by the caller */
__global__ __launch_bounds__(64) void resolve_kernel(DecodeParams P) {
    resolve_slot(P, threadIdx.x < P.top_k ? P.ids[threadIdx.x] : UINT32_MAX);
}

/* ---------------------------------------------------------------------- */
/* gate/up                                                                 */
/* ---------------------------------------------------------------------- */

struct GateUpSmem {
    float part[2 * kGU][4][64];
    float scl[2 * kGU][4][64];
};

/* grid (F / kGU, k), block 256; H <= 8192 (four 64-group stripes). */
__global__ __launch_bounds__(256) void gateup_kernel(DecodeParams P) {
    __shared__ GateUpSmem sm;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t slot = blockIdx.y, row0 = blockIdx.x * kGU;
    const uint32_t H = P.hidden, G = H / 32u;
    const k3_moe_expert ex = P.sel[slot];
    uint16_t *dst = P.act + (uint64_t)slot * P.ffn + row0;
    if (!ex.gate_packed) {
        if (threadIdx.x < (uint32_t)kGU) dst[threadIdx.x] = 0;
        return;
    }
    const uint32_t g = 64u * wave + lane;
    if (g < G) {
        const uint8_t *gp = (const uint8_t *)ex.gate_packed + (uint64_t)row0 * (H / 2u) + 16u * g;
        const uint8_t *up = (const uint8_t *)ex.up_packed + (uint64_t)row0 * (H / 2u) + 16u * g;
        const uint8_t *gs = (const uint8_t *)ex.gate_scales + (uint64_t)row0 * G + g;
        const uint8_t *us = (const uint8_t *)ex.up_scales + (uint64_t)row0 * G + g;
        uint4 w[2 * kGU];
        uint32_t sc[2 * kGU];
#pragma unroll
        for (int i = 0; i < kGU; i++) {
            w[i] = gload((const uint4 *)(gp + (uint64_t)i * (H / 2u)));
            w[kGU + i] = gload((const uint4 *)(up + (uint64_t)i * (H / 2u)));
            sc[i] = gload(gs + (uint64_t)i * G);
            sc[kGU + i] = gload(us + (uint64_t)i * G);
        }
        float xf[32];
        bf16x32_to_f32((const uint4 *)P.hidden_in + 4u * g, xf);
#pragma unroll
        for (int r = 0; r < 2 * kGU; r++) {
            sm.part[r][wave][lane] = fp4_group(w[r], xf);
            sm.scl[r][wave][lane] = e8m0_to_f32(sc[r]);
        }
    }
    __syncthreads();
    /* wave w: gate rows 2w, 2w+1 and the same up rows; lane l's groups
     * l, l+64, ... in order */
    constexpr int RPW = kGU / 4;
    const uint32_t stripes = (G + 63u) / 64u;
    float p[2 * RPW];
#pragma unroll
    for (int q = 0; q < 2 * RPW; q++) {
        const int r = (q / RPW) * kGU + (int)wave * RPW + (q % RPW);
        float acc = 0.0f;
        for (uint32_t j = 0; j < stripes; j++)
            if (64u * j + lane < G) acc = fmaf(sm.part[r][j][lane], sm.scl[r][j][lane], acc);
        p[q] = acc;
    }
    const float v = wave_sum_rows<2 * RPW>(p); /* lanes < 32: gate, lanes >= 32: up */
    const float u = __shfl_xor(v, 32, 64);
    const float gb = bf16_to_f32(f32_to_bf16(v)), ub = bf16_to_f32(f32_to_bf16(u));
    const uint16_t bits = f32_to_bf16(gated_act(gb, ub, P.activation, P.beta, P.linear_beta));
    /* gate row r of this wave sits on lanes 32 r / RPW .. (the up row r on
     * the same lanes + 32) */
    constexpr uint32_t kSpan = 32u / RPW;
    if (lane < 32u && (lane & (kSpan - 1u)) == 0u) dst[RPW * wave + lane / kSpan] = bits;
}

/* ---------------------------------------------------------------------- */
/* down                                                                    */
/* ---------------------------------------------------------------------- */

/*
 * Down projection per route slot, shaped like gateup_kernel so the weight
 * stream keeps many small blocks in flight: grid (H / (4 RB), k), block
 * 256; wave w of block (b, slot) computes rows (4b + w) RB .. + RB of slot
 * `slot` -- a contiguous RB-row stripe of its down matrix, all loads issued
 * at once. Lane l owns groups l, l + 64, ... (M of them: F <= 2048 M); per
 * row the group sum runs over the 32 columns in order, with 8-column
 * chunks of the activation converted once for the RB rows. Output y[slot,
 * d] = bf16(row sum), the reference's per-slot GEMV result
 * (k3_engine.cu:1058-1060).
 */
template <int M, int RB>
__global__ __launch_bounds__(256) void down_kernel(DecodeParams P) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t slot = blockIdx.y;
    const uint32_t row0 = (4u * blockIdx.x + wave) * RB;
    const uint32_t F = P.ffn, G = F / 32u;
    uint16_t *y = P.y + (uint64_t)slot * P.hidden + row0;
    const k3_moe_expert ex = P.sel[slot];
    if (!ex.down_packed) {
        if (lane < (uint32_t)RB) y[lane] = 0;
        return;
    }
    float acc[RB];
#pragma unroll
    for (int i = 0; i < RB; i++) acc[i] = 0.0f;
    const uint8_t *dp = (const uint8_t *)ex.down_packed + (uint64_t)row0 * (F / 2u);
    const uint8_t *ds = (const uint8_t *)ex.down_scales + (uint64_t)row0 * G;
    const uint4 *a4 = (const uint4 *)(P.act + (uint64_t)slot * F);
#pragma unroll
    for (int m = 0; m < M; m++) {
        const uint32_t g = lane + 64u * m;
        if (g < G) {
            uint4 w[RB], xr[4];
            uint32_t sc[RB];
#pragma unroll
            for (int i = 0; i < RB; i++) {
                w[i] = gload((const uint4 *)(dp + (uint64_t)i * (F / 2u) + 16u * g));
                sc[i] = gload(ds + (uint64_t)i * G + g);
            }
#pragma unroll
            for (int q = 0; q < 4; q++) xr[q] = gload(a4 + 4u * g + q);
            float gs[RB];
#pragma unroll
            for (int i = 0; i < RB; i++) gs[i] = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float x8[8] = {bf16_lo(xr[q].x), bf16_hi(xr[q].x), bf16_lo(xr[q].y),
                                     bf16_hi(xr[q].y), bf16_lo(xr[q].z), bf16_hi(xr[q].z),
                                     bf16_lo(xr[q].w), bf16_hi(xr[q].w)};
#pragma unroll
                for (int i = 0; i < RB; i++) {
                    const uint32_t wq = q == 0 ? w[i].x : q == 1 ? w[i].y : q == 2 ? w[i].z : w[i].w;
                    gs[i] = fp4_dot8(wq, x8, gs[i]);
                }
            }
#pragma unroll
            for (int i = 0; i < RB; i++) acc[i] = fmaf(gs[i], e8m0_to_f32(sc[i]), acc[i]);
        }
    }
    const float v = wave_sum_rows<RB>(acc);
    const int owner = wave_rows_owner<RB>();
    if ((lane & (64u / RB - 1u)) == 0u) y[owner] = f32_to_bf16(v);
}

/*
 * out[d] = bf16(residual[d] + bf16(sum_r w[r] * y[r, d])): fp32, rank order
 * from 0, product and sum rounded separately (k3_rocm_ops.cu:1452-1510).
 * One thread per output element.
 */
__global__ __launch_bounds__(256) void combine_kernel(DecodeParams P) {
    const uint32_t d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= P.hidden) return;
    /* every load is issued before the first use: one memory round trip */
    float wv[32], yv[32];
    const uint32_t live = *P.slot_mask;
    const uint16_t *rp = P.residual ? P.residual : P.y; /* unconditional load */
    const float r = bf16_to_f32(rp[d]);
#pragma unroll
    for (int s = 0; s < 32; s++) { /* unconditional loads (slot 0 stands in) */
        const uint32_t q = (uint32_t)s < P.top_k ? (uint32_t)s : 0u;
        wv[s] = P.weights[q];
        yv[s] = bf16_to_f32(P.y[(uint64_t)q * P.hidden + d]);
    }
    float c = 0.0f;
#pragma unroll
    for (int s = 0; s < 32; s++)
        if ((live >> s) & 1u) c = __fadd_rn(c, __fmul_rn(wv[s], yv[s]));
    const float cb = bf16_to_f32(f32_to_bf16(c));
    P.output[d] = P.residual ? f32_to_bf16(__fadd_rn(r, cb)) : f32_to_bf16(cb);
}

}  // namespace

bool decode_supported(const k3_moe_shape &s) {
    return s.hidden % (s.ffn <= 2048u ? 64u : 32u) == 0u && s.hidden <= 8192u && s.ffn % 32u == 0u && s.ffn <= 4096u &&
           s.top_k <= 32u && s.expert_count <= 1024u;
}

bool decode_launch(const DecodeParams &P, hipStream_t st, const StageMarker &mark) {
    mark(K3_MOE_STAGE_ROUTER);
    hipLaunchKernelGGL(router_kernel, dim3((P.expert_count + 3u) / 4u), dim3(256), 0, st, P);
    mark(K3_MOE_STAGE_TOPK);
    hipLaunchKernelGGL(topk_kernel, dim3(1), dim3(64), 0, st, P);
    return decode_launch_experts(P, st, mark, false);
}

bool decode_launch_experts(const DecodeParams &P, hipStream_t st, const StageMarker &mark,
                           bool resolve) {
    mark(K3_MOE_STAGE_PLAN);
    if (resolve) hipLaunchKernelGGL(resolve_kernel, dim3(1), dim3(64), 0, st, P);
    mark(K3_MOE_STAGE_GATE_UP);
    hipLaunchKernelGGL(gateup_kernel, dim3(P.ffn / kGU, P.top_k), dim3(256), 0, st, P);
    mark(K3_MOE_STAGE_DOWN);
    const dim3 block(256);
    if (P.ffn <= 2048u)
        hipLaunchKernelGGL(HIP_KERNEL_NAME(down_kernel<1, kDownRows>),
                           dim3(P.hidden / (4u * kDownRows), P.top_k), block, 0, st, P);
    else
        hipLaunchKernelGGL(HIP_KERNEL_NAME(down_kernel<2, kDownRows / 2>),
                           dim3(P.hidden / (2u * kDownRows), P.top_k), block, 0, st, P);
    mark(K3_MOE_STAGE_COMBINE);
    hipLaunchKernelGGL(combine_kernel, dim3((P.hidden + 255u) / 256u), block, 0, st, P);
    mark(K3_MOE_STAGE_END);
    return hipGetLastError() == hipSuccess;
}

}  // namespace k3
