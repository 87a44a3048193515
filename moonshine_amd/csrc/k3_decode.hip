/*
 * Single-token decode of the routed-MoE layer on gfx950: four kernels.
 *
 *   router_kernel   4 expert rows per block (one wave each, x staged in
 *                   LDS): logit, sigmoid score and order key per expert.
 *   topk_kernel     one wave selects the routes (k3_topk.h) and resolves
 *                   the k selected expert descriptors once, so the expert
 *                   kernels reach their weights through a single load.
 *   gateup_kernel   one block per (slot, 8 F-rows): each of its four waves
 *                   streams one 64-group K-stripe of the 8 gate and 8 up
 *                   rows (a coalesced 1 KB row-stripe per load), group sums
 *                   meet in LDS and are combined in the w64 lane order, then
 *                   the activation. 4096 blocks keep ~64 MB of loads in
 *                   flight.
 *   down_kernel     one block per 8 output rows for all k slots (each wave
 *                   streams contiguous 8-row stripes of four slots' down
 *                   matrices), then the rank-order weighted combine plus
 *                   the residual.
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
constexpr int kRB = 8;                /* output rows per down block */

/* ---------------------------------------------------------------------- */
/* router                                                                  */
/* ---------------------------------------------------------------------- */

/* Rows 4b..4b+3, w64 order (elements in chunks of 8; lane l owns chunks
 * l, l+64, ...; fmaf in column order; wave64 butterfly). */
__global__ __launch_bounds__(256) void router_kernel(DecodeParams P) {
    __shared__ uint4 xs[kRouterMaxChunks * 64];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t chunks = P.hidden / 8u;
    const uint32_t row = 4u * blockIdx.x + (threadIdx.x >> 6);
    const bool live = row < P.expert_count;
    /* this row's weights go out first; x is staged while they are in flight */
    uint4 wv[kRouterMaxChunks];
    if (live) {
        const uint4 *w4 = (const uint4 *)(P.router_weight + (uint64_t)row * P.hidden);
#pragma unroll
        for (int j = 0; j < kRouterMaxChunks; j++) {
            const uint32_t c = lane + 64u * j;
            if (c < chunks) wv[j] = w4[c];
        }
    }
    for (uint32_t c = threadIdx.x; c < chunks; c += blockDim.x)
        xs[c] = ((const uint4 *)P.hidden_in)[c];
    __syncthreads();
    if (!live) return;
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < kRouterMaxChunks; j++) {
        const uint32_t c = lane + 64u * j;
        if (c < chunks) {
            const uint4 xv = xs[c];
            a = fmaf(bf16_lo(wv[j].x), bf16_lo(xv.x), a); a = fmaf(bf16_hi(wv[j].x), bf16_hi(xv.x), a);
            a = fmaf(bf16_lo(wv[j].y), bf16_lo(xv.y), a); a = fmaf(bf16_hi(wv[j].y), bf16_hi(xv.y), a);
            a = fmaf(bf16_lo(wv[j].z), bf16_lo(xv.z), a); a = fmaf(bf16_hi(wv[j].z), bf16_hi(xv.z), a);
            a = fmaf(bf16_lo(wv[j].w), bf16_lo(xv.w), a); a = fmaf(bf16_hi(wv[j].w), bf16_hi(xv.w), a);
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

__device__ __forceinline__ void resolve_slots(const DecodeParams &P) {
    const uint32_t s = threadIdx.x;
    if (s < P.top_k) {
        const uint32_t e = P.ids[s];
        k3_moe_expert d{};
        if (e < P.expert_count) d = P.experts[e];
        P.sel[s] = d;
    }
}

/* one wave */
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
    topk_select_wave(key, score, P.top_k, P.scale, P.ids, P.weights, P.ids_copy, P.weights_copy,
                     sm);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
    resolve_slots(P);
}

/* descriptors for routes given by the caller */
__global__ __launch_bounds__(64) void resolve_kernel(DecodeParams P) { resolve_slots(P); }

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
    const uint32_t bits = f32_to_bf16(gated_act(gb, ub, P.activation, P.beta, P.linear_beta));
    /* lanes 0 and 32/RPW hold rows 2w and 2w+1 */
    const uint32_t hi = (uint32_t)__shfl_down((int)bits, 32u / RPW, 64);
    if (lane == 0u) *(uint32_t *)(dst + 2u * wave) = bits | (hi << 16);
}

/* ---------------------------------------------------------------------- */
/* down                                                                    */
/* ---------------------------------------------------------------------- */

/*
 * grid (H / kRB), block 256: the block computes output rows rb*kRB..+kRB
 * (a contiguous kRB-row stripe of each selected down matrix) for all k
 * slots -- wave w handles slots w, w + 4, ... one at a time, so the block
 * reads four kRB-row runs at once; lane l owns groups l, l + 64,
 * ... (M of them: F <= 2048 * M) -- then combines the k bf16 slot outputs
 * in rank order with the residual: out[d] = bf16(residual[d] +
 * bf16(sum_r w[r] * y[r, d])), product and sum rounded separately
 * (k3_rocm_ops.cu:1452-1510).
 */
template <int M>
__global__ __launch_bounds__(256) void down_kernel(DecodeParams P) {
    __shared__ float ys[32][kRB];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t waves = blockDim.x >> 6;
    const uint32_t row0 = blockIdx.x * kRB;
    const uint32_t F = P.ffn, G = F / 32u;
    for (uint32_t slot = wave; slot < P.top_k; slot += waves) {
        float acc[kRB];
#pragma unroll
        for (int i = 0; i < kRB; i++) acc[i] = 0.0f;
        const k3_moe_expert ex = P.sel[slot];
        if (ex.down_packed) {
            const uint8_t *dp = (const uint8_t *)ex.down_packed + (uint64_t)row0 * (F / 2u);
            const uint8_t *ds = (const uint8_t *)ex.down_scales + (uint64_t)row0 * G;
            uint4 w[kRB][M];
            uint32_t sc[kRB][M];
#pragma unroll
            for (int i = 0; i < kRB; i++)
#pragma unroll
                for (int m = 0; m < M; m++) {
                    const uint32_t g = lane + 64u * m;
                    if (g < G) {
                        w[i][m] = gload((const uint4 *)(dp + (uint64_t)i * (F / 2u) + 16u * g));
                        sc[i][m] = gload(ds + (uint64_t)i * G + g);
                    }
                }
            const uint4 *a4 = (const uint4 *)(P.act + (uint64_t)slot * F);
#pragma unroll
            for (int m = 0; m < M; m++) {
                const uint32_t g = lane + 64u * m;
                if (g < G) {
                    float xf[32];
                    bf16x32_to_f32(a4 + 4u * g, xf);
#pragma unroll
                    for (int i = 0; i < kRB; i++)
                        acc[i] = fmaf(fp4_group(w[i][m], xf), e8m0_to_f32(sc[i][m]), acc[i]);
                }
            }
        }
        const float v = wave_sum_rows<kRB>(acc);
        const int owner = wave_rows_owner<kRB>();
        if ((lane & (64u / kRB - 1u)) == 0u) ys[slot][owner] = bf16_to_f32(f32_to_bf16(v));
    }
    __syncthreads();
    if (threadIdx.x < (uint32_t)kRB) {
        const uint32_t d = row0 + threadIdx.x;
        float c = 0.0f;
        for (uint32_t s2 = 0; s2 < P.top_k; s2++)
            if (P.sel[s2].down_packed)
                c = __fadd_rn(c, __fmul_rn(P.weights[s2], ys[s2][threadIdx.x]));
        const float cb = bf16_to_f32(f32_to_bf16(c));
        P.output[d] = P.residual ? f32_to_bf16(__fadd_rn(bf16_to_f32(P.residual[d]), cb))
                                 : f32_to_bf16(cb);
    }
}

}  // namespace

bool decode_supported(const k3_moe_shape &s) {
    return s.hidden % 32u == 0u && s.hidden <= 8192u && s.ffn % 32u == 0u && s.ffn <= 4096u &&
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
        hipLaunchKernelGGL(HIP_KERNEL_NAME(down_kernel<1>), dim3(P.hidden / kRB), block, 0, st, P);
    else
        hipLaunchKernelGGL(HIP_KERNEL_NAME(down_kernel<2>), dim3(P.hidden / kRB), block, 0, st, P);
    mark(K3_MOE_STAGE_COMBINE); /* folded into down */
    mark(K3_MOE_STAGE_END);
    return hipGetLastError() == hipSuccess;
}

}  // namespace k3
