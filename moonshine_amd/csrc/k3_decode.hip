/*
 * Single-token decode of the routed-MoE layer on gfx950: three kernels.
 *
 *   router_topk_kernel  one wave per expert row (all of a row's loads in
 *                       flight at once); logits are published with
 *                       write-through agent-scope stores and the last block
 *                       to arrive runs the block radix-select top-k. No
 *                       agent-scope release fence is needed: on this part
 *                       such a fence is an L2 write-back, which measured
 *                       ~100 us across a few hundred blocks.
 *   gateup_kernel       one block per (slot, 4 F-rows); each of its four
 *                       waves streams one 64-group K-stripe of the 4 gate and
 *                       4 up rows (one coalesced 1 KB row-stripe per load),
 *                       group sums meet in LDS and are combined in the w64
 *                       lane order, then the activation. 4096 blocks keep
 *                       enough loads in flight to stream at ~6.3 TB/s.
 *   down_kernel         one block per (8 output rows, 4 slots), one wave per
 *                       slot; the slot outputs are published write-through
 *                       and the last block of a row block to arrive
 *                       combines all k slots in rank order with the
 *                       residual (small blocks refill the CUs far better
 *                       than one 16-wave block per row block did).
 *
 * A cooperative single-kernel variant was measured and dropped: the
 * cooperative launch alone cost ~18 us and its three agent-scope hand-offs
 * ~100 us on this part.
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

/* ---------------------------------------------------------------------- */
/* router row                                                              */
/* ---------------------------------------------------------------------- */

__device__ __forceinline__ float router_row(const uint16_t *__restrict__ w_row,
                                            const uint16_t *__restrict__ x, uint32_t chunks,
                                            uint32_t lane) {
    const uint4 *w4 = (const uint4 *)w_row;
    const uint4 *x4 = (const uint4 *)x;
    uint4 wv[kRouterMaxChunks], xv[kRouterMaxChunks];
#pragma unroll
    for (int j = 0; j < kRouterMaxChunks; j++) {
        const uint32_t c = lane + 64u * j;
        if (c < chunks) { wv[j] = w4[c]; xv[j] = x4[c]; }
    }
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < kRouterMaxChunks; j++) {
        const uint32_t c = lane + 64u * j;
        if (c < chunks) {
            a = fmaf(bf16_lo(wv[j].x), bf16_lo(xv[j].x), a); a = fmaf(bf16_hi(wv[j].x), bf16_hi(xv[j].x), a);
            a = fmaf(bf16_lo(wv[j].y), bf16_lo(xv[j].y), a); a = fmaf(bf16_hi(wv[j].y), bf16_hi(xv[j].y), a);
            a = fmaf(bf16_lo(wv[j].z), bf16_lo(xv[j].z), a); a = fmaf(bf16_hi(wv[j].z), bf16_hi(xv[j].z), a);
            a = fmaf(bf16_lo(wv[j].w), bf16_lo(xv[j].w), a); a = fmaf(bf16_hi(wv[j].w), bf16_hi(xv[j].w), a);
        }
    }
    return wave_sum(a);
}

/* ---------------------------------------------------------------------- */
/* kernels                                                                 */
/* ---------------------------------------------------------------------- */

/* s_waitcnt vmcnt(0): this wave's stores have reached the coherence point. */
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0x0F70); }


__global__ __launch_bounds__(256) void router_topk_kernel(DecodeParams P) {
    __shared__ TopkWaveSmem sm;
    __shared__ uint32_t s_last;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (row < P.expert_count) {
        const float v = router_row(P.router_weight + (uint64_t)row * P.hidden, P.hidden_in,
                                   P.hidden / 8u, lane);
        if (lane == 0u) {
            const float score = det_sigmoid(v);
            const uint32_t key = choice_key(score, P.router_bias[row]);
            __hip_atomic_store(P.logits + row, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(P.scores + row, score, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(P.keys + row, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0u)
        s_last = __hip_atomic_fetch_add(&P.sync->arrive_router, 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1u;
    __syncthreads();
    if (!s_last || threadIdx.x >= 64u) return;
    if (lane == 0u)
        __hip_atomic_store(&P.sync->arrive_router, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t key[kTopkSlots];
    float score[kTopkSlots];
#pragma unroll
    for (int j = 0; j < kTopkSlots; j++) {
        const uint32_t e = lane + 64u * j;
        key[j] = 0u;
        score[j] = 0.0f;
        if (e < P.expert_count) {
            key[j] = __hip_atomic_load(P.keys + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            score[j] = __hip_atomic_load(P.scores + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    topk_select_wave(key, score, P.top_k, P.scale, P.ids, P.weights, P.ids_copy, P.weights_copy,
                     sm);
}

template <int kGU>
struct GateUpSmem {
    float part[2 * kGU][4][64];
    float scl[2 * kGU][4][64];
};

/* grid (F / kGU, k), block 256; requires H <= 8192 (four 64-group stripes). */
template <int kGU>
__global__ __launch_bounds__(256) void gateup_kernel(DecodeParams P) {
    __shared__ GateUpSmem<kGU> sm;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t slot = blockIdx.y, row0 = blockIdx.x * kGU;
    const uint32_t H = P.hidden, G = H / 32u;
    const uint32_t e = P.ids[slot];
    uint16_t *dst = P.act + (uint64_t)slot * P.ffn + row0;
    if (e >= P.expert_count) {
        if (threadIdx.x < (uint32_t)kGU) dst[threadIdx.x] = 0;
        return;
    }
    const k3_moe_expert ex = P.experts[e];
    const uint32_t g = 64u * wave + lane;
    const bool gv = g < G;
    if (gv) {
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
    /* wave w: gate rows w*RPW .. +RPW and the same up rows; lane l's groups
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
    const float v = wave_sum_rows<2 * RPW>(p);   /* lanes < 32: gate, lanes >= 32: up */
    const float u = __shfl_xor(v, 32, 64);
    const int owner = wave_rows_owner<2 * RPW>();
    if (lane < 32u && (lane & (32u / RPW - 1u)) == 0u) {
        const float gb = bf16_to_f32(f32_to_bf16(v)), ub = bf16_to_f32(f32_to_bf16(u));
        dst[wave * RPW + owner] = f32_to_bf16(gated_act(gb, ub, P.activation, P.beta, P.linear_beta));
    }
}

/*
 * grid (H / RB, ceil(k / 4)), block 256: wave w computes RB output rows of
 * the down product for slot 4 * blockIdx.y + w (one slot per wave, lane l
 * owns groups l, l + 64, ... < F / 32, M of them). The four slot outputs
 * are published as bf16 with write-through stores; the last of the
 * ceil(k / 4) blocks of a row block to arrive combines all k slots in rank
 * order with the residual (and resets the row block's counter).
 */
template <int M, int RB>
__global__ __launch_bounds__(256) void down_kernel(DecodeParams P) {
    __shared__ float ybuf[4][RB];
    __shared__ uint32_t s_last;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t slot = 4u * blockIdx.y + wave;
    const uint32_t row0 = blockIdx.x * RB;
    const uint32_t F = P.ffn, G = F / 32u, H = P.hidden;
    const uint32_t e = slot < P.top_k ? P.ids[slot] : UINT32_MAX;
    float acc[RB];
#pragma unroll
    for (int i = 0; i < RB; i++) acc[i] = 0.0f;
    if (e < P.expert_count) {
        const k3_moe_expert ex = P.experts[e];
        const uint8_t *dp = (const uint8_t *)ex.down_packed + (uint64_t)row0 * (F / 2u);
        const uint8_t *ds = (const uint8_t *)ex.down_scales + (uint64_t)row0 * G;
        uint4 w[RB][M];
        uint32_t sc[RB][M];
#pragma unroll
        for (int i = 0; i < RB; i++)
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
                for (int i = 0; i < RB; i++)
                    acc[i] = fmaf(fp4_group(w[i][m], xf), e8m0_to_f32(sc[i][m]), acc[i]);
            }
        }
    }
    const float v = wave_sum_rows<RB>(acc);
    const int owner = wave_rows_owner<RB>();
    if ((lane & (64u / RB - 1u)) == 0u) ybuf[wave][owner] = v;
    __syncthreads();
    /* publish: thread t < 2 * RB writes rows (2 (t % (RB/2)), +1) of slot t / (RB/2) */
    if (threadIdx.x < 4u * (RB / 2)) {
        const uint32_t ws = threadIdx.x / (RB / 2), r = 2u * (threadIdx.x % (RB / 2));
        const uint32_t s2 = 4u * blockIdx.y + ws;
        if (s2 < P.top_k) {
            const uint32_t word = (uint32_t)f32_to_bf16(ybuf[ws][r]) |
                                  ((uint32_t)f32_to_bf16(ybuf[ws][r + 1]) << 16);
            __hip_atomic_store((uint32_t *)(P.slot_out + (uint64_t)s2 * H + row0 + r), word,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0u)
        s_last = __hip_atomic_fetch_add(&P.down_arrive[blockIdx.x], 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT) == gridDim.y - 1u;
    __syncthreads();
    if (!s_last) return;
    if (threadIdx.x == 0u)
        __hip_atomic_store(&P.down_arrive[blockIdx.x], 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    /* all k * RB / 2 words of this row block in one round trip */
    __shared__ float yall[32][RB];
    for (uint32_t t = threadIdx.x; t < P.top_k * (RB / 2); t += blockDim.x) {
        const uint32_t s2 = t / (RB / 2), r = 2u * (t % (RB / 2));
        const uint32_t word = __hip_atomic_load(
            (uint32_t *)(P.slot_out + (uint64_t)s2 * H + row0 + r), __ATOMIC_RELAXED,
            __HIP_MEMORY_SCOPE_AGENT);
        yall[s2][r] = bf16_to_f32((uint16_t)(word & 0xffffu));
        yall[s2][r + 1] = bf16_to_f32((uint16_t)(word >> 16));
    }
    __syncthreads();
    if (threadIdx.x < (uint32_t)RB) {
        const uint32_t row = row0 + threadIdx.x;
        float c = 0.0f;
        for (uint32_t s2 = 0; s2 < P.top_k; s2++)
            if (P.ids[s2] < P.expert_count)
                c = __fadd_rn(c, __fmul_rn(P.weights[s2], yall[s2][threadIdx.x]));
        const float cb = bf16_to_f32(f32_to_bf16(c));
        P.output[row] = P.residual
                            ? f32_to_bf16(__fadd_rn(bf16_to_f32(P.residual[row]), cb))
                            : f32_to_bf16(cb);
    }
}

__global__ void zero_words_kernel(uint32_t *w, uint32_t n) {
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) w[i] = 0u;
}

}  // namespace

bool decode_supported(const k3_moe_shape &s) {
    return s.hidden % 32u == 0u && s.hidden <= 8192u && s.ffn % 32u == 0u && s.ffn <= 4096u &&
           s.top_k <= 32u && s.expert_count <= 1024u;
}

bool decode_init_sync(DecodeSync *sync, hipStream_t st) {
    hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(1024), 0, st, (uint32_t *)sync,
                       (uint32_t)(sizeof(DecodeSync) / 4u));
    return hipGetLastError() == hipSuccess;
}

bool decode_launch(const DecodeParams &P, hipStream_t st, const StageMarker &mark) {
    mark(K3_MOE_STAGE_ROUTER);
    hipLaunchKernelGGL(router_topk_kernel, dim3((P.expert_count + 3u) / 4u), dim3(256), 0, st, P);
    mark(K3_MOE_STAGE_TOPK);
    return decode_launch_experts(P, st, mark);
}

bool decode_launch_experts(const DecodeParams &P, hipStream_t st, const StageMarker &mark) {
    mark(K3_MOE_STAGE_PLAN);
    mark(K3_MOE_STAGE_GATE_UP);
    hipLaunchKernelGGL(HIP_KERNEL_NAME(gateup_kernel<8>), dim3(P.ffn / 8u, P.top_k), dim3(256), 0,
                       st, P);
    mark(K3_MOE_STAGE_DOWN);
    const dim3 grid_down(P.hidden / 8u, (P.top_k + 3u) / 4u);
    if (P.ffn <= 2048u)
        hipLaunchKernelGGL(HIP_KERNEL_NAME(down_kernel<1, 8>), grid_down, dim3(256), 0, st, P);
    else
        hipLaunchKernelGGL(HIP_KERNEL_NAME(down_kernel<2, 8>), grid_down, dim3(256), 0, st, P);
    mark(K3_MOE_STAGE_COMBINE);
    mark(K3_MOE_STAGE_END);
    return hipGetLastError() == hipSuccess;
}

}  // namespace k3
