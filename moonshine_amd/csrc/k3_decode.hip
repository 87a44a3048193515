/*
 * Single-token decode of the routed-MoE layer on gfx950: five kernels.
 *
 *   router_kernel   2 expert rows per one-wave block (the hidden state is
 *                   read once for both): logit in the reference's order,
 *                   sigmoid score and order key per expert.
 *   topk_kernel     one wave selects the routes (k3_topk.h) and resolves
 *                   the k selected expert descriptors once (their loads
 *                   start before ranking), so the expert kernels reach
 *                   their weights through a single load.
 *   gateup_kernel   one block per (slot, 8 F-rows; 16 in two sets when
 *                   H <= 4096): each wave streams one 64-group K-stripe of
 *                   8 gate and 8 up rows (a coalesced 1 KB row-stripe per
 *                   load), group sums meet in LDS and are combined in the
 *                   w64 lane order, then the activation. 4096 blocks at
 *                   the K3 shape keep ~64 MB of loads in flight.
 *   down_kernel     one block per (slot, 4 x 8 rows): each wave streams a
 *                   contiguous 8-row stripe of the slot's down matrix
 *                   (8 KB in flight per wave) against the activation
 *                   staged once per block in LDS, and writes bf16 y[slot].
 *   combine_kernel  rank-order weighted sum of the k slot rows plus the
 *                   residual.
 *
 * A K3-native layer runs the same kernels with the router reading the
 * model's hidden state (router_in, router_cols) and the experts the latent.
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

constexpr int kGU = 8;                /* gate (and up) rows per gate/up block */
/* rows per down wave (F <= 2048): 8 gives 3584 blocks for the K3 shape,
 * enough for an even tail (16 rows: 1.75 rounds of resident blocks, ~1.5
 * us slower per layer; 4 rows: no better than 8) */
constexpr int kDownRows = 8;

/* ---------------------------------------------------------------------- */
/* router                                                                  */
/* ---------------------------------------------------------------------- */

/* One wave per block computes rows 2b and 2b+1 (router_rows_wave): the
 * hidden state is read once for the two rows, since a CU's L2 read
 * bandwidth, not HBM, bounds this kernel and rereading x per row would
 * cost as much as a third of the weights. */
__global__ __launch_bounds__(64) void router_kernel(DecodeParams P) {
    const RouterRows R{P.router_weight, P.router_bias, P.router_in, P.logits,
                       P.scores,        P.keys,        P.expert_count, P.router_cols};
    router_rows_wave<2>(R, 2u * blockIdx.x);
}

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

/* Descriptor hand-off of the decode top-k: each candidate lane starts the
 * load of its expert's descriptor before ranking, and the lane whose
 * candidate takes rank r stores it to slot r. */
struct ResolveHooks {
    const DecodeParams &P;
    uint32_t *live_bits; /* LDS: bit r = slot r has an expert */
    k3_moe_expert d{};
    __device__ __forceinline__ void candidate(uint32_t id) { d = P.experts[id]; }
    __device__ __forceinline__ void selected(uint32_t rank) {
        P.sel[rank] = d;
        if (d.down_packed) atomicOr(live_bits, 1u << rank);
    }
};

/* One wave: select and resolve; slots past the selected routes get empty
 * descriptors. */
__global__ __launch_bounds__(64) void topk_kernel(DecodeParams P) {
    __shared__ TopkWaveSmem sm;
    __shared__ uint32_t live_bits;
    const uint32_t lane = threadIdx.x;
    if (lane == 0u) live_bits = 0u;
    uint32_t key[kTopkSlots];
    float score[kTopkSlots];
#pragma unroll
    for (int j = 0; j < kTopkSlots; j++) {
        const uint32_t e = lane + 64u * j;
        key[j] = e < P.expert_count ? P.keys[e] : 0u;
        score[j] = e < P.expert_count ? P.scores[e] : 0.0f;
    }
    const uint32_t id = topk_select_wave(key, score, P.top_k, P.scale, P.ids, P.weights,
                                         P.ids_copy, P.weights_copy, sm,
                                         ResolveHooks{P, &live_bits});
    if (lane < P.top_k && id == UINT32_MAX) P.sel[lane] = k3_moe_expert{};
    wave_fence();
    if (lane == 0u) *P.slot_mask = live_bits;
}

/* descriptors for routes given by the caller */
__global__ __launch_bounds__(64) void resolve_kernel(DecodeParams P) {
    resolve_slot(P, threadIdx.x < P.top_k ? P.ids[threadIdx.x] : UINT32_MAX);
}

/* ---------------------------------------------------------------------- */
/* gate/up                                                                 */
/* ---------------------------------------------------------------------- */

/* NS row sets of kGU gate and kGU up rows per block: NS = 2 when the
 * input has at most two 64-group stripes (H <= 4096), so that all four
 * waves load (two stripes x two sets) instead of two. */
template <int NS>
struct GateUpSmem {
    float part[NS][2 * kGU][4 / NS][64];
    uint32_t scl[2 * NS * kGU][64]; /* raw E8M0 bytes: gate rows, then up rows */
};

/* grid (F / (NS kGU), k), block 256; H <= 4096 NS (64-group stripes per
 * set: 4 / NS). */
template <int NS>
__global__ __launch_bounds__(256) void gateup_kernel(DecodeParams P) {
    __shared__ GateUpSmem<NS> sm;
    constexpr int SW = 4 / NS;    /* waves (stripes) per set */
    constexpr int NR = NS * kGU;  /* gate rows per block */
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t set = wave / SW, stripe = wave % SW;
    const uint32_t slot = blockIdx.y, row0 = blockIdx.x * NR;
    const uint32_t H = P.hidden, G = H / 32u;
    const k3_moe_expert ex = P.sel[slot];
    uint16_t *dst = P.act + (uint64_t)slot * P.ffn + row0;
    if (!ex.gate_packed) {
        if (threadIdx.x < (uint32_t)NR) dst[threadIdx.x] = 0;
        return;
    }
    const uint32_t g = 64u * stripe + lane;
    const uint8_t *gs = (const uint8_t *)ex.gate_scales + (uint64_t)row0 * G;
    const uint8_t *us = (const uint8_t *)ex.up_scales + (uint64_t)row0 * G;
    /* the block's scales are two contiguous runs of NR G bytes (gate, up):
     * fetched as whole lines of dwords, thread-contiguous, instead of a
     * byte load per row and wave */
    const bool words = G % 4u == 0u && (((uintptr_t)gs | (uintptr_t)us) & 3u) == 0u;
    const uint32_t t = threadIdx.x, nd = NR * G / 4u; /* dwords per run */
    const uint32_t srow0 = set * kGU; /* this wave's first row in the block */
    uint4 w[2 * kGU];
    uint32_t sw[4];
    /* 8-mod-16 tensor starts (real checkpoint spans) load as 8-byte pairs */
    const bool a16 = (((uintptr_t)ex.gate_packed | (uintptr_t)ex.up_packed) % 16u) == 0u;
    if (g < G) {
        const uint8_t *gp = (const uint8_t *)ex.gate_packed + (uint64_t)(row0 + srow0) * (H / 2u) + 16u * g;
        const uint8_t *up = (const uint8_t *)ex.up_packed + (uint64_t)(row0 + srow0) * (H / 2u) + 16u * g;
#pragma unroll
        for (int i = 0; i < kGU; i++) {
            w[i] = gload16_nt(gp + (uint64_t)i * (H / 2u), a16);
            w[kGU + i] = gload16_nt(up + (uint64_t)i * (H / 2u), a16);
        }
    }
    if (words) {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const uint32_t d = t + 256u * (uint32_t)k;
            if (d < nd) {
                sw[k] = gload_nt((const uint32_t *)(gs + 4u * d));
                sw[2 + k] = gload_nt((const uint32_t *)(us + 4u * d));
            }
        }
    }
    if (g < G) {
        float xf[32];
        bf16x32_to_f32((const uint4 *)P.hidden_in + 4u * g, xf);
#pragma unroll
        for (int r = 0; r < 2 * kGU; r++) sm.part[set][r][stripe][lane] = fp4_group(w[r], xf);
    }
    uint8_t *sb = (uint8_t *)sm.scl;
    if (words) {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const uint32_t d = t + 256u * (uint32_t)k;
            if (d < nd) { /* byte 4 d: row 4 d / G, group 4 d % G (G % 4 == 0) */
                const uint32_t r = 4u * d / G, c4 = (4u * d % G) / 4u;
                sm.scl[r][c4] = sw[k];
                sm.scl[NR + r][c4] = sw[2 + k];
            }
        }
    } else if (g < G) {
#pragma unroll
        for (int i = 0; i < kGU; i++) {
            const uint32_t r = srow0 + (uint32_t)i;
            sb[256u * r + g] = (uint8_t)gload(gs + (uint64_t)r * G + g);
            sb[256u * (NR + r) + g] = (uint8_t)gload(us + (uint64_t)r * G + g);
        }
    }
    __syncthreads();
    /* wave w: gate rows RPW w .. RPW w + RPW - 1 and the same up rows; lane
     * l's groups l, l+64, ... in order */
    constexpr int RPW = NR / 4;
    const uint32_t stripes = (G + 63u) / 64u;
    float p[2 * RPW];
#pragma unroll
    for (int q = 0; q < 2 * RPW; q++) {
        const uint32_t gr = RPW * wave + (uint32_t)(q % RPW); /* gate row in the block */
        const uint32_t rs = gr / kGU, ri = gr % kGU + (q < RPW ? 0u : (uint32_t)kGU);
        const uint32_t sr = q < RPW ? gr : NR + gr;
        float acc = 0.0f;
        for (uint32_t j = 0; j < stripes; j++)
            if (64u * j + lane < G)
                acc = fmaf(sm.part[rs][ri][j][lane], e8m0_to_f32(sb[256u * sr + 64u * j + lane]), acc);
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
 * at once. The block stages the slot's activation in LDS once and each
 * wave its RB x F/32 scale bytes (one contiguous run) with dword loads:
 * the per-CU L2 request rate, not HBM, bounds this kernel, and per-wave
 * activation reads and per-row byte loads of the scales added a third
 * to the weight stream's requests. Lane l owns groups l, l + 64, ... (M
 * of them: F <= 2048 M); per
 * row the group sum runs over the 32 columns in order, with 8-column
 * chunks of the activation converted once for the RB rows. Output y[slot,
 * d] = bf16(row sum), the reference's per-slot GEMV result
 * (k3_engine.cu:1058-1060).
 */
template <int M, int RB>
__global__ __launch_bounds__(256) void down_kernel(DecodeParams P) {
    static_assert(RB * 64 * M <= 1024, "a wave's scale block is at most 1 KB");
    /* the slot's activation, chunk (g, q) (8 columns, 32 g + 8 q) at
     * q * 64 M + g, so lane-consecutive reads are bank-consecutive */
    __shared__ uint4 xs[4 * 64 * M];
    __shared__ uint32_t ssc[4][256]; /* each wave's RB x G scale bytes */
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, t = threadIdx.x;
    const uint32_t slot = blockIdx.y;
    const uint32_t row0 = (4u * blockIdx.x + wave) * RB;
    const uint32_t F = P.ffn, G = F / 32u;
    uint16_t *y = P.y + (uint64_t)slot * P.hidden + row0;
    const k3_moe_expert ex = P.sel[slot];
    if (!ex.down_packed) { /* uniform over the block */
        if (lane < (uint32_t)RB) y[lane] = 0;
        return;
    }
    const uint8_t *dp = (const uint8_t *)ex.down_packed + (uint64_t)row0 * (F / 2u);
    const uint8_t *ds = (const uint8_t *)ex.down_scales + (uint64_t)row0 * G;
    const uint4 *a4 = (const uint4 *)(P.act + (uint64_t)slot * F);
    /* issue order: the first weight stripe, then the block's activation
     * (one load per thread instead of one per wave) and the wave's scale
     * bytes (RB G contiguous bytes, dword loads when aligned) */
    uint4 w[M][RB]; /* every stripe's weights issued up front: one round trip */
    const bool a16 = ((uintptr_t)ex.down_packed % 16u) == 0u;
#pragma unroll
    for (int m = 0; m < M; m++) {
        if (lane + 64u * m < G) {
#pragma unroll
            for (int i = 0; i < RB; i++)
                w[m][i] = gload16_nt(dp + (uint64_t)i * (F / 2u) + 16u * (lane + 64u * m), a16);
        }
    }
    uint4 xa[M];
#pragma unroll
    for (int k = 0; k < M; k++) {
        const uint32_t c = t + 256u * k;
        if (c < 4u * G) xa[k] = gload(a4 + c);
    }
    const uint32_t nbytes = RB * G;
    uint32_t sw[4];
    const bool words = ((uintptr_t)ds & 3u) == 0u;
    if (words) {
        const uint32_t *dw = (const uint32_t *)ds;
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (4u * (lane + 64u * k) < nbytes) sw[k] = gload_nt(dw + lane + 64u * k);
    }
#pragma unroll
    for (int k = 0; k < M; k++) {
        const uint32_t c = t + 256u * k;
        if (c < 4u * G) xs[(c & 3u) * 64u * M + (c >> 2)] = xa[k];
    }
    if (words) {
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (4u * (lane + 64u * k) < nbytes) ssc[wave][lane + 64u * k] = sw[k];
    } else {
        uint8_t *sb = (uint8_t *)ssc[wave];
        for (uint32_t b = lane; b < nbytes; b += 64u) sb[b] = (uint8_t)gload(ds + b);
    }
    __syncthreads();
    const uint8_t *sb = (const uint8_t *)ssc[wave];
    float acc[RB];
#pragma unroll
    for (int i = 0; i < RB; i++) acc[i] = 0.0f;
#pragma unroll
    for (int m = 0; m < M; m++) {
        const uint32_t g = lane + 64u * m;
        if (g < G) {
            uint4 xr[4];
#pragma unroll
            for (int q = 0; q < 4; q++) xr[q] = xs[q * 64 * M + g];
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
                    const uint32_t wq = q == 0 ? w[m][i].x : q == 1 ? w[m][i].y : q == 2 ? w[m][i].z : w[m][i].w;
                    gs[i] = fp4_dot8(wq, x8, gs[i]);
                }
            }
#pragma unroll
            for (int i = 0; i < RB; i++)
                acc[i] = fmaf(gs[i], e8m0_to_f32(sb[(uint32_t)i * G + g]), acc[i]);
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
    /* down grids: H / 32 blocks (F <= 2048) or H / 16 (F <= 4096) */
    return s.hidden % 32u == 0u && s.hidden <= 8192u && s.ffn % 32u == 0u && s.ffn <= 4096u &&
           s.top_k <= 32u && s.expert_count <= 1024u;
}

bool decode_launch_route(const DecodeParams &P, hipStream_t st, const StageMarker &mark) {
    mark(K3_MOE_STAGE_ROUTER);
    hipLaunchKernelGGL(router_kernel, dim3((P.expert_count + 1u) / 2u), dim3(64), 0, st, P);
    return hipGetLastError() == hipSuccess && decode_launch_topk(P, st, mark);
}

bool decode_launch_topk(const DecodeParams &P, hipStream_t st, const StageMarker &mark) {
    mark(K3_MOE_STAGE_TOPK);
    hipLaunchKernelGGL(topk_kernel, dim3(1), dim3(64), 0, st, P);
    return hipGetLastError() == hipSuccess;
}

bool decode_launch(const DecodeParams &P, hipStream_t st, const StageMarker &mark) {
    return decode_launch_route(P, st, mark) && decode_launch_experts(P, st, mark, false);
}

bool decode_launch_experts(const DecodeParams &P, hipStream_t st, const StageMarker &mark,
                           bool resolve) {
    mark(K3_MOE_STAGE_PLAN);
    if (resolve) hipLaunchKernelGGL(resolve_kernel, dim3(1), dim3(64), 0, st, P);
    mark(K3_MOE_STAGE_GATE_UP);
    if (P.hidden <= 4096u && P.ffn % (2u * kGU) == 0u)
        hipLaunchKernelGGL(HIP_KERNEL_NAME(gateup_kernel<2>), dim3(P.ffn / (2u * kGU), P.top_k),
                           dim3(256), 0, st, P);
    else
        hipLaunchKernelGGL(HIP_KERNEL_NAME(gateup_kernel<1>), dim3(P.ffn / kGU, P.top_k),
                           dim3(256), 0, st, P);
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
