/*
 * libk3moe — gfx950 kernels behind the routed-MoE entry points that
 * Moonshine declares in k3_rocm_ops.h. Signatures, argument validation and
 * return conventions follow the reference launchers; the kernels are
 * written for CDNA4 wave64.
 *
 * Reduction orders ("w64"):
 *   bf16 -> f32 rows: elements in chunks of 8, lane l owns chunks l, l+64,
 *     ..., acc = fmaf(w, x, acc) in column order, then a wave64 butterfly.
 *   MXFP4 rows: lane l owns 32-column groups l, l+64, ...; each group is
 *     gs = fmaf(e2m1, x, gs) over its 32 columns, then acc = fmaf(gs,
 *     2^(e-127), acc); wave64 butterfly; bf16 round.
 *   Q8-128 rows: the MXFP4 skeleton with int8 codes: gs = fmaf(q, x, gs)
 *     over a 32-column group (each product exact), acc = fmaf(gs,
 *     scale[group / 4], acc); wave64 butterfly; bf16 round.
 *   bf16 -> bf16 rows: the bf16 -> f32 order, rounded once to bf16.
 * Every token row of a batch uses the same order as the single-vector form,
 * so batch == sequential and results do not depend on the batch tile.
 */
#include "k3_device.h"
#include "k3_internal.h"
#include "k3_topk.h"
#include "../../include/k3_rocm_ops.h"

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

using namespace k3;

namespace {

constexpr uint32_t kThreads = 256;
constexpr uint32_t kWavesPerBlock = kThreads / kWave;

inline uint32_t grid_cap(uint64_t blocks) {
    return (uint32_t)(blocks > 65535u ? 65535u : (blocks ? blocks : 1u));
}

/* ------------------------------------------------------------------------ */
/* bf16 weights x bf16 inputs -> f32 (router logits)                         */
/* ------------------------------------------------------------------------ */

template <int TT, bool B16 = false>
__global__ __launch_bounds__(256) void bf16_rows_f32_kernel(
        void *__restrict__ out, const uint16_t *__restrict__ weights,
        const uint16_t *__restrict__ input, uint32_t tokens, uint32_t rows,
        uint32_t cols, uint32_t vec_ok) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const uint32_t t0 = blockIdx.y * TT;
    if (row >= rows) return;
    const uint32_t active = tokens - t0 < (uint32_t)TT ? tokens - t0 : (uint32_t)TT;
    float acc[TT];
#pragma unroll
    for (int t = 0; t < TT; t++) acc[t] = 0.0f;
    const uint16_t *w = weights + (uint64_t)row * cols;
    const uint32_t chunks = (cols + 7u) / 8u;
    if (vec_ok) {
        const uint4 *w4 = (const uint4 *)w;
        for (uint32_t c = lane; c < chunks; c += 64u) {
            const uint4 wv = w4[c];
            const float wf[8] = {bf16_lo(wv.x), bf16_hi(wv.x), bf16_lo(wv.y), bf16_hi(wv.y),
                                 bf16_lo(wv.z), bf16_hi(wv.z), bf16_lo(wv.w), bf16_hi(wv.w)};
#pragma unroll
            for (int t = 0; t < TT; t++) {
                if ((uint32_t)t < active) {
                    const uint4 xv = ((const uint4 *)(input + (uint64_t)(t0 + t) * cols))[c];
                    float a = acc[t];
                    a = fmaf(wf[0], bf16_lo(xv.x), a); a = fmaf(wf[1], bf16_hi(xv.x), a);
                    a = fmaf(wf[2], bf16_lo(xv.y), a); a = fmaf(wf[3], bf16_hi(xv.y), a);
                    a = fmaf(wf[4], bf16_lo(xv.z), a); a = fmaf(wf[5], bf16_hi(xv.z), a);
                    a = fmaf(wf[6], bf16_lo(xv.w), a); a = fmaf(wf[7], bf16_hi(xv.w), a);
                    acc[t] = a;
                }
            }
        }
    } else {
        for (uint32_t c = lane; c < chunks; c += 64u) {
            const uint32_t end = 8u * c + 8u < cols ? 8u * c + 8u : cols;
            for (uint32_t i = 8u * c; i < end; i++) {
                const float wf = bf16_to_f32(w[i]);
#pragma unroll
                for (int t = 0; t < TT; t++)
                    if ((uint32_t)t < active)
                        acc[t] = fmaf(wf, bf16_to_f32(input[(uint64_t)(t0 + t) * cols + i]), acc[t]);
            }
        }
    }
    const float v = wave_sum_rows<TT>(acc);
    const int owner = wave_rows_owner<TT>();
    if ((lane & (64u / TT - 1u)) == 0u && (uint32_t)owner < active) {
        const uint64_t o = (uint64_t)(t0 + owner) * rows + row;
        if constexpr (B16)
            ((uint16_t *)out)[o] = f32_to_bf16(v);
        else
            ((float *)out)[o] = v;
    }
}

template <int TT, bool B16 = false>
bool launch_bf16_rows_f32(void *out, const void *w, const void *x, uint32_t tokens,
                          uint32_t rows, uint32_t cols, hipStream_t s) {
    const uint32_t vec_ok = (cols % 8u == 0u) && (((uintptr_t)w | (uintptr_t)x) % 16u == 0u);
    dim3 grid((rows + kWavesPerBlock - 1u) / kWavesPerBlock, (tokens + TT - 1u) / TT);
    hipLaunchKernelGGL(HIP_KERNEL_NAME(bf16_rows_f32_kernel<TT, B16>), grid, dim3(kThreads), 0, s,
                       out, (const uint16_t *)w, (const uint16_t *)x, tokens, rows, cols, vec_ok);
    return hipGetLastError() == hipSuccess;
}

/*
 * Router logits (f32 output) in the reference's order, k3_rocm_ops.cu:359-425
 * and 512-661: thread t of 256 sums the quads t, t + 256, ...; the quad's
 * arithmetic is ref_quad; the LDS tree 128 -> 1 finishes. One wave per
 * weight row and TT tokens per wave (the token tile changes no bit).
 *   vec (16-byte rows): chunk c = lane + 64 j holds quads 2c and 2c + 1
 *     (ref_chunk); the four partials of each token meet in
 *     wave_sum_rows<2 TT> (rows 2t, 2t + 1 = levels 128 .. 2 of token t) and
 *     the last level adds rows 2t and 2t + 1, which sit 32 / TT lanes apart.
 *   otherwise: lane l owns partials l, l + 64, l + 128, l + 192, each summed
 *     as the reference's quad (cols % 4 == 0), pair (cols % 2 == 0: p1 then
 *     p0, :395-405) or element (fmaf, :407-411) path, from scalar loads;
 *     levels 128 and 64 in the lane, then wave_sum_rows<TT>.
 */
template <int TT>
__global__ __launch_bounds__(256) void bf16_rows_ref_kernel(
        float *__restrict__ out, const uint16_t *__restrict__ weights,
        const uint16_t *__restrict__ input, uint32_t tokens, uint32_t rows, uint32_t cols,
        uint32_t vec_ok) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const uint32_t t0 = blockIdx.y * TT;
    if (row >= rows) return;
    const uint32_t active = tokens - t0 < (uint32_t)TT ? tokens - t0 : (uint32_t)TT;
    const uint16_t *w = weights + (uint64_t)row * cols;
    float v;
    int owner;
    if (vec_ok) {
        float acc[TT][4];
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[t][i] = 0.0f;
        const uint4 *w4 = (const uint4 *)w;
        const uint32_t chunks = cols / 8u;
        for (uint32_t c = lane, j = 0; c < chunks; c += 64u, j++) {
            const uint4 wv = w4[c];
#pragma unroll
            for (int t = 0; t < TT; t++)
                if ((uint32_t)t < active)
                    ref_chunk(acc[t], (int)(j & 1u),  wv,
                              ((const uint4 *)(input + (uint64_t)(t0 + t) * cols))[c]);
        }
        float p[2 * TT];
#pragma unroll
        for (int t = 0; t < TT; t++) {
            p[2 * t] = __fadd_rn(acc[t][0], acc[t][2]);
            p[2 * t + 1] = __fadd_rn(acc[t][1], acc[t][3]);
        }
        v = wave_sum_rows<2 * TT>(p);
        v = __fadd_rn(v, __shfl_xor(v, 32 / TT, 64));
        owner = wave_rows_owner<2 * TT>() / 2;
    } else {
        const uint32_t mode = cols % 4u == 0u ? 0u : cols % 2u == 0u ? 1u : 2u;
        const uint32_t step = mode == 0u ? 4u : mode == 1u ? 2u : 1u;
        const uint32_t units = cols / step;
        float part[TT][4];
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int m = 0; m < 4; m++) part[t][m] = 0.0f;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            for (uint32_t u = lane + 64u * (uint32_t)m; u < units; u += 256u) {
                const uint16_t *wu = w + (uint64_t)u * step;
                float wf[4];
                for (uint32_t i = 0; i < step; i++) wf[i] = bf16_to_f32(wu[i]);
#pragma unroll
                for (int t = 0; t < TT; t++) {
                    if ((uint32_t)t >= active) continue;
                    const uint16_t *xu = input + (uint64_t)(t0 + t) * cols + (uint64_t)u * step;
                    float s = part[t][m];
                    if (mode == 0u) {
                        const float p2 = __fmul_rn(wf[2], bf16_to_f32(xu[2]));
                        const float p3 = __fmul_rn(wf[3], bf16_to_f32(xu[3]));
                        s = __fadd_rn(s, __fadd_rn(fmaf(wf[1], bf16_to_f32(xu[1]), p2),
                                                   fmaf(wf[0], bf16_to_f32(xu[0]), p3)));
                    } else if (mode == 1u) {
                        s = __fadd_rn(s, __fmul_rn(wf[1], bf16_to_f32(xu[1])));
                        s = __fadd_rn(s, __fmul_rn(wf[0], bf16_to_f32(xu[0])));
                    } else {
                        s = fmaf(wf[0], bf16_to_f32(xu[0]), s);
                    }
                    part[t][m] = s;
                }
            }
        }
        float p[TT];
#pragma unroll
        for (int t = 0; t < TT; t++)
            p[t] = __fadd_rn(__fadd_rn(part[t][0], part[t][2]), __fadd_rn(part[t][1], part[t][3]));
        v = wave_sum_rows<TT>(p);
        owner = wave_rows_owner<TT>();
    }
    const uint32_t lanes_per = 64u / TT;
    if ((lane & (lanes_per - 1u)) == 0u && (uint32_t)owner < active)
        out[(uint64_t)(t0 + owner) * rows + row] = v;
}

template <int TT>
bool launch_bf16_rows_ref(float *out, const void *w, const void *x, uint32_t tokens,
                          uint32_t rows, uint32_t cols, hipStream_t s) {
    const uint32_t vec_ok = (cols % 8u == 0u) && (((uintptr_t)w | (uintptr_t)x) % 16u == 0u);
    dim3 grid((rows + kWavesPerBlock - 1u) / kWavesPerBlock, (tokens + TT - 1u) / TT);
    hipLaunchKernelGGL(HIP_KERNEL_NAME(bf16_rows_ref_kernel<TT>), grid, dim3(kThreads), 0, s, out,
                       (const uint16_t *)w, (const uint16_t *)x, tokens, rows, cols, vec_ok);
    return hipGetLastError() == hipSuccess;
}

/*
 * The same w64 order for many tokens at once (router logits of a prefill
 * batch), as a register-blocked GEMM: a block computes 32 tokens x 16 rows.
 * Wave w (of 8) owns tokens 8 (w / 2) .. +8 and rows 8 (w % 2) .. +8; lane l
 * keeps the 64 partial sums of its own chunks l, l + 64, ... -- exactly the
 * per-lane partials of bf16_rows_f32_kernel -- and the wave64 butterfly of
 * wave_sum_rows<64> finishes all 64 outputs at once, so the logits are
 * bit-identical to the one-wave-per-row kernel.
 *
 * A K step covers 512 columns (64 chunks of 8). The step's bf16 tiles are
 * loaded into registers one step ahead, then written to LDS as fp32 in two
 * planes (elements 0-3 and 4-7 of each chunk), so every fragment read is a
 * lane-contiguous ds_read_b128 and no conversion sits in the FMA loop.
 * Out-of-range tokens/rows/chunks load zeros: fmaf(0, 0, acc) == acc
 * for every acc the loop can hold (+0 + +0 = +0), so padding changes no bit.
 *
 * Block order is XCD-aware: workgroups are dealt to the eight XCDs round
 * robin, and XCD x walks (token tile, its contiguous range of row tiles)
 * with the row tiles fastest, so its 16-row weight slices stay in its own
 * L2 and each token tile is fetched once per XCD.
 */
constexpr int kGT = 32, kGE = 16, kGThreads = 512;
constexpr uint32_t kGemmMinTokens = 128;

template <bool B16>
__global__ __launch_bounds__(512) void bf16_gemm_w64_kernel(
        void *__restrict__ out, const uint16_t *__restrict__ weights,
        const uint16_t *__restrict__ input, uint32_t tokens, uint32_t rows, uint32_t cols,
        uint32_t row_tiles, uint32_t xcd_groups) {
    __shared__ float4 xs[2][kGT][64];
    __shared__ float4 wsm[2][kGE][64];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    /* block -> (token tile, row tile) */
    uint32_t tt, et;
    {
        const uint32_t L = blockIdx.x;
        if (xcd_groups) {
            const uint32_t x = L & 7u, j = L >> 3;
            const uint32_t base = row_tiles >> 3, rem = row_tiles & 7u;
            const uint32_t cnt = base + (x < rem ? 1u : 0u);
            const uint32_t start = x * base + (x < rem ? x : rem);
            const uint32_t token_tiles = (tokens + kGT - 1u) / kGT;
            if (cnt == 0u || j >= token_tiles * cnt) return;
            tt = j / cnt;
            et = start + j % cnt;
        } else {
            tt = L / row_tiles;
            et = L % row_tiles;
        }
    }
    const uint32_t t0 = tt * kGT, e0 = et * kGE;
    const uint32_t chunks = cols / 8u, nsteps = (chunks + 63u) / 64u;
    const uint4 *x4 = (const uint4 *)input, *w4 = (const uint4 *)weights;
    /* this thread's 6 staging items: items < 2048 are x (token i / 64,
     * chunk i % 64), the rest weight rows */
    constexpr int kItems = (kGT + kGE) * 64 / kGThreads;
    uint4 reg[kItems];
    auto load_step = [&](uint32_t s) {
#pragma unroll
        for (int q = 0; q < kItems; q++) {
            const uint32_t it = tid + (uint32_t)q * kGThreads;
            const uint32_t c = 64u * s + (it & 63u);
            uint4 v = make_uint4(0u, 0u, 0u, 0u);
            if (it < (uint32_t)kGT * 64u) {
                const uint32_t t = t0 + (it >> 6);
                if (t < tokens && c < chunks) v = x4[(uint64_t)t * chunks + c];
            } else {
                const uint32_t e = e0 + ((it >> 6) - (uint32_t)kGT);
                if (e < rows && c < chunks) v = w4[(uint64_t)e * chunks + c];
            }
            reg[q] = v;
        }
    };
    const uint32_t wt = wave >> 1, we = wave & 1u;
    float acc[64];
#pragma unroll
    for (int i = 0; i < 64; i++) acc[i] = 0.0f;
    load_step(0u);
    for (uint32_t s = 0; s < nsteps; s++) {
        __syncthreads(); /* the previous step's reads are done */
#pragma unroll
        for (int q = 0; q < kItems; q++) {
            const uint32_t it = tid + (uint32_t)q * kGThreads;
            const uint4 v = reg[q];
            const float4 p0 = make_float4(bf16_lo(v.x), bf16_hi(v.x), bf16_lo(v.y), bf16_hi(v.y));
            const float4 p1 = make_float4(bf16_lo(v.z), bf16_hi(v.z), bf16_lo(v.w), bf16_hi(v.w));
            const uint32_t r = it >> 6, c = it & 63u;
            if (it < (uint32_t)kGT * 64u) {
                xs[0][r][c] = p0;
                xs[1][r][c] = p1;
            } else {
                wsm[0][r - kGT][c] = p0;
                wsm[1][r - kGT][c] = p1;
            }
        }
        __syncthreads();
        if (s + 1u < nsteps) load_step(s + 1u);
#pragma unroll
        for (int p = 0; p < 2; p++) {
            float4 xv[8], wv[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                xv[i] = xs[p][8u * wt + i][lane];
                wv[i] = wsm[p][8u * we + i][lane];
            }
#pragma unroll
            for (int t = 0; t < 8; t++)
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    float a = acc[8 * t + e];
                    a = fmaf(wv[e].x, xv[t].x, a);
                    a = fmaf(wv[e].y, xv[t].y, a);
                    a = fmaf(wv[e].z, xv[t].z, a);
                    a = fmaf(wv[e].w, xv[t].w, a);
                    acc[8 * t + e] = a;
                }
        }
    }
    const float v = wave_sum_rows<64>(acc);
    const int owner = wave_rows_owner<64>();
    const uint32_t t = t0 + 8u * wt + (uint32_t)(owner >> 3);
    const uint32_t e = e0 + 8u * we + (uint32_t)(owner & 7);
    if (t < tokens && e < rows) {
        if constexpr (B16)
            ((uint16_t *)out)[(uint64_t)t * rows + e] = f32_to_bf16(v);
        else
            ((float *)out)[(uint64_t)t * rows + e] = v;
    }
}

template <bool B16>
bool launch_bf16_gemm_w64(void *out, const void *w, const void *x, uint32_t tokens,
                          uint32_t rows, uint32_t cols, hipStream_t s) {
    const uint32_t token_tiles = (tokens + kGT - 1u) / kGT;
    const uint32_t row_tiles = (rows + kGE - 1u) / kGE;
    const uint32_t xcd = row_tiles >= 8u ? 1u : 0u;
    const uint64_t blocks = xcd ? 8ull * token_tiles * ((row_tiles + 7u) / 8u)
                                : (uint64_t)token_tiles * row_tiles;
    if (blocks > 0x7fffffffull) return false;
    hipLaunchKernelGGL(HIP_KERNEL_NAME(bf16_gemm_w64_kernel<B16>), dim3((uint32_t)blocks), dim3(kGThreads), 0, s, out,
                       (const uint16_t *)w, (const uint16_t *)x, tokens, rows, cols, row_tiles,
                       xcd);
    return hipGetLastError() == hipSuccess;
}

/*
 * Router logits of many tokens (f32, T >= 128) in the reference's order as
 * a blocked GEMM: a block computes 16 tokens x 8 weight rows; a K step is
 * 1024 columns (256 quads), so each of the reference's 256 partials of an
 * output gets exactly one quad per step. Wave w takes partials 64 (w % 4) +
 * lane (its K quarter) of tokens 8 (w / 4) .. + 8 and all 8 rows: one
 * accumulator per output, the quad summed by ref_quad, the quads of a
 * partial in K order as the reference's thread adds them. At the end the
 * K quarters meet in LDS as the reference's tree levels 128 (quarters q
 * and q + 2) and 64 (quarters 0 and 1), and wave_sum_rows<64> does levels
 * 32 .. 1. Out-of-range tokens/rows/columns stage zeros: a zero quad adds
 * +0, which changes no partial (a partial is never -0). The step's bf16
 * tiles are loaded into registers one step ahead and staged in LDS as fp32
 * quads, so each fragment read is one lane-contiguous ds_read_b128. Block
 * order is XCD-aware as in bf16_gemm_w64_kernel.
 */
constexpr int kQT = 16, kQE = 8, kQThreads = 512;

__device__ __forceinline__ float ref_quad_f4(const float4 &w, const float4 &x) {
    const float p2 = __fmul_rn(w.z, x.z), p3 = __fmul_rn(w.w, x.w);
    return __fadd_rn(fmaf(w.y, x.y, p2), fmaf(w.x, x.x, p3));
}

__global__ __launch_bounds__(512) void bf16_gemm_ref_kernel(
        float *__restrict__ out, const uint16_t *__restrict__ weights,
        const uint16_t *__restrict__ input, uint32_t tokens, uint32_t rows, uint32_t cols,
        uint32_t row_tiles, uint32_t xcd_groups) {
    __shared__ float4 xs[kQT][256];
    __shared__ float4 wsm[kQE][256];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    uint32_t tt, et;
    {
        const uint32_t L = blockIdx.x;
        if (xcd_groups) {
            const uint32_t x = L & 7u, j = L >> 3;
            const uint32_t base = row_tiles >> 3, rem = row_tiles & 7u;
            const uint32_t cnt = base + (x < rem ? 1u : 0u);
            const uint32_t start = x * base + (x < rem ? x : rem);
            const uint32_t token_tiles = (tokens + kQT - 1u) / kQT;
            if (cnt == 0u || j >= token_tiles * cnt) return;
            tt = j / cnt;
            et = start + j % cnt;
        } else {
            tt = L / row_tiles;
            et = L % row_tiles;
        }
    }
    const uint32_t t0 = tt * kQT, e0 = et * kQE;
    const uint32_t chunks = cols / 8u, nsteps = (chunks + 127u) / 128u;
    const uint4 *x4 = (const uint4 *)input, *w4 = (const uint4 *)weights;
    /* staging items: 16 token rows then 8 weight rows, 128 chunks each */
    constexpr int kItems = (kQT + kQE) * 128 / kQThreads;
    uint4 reg[kItems];
    auto load_step = [&](uint32_t s) {
#pragma unroll
        for (int q = 0; q < kItems; q++) {
            const uint32_t it = tid + (uint32_t)q * kQThreads;
            const uint32_t r = it >> 7, c = 128u * s + (it & 127u);
            uint4 v = make_uint4(0u, 0u, 0u, 0u);
            if (r < (uint32_t)kQT) {
                if (t0 + r < tokens && c < chunks) v = x4[(uint64_t)(t0 + r) * chunks + c];
            } else if (e0 + r - kQT < rows && c < chunks) {
                v = w4[(uint64_t)(e0 + r - kQT) * chunks + c];
            }
            reg[q] = v;
        }
    };
    const uint32_t kq = wave & 3u, tg = wave >> 2, qi = 64u * kq + lane;
    float acc[64];
#pragma unroll
    for (int i = 0; i < 64; i++) acc[i] = 0.0f;
    load_step(0u);
    for (uint32_t s = 0; s < nsteps; s++) {
        __syncthreads(); /* the previous step's reads are done */
#pragma unroll
        for (int q = 0; q < kItems; q++) {
            const uint32_t it = tid + (uint32_t)q * kQThreads;
            const uint4 v = reg[q];
            const float4 a = make_float4(bf16_lo(v.x), bf16_hi(v.x), bf16_lo(v.y), bf16_hi(v.y));
            const float4 b = make_float4(bf16_lo(v.z), bf16_hi(v.z), bf16_lo(v.w), bf16_hi(v.w));
            const uint32_t r = it >> 7, c = it & 127u;
            float4 *dst = r < (uint32_t)kQT ? &xs[r][2u * c] : &wsm[r - kQT][2u * c];
            dst[0] = a;
            dst[1] = b;
        }
        __syncthreads();
        if (s + 1u < nsteps) load_step(s + 1u);
        float4 wv[kQE];
#pragma unroll
        for (int e = 0; e < kQE; e++) wv[e] = wsm[e][qi];
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const float4 xv = xs[8u * tg + t][qi];
#pragma unroll
            for (int e = 0; e < kQE; e++)
                acc[8 * t + e] = __fadd_rn(acc[8 * t + e], ref_quad_f4(wv[e], xv));
        }
    }
    /* tree levels 128 and 64 across the K quarters, through LDS */
    float *red = (float *)&xs[0][0]; /* [2 token groups][2][64 outputs][64 lanes] */
    __syncthreads();
    if (kq >= 2u) {
#pragma unroll
        for (int i = 0; i < 64; i++) red[((tg * 2u + kq - 2u) * 64u + i) * 64u + lane] = acc[i];
    }
    __syncthreads();
    if (kq < 2u) {
#pragma unroll
        for (int i = 0; i < 64; i++)
            acc[i] = __fadd_rn(acc[i], red[((tg * 2u + kq) * 64u + i) * 64u + lane]);
    }
    __syncthreads();
    if (kq == 1u) {
#pragma unroll
        for (int i = 0; i < 64; i++) red[(tg * 64u + i) * 64u + lane] = acc[i];
    }
    __syncthreads();
    if (kq != 0u) return;
#pragma unroll
    for (int i = 0; i < 64; i++) acc[i] = __fadd_rn(acc[i], red[(tg * 64u + i) * 64u + lane]);
    const float v = wave_sum_rows<64>(acc);
    const int owner = wave_rows_owner<64>();
    const uint32_t t = t0 + 8u * tg + (uint32_t)(owner >> 3);
    const uint32_t e = e0 + (uint32_t)(owner & 7);
    if (t < tokens && e < rows) out[(uint64_t)t * rows + e] = v;
}

bool launch_bf16_gemm_ref(float *out, const void *w, const void *x, uint32_t tokens,
                          uint32_t rows, uint32_t cols, hipStream_t s) {
    const uint32_t token_tiles = (tokens + kQT - 1u) / kQT;
    const uint32_t row_tiles = (rows + kQE - 1u) / kQE;
    const uint32_t xcd = row_tiles >= 8u ? 1u : 0u;
    const uint64_t blocks = xcd ? 8ull * token_tiles * ((row_tiles + 7u) / 8u)
                                : (uint64_t)token_tiles * row_tiles;
    if (blocks > 0x7fffffffull) return false;
    hipLaunchKernelGGL(bf16_gemm_ref_kernel, dim3((uint32_t)blocks), dim3(kQThreads), 0, s, out,
                       (const uint16_t *)w, (const uint16_t *)x, tokens, rows, cols, row_tiles,
                       xcd);
    return hipGetLastError() == hipSuccess;
}

/* ------------------------------------------------------------------------ */
/* router top-k                                                              */
/* ------------------------------------------------------------------------ */

/* One wave per token (4 tokens per block): sigmoid, choice keys and the
 * wave radix select of k3_topk.h. */
__global__ __launch_bounds__(256) void router_topk_kernel(
        uint32_t *__restrict__ ids_out, float *__restrict__ w_out,
        uint32_t *ids_copy, float *w_copy,
        const float *__restrict__ logits, const float *__restrict__ bias,
        uint32_t tokens, uint32_t experts, uint32_t top_k, float scale) {
    __shared__ TopkWaveSmem sm[4];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t t = blockIdx.x * 4u + wave;
    if (t >= tokens) return;
    const float *lg = logits + (uint64_t)t * experts;
    uint32_t key[kTopkSlots];
    float score[kTopkSlots];
#pragma unroll
    for (int j = 0; j < kTopkSlots; j++) {
        const uint32_t e = lane + 64u * j;
        key[j] = 0u;
        score[j] = 0.0f;
        if (e < experts) {
            score[j] = det_sigmoid(lg[e]);
            key[j] = choice_key(router_sigmoid(lg[e]), bias[e]);
        }
    }
    const uint64_t o = (uint64_t)t * top_k;
    topk_select_wave(key, score, top_k, scale, ids_out + o, w_out + o,
                     ids_copy ? ids_copy + o : nullptr, w_copy ? w_copy + o : nullptr, sm[wave]);
}

/* ------------------------------------------------------------------------ */
/* MXFP4 rows (generic GEMV / GEMM behind the reference ABI)                 */
/* ------------------------------------------------------------------------ */

__device__ __forceinline__ uint4 load_group(const uint8_t *p, uint32_t align16) {
    if (align16) return *(const uint4 *)p;
    /* 8-byte aligned starts occur in real checkpoints (k3_rocm_ops.cu:207-223). */
    const uint2 a = ((const uint2 *)p)[0], b = ((const uint2 *)p)[1];
    return make_uint4(a.x, a.y, b.x, b.y);
}

template <int TT>
__global__ __launch_bounds__(256) void mxfp4_rows_kernel(
        uint16_t *__restrict__ out, const uint8_t *__restrict__ packed,
        const uint8_t *__restrict__ scales, const uint16_t *__restrict__ input,
        uint32_t tokens, uint32_t rows, uint32_t cols, uint32_t align16) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const uint32_t t0 = blockIdx.y * TT;
    if (row >= rows) return;
    const uint32_t active = tokens - t0 < (uint32_t)TT ? tokens - t0 : (uint32_t)TT;
    const uint32_t groups = cols / 32u;
    const uint8_t *prow = packed + (uint64_t)row * (cols / 2u);
    const uint8_t *srow = scales + (uint64_t)row * groups;
    float acc[TT];
#pragma unroll
    for (int t = 0; t < TT; t++) acc[t] = 0.0f;
    for (uint32_t g = lane; g < groups; g += 64u) {
        const uint4 wv = load_group(prow + 16u * g, align16);
        const float sc = e8m0_to_f32(srow[g]);
#pragma unroll
        for (int t = 0; t < TT; t++) {
            if ((uint32_t)t < active) {
                float xf[32];
                bf16x32_to_f32((const uint4 *)(input + (uint64_t)(t0 + t) * cols) + 4u * g, xf);
                acc[t] = fmaf(fp4_group(wv, xf), sc, acc[t]);
            }
        }
    }
    const float v = wave_sum_rows<TT>(acc);
    const int owner = wave_rows_owner<TT>();
    if ((lane & (64u / TT - 1u)) == 0u && (uint32_t)owner < active)
        out[(uint64_t)(t0 + owner) * rows + row] = f32_to_bf16(v);
}

template <int TT>
bool launch_mxfp4_rows(void *out, const void *p, const void *s, const void *x,
                       uint32_t tokens, uint32_t rows, uint32_t cols, hipStream_t st) {
    const uint32_t align16 = ((uintptr_t)p % 16u) == 0u;
    dim3 grid((rows + kWavesPerBlock - 1u) / kWavesPerBlock, (tokens + TT - 1u) / TT);
    hipLaunchKernelGGL(HIP_KERNEL_NAME(mxfp4_rows_kernel<TT>), grid, dim3(kThreads), 0, st,
                       (uint16_t *)out, (const uint8_t *)p, (const uint8_t *)s,
                       (const uint16_t *)x, tokens, rows, cols, align16);
    return hipGetLastError() == hipSuccess;
}

/* ------------------------------------------------------------------------ */
/* Q8-128 static projections                                                 */
/* ------------------------------------------------------------------------ */

/* 32 int8 codes of a group: 16-byte aligned rows load two uint4, 8-byte
 * aligned ones four uint2 (the reference reads 8-byte octets). */
__device__ __forceinline__ void load_q8_group(const int8_t *p, uint32_t align16, uint4 &a,
                                              uint4 &b) {
    if (align16) {
        a = ((const uint4 *)p)[0];
        b = ((const uint4 *)p)[1];
        return;
    }
    const uint2 *q = (const uint2 *)p;
    const uint2 c0 = q[0], c1 = q[1], c2 = q[2], c3 = q[3];
    a = make_uint4(c0.x, c0.y, c1.x, c1.y);
    b = make_uint4(c2.x, c2.y, c3.x, c3.y);
}

/* gs = fmaf(q_i, x_i, gs) over the group's 32 columns in order. */
__device__ __forceinline__ float q8_group(const uint4 &a, const uint4 &b, const float *x) {
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float gs = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++)
#pragma unroll
        for (int i = 0; i < 4; i++)
            gs = fmaf((float)(int8_t)(w[k] >> (8 * i)), x[4 * k + i], gs);
    return gs;
}

/* One wave per row (tokens in tiles of TT); order in the file header. */
template <int TT>
__global__ __launch_bounds__(256) void q8_rows_kernel(
        uint16_t *__restrict__ out, const int8_t *__restrict__ codes,
        const float *__restrict__ scales, const uint16_t *__restrict__ input,
        uint32_t tokens, uint32_t rows, uint32_t cols, uint32_t align16) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const uint32_t t0 = blockIdx.y * TT;
    if (row >= rows) return;
    const uint32_t active = tokens - t0 < (uint32_t)TT ? tokens - t0 : (uint32_t)TT;
    const uint32_t groups = cols / 32u;
    const int8_t *qrow = codes + (uint64_t)row * cols;
    const float *srow = scales + (uint64_t)row * (cols / 128u);
    float acc[TT];
#pragma unroll
    for (int t = 0; t < TT; t++) acc[t] = 0.0f;
    for (uint32_t g = lane; g < groups; g += 64u) {
        uint4 a, b;
        load_q8_group(qrow + 32u * g, align16, a, b);
        const float sc = srow[g >> 2];
#pragma unroll
        for (int t = 0; t < TT; t++) {
            if ((uint32_t)t < active) {
                float xf[32];
                bf16x32_to_f32((const uint4 *)(input + (uint64_t)(t0 + t) * cols) + 4u * g, xf);
                acc[t] = fmaf(q8_group(a, b, xf), sc, acc[t]);
            }
        }
    }
    const float v = wave_sum_rows<TT>(acc);
    const int owner = wave_rows_owner<TT>();
    if ((lane & (64u / TT - 1u)) == 0u && (uint32_t)owner < active)
        out[(uint64_t)(t0 + owner) * rows + row] = f32_to_bf16(v);
}

template <int TT>
bool launch_q8_rows(void *out, const void *q, const void *s, const void *x, uint32_t tokens,
                    uint32_t rows, uint32_t cols, hipStream_t st) {
    const uint32_t align16 = ((uintptr_t)q % 16u) == 0u;
    dim3 grid((rows + kWavesPerBlock - 1u) / kWavesPerBlock, (tokens + TT - 1u) / TT);
    hipLaunchKernelGGL(HIP_KERNEL_NAME(q8_rows_kernel<TT>), grid, dim3(kThreads), 0, st,
                       (uint16_t *)out, (const int8_t *)q, (const float *)s, (const uint16_t *)x,
                       tokens, rows, cols, align16);
    return hipGetLastError() == hipSuccess;
}

/* RMSNorm pieces shared by rms_norm_kernel and the normalising GEMV, so
 * that both produce the same bits. Thread t of a 256-thread block owns the
 * 8-element chunks t + 256 j (j < kRmsChunks) of the vector. */
constexpr int kRmsChunks = 4; /* 8-element chunks per thread: hidden <= 8192 */

__device__ __forceinline__ float rms_sumsq(const uint4 (&xv)[kRmsChunks], uint32_t t,
                                           uint32_t chunks) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kRmsChunks; j++) {
        if (t + 256u * (uint32_t)j < chunks) {
            const uint32_t u[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                s = fmaf(bf16_lo(u[q]), bf16_lo(u[q]), s);
                s = fmaf(bf16_hi(u[q]), bf16_hi(u[q]), s);
            }
        }
    }
    return s;
}

/* 1 / sqrt(total / hidden + eps) from the four per-wave sums. */
__device__ __forceinline__ float rms_inv(const float (&part)[4], uint32_t hidden, float eps) {
    const float total = __fadd_rn(__fadd_rn(part[0], part[1]), __fadd_rn(part[2], part[3]));
    return __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(total, (float)hidden), eps)));
}

/* Two packed bf16 of x, scaled: bf16((x * inv) * w). */
__device__ __forceinline__ uint32_t rms_apply2(uint32_t u, uint32_t w, float inv) {
    const uint32_t lo = f32_to_bf16(__fmul_rn(__fmul_rn(bf16_lo(u), inv), bf16_lo(w)));
    const uint32_t hi = f32_to_bf16(__fmul_rn(__fmul_rn(bf16_hi(u), inv), bf16_hi(w)));
    return lo | (hi << 16);
}

/*
 * Single-vector Q8-128 projections for cols <= 8192, R rows per row set
 * and RS row sets per block of 256 threads: the 4 / RS waves of a row set
 * split K into 64-group stripes (RS = 2 needs cols <= 4096, RS = 4 cols <=
 * 2048). Each lane loads its group of x once for all R rows; the unscaled
 * group sums and their scales meet in LDS, and lane l then chains acc =
 * fmaf(gs, scale, acc) over its groups l, l + 64, ... in order -- exactly
 * q8_rows_kernel's per lane sequence -- before the same wave64 butterfly,
 * so the outputs are bit-identical to it. One wave per row re-read x from
 * L2 for every row, twice the bytes of the int8 weight row itself.
 *
 * DUAL (RS = 1): rows r of two matrices (gate, up) per block and out =
 * bf16(act(bf16(gate), bf16(up))), the shared expert's gate/up/activation
 * in one pass. Otherwise out = bf16(v), or with the epilogue addends
 * bf16(add2 + bf16(add1 + bf16(v))) (two bf16 adds, in that order).
 *
 * NORM: x is first replaced by rms_norm_kernel's output for (x, norm_w,
 * eps), bit for bit: every block recomputes the sum of squares in that
 * kernel's order from the vector and norm weight it loads before the
 * weight rows, normalises its own chunks into LDS and reads its groups
 * back, which saves the norm's launch and its round trip through memory.
 */
constexpr int kQ8DualRows = 8; /* rows per block of the DUAL kernel */

template <bool DUAL, int R, int RS, bool NORM>
struct Q8GemvSmem {
    static constexpr int NM = DUAL ? 2 : 1, SPS = 4 / RS, RB = R * RS;
    float part[NM * RB][SPS][64];
    float scl[NM * RB][SPS][64];
    float npart[4];
    uint4 xn[NORM ? 8192 / 8 : 1]; /* the normalised vector */
};

struct Q8GemvArgs {
    uint16_t *out;
    const int8_t *codes_a;
    const float *scales_a;
    const int8_t *codes_b;
    const float *scales_b;
    const uint16_t *x;
    uint32_t rows, cols, align16;
    const uint16_t *add1, *add2;
    uint32_t act_kind;
    float beta, lb;
    const uint16_t *norm_w;
    float eps;
};

/* Block `bid` of a q8_gemv launch (the kernel body, shared by the launches
 * that run two projections as one grid). */
template <bool DUAL, int R, int RS, bool NORM>
__device__ __forceinline__ void q8_gemv_block(Q8GemvSmem<DUAL, R, RS, NORM> &sm, uint32_t bid,
                                              const Q8GemvArgs &A) {
    static_assert(RS == 1 || RS == 2 || RS == 4, "row sets");
    static_assert(!DUAL || RS == 1, "DUAL uses one row set");
    constexpr int NM = DUAL ? 2 : 1, SPS = 4 / RS, RB = R * RS;
    static_assert(RB >= 4, "at least one row per wave in the reduction");
    auto &part = sm.part;
    auto &scl = sm.scl;
    auto &npart = sm.npart;
    auto &xn = sm.xn;
    uint16_t *__restrict__ out = A.out;
    const int8_t *__restrict__ codes_a = A.codes_a;
    const float *__restrict__ scales_a = A.scales_a;
    const int8_t *__restrict__ codes_b = A.codes_b;
    const float *__restrict__ scales_b = A.scales_b;
    const uint16_t *__restrict__ x = A.x;
    const uint32_t rows = A.rows, cols = A.cols, align16 = A.align16;
    const uint16_t *__restrict__ add1 = A.add1;
    const uint16_t *__restrict__ add2 = A.add2;
    const uint16_t *__restrict__ norm_w = A.norm_w;
    const uint32_t act_kind = A.act_kind;
    const float beta = A.beta, lb = A.lb, eps = A.eps;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t set = wave / SPS, stripe = wave % SPS;
    const uint32_t row0 = bid * RB + set * R;
    const uint32_t groups = cols / 32u, g = 64u * stripe + lane;
    const bool active = g < groups;
    /* NORM: the vector and the norm weight first, so that waiting for them
     * does not wait for the weight rows (loads complete in issue order) */
    uint4 xv[NORM ? kRmsChunks : 1], nv[NORM ? kRmsChunks : 1];
    const uint32_t chunks = cols / 8u;
    if constexpr (NORM) {
#pragma unroll
        for (int j = 0; j < kRmsChunks; j++) {
            const uint32_t c = threadIdx.x + 256u * (uint32_t)j;
            if (c < chunks) {
                xv[j] = ((const uint4 *)x)[c];
                nv[j] = ((const uint4 *)norm_w)[c];
            }
        }
    }
    uint4 wa[NM * R], wb[NM * R];
    float sc[NM * R];
    if (active) {
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const int8_t *q = m ? codes_b : codes_a;
            const float *sp = m ? scales_b : scales_a;
#pragma unroll
            for (int i = 0; i < R; i++) {
                const uint32_t r = row0 + (uint32_t)i < rows ? row0 + (uint32_t)i : rows - 1u;
                load_q8_group(q + (uint64_t)r * cols + 32u * g, align16, wa[m * R + i],
                              wb[m * R + i]);
                sc[m * R + i] = sp[(uint64_t)r * (cols / 128u) + (g >> 2)];
            }
        }
    }
    float xf[32];
    if constexpr (NORM) {
        /* rms_norm_kernel's sum, then each thread normalises its own chunks
         * into LDS and every lane reads its group back */
        const uint32_t t = threadIdx.x;
        const float s = wave_sum(rms_sumsq(xv, t, chunks));
        if (lane == 0u) npart[wave] = s;
        __syncthreads();
        const float inv = rms_inv(npart, cols, eps);
#pragma unroll
        for (int j = 0; j < kRmsChunks; j++) {
            const uint32_t c = t + 256u * (uint32_t)j;
            if (c < chunks)
                xn[c] = make_uint4(rms_apply2(xv[j].x, nv[j].x, inv),
                                   rms_apply2(xv[j].y, nv[j].y, inv),
                                   rms_apply2(xv[j].z, nv[j].z, inv),
                                   rms_apply2(xv[j].w, nv[j].w, inv));
        }
        __syncthreads();
        if (active) bf16x32_to_f32(xn + 4u * g, xf);
    } else {
        if (active) bf16x32_to_f32((const uint4 *)x + 4u * g, xf);
    }
    if (active) {
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int i = 0; i < R; i++) {
                const int pr = m * RB + (int)set * R + i;
                part[pr][stripe][lane] = q8_group(wa[m * R + i], wb[m * R + i], xf);
                scl[pr][stripe][lane] = sc[m * R + i];
            }
    }
    __syncthreads();
    constexpr int RPW = RB / 4; /* rows per wave (per matrix) in the reduction */
    const uint32_t stripes = (groups + 63u) / 64u;
    float p[NM * RPW];
#pragma unroll
    for (int q = 0; q < NM * RPW; q++) {
        const int i = (q / RPW) * RB + (int)wave * RPW + (q % RPW);
        float acc = 0.0f;
        for (uint32_t j = 0; j < stripes; j++)
            if (64u * j + lane < groups) acc = fmaf(part[i][j][lane], scl[i][j][lane], acc);
        p[q] = acc;
    }
    const float v = wave_sum_rows<NM * RPW>(p);
    const uint32_t base = bid * RB + RPW * wave;
    if constexpr (DUAL) {
        /* lanes < 32: gate rows, lanes >= 32: the same up rows */
        const float u = __shfl_xor(v, 32, 64);
        const float gb = bf16_to_f32(f32_to_bf16(v)), ub = bf16_to_f32(f32_to_bf16(u));
        constexpr uint32_t kSpan = 32u / RPW;
        const uint32_t row = base + lane / kSpan;
        if (lane < 32u && (lane & (kSpan - 1u)) == 0u && row < rows)
            out[row] = f32_to_bf16(gated_act(gb, ub, act_kind, beta, lb));
    } else {
        const int owner = wave_rows_owner<RPW>();
        const uint32_t row = base + (uint32_t)owner;
        if ((lane & (64u / RPW - 1u)) == 0u && row < rows) {
            float r = bf16_to_f32(f32_to_bf16(v));
            if (add1) r = bf16_to_f32(f32_to_bf16(__fadd_rn(bf16_to_f32(add1[row]), r)));
            if (add2) r = __fadd_rn(bf16_to_f32(add2[row]), r);
            out[row] = f32_to_bf16(r);
        }
    }
}

template <bool DUAL, int R, int RS, bool NORM>
__global__ __launch_bounds__(256) void q8_gemv_kernel(Q8GemvArgs A) {
    __shared__ Q8GemvSmem<DUAL, R, RS, NORM> sm;
    q8_gemv_block<DUAL, R, RS, NORM>(sm, blockIdx.x, A);
}

/* Two independent single-vector projections as one grid: blocks [0, nd)
 * run the fused gate/up/activation (DUAL, 8 rows), the rest a plain
 * projection (4 rows). One launch ramp and tail instead of two. With nr >
 * 0, blocks [0, nr) first compute router rows on the same x
 * (router_rows_wave, kPairRouterRows per wave): their latency-bound loads
 * then overlap the projections' streaming instead of running as a launch
 * of their own. */
constexpr int kPairRouterRows = 1;

__global__ __launch_bounds__(256) void q8_gemv_pair_kernel(Q8GemvArgs D, Q8GemvArgs S,
                                                           RouterRows R, uint32_t nd,
                                                           uint32_t nr) {
    __shared__ union {
        Q8GemvSmem<true, 8, 1, false> d;
        Q8GemvSmem<false, 4, 1, false> s;
    } sm;
    if (blockIdx.x < nr) {
        router_rows_wave<kPairRouterRows>(
            R, (blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6)) * kPairRouterRows);
        return;
    }
    const uint32_t b = blockIdx.x - nr;
    if (b < nd)
        q8_gemv_block<true, 8, 1, false>(sm.d, b, D);
    else
        q8_gemv_block<false, 4, 1, false>(sm.s, b - nd, S);
}

/* One wave per 128-element block: scale = max|w| / 127 (1 for an all-zero
 * block), code = clamp(rint(w / scale), -127, 127) with IEEE division;
 * a NaN weight codes as 0 (k3_rocm_ops.cu:662-697). */
__global__ __launch_bounds__(256) void q8_quantize_kernel(int8_t *__restrict__ codes,
                                                          float *__restrict__ scales,
                                                          const uint16_t *__restrict__ w,
                                                          uint64_t blocks) {
    const uint64_t blk = (uint64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    if (blk >= blocks) return;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t pair = ((const uint32_t *)(w + 128u * blk))[lane];
    const float v0 = bf16_lo(pair), v1 = bf16_hi(pair);
    float m = fmaxf(fabsf(v0), fabsf(v1));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    const float sc = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
    auto code = [&](float v) -> uint32_t {
        float r = rintf(__fdiv_rn(v, sc));
        if (r != r) r = 0.0f;
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        return (uint32_t)(uint8_t)(int8_t)(int)r;
    };
    ((uint16_t *)(codes + 128u * blk))[lane] = (uint16_t)(code(v0) | (code(v1) << 8));
    if (lane == 0u) scales[blk] = sc;
}

/* w = bf16(q * scale) (k3_rocm_ops.cu:699-711). */
__global__ void q8_dequantize_kernel(uint16_t *__restrict__ w, const int8_t *__restrict__ codes,
                                     const float *__restrict__ scales, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)blockDim.x * gridDim.x)
        w[i] = f32_to_bf16(__fmul_rn((float)codes[i], scales[i / 128u]));
}

/* ------------------------------------------------------------------------ */
/* elementwise                                                               */
/* ------------------------------------------------------------------------ */

__global__ void gated_act_kernel(uint16_t *__restrict__ out, const uint16_t *__restrict__ gate,
                                 const uint16_t *__restrict__ up, uint64_t n, uint32_t kind,
                                 float beta, float lb) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)blockDim.x * gridDim.x)
        out[i] = f32_to_bf16(gated_act(bf16_to_f32(gate[i]), bf16_to_f32(up[i]), kind, beta, lb));
}

/* out[t, d] = bf16(sum_r w[t, r] * v[t, r, d]) in rank order, products and
 * sums rounded separately (k3_rocm_ops.cu:1452-1474). */
__global__ void weighted_sum_kernel(uint16_t *__restrict__ out, const uint16_t *__restrict__ v,
                                    const float *__restrict__ w, uint32_t count, uint32_t hidden) {
    const uint32_t t = blockIdx.y;
    const uint16_t *vt = v + (uint64_t)t * count * hidden;
    const float *wt = w + (uint64_t)t * count;
    for (uint32_t d = blockIdx.x * blockDim.x + threadIdx.x; d < hidden; d += blockDim.x * gridDim.x) {
        float sum = 0.0f;
        for (uint32_t r = 0; r < count; r++)
            sum = __fadd_rn(sum, __fmul_rn(wt[r], bf16_to_f32(vt[(uint64_t)r * hidden + d])));
        out[(uint64_t)t * hidden + d] = f32_to_bf16(sum);
    }
}

template <bool Scatter>
__global__ void copy_rows_kernel(uint16_t *__restrict__ out, const uint16_t *__restrict__ in,
                                 const uint32_t *__restrict__ ids, uint32_t row_count,
                                 uint32_t row_size) {
    const uint64_t n = (uint64_t)row_count * row_size;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)blockDim.x * gridDim.x) {
        const uint32_t r = (uint32_t)(i / row_size), c = (uint32_t)(i % row_size);
        const uint64_t j = (uint64_t)ids[r] * row_size + c;
        if (Scatter) out[j] = in[i];
        else out[i] = in[j];
    }
}

__global__ void add_kernel(uint16_t *__restrict__ out, const uint16_t *__restrict__ a,
                           const uint16_t *__restrict__ b, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)blockDim.x * gridDim.x)
        out[i] = f32_to_bf16(__fadd_rn(bf16_to_f32(a[i]), bf16_to_f32(b[i])));
}

/* One block of 256 threads per vector. Order: thread t owns 8-element
 * chunks t, t + 256, ... (elements in order within a chunk), s =
 * fmaf(v, v, s); a wave64 butterfly per wave; total = (w0 + w1) + (w2 +
 * w3); inv = 1 / sqrt(total / hidden + eps) (IEEE); out = bf16((x * inv) *
 * weight). hidden <= 8192 with 16-byte rows keeps the vector in registers
 * (every load issued up front: one memory round trip); otherwise the same
 * order element by element. */
__global__ __launch_bounds__(256) void rms_norm_kernel(uint16_t *__restrict__ out,
                                                       const uint16_t *__restrict__ in,
                                                       const uint16_t *__restrict__ weight,
                                                       uint32_t hidden, float eps, uint32_t vec) {
    __shared__ float part[4];
    const uint32_t t = threadIdx.x;
    const uint16_t *x = in + (uint64_t)blockIdx.x * hidden;
    uint16_t *o = out + (uint64_t)blockIdx.x * hidden;
    const uint32_t chunks = (hidden + 7u) / 8u;
    if (vec) {
        uint4 xv[kRmsChunks], wv[kRmsChunks];
#pragma unroll
        for (int j = 0; j < kRmsChunks; j++) {
            const uint32_t c = t + 256u * (uint32_t)j;
            if (c < chunks) {
                xv[j] = ((const uint4 *)x)[c];
                wv[j] = ((const uint4 *)weight)[c];
            }
        }
        const float s = wave_sum(rms_sumsq(xv, t, chunks));
        if ((t & 63u) == 0u) part[t >> 6] = s;
        __syncthreads();
        const float inv = rms_inv(part, hidden, eps);
#pragma unroll
        for (int j = 0; j < kRmsChunks; j++) {
            const uint32_t c = t + 256u * (uint32_t)j;
            if (c < chunks)
                ((uint4 *)o)[c] = make_uint4(rms_apply2(xv[j].x, wv[j].x, inv),
                                             rms_apply2(xv[j].y, wv[j].y, inv),
                                             rms_apply2(xv[j].z, wv[j].z, inv),
                                             rms_apply2(xv[j].w, wv[j].w, inv));
        }
        return;
    }
    float s = 0.0f;
    for (uint32_t c = t; c < chunks; c += 256u) {
        const uint32_t end = 8u * c + 8u < hidden ? 8u * c + 8u : hidden;
        for (uint32_t d = 8u * c; d < end; d++) {
            const float v = bf16_to_f32(x[d]);
            s = fmaf(v, v, s);
        }
    }
    s = wave_sum(s);
    if ((t & 63u) == 0u) part[t >> 6] = s;
    __syncthreads();
    const float inv = rms_inv(part, hidden, eps);
    for (uint32_t d = t; d < hidden; d += 256u)
        o[d] = f32_to_bf16(__fmul_rn(__fmul_rn(bf16_to_f32(x[d]), inv), bf16_to_f32(weight[d])));
}

}  // namespace

namespace {
/* f32 router logits: the reference's order on every path */
bool launch_bf16_ref_any(float *out, const void *w, const void *x, uint32_t tokens,
                         uint32_t rows, uint32_t cols, hipStream_t s) {
    if (tokens == 1u) return launch_bf16_rows_ref<1>(out, w, x, 1u, rows, cols, s);
    if (tokens <= 4u) return launch_bf16_rows_ref<4>(out, w, x, tokens, rows, cols, s);
    if (tokens >= kGemmMinTokens && cols % 8u == 0u && ((uintptr_t)w | (uintptr_t)x) % 16u == 0u)
        return launch_bf16_gemm_ref(out, w, x, tokens, rows, cols, s);
    return launch_bf16_rows_ref<16>(out, w, x, tokens, rows, cols, s);
}

template <bool B16>
bool launch_bf16_rows_any(void *out, const void *w, const void *x, uint32_t tokens,
                          uint32_t rows, uint32_t cols, hipStream_t s) {
    if (tokens == 1u) return launch_bf16_rows_f32<1, B16>(out, w, x, 1u, rows, cols, s);
    if (tokens <= 4u) return launch_bf16_rows_f32<4, B16>(out, w, x, tokens, rows, cols, s);
    /* many tokens: the blocked GEMM (same bits); it needs 16-byte rows */
    if (tokens >= kGemmMinTokens && cols % 8u == 0u && ((uintptr_t)w | (uintptr_t)x) % 16u == 0u)
        return launch_bf16_gemm_w64<B16>(out, w, x, tokens, rows, cols, s);
    return launch_bf16_rows_f32<16, B16>(out, w, x, tokens, rows, cols, s);
}
}  // namespace

bool k3::launch_bf16_rows_f32_any(float *out, const void *w, const void *x, uint32_t tokens,
                                  uint32_t rows, uint32_t cols, hipStream_t s) {
    return launch_bf16_ref_any(out, w, x, tokens, rows, cols, s);
}

bool k3::launch_bf16_rows_bf16_any(uint16_t *out, const void *w, const void *x, uint32_t tokens,
                                   uint32_t rows, uint32_t cols, hipStream_t s) {
    return launch_bf16_rows_any<true>(out, w, x, tokens, rows, cols, s);
}

bool k3::launch_router_topk(uint32_t *ids, float *w, uint32_t *ids2, float *w2,
                            const float *logits, const float *bias, uint32_t tokens,
                            uint32_t experts, uint32_t top_k, float scale, hipStream_t s) {
    hipLaunchKernelGGL(router_topk_kernel, dim3((tokens + 3u) / 4u), dim3(256), 0, s, ids, w, ids2,
                       w2, logits, bias, tokens, experts, top_k, scale);
    return hipGetLastError() == hipSuccess;
}

/* ======================================================================== */
/* C ABI                                                                     */
/* ======================================================================== */

extern "C" bool k3_rocm_situ_bf16(void *output, const void *gate, const void *up,
                                  uint64_t element_count, float beta, float linear_beta,
                                  void *stream) {
    if (!output || !gate || !up || element_count == 0u || !(beta > 0.0f) ||
        !(linear_beta > 0.0f))
        return false;
    hipLaunchKernelGGL(gated_act_kernel, dim3(grid_cap((element_count + 255u) / 256u)),
                       dim3(256), 0, (hipStream_t)stream, (uint16_t *)output,
                       (const uint16_t *)gate, (const uint16_t *)up, element_count, 0u, beta,
                       linear_beta);
    return hipGetLastError() == hipSuccess;
}

extern "C" bool k3_rocm_swiglu_bf16(void *output, const void *gate, const void *up,
                                    uint64_t element_count, void *stream) {
    if (!output || !gate || !up || element_count == 0u) return false;
    hipLaunchKernelGGL(gated_act_kernel, dim3(grid_cap((element_count + 255u) / 256u)),
                       dim3(256), 0, (hipStream_t)stream, (uint16_t *)output,
                       (const uint16_t *)gate, (const uint16_t *)up, element_count, 1u, 1.0f,
                       1.0f);
    return hipGetLastError() == hipSuccess;
}

extern "C" bool k3_rocm_mxfp4_gemm_tiled_bf16(void *output, const void *packed,
                                              const void *scales, const void *input,
                                              uint32_t vector_count, uint32_t rows,
                                              uint32_t columns, uint32_t batch_tile,
                                              void *stream) {
    if (!output || !packed || !scales || !input || vector_count == 0u ||
        vector_count > 65535u || rows == 0u || columns == 0u || columns % 32u != 0u ||
        ((uintptr_t)packed % 8u) != 0u || ((uintptr_t)input % 16u) != 0u)
        return false;
    const hipStream_t s = (hipStream_t)stream;
    switch (batch_tile) {
        case 16u: return launch_mxfp4_rows<16>(output, packed, scales, input, vector_count, rows, columns, s);
        case 32u: return launch_mxfp4_rows<32>(output, packed, scales, input, vector_count, rows, columns, s);
        case 64u: return launch_mxfp4_rows<64>(output, packed, scales, input, vector_count, rows, columns, s);
        default: return false;
    }
}

extern "C" bool k3_rocm_mxfp4_gemm_bf16(void *output, const void *packed, const void *scales,
                                        const void *input, uint32_t vector_count, uint32_t rows,
                                        uint32_t columns, void *stream) {
    if (!output || !packed || !scales || !input || vector_count == 0u ||
        vector_count > 65535u || rows == 0u || columns == 0u || columns % 32u != 0u ||
        ((uintptr_t)packed % 8u) != 0u || ((uintptr_t)input % 16u) != 0u)
        return false;
    const hipStream_t s = (hipStream_t)stream;
    if (vector_count == 1u)
        return launch_mxfp4_rows<1>(output, packed, scales, input, 1u, rows, columns, s);
    if (vector_count <= 4u)
        return launch_mxfp4_rows<4>(output, packed, scales, input, vector_count, rows, columns, s);
    return launch_mxfp4_rows<16>(output, packed, scales, input, vector_count, rows, columns, s);
}

extern "C" bool k3_rocm_mxfp4_gemv_bf16(void *output, const void *packed, const void *scales,
                                        const void *input, uint32_t rows, uint32_t columns,
                                        void *stream) {
    return k3_rocm_mxfp4_gemm_bf16(output, packed, scales, input, 1u, rows, columns, stream);
}

extern "C" bool k3_rocm_bf16_gemm_tiled_f32(void *output, const void *weights,
                                            const void *input, uint32_t vector_count,
                                            uint32_t rows, uint32_t columns,
                                            uint32_t batch_tile, void *stream) {
    if (!output || !weights || !input || vector_count == 0u || vector_count > 65535u ||
        rows == 0u || columns == 0u)
        return false;
    /* the tile changes no bit of the reference's per-row order */
    if (batch_tile != 16u && batch_tile != 32u && batch_tile != 64u) return false;
    return k3::launch_bf16_rows_f32_any((float *)output, weights, input, vector_count, rows,
                                        columns, (hipStream_t)stream);
}

extern "C" bool k3_rocm_bf16_gemm_f32(void *output, const void *weights, const void *input,
                                      uint32_t vector_count, uint32_t rows, uint32_t columns,
                                      void *stream) {
    if (!output || !weights || !input || vector_count == 0u || vector_count > 65535u ||
        rows == 0u || columns == 0u)
        return false;
    return k3::launch_bf16_rows_f32_any((float *)output, weights, input, vector_count, rows,
                                        columns, (hipStream_t)stream);
}

extern "C" bool k3_rocm_bf16_gemv_f32(void *output, const void *weights, const void *input,
                                      uint32_t rows, uint32_t columns, void *stream) {
    return k3_rocm_bf16_gemm_f32(output, weights, input, 1u, rows, columns, stream);
}

extern "C" bool k3_rocm_router_topk_f32_batch(void *expert_ids, void *expert_weights,
                                              const void *logits, const void *correction_bias,
                                              uint32_t vector_count, uint32_t expert_count,
                                              uint32_t top_k, float scaling_factor,
                                              void *stream) {
    if (!expert_ids || !expert_weights || !logits || !correction_bias || vector_count == 0u ||
        vector_count > 65535u || expert_count == 0u || top_k == 0u || top_k > expert_count ||
        expert_count > 1024u || top_k > 32u || !(scaling_factor > 0.0f))
        return false;
    return k3::launch_router_topk((uint32_t *)expert_ids, (float *)expert_weights, nullptr,
                                  nullptr, (const float *)logits,
                                  (const float *)correction_bias, vector_count, expert_count,
                                  top_k, scaling_factor, (hipStream_t)stream);
}

extern "C" bool k3_rocm_router_topk_f32(void *expert_ids, void *expert_weights,
                                        const void *logits, const void *correction_bias,
                                        uint32_t expert_count, uint32_t top_k,
                                        float scaling_factor, void *stream) {
    return k3_rocm_router_topk_f32_batch(expert_ids, expert_weights, logits, correction_bias, 1u,
                                         expert_count, top_k, scaling_factor, stream);
}

extern "C" bool k3_rocm_weighted_sum_bf16_batch(void *output, const void *vectors,
                                                const void *weights, uint32_t token_count,
                                                uint32_t vector_count, uint32_t hidden_size,
                                                void *stream) {
    if (!output || !vectors || !weights || token_count == 0u || token_count > 65535u ||
        vector_count == 0u || hidden_size == 0u)
        return false;
    hipLaunchKernelGGL(weighted_sum_kernel, dim3((hidden_size + 255u) / 256u, token_count),
                       dim3(256), 0, (hipStream_t)stream, (uint16_t *)output,
                       (const uint16_t *)vectors, (const float *)weights, vector_count,
                       hidden_size);
    return hipGetLastError() == hipSuccess;
}

extern "C" bool k3_rocm_weighted_sum_bf16(void *output, const void *vectors, const void *weights,
                                          uint32_t vector_count, uint32_t hidden_size,
                                          void *stream) {
    return k3_rocm_weighted_sum_bf16_batch(output, vectors, weights, 1u, vector_count,
                                           hidden_size, stream);
}

static bool copy_rows(bool scatter, void *output, const void *input, const void *row_ids,
                      uint32_t row_count, uint32_t row_size, void *stream) {
    if (!output || !input || !row_ids || row_count == 0u || row_size == 0u) return false;
    const uint64_t n = (uint64_t)row_count * row_size;
    const dim3 grid(grid_cap((n + 255u) / 256u));
    if (scatter)
        hipLaunchKernelGGL(HIP_KERNEL_NAME(copy_rows_kernel<true>), grid, dim3(256), 0,
                           (hipStream_t)stream, (uint16_t *)output, (const uint16_t *)input,
                           (const uint32_t *)row_ids, row_count, row_size);
    else
        hipLaunchKernelGGL(HIP_KERNEL_NAME(copy_rows_kernel<false>), grid, dim3(256), 0,
                           (hipStream_t)stream, (uint16_t *)output, (const uint16_t *)input,
                           (const uint32_t *)row_ids, row_count, row_size);
    return hipGetLastError() == hipSuccess;
}

extern "C" bool k3_rocm_gather_rows_bf16(void *output, const void *input, const void *row_ids,
                                         uint32_t row_count, uint32_t row_size, void *stream) {
    return copy_rows(false, output, input, row_ids, row_count, row_size, stream);
}

extern "C" bool k3_rocm_scatter_rows_bf16(void *output, const void *input, const void *row_ids,
                                          uint32_t row_count, uint32_t row_size, void *stream) {
    return copy_rows(true, output, input, row_ids, row_count, row_size, stream);
}

extern "C" bool k3_rocm_add_bf16(void *output, const void *left, const void *right,
                                 uint64_t element_count, void *stream) {
    if (!output || !left || !right || element_count == 0u) return false;
    hipLaunchKernelGGL(add_kernel, dim3(grid_cap((element_count + 255u) / 256u)), dim3(256), 0,
                       (hipStream_t)stream, (uint16_t *)output, (const uint16_t *)left,
                       (const uint16_t *)right, element_count);
    return hipGetLastError() == hipSuccess;
}

extern "C" bool k3_rocm_rms_norm_bf16(void *output, const void *input, const void *weight,
                                      uint32_t vector_count, uint32_t hidden_size, float epsilon,
                                      void *stream) {
    if (!output || !input || !weight || vector_count == 0u || hidden_size == 0u) return false;
    const uint32_t vec = hidden_size % 8u == 0u && hidden_size <= 256u * 8u * kRmsChunks &&
                         (((uintptr_t)output | (uintptr_t)input | (uintptr_t)weight) % 16u) == 0u;
    hipLaunchKernelGGL(rms_norm_kernel, dim3(vector_count), dim3(256), 0, (hipStream_t)stream,
                       (uint16_t *)output, (const uint16_t *)input, (const uint16_t *)weight,
                       hidden_size, epsilon, vec);
    return hipGetLastError() == hipSuccess;
}

/* ------------------------------------------------------------------------ */
/* bf16 -> bf16 and Q8-128 static projections                                */
/* ------------------------------------------------------------------------ */

extern "C" bool k3_rocm_bf16_gemm_tiled_bf16(void *output, const void *weights,
                                             const void *input, uint32_t vector_count,
                                             uint32_t rows, uint32_t columns,
                                             uint32_t batch_tile, void *stream) {
    if (!output || !weights || !input || vector_count == 0u || vector_count > 65535u ||
        rows == 0u || columns == 0u)
        return false;
    const hipStream_t s = (hipStream_t)stream;
    switch (batch_tile) {
        case 16u: return launch_bf16_rows_f32<16, true>(output, weights, input, vector_count, rows, columns, s);
        case 32u: return launch_bf16_rows_f32<32, true>(output, weights, input, vector_count, rows, columns, s);
        case 64u: return launch_bf16_rows_f32<64, true>(output, weights, input, vector_count, rows, columns, s);
        default: return false;
    }
}

extern "C" bool k3_rocm_bf16_gemm_bf16(void *output, const void *weights, const void *input,
                                       uint32_t vector_count, uint32_t rows, uint32_t columns,
                                       void *stream) {
    if (!output || !weights || !input || vector_count == 0u || vector_count > 65535u ||
        rows == 0u || columns == 0u)
        return false;
    return k3::launch_bf16_rows_bf16_any((uint16_t *)output, weights, input, vector_count, rows,
                                         columns, (hipStream_t)stream);
}

extern "C" bool k3_rocm_bf16_gemv_bf16(void *output, const void *weights, const void *input,
                                       uint32_t rows, uint32_t columns, void *stream) {
    return k3_rocm_bf16_gemm_bf16(output, weights, input, 1u, rows, columns, stream);
}

extern "C" bool k3_rocm_bf16_quantize_q8_128(void *quantized, void *scales, const void *weights,
                                             uint32_t rows, uint32_t columns, void *stream) {
    if (!quantized || !scales || !weights || rows == 0u || columns == 0u || columns % 128u != 0u ||
        ((uintptr_t)weights % 4u) != 0u || ((uintptr_t)quantized % 2u) != 0u)
        return false;
    const uint64_t blocks = (uint64_t)rows * (columns / 128u);
    const uint64_t grid = (blocks + kWavesPerBlock - 1u) / kWavesPerBlock;
    if (grid > 0x7fffffffull) return false;
    hipLaunchKernelGGL(q8_quantize_kernel, dim3((uint32_t)grid), dim3(kThreads), 0,
                       (hipStream_t)stream, (int8_t *)quantized, (float *)scales,
                       (const uint16_t *)weights, blocks);
    return hipGetLastError() == hipSuccess;
}

extern "C" bool k3_rocm_q8_128_dequantize_bf16(void *weights, const void *quantized,
                                               const void *scales, uint32_t rows,
                                               uint32_t columns, void *stream) {
    if (!weights || !quantized || !scales || rows == 0u || columns == 0u || columns % 128u != 0u)
        return false;
    const uint64_t n = (uint64_t)rows * columns;
    hipLaunchKernelGGL(q8_dequantize_kernel, dim3(grid_cap((n + 255u) / 256u)), dim3(256), 0,
                       (hipStream_t)stream, (uint16_t *)weights, (const int8_t *)quantized,
                       (const float *)scales, n);
    return hipGetLastError() == hipSuccess;
}

static bool q8_args_ok(const void *output, const void *quantized, const void *scales,
                       const void *input, uint32_t vector_count, uint32_t rows,
                       uint32_t columns) {
    return output && quantized && scales && input && vector_count != 0u &&
           vector_count <= 65535u && rows != 0u && columns != 0u && columns % 128u == 0u &&
           ((uintptr_t)quantized % 8u) == 0u && ((uintptr_t)input % 16u) == 0u &&
           ((uintptr_t)scales % 4u) == 0u;
}

extern "C" bool k3_rocm_q8_128_gemm_tiled_bf16(void *output, const void *quantized,
                                               const void *scales, const void *input,
                                               uint32_t vector_count, uint32_t rows,
                                               uint32_t columns, uint32_t batch_tile,
                                               void *stream) {
    if (!q8_args_ok(output, quantized, scales, input, vector_count, rows, columns)) return false;
    const hipStream_t s = (hipStream_t)stream;
    switch (batch_tile) {
        case 16u: return launch_q8_rows<16>(output, quantized, scales, input, vector_count, rows, columns, s);
        case 32u: return launch_q8_rows<32>(output, quantized, scales, input, vector_count, rows, columns, s);
        case 64u: return launch_q8_rows<64>(output, quantized, scales, input, vector_count, rows, columns, s);
        default: return false;
    }
}

extern "C" bool k3_rocm_q8_128_gemm_bf16(void *output, const void *quantized, const void *scales,
                                         const void *input, uint32_t vector_count, uint32_t rows,
                                         uint32_t columns, void *stream) {
    if (!q8_args_ok(output, quantized, scales, input, vector_count, rows, columns)) return false;
    const hipStream_t s = (hipStream_t)stream;
    if (vector_count == 1u) {
        if (k3::q8_gemv_fits(columns, quantized, input))
            return k3::launch_q8_gemv((uint16_t *)output, quantized, scales, input, rows, columns,
                                      nullptr, nullptr, s);
        return launch_q8_rows<1>(output, quantized, scales, input, 1u, rows, columns, s);
    }
    if (vector_count <= 4u)
        return launch_q8_rows<4>(output, quantized, scales, input, vector_count, rows, columns, s);
    return launch_q8_rows<16>(output, quantized, scales, input, vector_count, rows, columns, s);
}

extern "C" bool k3_rocm_q8_128_gemv_bf16(void *output, const void *quantized, const void *scales,
                                         const void *input, uint32_t rows, uint32_t columns,
                                         void *stream) {
    return k3_rocm_q8_128_gemm_bf16(output, quantized, scales, input, 1u, rows, columns, stream);
}

bool k3::q8_gemv_fits(uint32_t cols, const void *codes, const void *x) {
    return cols != 0u && cols % 128u == 0u && cols <= 8192u && ((uintptr_t)codes % 8u) == 0u &&
           ((uintptr_t)x % 16u) == 0u;
}

namespace {

template <int R, int RS, bool NORM>
void q8_gemv_launch(uint16_t *out, const void *codes, const void *scales, const void *x,
                    uint32_t rows, uint32_t cols, uint32_t align16, const uint16_t *add1,
                    const uint16_t *add2, const uint16_t *norm_w, float eps, hipStream_t st) {
    constexpr uint32_t rb = R * RS;
    const Q8GemvArgs A{out, (const int8_t *)codes, (const float *)scales, nullptr, nullptr,
                       (const uint16_t *)x, rows, cols, align16, add1, add2, 0u, 1.0f, 1.0f,
                       norm_w, eps};
    hipLaunchKernelGGL(HIP_KERNEL_NAME(q8_gemv_kernel<false, R, RS, NORM>), dim3((rows + rb - 1u) / rb),
                       dim3(256), 0, st, A);
}

/* Row blocking measured on cold weights (one MI355X): 4 rows per set beats
 * 8 and 16 on every single-matrix shape of the K3 layer (e.g. 7168 x 6144:
 * 10.6 us against 13.3 us for 8 rows), as more, smaller blocks spread the
 * stream over all CUs; with the norm prologue two row sets per block pay
 * it over 8 rows (7168 x 3584: 9.6 us against 12.3 us for one set). */
template <bool NORM>
void q8_gemv_dispatch(uint16_t *out, const void *codes, const void *scales, const void *x,
                      uint32_t rows, uint32_t cols, uint32_t align16, const uint16_t *add1,
                      const uint16_t *add2, const uint16_t *norm_w, float eps, hipStream_t st) {
    if (NORM && cols <= 4096u)
        q8_gemv_launch<4, 2, NORM>(out, codes, scales, x, rows, cols, align16, add1, add2, norm_w, eps, st);
    else
        q8_gemv_launch<4, 1, NORM>(out, codes, scales, x, rows, cols, align16, add1, add2, norm_w, eps, st);
}

}  // namespace

bool k3::launch_q8_gemv(uint16_t *out, const void *codes, const void *scales, const void *x,
                        uint32_t rows, uint32_t cols, const uint16_t *add1, const uint16_t *add2,
                        hipStream_t st) {
    if (!q8_gemv_fits(cols, codes, x) || rows == 0u) return false;
    const uint32_t align16 = ((uintptr_t)codes % 16u) == 0u;
    q8_gemv_dispatch<false>(out, codes, scales, x, rows, cols, align16, add1, add2, nullptr, 0.0f,
                            st);
    return hipGetLastError() == hipSuccess;
}

bool k3::launch_q8_gemv_norm(uint16_t *out, const void *codes, const void *scales, const void *x,
                             const void *norm_weight, float eps, uint32_t rows, uint32_t cols,
                             hipStream_t st) {
    if (!q8_gemv_fits(cols, codes, x) || rows == 0u || !norm_weight ||
        ((uintptr_t)norm_weight % 16u) != 0u)
        return false;
    const uint32_t align16 = ((uintptr_t)codes % 16u) == 0u;
    q8_gemv_dispatch<true>(out, codes, scales, x, rows, cols, align16, nullptr, nullptr,
                           (const uint16_t *)norm_weight, eps, st);
    return hipGetLastError() == hipSuccess;
}

bool k3::launch_q8_gateup(uint16_t *act, const void *gate_codes, const void *gate_scales,
                          const void *up_codes, const void *up_scales, const void *x,
                          uint32_t rows, uint32_t cols, uint32_t kind, float beta, float lb,
                          hipStream_t st) {
    if (!q8_gemv_fits(cols, gate_codes, x) || !q8_gemv_fits(cols, up_codes, x) || rows == 0u)
        return false;
    const uint32_t align16 = (((uintptr_t)gate_codes | (uintptr_t)up_codes) % 16u) == 0u;
    const Q8GemvArgs A{act, (const int8_t *)gate_codes, (const float *)gate_scales,
                       (const int8_t *)up_codes, (const float *)up_scales, (const uint16_t *)x,
                       rows, cols, align16, nullptr, nullptr, kind, beta, lb, nullptr, 0.0f};
    hipLaunchKernelGGL(HIP_KERNEL_NAME(q8_gemv_kernel<true, kQ8DualRows, 1, false>),
                       dim3((rows + kQ8DualRows - 1u) / kQ8DualRows), dim3(256), 0, st, A);
    return hipGetLastError() == hipSuccess;
}

bool k3::launch_q8_gateup_and_gemv(uint16_t *act, const void *gate_codes,
                                   const void *gate_scales, const void *up_codes,
                                   const void *up_scales, const void *x, uint32_t rows,
                                   uint32_t cols, uint32_t kind, float beta, float lb,
                                   uint16_t *out, const void *codes, const void *scales,
                                   uint32_t out_rows, const RouterRows *router,
                                   hipStream_t st) {
    if (!q8_gemv_fits(cols, gate_codes, x) || !q8_gemv_fits(cols, up_codes, x) ||
        !q8_gemv_fits(cols, codes, x) || rows == 0u || out_rows == 0u)
        return false;
    RouterRows R{};
    uint32_t nr = 0u;
    if (router) {
        R = *router;
        if (R.x != x || R.cols != cols || R.cols % 8u != 0u || R.cols > 8u * 64u * kRouterMaxChunks ||
            ((uintptr_t)R.weight % 16u) != 0u || R.rows == 0u)
            return false;
        constexpr uint32_t per_block = kWavesPerBlock * kPairRouterRows;
        nr = (R.rows + per_block - 1u) / per_block;
    }
    const uint32_t a16d = (((uintptr_t)gate_codes | (uintptr_t)up_codes) % 16u) == 0u;
    const uint32_t a16s = ((uintptr_t)codes % 16u) == 0u;
    const Q8GemvArgs D{act, (const int8_t *)gate_codes, (const float *)gate_scales,
                       (const int8_t *)up_codes, (const float *)up_scales, (const uint16_t *)x,
                       rows, cols, a16d, nullptr, nullptr, kind, beta, lb, nullptr, 0.0f};
    const Q8GemvArgs S{out, (const int8_t *)codes, (const float *)scales, nullptr, nullptr,
                       (const uint16_t *)x, out_rows, cols, a16s, nullptr, nullptr, 0u, 1.0f,
                       1.0f, nullptr, 0.0f};
    const uint32_t nd = (rows + kQ8DualRows - 1u) / kQ8DualRows, ns = (out_rows + 3u) / 4u;
    hipLaunchKernelGGL(q8_gemv_pair_kernel, dim3(nr + nd + ns), dim3(256), 0, st, D, S, R, nd,
                       nr);
    return hipGetLastError() == hipSuccess;
}
