/*
 * Static projections of a token batch on bf16 MFMA, for the MXFP8
 * precisions of the K3-native block (the exact precision keeps the VALU
 * rows kernels of k3_rocm_q8_128_gemm_bf16 / k3_rocm_bf16_gemm_bf16,
 * k3_rocm_ops.cu:663-835, 1694-2038, and their bits).
 *
 *   out[t, r] = bf16(sum_b s[r, b] * sum_{k in block b} q[r, k] x[t, k])   Q8-128
 *   out[t, r] = bf16(sum_k w[r, k] x[t, k])                                bf16
 *
 * Int8 codes are exact in bf16 (|q| <= 127 has at most 7 significant
 * bits), so every product is the exact product and only the fp32
 * summation order differs from the exact kernels (which sum 32-column
 * groups and scale each): a tolerance of fp32 reassociation, far inside
 * one bf16 rounding of the output.
 *
 * Block tile 128 tokens x 128 rows, 8 waves of 32 x 64 (2 x 4
 * V_MFMA_F32_16X16X32_BF16 tiles), K steps of 64 through two LDS buffers
 * (rows padded to 144 bytes), global loads two steps ahead. Codes are
 * converted to bf16 on their way into LDS. A Q8-128 block is two K steps:
 * its four MFMAs per tile chain in a block sum that is then scaled into
 * the accumulator with one fma per output; the next block's scales are
 * loaded a block ahead. Tiles are dealt to the XCDs in contiguous ranges,
 * a token tile's row tiles together.
 */
#include "k3_device.h"
#include "k3_internal.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace k3 {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr uint32_t kPT = 128, kPK = 64, kPPad = 144;

typedef uint8_t ProjStage[2][kPT * kPPad]; /* [A tokens | B weight rows] */

struct ProjArgs {
    uint16_t *out;        /* [T, N] bf16 */
    const uint16_t *x;    /* [T, K] bf16 */
    const void *w;        /* [N, K] int8 codes or bf16 */
    const float *scales;  /* [N, K / 128] (Q8-128) */
    uint32_t T, N, K;
};

/* Eight int8 codes as eight bf16 (exact). */
__device__ __forceinline__ uint4 codes_to_bf16(uint2 v) {
    uint32_t o[4];
    const uint32_t u[2] = {v.x, v.y};
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const float lo = (float)(int8_t)(u[h] >> (16 * p));
            const float hi = (float)(int8_t)(u[h] >> (16 * p + 8));
            o[2 * h + p] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
        }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

/* The thread's two rows of one K step: x as 16 bytes, weights as 16
 * (bf16) or 8 (codes) bytes, converted to bf16 on the store. */
template <bool Q8>
using WeightPiece = typename std::conditional<Q8, uint2, uint4>::type;

template <bool Q8>
__device__ __forceinline__ void proj_load(uint4 &a0, uint4 &a1, WeightPiece<Q8> &b0,
                                          WeightPiece<Q8> &b1, const uint8_t *xb,
                                          const uint8_t *wb, uint32_t ao0, uint32_t ao1,
                                          uint32_t bo0, uint32_t bo1, uint32_t s) {
    const uint32_t ka = 2u * kPK * s, kw = (Q8 ? 1u : 2u) * kPK * s;
    a0 = *(const uint4 *)(xb + ao0 + ka);
    a1 = *(const uint4 *)(xb + ao1 + ka);
    b0 = *(const WeightPiece<Q8> *)(wb + bo0 + kw);
    b1 = *(const WeightPiece<Q8> *)(wb + bo1 + kw);
}

__device__ __forceinline__ uint4 as_bf16x8(uint2 codes) { return codes_to_bf16(codes); }
__device__ __forceinline__ uint4 as_bf16x8(uint4 bf16) { return bf16; }

template <bool Q8>
__device__ __forceinline__ void proj_store(ProjStage &buf, uint32_t off, const uint4 &a0,
                                           const uint4 &a1, const WeightPiece<Q8> &b0,
                                           const WeightPiece<Q8> &b1) {
    constexpr uint32_t R64 = 64u * kPPad;
    *(uint4 *)(buf[0] + off) = a0;
    *(uint4 *)(buf[0] + off + R64) = a1;
    *(uint4 *)(buf[1] + off) = as_bf16x8(b0);
    *(uint4 *)(buf[1] + off + R64) = as_bf16x8(b1);
}

/* acc[i][j] += A(wave rows i) . B(wave rows j) over one K step. */
__device__ __forceinline__ void proj_compute(f32x4_t (&acc)[2][4], const ProjStage &buf,
                                             uint32_t a_off, uint32_t b_off) {
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        bf16x8_t af[2], bf[4];
#pragma unroll
        for (int i = 0; i < 2; i++)
            af[i] = __builtin_bit_cast(bf16x8_t, *(const uint4 *)(buf[0] + a_off + 16u * kPPad * i +
                                                                  64u * ks));
#pragma unroll
        for (int j = 0; j < 4; j++)
            bf[j] = __builtin_bit_cast(bf16x8_t, *(const uint4 *)(buf[1] + b_off + 16u * kPPad * j +
                                                                  64u * ks));
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
}

template <bool Q8>
__global__ __launch_bounds__(512) void proj_mfma_kernel(ProjArgs P) {
    __shared__ __attribute__((aligned(16))) ProjStage lds[2];
    const uint32_t T = P.T, N = P.N, K = P.K;
    const uint32_t ntt = (T + kPT - 1u) / kPT, nnt = (N + kPT - 1u) / kPT;
    const uint32_t works = ntt * nnt, per = (works + 7u) / 8u;
    const uint32_t L = blockIdx.x, j8 = L >> 3, wk = (L & 7u) * per + j8;
    if (j8 >= per || wk >= works) return;
    const uint32_t t0 = (wk / nnt) * kPT, n0 = (wk % nnt) * kPT;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1u, g = lane >> 4, c = lane & 15u;
    /* thread tid loads piece tid % 8 (8 columns) of rows tid / 8 and tid /
     * 8 + 64; rows past T or N clamp to the last one (not stored) */
    const uint32_t r0 = tid >> 3, pc = tid & 7u;
    constexpr uint32_t wbytes = Q8 ? 1u : 2u;
    uint32_t ao[2], bo[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const uint32_t ta = t0 + r0 + 64u * i, nb = n0 + r0 + 64u * i;
        ao[i] = ((ta < T ? ta : T - 1u) * K + 8u * pc) * 2u;
        bo[i] = ((nb < N ? nb : N - 1u) * K + 8u * pc) * wbytes;
    }
    const uint8_t *xb = (const uint8_t *)P.x, *wb = (const uint8_t *)P.w;
    const uint32_t soff = r0 * kPPad + 16u * pc;
    const uint32_t a_off = (32u * wm + c) * kPPad + 16u * g;
    const uint32_t b_off = (64u * wn + c) * kPPad + 16u * g;
    /* Q8: the scales of this lane's four weight rows (one per n-tile) */
    const uint32_t nblk = K / 128u;
    const float *srow[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t r = n0 + 64u * wn + 16u * (uint32_t)j + c;
        srow[j] = P.scales + (uint64_t)(r < N ? r : N - 1u) * nblk;
    }
    f32x4_t acc[2][4], blk[2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            blk[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
    float sc[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if constexpr (Q8) {
#pragma unroll
        for (int j = 0; j < 4; j++) sc[j] = srow[j][0];
    }
    const uint32_t nsteps = K / kPK, last = nsteps - 1u;
    /* two register sets: step s + 2's loads are issued at the start of
     * step s; loads and stores are unconditional (steps past the end
     * reload the last one into a buffer nobody reads) */
    uint4 a0, a1, p0, p1;
    WeightPiece<Q8> b0, b1, q0, q1;
    proj_load<Q8>(a0, a1, b0, b1, xb, wb, ao[0], ao[1], bo[0], bo[1], 0u);
    proj_load<Q8>(p0, p1, q0, q1, xb, wb, ao[0], ao[1], bo[0], bo[1], 1u < last ? 1u : last);
    proj_store<Q8>(lds[0], soff, a0, a1, b0, b1);
    __syncthreads();
    for (uint32_t s = 0; s < nsteps; s += 2u) {
        /* Q8: steps s, s + 1 are 128-column block s / 2 (K % 128 == 0);
         * the next block's scales load during this block's two steps */
        float nx[4] = {1.0f, 1.0f, 1.0f, 1.0f};
        if constexpr (Q8) {
            const uint32_t b1 = s / 2u + 1u < nblk ? s / 2u + 1u : s / 2u;
#pragma unroll
            for (int j = 0; j < 4; j++) nx[j] = srow[j][b1];
        }
        proj_load<Q8>(a0, a1, b0, b1, xb, wb, ao[0], ao[1], bo[0], bo[1],
                      s + 2u < last ? s + 2u : last);
        if constexpr (Q8) proj_compute(blk, lds[0], a_off, b_off);
        else proj_compute(acc, lds[0], a_off, b_off);
        proj_store<Q8>(lds[1], soff, p0, p1, q0, q1);
        __syncthreads();
        if (s + 1u < nsteps) {
            proj_load<Q8>(p0, p1, q0, q1, xb, wb, ao[0], ao[1], bo[0], bo[1],
                          s + 3u < last ? s + 3u : last);
            if constexpr (Q8) proj_compute(blk, lds[1], a_off, b_off);
            else proj_compute(acc, lds[1], a_off, b_off);
            proj_store<Q8>(lds[0], soff, a0, a1, b0, b1);
            __syncthreads();
        }
        if constexpr (Q8) {
            /* acc += scale * block sum */
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[i][j][r] = fmaf(blk[i][j][r], sc[j], acc[i][j][r]);
                    blk[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
                }
#pragma unroll
            for (int j = 0; j < 4; j++) sc[j] = nx[j];
        }
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t n = n0 + 64u * wn + 16u * (uint32_t)j + c;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t t = t0 + 32u * wm + 16u * (uint32_t)i + 4u * g + (uint32_t)r;
                if (t < T && n < N) P.out[(uint64_t)t * N + n] = f32_to_bf16(acc[i][j][r]);
            }
        }
}

}  // namespace

bool proj_mfma_supported(uint32_t tokens, uint32_t rows, uint32_t cols, bool q8,
                         const void *weights, const void *x) {
    const uint64_t xbytes = 2ull * tokens * cols, wbytes = (q8 ? 1ull : 2ull) * rows * cols;
    return tokens > 0u && rows > 0u && cols > 0u && cols % (q8 ? 128u : kPK) == 0u &&
           xbytes < (1ull << 31) && wbytes < (1ull << 31) &&
           ((uintptr_t)x % 16u) == 0u && ((uintptr_t)weights % (q8 ? 8u : 16u)) == 0u;
}

bool launch_proj_mfma(uint16_t *out, const void *x, const void *weights, const float *scales,
                      uint32_t T, uint32_t N, uint32_t K, bool q8, hipStream_t st) {
    if (!proj_mfma_supported(T, N, K, q8, weights, x) || (q8 && !scales)) return false;
    const uint32_t works = ((T + kPT - 1u) / kPT) * ((N + kPT - 1u) / kPT);
    const ProjArgs A{out, (const uint16_t *)x, weights, scales, T, N, K};
    const dim3 grid(8u * ((works + 7u) / 8u));
    if (q8)
        hipLaunchKernelGGL(HIP_KERNEL_NAME(proj_mfma_kernel<true>), grid, dim3(512), 0, st, A);
    else
        hipLaunchKernelGGL(HIP_KERNEL_NAME(proj_mfma_kernel<false>), grid, dim3(512), 0, st, A);
    return hipGetLastError() == hipSuccess;
}

}  // namespace k3

extern "C" bool k3_moe_proj_mfma_bf16(void *output, const void *weights, const float *scales,
                                      const void *input, uint32_t vector_count, uint32_t rows,
                                      uint32_t columns, bool q8, void *stream) {
    if (!output || !weights || !input) return false;
    return k3::launch_proj_mfma((uint16_t *)output, input, weights, scales, vector_count, rows,
                                columns, q8, (hipStream_t)stream);
}
