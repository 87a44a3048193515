/*
 * Grouped MXFP4 expert products on gfx950 scaled MFMA (prefill and batched
 * tokens). Replaces the per-expert k3_rocm_mxfp4_gemm_tiled_bf16 calls of
 * launch_prefill_expert (k3_engine_prefill.inc:962-990): one launch per
 * tile-size class covers every selected expert of the layer.
 *
 *   x_split_kernel      bf16 values -> MXFP8 hi (and lo) codes + scales per
 *                       32 (the k3_moe_mx8_quantize_bf16 ABI)
 *   x_split_rows_kernel token rows -> E4M3 hi (and lo) codes, one scale
 *                       per row and term
 *   tile_build_kernel   plan -> per-class tile lists (16/64/96/128-row tiles)
 *   gateup_mfma_kernel  act = bf16(f(bf16(x.Wg), bf16(x.Wu))), written as
 *                       MXFP8 hi/lo of the activation (blocks of 32 along F)
 *   down_mfma_kernel    y[route] = bf16(act . Wd) for the route's slot
 *
 * MFMA operand layout (V_MFMA_SCALE_F32_16X16X128_F8F6F4, measured on the
 * part): lane l = 16 g + c supplies row c of the 16 x 128 slice. An FP8
 * operand carries K bytes [16g, 16g + 16) and [64 + 16g, 64 + 16g + 16); an
 * FP4 operand carries K [32g, 32g + 32) (16 bytes, low nibble = even k).
 * Both scale operands are the E8M0 byte of K block g of the lane's row.
 * Output: lane l holds rows 4g + i (i < 4) of column c.
 *
 * Tiles: by the expert's row count, a block computes 16, 64, 96 or 128
 * activation rows against 128, 256 or 512 weight rows with 2 to 8 waves
 * (the Cls* configurations below); K advances 128 or 256 per step through
 * a 2- or 3-stage LDS ring filled by direct-to-LDS loads.
 */
#include "k3_device.h"
#include "k3_lds.h"
#include "k3_mfma.h"
#include "../../include/k3_moe.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace k3 {
namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kTileRows[kTileClasses] = {16u, 64u, 96u, 128u};

__device__ __forceinline__ float bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

/* ---------------------------------------------------------------------- */
/* activation split                                                        */
/* ---------------------------------------------------------------------- */

/* One thread per 32-element block of the [T, H] bf16 rows. */
template <int TERMS>
__global__ __launch_bounds__(256) void x_split_kernel(MfmaBuffers B, const uint16_t *__restrict__ x,
                                                      uint64_t blocks) {
    const uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= blocks) return;
    float v[32];
    bf16x32_to_f32((const uint4 *)(x + 32u * b), v);
#pragma unroll
    for (int t = 0; t < TERMS; t++) {
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
        const uint32_t sb = mx8_scale_byte(amax);
        const float inv = mx8_inv_scale(sb), sc = e8m0_to_f32(sb);
        uint32_t w[8];
#pragma unroll
        for (int q = 0; q < 8; q++) {
            float *u = v + 4 * q;
            uint32_t word = e4m3x2<false>(__fmul_rn(u[0], inv), __fmul_rn(u[1], inv), 0u);
            word = e4m3x2<true>(__fmul_rn(u[2], inv), __fmul_rn(u[3], inv), word);
            if (TERMS == 2 && t == 0) {
                u[0] = __fsub_rn(u[0], __fmul_rn(e4m3_byte<0>(word), sc));
                u[1] = __fsub_rn(u[1], __fmul_rn(e4m3_byte<1>(word), sc));
                u[2] = __fsub_rn(u[2], __fmul_rn(e4m3_byte<2>(word), sc));
                u[3] = __fsub_rn(u[3], __fmul_rn(e4m3_byte<3>(word), sc));
            }
            w[q] = word;
        }
        uint4 *dst = (uint4 *)(B.xq[t] + 32u * b);
        dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
        dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
        B.xs[t][b] = (uint8_t)sb;
    }
}

/* Maximum over the 256 threads of a block (values >= 0; NaN ignored). */
__device__ __forceinline__ float block_max256(float m, float *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    __syncthreads(); /* red is reused by consecutive calls */
    if ((threadIdx.x & 63u) == 0u) red[threadIdx.x >> 6] = m;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

/* Codes of 8 values under one scale (inverse inv), and their residuals
 * v - code x sc in v (exact products, one rounding). */
template <bool Residual>
__device__ __forceinline__ uint2 e4m3x8(float (&v)[8], float inv, float sc) {
    uint32_t w[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        float *u = v + 4 * h;
        uint32_t word = e4m3x2<false>(__fmul_rn(u[0], inv), __fmul_rn(u[1], inv), 0u);
        word = e4m3x2<true>(__fmul_rn(u[2], inv), __fmul_rn(u[3], inv), word);
        if constexpr (Residual) {
            u[0] = __fsub_rn(u[0], __fmul_rn(e4m3_byte<0>(word), sc));
            u[1] = __fsub_rn(u[1], __fmul_rn(e4m3_byte<1>(word), sc));
            u[2] = __fsub_rn(u[2], __fmul_rn(e4m3_byte<2>(word), sc));
            u[3] = __fsub_rn(u[3], __fmul_rn(e4m3_byte<3>(word), sc));
        }
        w[h] = word;
    }
    return make_uint2(w[0], w[1]);
}

__device__ __forceinline__ void bf16x8_to_f32(uint4 p, float (&v)[8]) {
    const uint32_t d[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[2 * i] = bf16_lo(d[i]);
        v[2 * i + 1] = bf16_hi(d[i]);
    }
}

/*
 * One block of 256 threads per token row of [T, H] bf16 (H % 8 == 0): the
 * row's E4M3 codes under one E8M0 scale per term (the scale rule of the
 * 32-element MXFP8 blocks applied to the whole row), hi and, for two
 * terms, lo = x - hi under its own scale. With M > 0 (H <= 2048 M) each
 * thread keeps its M chunks of 8 values in registers and the row is read
 * once; M = 0 reads it once per pass (maximum, residual maximum, codes),
 * from L2 after the first. With one scale per row the MFMA lanes hold
 * their rows' scales in registers for the whole K loop instead of staging
 * scale bytes per step.
 */
template <int TERMS, int M>
__global__ __launch_bounds__(256) void x_split_rows_kernel(MfmaBuffers B,
                                                           const uint16_t *__restrict__ x,
                                                           uint32_t H) {
    __shared__ float red[4];
    const uint32_t row = blockIdx.x, chunks = H / 8u;
    const uint4 *src = (const uint4 *)(x + (uint64_t)row * H);
    uint2 *hq = (uint2 *)(B.xq[0] + (uint64_t)row * H);
    uint2 *lq = (uint2 *)(B.xq[TERMS - 1] + (uint64_t)row * H);
    uint32_t s0, s1 = 0u;
    if constexpr (M > 0) {
        float v[M][8];
        bool live[M];
#pragma unroll
        for (int m = 0; m < M; m++) {
            const uint32_t q = threadIdx.x + 256u * (uint32_t)m;
            live[m] = q < chunks;
            bf16x8_to_f32(live[m] ? src[q] : make_uint4(0u, 0u, 0u, 0u), v[m]);
        }
        float amax = 0.0f;
#pragma unroll
        for (int m = 0; m < M; m++)
#pragma unroll
            for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[m][i]));
        s0 = mx8_scale_byte(block_max256(amax, red));
        const float inv0 = mx8_inv_scale(s0), sc0 = e8m0_to_f32(s0);
        uint2 h[M];
#pragma unroll
        for (int m = 0; m < M; m++) h[m] = e4m3x8<TERMS == 2>(v[m], inv0, sc0);
        if constexpr (TERMS == 2) {
            float rmax = 0.0f; /* padding chunks hold zeros: residual 0 */
#pragma unroll
            for (int m = 0; m < M; m++)
#pragma unroll
                for (int i = 0; i < 8; i++) rmax = fmaxf(rmax, fabsf(v[m][i]));
            s1 = mx8_scale_byte(block_max256(rmax, red));
        }
        const float inv1 = mx8_inv_scale(s1);
#pragma unroll
        for (int m = 0; m < M; m++) {
            if (!live[m]) continue;
            const uint32_t q = threadIdx.x + 256u * (uint32_t)m;
            hq[q] = h[m];
            if constexpr (TERMS == 2) lq[q] = e4m3x8<false>(v[m], inv1, 0.0f);
        }
    } else {
        float amax = 0.0f;
        for (uint32_t q = threadIdx.x; q < chunks; q += 256u) {
            float v[8];
            bf16x8_to_f32(src[q], v);
#pragma unroll
            for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[i]));
        }
        s0 = mx8_scale_byte(block_max256(amax, red));
        const float inv0 = mx8_inv_scale(s0), sc0 = e8m0_to_f32(s0);
        if constexpr (TERMS == 2) {
            float rmax = 0.0f;
            for (uint32_t q = threadIdx.x; q < chunks; q += 256u) {
                float v[8];
                bf16x8_to_f32(src[q], v);
                (void)e4m3x8<true>(v, inv0, sc0);
#pragma unroll
                for (int i = 0; i < 8; i++) rmax = fmaxf(rmax, fabsf(v[i]));
            }
            s1 = mx8_scale_byte(block_max256(rmax, red));
        }
        const float inv1 = mx8_inv_scale(s1);
        for (uint32_t q = threadIdx.x; q < chunks; q += 256u) {
            float v[8];
            bf16x8_to_f32(src[q], v);
            hq[q] = e4m3x8<TERMS == 2>(v, inv0, sc0);
            if constexpr (TERMS == 2) lq[q] = e4m3x8<false>(v, inv1, 0.0f);
        }
    }
    if (threadIdx.x == 0u) {
        B.xs[0][row] = (uint8_t)s0;
        if constexpr (TERMS == 2) B.xs[1][row] = (uint8_t)s1;
    }
}

/* x_split_rows_kernel<TERMS, M> for H: registers up to H = 8192. */
template <int TERMS>
void launch_split_rows(const MfmaBuffers &B, const uint16_t *x, uint32_t rows, uint32_t H,
                       hipStream_t st) {
    if (H <= 2048u)
        hipLaunchKernelGGL(HIP_KERNEL_NAME(x_split_rows_kernel<TERMS, 1>), dim3(rows), dim3(256),
                           0, st, B, x, H);
    else if (H <= 8192u)
        hipLaunchKernelGGL(HIP_KERNEL_NAME(x_split_rows_kernel<TERMS, 4>), dim3(rows), dim3(256),
                           0, st, B, x, H);
    else
        hipLaunchKernelGGL(HIP_KERNEL_NAME(x_split_rows_kernel<TERMS, 0>), dim3(rows), dim3(256),
                           0, st, B, x, H);
}

/* ---------------------------------------------------------------------- */
/* tile lists                                                              */
/* ---------------------------------------------------------------------- */

/* One block of 1024 threads (thread e = expert e). Class 0: experts with
 * <= 16 rows (one 16-row tile), class 1: <= 64 rows (one 64-row tile),
 * class 2: <= 96 rows (one 96-row tile), class 3: 128-row tiles (the last
 * one partial). Tiles are listed in expert order. The 8-mod-16 tensor
 * starts of real checkpoint spans (about a quarter of the shipped tensors,
 * k3_rocm_ops.cu:207-223) take the MFMA kernels like aligned ones: the
 * 16-byte direct-to-LDS loads return the right bytes from 8-byte aligned
 * sources on gfx950 (measured, register and LDS forms). For the MFMA
 * kernels (all == 0) an expert with a tensor that is not even 8-byte
 * aligned gets no tiles, and B.unaligned hands it to the exact grouped
 * kernels. With all != 0 (the exact kernels' own tile list) every selected
 * expert gets tiles. */
__global__ __launch_bounds__(1024) void tile_build_kernel(MfmaBuffers B,
                                                          const uint32_t *__restrict__ counts,
                                                          const uint32_t *__restrict__ offsets,
                                                          const k3_moe_expert *__restrict__ experts,
                                                          uint32_t E, uint32_t all) {
    __shared__ uint32_t wave_tot[kTileClasses][16];
    __shared__ uint32_t odd_count;
    if (threadIdx.x == 0u) odd_count = 0u;
    __syncthreads();
    const uint32_t e = threadIdx.x, lane = e & 63u, wave = e >> 6;
    const uint32_t n = e < E ? counts[e] : 0u;
    bool odd = false;
    if (n != 0u && !all) {
        const k3_moe_expert ex = experts[e];
        odd = (((uintptr_t)ex.gate_packed | (uintptr_t)ex.gate_scales | (uintptr_t)ex.down_packed |
                (uintptr_t)ex.down_scales | (uintptr_t)ex.up_packed | (uintptr_t)ex.up_scales) %
               8u) != 0u;
    }
    if (odd) B.unaligned[1u + atomicAdd(&odd_count, 1u)] = e;
    constexpr int kLast = kTileClasses - 1; /* the multi-tile class */
    const int cls = n == 0u || odd ? kTileClasses
                                   : (n <= 16u ? 0 : (n <= 64u ? 1 : (n <= 96u ? 2 : kLast)));
    uint32_t nt[kTileClasses], inc[kTileClasses];
#pragma unroll
    for (int c = 0; c < kTileClasses; c++) {
        nt[c] = cls == c ? (c == kLast ? (n + 127u) / 128u : 1u) : 0u;
        inc[c] = nt[c];
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1)
#pragma unroll
        for (int c = 0; c < kTileClasses; c++) {
            const uint32_t a = __shfl_up(inc[c], o, 64);
            if ((int)lane >= o) inc[c] += a;
        }
    if (lane == 63u)
        for (int c = 0; c < kTileClasses; c++) wave_tot[c][wave] = inc[c];
    __syncthreads();
    uint32_t base_idx = 0u;
    for (int c = 0; c < kTileClasses; c++) {
        uint32_t before = 0u, total = 0u;
        for (uint32_t w = 0; w < blockDim.x / 64u; w++) {
            if (w < wave) before += wave_tot[c][w];
            total += wave_tot[c][w];
        }
        if (cls == c) {
            const uint32_t first = before + inc[c] - nt[c];
            for (uint32_t q = 0; q < nt[c]; q++) {
                uint32_t *t = B.tiles + 3u * (base_idx + first + q);
                const uint32_t r0 = q * kTileRows[c];
                t[0] = e;
                t[1] = offsets[e] + r0;
                t[2] = n - r0 < kTileRows[c] ? n - r0 : kTileRows[c];
            }
        }
        if (e == 0u) B.tile_count[c] = total;
        base_idx += B.tile_cap[c];
    }
    if (e == 0u) B.unaligned[0] = odd_count; /* after the barrier above */
}

/* ---------------------------------------------------------------------- */
/* MFMA core: LDS ring fed by direct-to-LDS loads                          */
/* ---------------------------------------------------------------------- */

/*
 * Block tile: MW x NW waves; wave tile (16 WM activation rows) x (16 WN
 * weight rows). Per K step of 128 the block stages in LDS
 *   A   TERMS x (BM / 16) x 2 chunks of 1 KB: chunk (t, i, h) holds the
 *       step's full 128 bytes of the 8 rows 16 i + 8 h + r (r < 8), slot
 *       8 r + q' holding 16-byte piece p = q' ^ a_swizzle(r, h) -- one
 *       instruction fetches eight whole 128-byte lines;
 *   B   BN / 16 chunks of 1 KB: lane order FP4 fragments of 16 rows;
 *   SA  TERMS x max(BM, 64) dwords: the 4 E8M0 bytes of each row's step;
 *   SB  BN dwords.
 * Every chunk is written by one global_load_lds instruction (lane l's 16 or
 * 4 bytes land at chunk + 16 l or + 4 l). B fragments are read back with
 * ds_read_b128 at lane * 16; an A fragment (row c, pieces g and 4 + g) is
 * read at the swizzled slot, which puts the 16 lanes of each read pass on
 * 16 different 16-byte bank groups. Chunks are dealt to the waves in equal
 * numbers per kind; the A scale chunks of small tiles (fewer than the
 * waves) go to the first waves.
 */
/* How the chunks of one kind are dealt to the block's W waves: N >= W
 * chunks must split evenly (wave w takes w, w + W, ...); fewer go one each
 * to the first N waves. */
template <int N, int W>
struct Deal {
    static constexpr bool partial = N < W;
    static constexpr int per = N == 0 ? 0 : (partial ? 1 : N / W);
    static_assert(partial || N % W == 0, "chunks split evenly over the waves");
};

template <int MW_, int NW_, int WM_, int WN_, int TERMS_, int STAGES_, int KS_ = 1, int BAUX_ = 0>
struct TileCfg {
    static constexpr int MW = MW_, NW = NW_, WM = WM_, WN = WN_, TERMS = TERMS_;
    static constexpr int STAGES = STAGES_, NWV = MW * NW, THREADS = 64 * NWV;
    /* KS: 128-column K slices per stage. With KS = 2 a stage holds 128
     * bytes of every weight row, so B chunks are whole 128-byte lines too
     * (8 rows each, the A layout); KS = 1 keeps the 16-row lane-order
     * fragments of 64 bytes per row. */
    static constexpr int KS = KS_, KSTEP = 128 * KS;
    /* cache policy of the weight DMA (2 = non-temporal): classes whose
     * experts own a single tile read every weight byte once per launch, so
     * streaming them past L2 keeps the activations resident */
    static constexpr int BAUX = BAUX_;
    static constexpr int BM = MW * 16 * WM, BN = NW * 16 * WN;
    static constexpr int A_CH = KS * TERMS * (BM / 16) * 2, B_CH = KS == 2 ? BN / 8 : BN / 16;
    /* E8M0 scales live outside the stages, in two scale buffers: a scale
     * block holds 16 bytes of every row (SQ stages' worth, 4 scales per 128
     * K), so a row's scales arrive in one 16-byte request per SQ stages
     * instead of a 4-byte request per stage. Chunk = 64 rows x 16 B. With
     * SBH = 2 a scale block holds two such 16-byte records per weight row
     * (the row's next 32 bytes, fetched together: one touch per scale line
     * in half as many blocks), the second in a second SB region. */
    static constexpr int SBH = 1;
    static constexpr int SQ = 4 / KS;
    static constexpr int SA_ROWS = (BM + 63) / 64 * 64; /* whole 64-row scale chunks */
    static constexpr int SA_CH = TERMS * SA_ROWS / 64, SB_CH = BN / 64;
    static constexpr int OFF_A = 0, OFF_B = OFF_A + A_CH * 1024, STAGE = OFF_B + B_CH * 1024;
    static constexpr int OFF_SA = 0, OFF_SB = SA_CH * 1024, SBUF = (SA_CH + SB_CH) * 1024;
    static constexpr int LDS = STAGE * STAGES + 2 * SBUF;
    /* eight waves (two per SIMD, register-bound) read A fragment q + 1
     * under the MFMAs of fragment q; smaller blocks read all fragments
     * in two halves */
    static constexpr bool SEQ = NWV > 4;
    static_assert(KS == 1 || KS == 2, "one or two K slices per stage");
    using DA = Deal<A_CH, NWV>;
    using DB = Deal<B_CH, NWV>;
    using DSA = Deal<SA_CH, NWV>;
    using DSB = Deal<SB_CH, NWV>;
    /* loads per step of a wave holding the kinds flagged in `mask`
     * (bit 3 A, 2 B, 1 SA, 0 SB) */
    /* (scale blocks are issued first in their stage's batch and are not
     * counted: waiting on the count of A and B loads alone covers them) */
    static constexpr int loads(int mask) {
        return ((mask & 8) ? DA::per : 0) + ((mask & 4) ? DB::per : 0);
    }
    /* activation scales: per row in registers (RowScaled) or staged */
    static constexpr bool AROW = false;
    static_assert(LDS <= 160 * 1024, "LDS");
    static_assert(loads(15) < 32, "vmcnt budget for one step in flight");
};

/* A tile class for the gate/up kernel: the token rows carry one scale per
 * row and term (x_split_rows_kernel), held in registers, so no activation
 * scale chunks are staged or read per step. */
template <class C>
struct RowScaled : C {
    static constexpr bool AROW = true;
    /* the freed activation scale space takes weight scale blocks of two
     * records per row */
    static constexpr int SBH = 2, SQ = SBH * 4 / C::KS;
    static constexpr int SA_CH = 0, OFF_SA = 0, OFF_SB = 0, SBUF = SBH * C::SB_CH * 1024;
    static constexpr int LDS = C::STAGE * C::STAGES + 2 * SBUF;
    static_assert(LDS <= 160 * 1024, "LDS");
    using DSA = Deal<0, C::NWV>;
};


/* Per-lane source pointers of the chunks this wave loads, and which kinds
 * it holds (index q of a kind is chunk q * NWV + wave, or chunk `wave`). */
template <class C>
struct Loader {
    const uint8_t *a[C::DA::per > 0 ? C::DA::per : 1];
    const uint8_t *b[C::DB::per > 0 ? C::DB::per : 1];
    const uint8_t *sa[C::DSA::per > 0 ? C::DSA::per : 1];
    const uint8_t *sb[C::DSB::per > 0 ? C::DSB::per : 1];
    uint32_t mask;      /* kinds held: bit 3 A, 2 B, 1 SA, 0 SB */
    uint32_t sa_stride; /* bytes between consecutive scale blocks of an SA row */
    uint32_t sb_recs;   /* 16-byte scale records per weight row (K / 512) */
};

/* chunk index of slot q of a kind for this wave */
template <class D, int W>
__device__ __forceinline__ int chunk_of(int q, uint32_t wave) {
    return D::partial ? (int)wave : q * W + (int)wave;
}

template <class C>
__device__ __forceinline__ uint32_t kinds_held(uint32_t wave) {
    auto has = [&](bool partial, int n) { return !partial || (int)wave < n; };
    return (has(C::DA::partial, C::A_CH) ? 8u : 0u) | (has(C::DB::partial, C::B_CH) ? 4u : 0u) |
           (has(C::DSA::partial, C::SA_CH) ? 2u : 0u) | (has(C::DSB::partial, C::SB_CH) ? 1u : 0u);
}

template <class C>
__device__ __forceinline__ void issue_step(const Loader<C> &L, uint8_t *stage, uint32_t s,
                                           uint32_t wave, uint8_t *sbuf0, uint8_t *sbuf1) {
    constexpr int W = C::NWV;
    if (s % (uint32_t)C::SQ == 0u) { /* scale block s / SQ, before the stage's data */
        const uint32_t b = s / (uint32_t)C::SQ;
        uint8_t *sbuf = (b & 1u) ? sbuf1 : sbuf0;
        if (L.mask & 2u) {
#pragma unroll
            for (int q = 0; q < C::DSA::per; q++)
                dma<16>(L.sa[q] + L.sa_stride * b, sbuf + C::OFF_SA + 1024 * chunk_of<typename C::DSA, W>(q, wave));
        }
        if (L.mask & 1u) {
#pragma unroll
            for (int q = 0; q < C::DSB::per; q++)
#pragma unroll
                for (int h = 0; h < C::SBH; h++)
                    if (h == 0 || C::SBH * b + (uint32_t)h < L.sb_recs) /* not past the row */
                    dma<16>(L.sb[q] + 16u * (C::SBH * b + (uint32_t)h),
                            sbuf + C::OFF_SB + 1024 * (h * C::SB_CH + chunk_of<typename C::DSB, W>(q, wave)));
        }
    }
    if (L.mask & 8u) {
#pragma unroll
        for (int q = 0; q < C::DA::per; q++)
            dma<16>(L.a[q] + (uint32_t)C::KSTEP * s, stage + C::OFF_A + 1024 * chunk_of<typename C::DA, W>(q, wave));
    }
    if (L.mask & 4u) {
#pragma unroll
        for (int q = 0; q < C::DB::per; q++)
            dma<16, C::BAUX>(L.b[q] + (uint32_t)(C::KSTEP / 2) * s, stage + C::OFF_B + 1024 * chunk_of<typename C::DB, W>(q, wave));
    }
}

/* Wait until this wave's loads of the current step have landed; with
 * `ahead`, the following step's loads may stay in flight. */
template <class C>
__device__ __forceinline__ void wait_step(const Loader<C> &L, int ahead);

template <class C>
__device__ __forceinline__ void wait_step(const Loader<C> &L, int ahead) {
    if (ahead <= 0) {
        wait_vm<0>();
        return;
    }
    static_for<16>([&](auto M) {
        if (L.mask == (uint32_t)decltype(M)::value) wait_vm<C::loads(decltype(M)::value)>();
    });
}


/*
 * One K step from a staged LDS buffer. The (term, row-block) fragment list
 * is read in two halves: the B fragments and the first half of the A
 * fragments, then the second half; the first half's MFMAs are issued as
 * soon as its reads have landed (lgkmcnt(count of the second half's
 * reads)), so the second half's LDS reads run under them.
 */
/* Activation scale bytes of a wave's rows when they are per row (C::AROW):
 * v[t][i] for term t, row block i (lane row c). */
template <class C>
struct RowScales {
    uint32_t v[C::TERMS][C::WM];
};

template <class C, int KSI>
__device__ __forceinline__ void mfma_slice(f32x4 (&acc)[C::WM][C::WN], const uint8_t *st,
                                           const uint8_t *sbuf, uint32_t sq, uint32_t wm,
                                           uint32_t wn, uint32_t live, const RowScales<C> &rs) {
    constexpr int NA = C::TERMS * C::WM, H1 = (NA + 1) / 2, H2 = NA - H1;
    /* LDS reads per A fragment: two code halves (+ its scale dword) */
    constexpr int RA = C::AROW ? 2 : 3;
    static_assert(RA * H2 < 16, "second-half reads fit the lgkm counter");
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t g = lane >> 4, c = lane & 15u;
    const uint32_t base = lds_addr(st);
    const uint32_t a_lo = base + a_slot(c, g) + 2048u * C::WM * wm;
    const uint32_t a_hi = base + a_slot(c, 4u + g) + 2048u * C::WM * wm;
    /* region bases in the address registers keep the immediates 16-bit;
     * slice KSI's A chunks, scales and (KS = 2) B pieces 4 KSI + g */
    const uint32_t b_base = C::KS == 2
        ? base + C::OFF_B + a_slot(c, 4u * KSI + g) + 2048u * C::WN * wn
        : base + C::OFF_B + 16u * lane + 1024u * C::WN * wn;
    /* scales: row r's dword for K slice kq at 16 r + 4 (kq % 4) of record
     * kq / 4 (SB records are regions of SB_CH KB) */
    const uint32_t kq = C::KS * sq + KSI; /* 128-column slice within the scale block */
    const uint32_t sbase = lds_addr(sbuf) + 16u * c + 4u * (kq & 3u);
    const uint32_t sa_base = sbase + C::OFF_SA + 256u * C::WM * wm;
    const uint32_t sb_base = sbase + C::OFF_SB + 1024u * C::SB_CH * (kq >> 2) + 256u * C::WN * wn;
    u32x4_t alo[NA], ahi[NA], bv[C::WN];
    uint32_t saw[NA], sbw[C::WN];
    auto read_a = [&](auto I) {
        constexpr int q = decltype(I)::value, t = q / C::WM, i = q % C::WM;
        constexpr int off = C::OFF_A + 2048 * ((KSI * C::TERMS + t) * (C::BM / 16) + i);
        alo[q] = ds_read16<off>(a_lo);
        ahi[q] = ds_read16<off>(a_hi);
        if constexpr (!C::AROW) saw[q] = ds_read4<16 * (t * C::SA_ROWS + 16 * i)>(sa_base);
    };
    auto mfmas = [&](auto Q) {
        constexpr int q = decltype(Q)::value, i = q % C::WM;
        const i32x8 af = i32x8{(int)alo[q].x, (int)alo[q].y, (int)alo[q].z, (int)alo[q].w,
                               (int)ahi[q].x, (int)ahi[q].y, (int)ahi[q].z, (int)ahi[q].w};
        int sa;
        if constexpr (C::AROW)
            sa = (int)rs.v[q / C::WM][i];
        else
            sa = (int)((saw[q] >> (8u * g)) & 255u);
        if ((uint32_t)i >= live) return; /* row block past the tile's rows */
        static_for<C::WN>([&](auto J) {
            constexpr int j = decltype(J)::value;
            const i32x8 bf = i32x8{(int)bv[j].x, (int)bv[j].y, (int)bv[j].z, (int)bv[j].w, 0, 0, 0, 0};
            const int sb = (int)((sbw[j] >> (8u * g)) & 255u);
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af, bf, acc[i][j], 0, 4, 0,
                                                                         sa, 0, sb);
        });
    };
    static_for<C::WN>([&](auto J) {
        constexpr int j = decltype(J)::value;
        bv[j] = ds_read16<(C::KS == 2 ? 2048 : 1024) * j>(b_base);
        sbw[j] = ds_read4<256 * j>(sb_base);
    });
    if constexpr (C::SEQ) {
        /* Software pipeline over the A fragments (two waves per SIMD):
         * the reads of fragment q + 1 are issued before the MFMAs of
         * fragment q, so the LDS reads run under the matrix pipe instead
         * of in a read phase with no MFMA in flight. LDS reads complete in
         * order, so lgkmcnt(RA) = all but fragment q + 1. */
        read_a(std::integral_constant<int, 0>{});
        static_for<NA>([&](auto Q) {
            constexpr int q = decltype(Q)::value;
            if constexpr (q + 1 < NA) {
                read_a(std::integral_constant<int, q + 1>{});
                wait_lgkm<RA>();
            } else {
                wait_lgkm<0>();
            }
            if constexpr (q == 0) {
                static_for<C::WN>([&](auto J) {
                    after_wait(bv[decltype(J)::value]);
                    after_wait(sbw[decltype(J)::value]);
                });
            }
            after_wait(alo[q]);
            after_wait(ahi[q]);
            if constexpr (!C::AROW) after_wait(saw[q]);
            mfmas(Q);
            __builtin_amdgcn_sched_barrier(0);
        });
        return;
    }
    static_for<H1>([&](auto I) { read_a(I); });
    static_for<H2>([&](auto I) { read_a(std::integral_constant<int, H1 + decltype(I)::value>{}); });
    /* first half (and B) landed */
    wait_lgkm<RA * H2>();
    static_for<C::WN>([&](auto J) {
        after_wait(bv[decltype(J)::value]);
        after_wait(sbw[decltype(J)::value]);
    });
    static_for<H1>([&](auto I) {
        after_wait(alo[decltype(I)::value]);
        after_wait(ahi[decltype(I)::value]);
        if constexpr (!C::AROW) after_wait(saw[decltype(I)::value]);
    });
    static_for<H1>([&](auto I) { mfmas(I); });
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkm<0>();
    static_for<H2>([&](auto I) {
        constexpr int q = H1 + decltype(I)::value;
        after_wait(alo[q]);
        after_wait(ahi[q]);
        if constexpr (!C::AROW) after_wait(saw[q]);
    });
    static_for<H2>([&](auto I) { mfmas(std::integral_constant<int, H1 + decltype(I)::value>{}); });
}

/* One staged step: its K slices in order. */
template <class C>
__device__ __forceinline__ void mfma_step(f32x4 (&acc)[C::WM][C::WN], const uint8_t *st,
                                          const uint8_t *sbuf0, const uint8_t *sbuf1, uint32_t s,
                                          uint32_t wm, uint32_t wn, uint32_t live,
                                          const RowScales<C> &rs) {
    const uint32_t b = s / (uint32_t)C::SQ, sq = s % (uint32_t)C::SQ;
    const uint8_t *sbuf = (b & 1u) ? sbuf1 : sbuf0;
    mfma_slice<C, 0>(acc, st, sbuf, sq, wm, wn, live, rs);
    if constexpr (C::KS == 2) {
        __builtin_amdgcn_sched_barrier(0);
        mfma_slice<C, 1>(acc, st, sbuf, sq, wm, wn, live, rs);
    }
}

/* Step s of the ring: wait for this wave's loads of step s (one later step
 * may stay in flight), barrier (every wave's loads of s have landed and
 * every wave is done reading the buffer refilled next), refill `nxt` with
 * step s + 2, compute from `cur`. */
template <class C>
__device__ __forceinline__ void ring_step(f32x4 (&acc)[C::WM][C::WN], const Loader<C> &L,
                                          const uint8_t *cur, uint8_t *nxt, uint32_t s,
                                          uint32_t nsteps, uint32_t wm, uint32_t wn,
                                          uint8_t *sbuf0, uint8_t *sbuf1, uint32_t live,
                                          const RowScales<C> &rs) {
    wait_step<C>(L, s + 1u < nsteps ? 1 : 0);
    __builtin_amdgcn_s_barrier();
    if (s + 2u < nsteps) issue_step<C>(L, nxt, s + 2u, threadIdx.x >> 6, sbuf0, sbuf1);
    mfma_step<C>(acc, cur, sbuf0, sbuf1, s, wm, wn, live, rs);
}

/* 16-row blocks of wave row wm that hold tile rows (< rows): MFMAs of
 * the others are skipped (their fragments are still read, which keeps the
 * LDS wait counts fixed). Wave-uniform. */
template <class C>
__device__ __forceinline__ uint32_t live_blocks(uint32_t rows, uint32_t wm) {
    const uint32_t r0 = 16u * (uint32_t)C::WM * wm;
    const uint32_t n = rows > r0 ? (rows - r0 + 15u) / 16u : 0u;
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)(n < (uint32_t)C::WM ? n : (uint32_t)C::WM));
}

/*
 * acc[i][j] += A(wave rows i) . W(wave rows j)^T over K (K % 128 == 0)
 * through three LDS buffers. They are distinct __shared__ arrays and the
 * loop is unrolled by three so every access names its buffer statically:
 * the compiler then sees that the in-flight direct-to-LDS loads target
 * other buffers than the ones being read and does not drain them.
 */
template <class C>
__device__ __forceinline__ void mfma_pipeline(f32x4 (&acc)[C::WM][C::WN], const Loader<C> &L,
                                              uint8_t *b0, uint8_t *b1, uint8_t *b2, uint8_t *sbuf0,
                                              uint8_t *sbuf1, uint32_t K, uint32_t wm,
                                              uint32_t wn, uint32_t live, const RowScales<C> &rs) {
    static_assert(C::STAGES == 2 || C::STAGES == 3, "two or three buffers");
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t nsteps = K / (uint32_t)C::KSTEP;
    if constexpr (C::STAGES == 2) {
        /* Two buffers, for tiles whose stage is too big for three: the
         * step is long (one wave per SIMD, WM x WN x TERMS MFMAs each), so
         * issuing step s + 1's loads at the start of step s hides them. */
        auto step2 = [&](uint32_t s, const uint8_t *cur, uint8_t *nxt) __attribute__((always_inline)) {
            wait_vm<0>();
            __builtin_amdgcn_s_barrier();
            if (s + 1u < nsteps) issue_step<C>(L, nxt, s + 1u, wave, sbuf0, sbuf1);
            mfma_step<C>(acc, cur, sbuf0, sbuf1, s, wm, wn, live, rs);
        };
        issue_step<C>(L, b0, 0u, wave, sbuf0, sbuf1);
        for (uint32_t s = 0; s < nsteps; s += 2u) {
            step2(s, b0, b1);
            if (s + 1u < nsteps) step2(s + 1u, b1, b0);
        }
        return;
    }
    issue_step<C>(L, b0, 0u, wave, sbuf0, sbuf1);
    if (nsteps > 1u) issue_step<C>(L, b1, 1u, wave, sbuf0, sbuf1);
    for (uint32_t s = 0; s < nsteps; s += 3u) {
        ring_step<C>(acc, L, b0, b2, s, nsteps, wm, wn, sbuf0, sbuf1, live, rs);
        if (s + 1u < nsteps)
            ring_step<C>(acc, L, b1, b0, s + 1u, nsteps, wm, wn, sbuf0, sbuf1, live, rs);
        if (s + 2u < nsteps)
            ring_step<C>(acc, L, b2, b1, s + 2u, nsteps, wm, wn, sbuf0, sbuf1, live, rs);
    }
}

/* ---------------------------------------------------------------------- */
/* XCD-aware work order                                                    */
/* ---------------------------------------------------------------------- */

/*
 * Workgroups are dealt to the eight XCDs round robin by linear id, and each
 * XCD has its own L2. Work item w = (tile w / cols, column block w % cols);
 * XCD x takes the contiguous range [x per, (x + 1) per) of the works. Tiles
 * are listed in expert order, so the ~32 blocks an XCD runs at once are
 * about 4 consecutive tiles (the same expert, for heavy experts) x 8
 * column blocks: they share ~4 activation tiles and 8 weight slices in
 * that L2 instead of fetching 32 different pairs through the fabric. The
 * column runs fastest so a tile's column blocks (equal run times) start
 * together as CUs free up and read the tile's activation lines while they
 * are still in L2; with the tile fastest they drifted apart after the
 * first round of blocks (cfg4 gate/up memory reads +9%, layer +2.4%).
 * L is the block's index in its class's grid (grids are multiples of 8, so
 * a class placed after another keeps L % 8 = XCD). Returns false for
 * blocks beyond the work count.
 */
__device__ __forceinline__ bool xcd_work(uint32_t L, uint32_t ntiles, uint32_t cols,
                                         uint32_t &tile, uint32_t &col) {
    const uint32_t works = ntiles * cols, per = (works + 7u) / 8u;
    const uint32_t j = L >> 3;
    const uint32_t w = (L & 7u) * per + j;
    if (j >= per || w >= works) return false;
    tile = w / cols;
    col = w % cols;
    return true;
}

/* Blocks for up to `cap` tiles of `cols` column blocks: xcd_work needs
 * 8 ceil(cap cols / 8). */
inline uint32_t xcd_grid(uint32_t cap, uint32_t cols) {
    const uint64_t works = (uint64_t)cap * cols;
    return (uint32_t)(8u * ((works + 7u) / 8u));
}

/* ---------------------------------------------------------------------- */
/* gate/up                                                                 */
/* ---------------------------------------------------------------------- */

struct GateUpArgs {
    MfmaBuffers B;
    const uint32_t *tiles;       /* this class's list */
    const uint32_t *tile_count;  /* this class's count */
    const uint32_t *token_index;
    const k3_moe_expert *experts;
    uint32_t H, F, kind;
    float beta, lb;
};

/*
 * Gate/up epilogue for activation kind KIND: lane (g, c) holds, for each of
 * its rows, the gate and up sums of G = WN / 2 consecutive f-columns fw0 +
 * G c + j. Each row's activation is rounded to bf16 and split into MXFP8
 * terms per 32-column block (32 / G lanes of one DPP row: maximum by DPP),
 * and each lane writes its G codes of a row and term with one store.
 */
template <class C, uint32_t KIND>
__device__ __forceinline__ void gateup_epilogue(const f32x4 (&acc)[C::WM][C::WN],
                                                const GateUpArgs &A, uint32_t row0, uint32_t rows,
                                                uint32_t fw0, uint32_t wm, uint32_t g, uint32_t c) {
    constexpr int G = C::WN / 2, LB = 32 / G;
    static_assert(G == 2 || G == 4, "two or four columns per lane");
    const uint32_t F = A.F;
    /* template loops: the rows must unroll fully (acc indices constant)
     * even where the activation's body exceeds the unroller's budget */
    static_for<C::WM * 4>([&](auto IR) {
        constexpr int i = decltype(IR)::value / 4, r = decltype(IR)::value % 4;
        const uint32_t lr = 16u * (wm * C::WM + (uint32_t)i) + 4u * g + (uint32_t)r;
        const uint64_t prow = (uint64_t)row0 + (lr < rows ? lr : 0u);
        float v[G];
        if constexpr (KIND == 1u) {
            /* SwiGLU g sigmoid(g) u with the sigmoid from the hardware
             * exp2 and reciprocal (each within 1 ulp): this path's
             * two-term split already carries ~2^-16 relative error,
             * and the value is rounded to bf16 first */
#pragma unroll
            for (int j = 0; j < G; j += 2) {
                const float2 gg = bf16r2(acc[i][j][r], acc[i][j + 1][r]);
                const float2 uu = bf16r2(acc[i][G + j][r], acc[i][G + j + 1][r]);
                const float g2[2] = {gg.x, gg.y}, u2[2] = {uu.x, uu.y};
                float h[2];
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    const float e = __builtin_amdgcn_exp2f(__fmul_rn(g2[k], -1.44269502162933349609375f));
                    const float sg = __builtin_amdgcn_rcpf(__fadd_rn(1.0f, e));
                    h[k] = __fmul_rn(__fmul_rn(g2[k], sg), u2[k]);
                }
                const float2 hh = bf16r2(h[0], h[1]);
                v[j] = hh.x;
                v[j + 1] = hh.y;
            }
        } else {
#pragma unroll
            for (int j = 0; j < G; j++) {
                v[j] = bf16r(gated_act(bf16r(acc[i][j][r]), bf16r(acc[i][G + j][r]), KIND,
                                       A.beta, A.lb));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int t = 0; t < C::TERMS; t++) {
            float amax = fabsf(v[0]);
#pragma unroll
            for (int j = 1; j < G; j++) amax = fmaxf(amax, fabsf(v[j]));
            amax = row_group_max<LB>(amax);
            const uint32_t sbyte = mx8_scale_byte(amax);
            const float inv = mx8_inv_scale(sbyte), sc = e8m0_to_f32(sbyte);
            /* code x scale is exact (a 4-bit significand times a power
             * of two at or above 2^-127), so the residual is one fma */
            uint32_t w = e4m3x2_raw<false>(__fmul_rn(v[0], inv), __fmul_rn(v[1], inv), 0u);
            if constexpr (G == 4)
                w = e4m3x2_raw<true>(__fmul_rn(v[2], inv), __fmul_rn(v[3], inv), w);
            if (C::TERMS == 2 && t == 0) {
                v[0] = fmaf(-e4m3_byte<0>(w), sc, v[0]);
                v[1] = fmaf(-e4m3_byte<1>(w), sc, v[1]);
                if constexpr (G == 4) {
                    v[2] = fmaf(-e4m3_byte<2>(w), sc, v[2]);
                    v[3] = fmaf(-e4m3_byte<3>(w), sc, v[3]);
                }
            }
            if (lr < rows) {
                uint8_t *dst = A.B.aq[t] + prow * F + fw0 + (uint32_t)G * c;
                if constexpr (G == 4)
                    *(uint32_t *)dst = w;
                else
                    *(uint16_t *)dst = (uint16_t)w;
                if (c % (uint32_t)LB == 0u) { /* block-major: [kb / 16][route][kb % 16] */
                    const uint32_t kb = fw0 / 32u + c / (uint32_t)LB;
                    A.B.as[t][(((uint64_t)(kb >> 4) * A.B.routes + prow) << 4) + (kb & 15u)] =
                        (uint8_t)sbyte;
                }
            }
        }
        /* one row at a time: interleaving rows raises the register
         * pressure past the 128-row class's budget */
        __builtin_amdgcn_sched_barrier(0);
    });
}

/*
 * One gate/up block of class C (blk: its index in the class's grid, b0 ..
 * sbuf1: its LDS ring). The block's
 * BN weight rows are BN / 2 gate rows and the same up rows: wave column wn
 * owns f-columns f0 + 8 WN wn .. + 8 WN, n-subtiles j < WN / 2 gate and
 * j >= WN / 2 up, so gate and up of a column meet in one lane (wrow gives
 * each lane WN / 2 consecutive columns). Epilogue: gateup_epilogue.
 */
template <class C, uint32_t KIND>
__device__ __forceinline__ void gateup_block(const GateUpArgs &A, uint32_t blk, uint8_t *b0,
                                             uint8_t *b1, uint8_t *b2, uint8_t *sbuf0,
                                             uint8_t *sbuf1) {
    uint32_t tile, colb;
    if (!xcd_work(blk, *A.tile_count, A.F / (uint32_t)(C::BN / 2), tile, colb)) return;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t g = lane >> 4, c = lane & 15u;
    const uint32_t wm = wave / C::NW, wn = wave % C::NW;
    const uint32_t e = A.tiles[3u * tile], row0 = A.tiles[3u * tile + 1u];
    const uint32_t rows = A.tiles[3u * tile + 2u];
    const uint32_t H = A.H, F = A.F;
    const k3_moe_expert ex = A.experts[e];
    constexpr int FW = 8 * C::WN; /* f-columns per wave column */
    constexpr int G = C::WN / 2;  /* gate (and up) columns per lane and row */
    const uint32_t f0 = colb * (uint32_t)(C::BN / 2);
    /* weight row of block subtile J, lane row c: gate rows for the first
     * half of each wave column's subtiles, up rows (offset by F) after.
     * Lane row c of gate subtile j takes f-column G c + j, so each lane's
     * accumulators hold G consecutive columns of every row (one packed
     * store per row and term in the epilogue). */
    auto wrow = [&](int J, uint32_t cc) -> uint32_t {
        const int wcol = J / C::WN, j = J % C::WN;
        const uint32_t f = f0 + (uint32_t)(FW * wcol) + (uint32_t)G * cc + (uint32_t)(j % G);
        return j < G ? f : F + f; /* rows >= F address the up tensor */
    };
    auto tok = [&](uint32_t r) -> uint32_t {
        return A.token_index[row0 + (r < rows ? r : 0u)];
    };
    auto a_row = [&](int t, uint32_t r) -> const uint8_t * {
        return A.B.xq[t] + (uint64_t)tok(r) * H;
    };
    Loader<C> L;
    {
        const uint8_t *gp = (const uint8_t *)ex.gate_packed, *up = (const uint8_t *)ex.up_packed;
        const uint8_t *gs = (const uint8_t *)ex.gate_scales, *us = (const uint8_t *)ex.up_scales;
        auto wr_codes = [&](int J, uint32_t cc) -> const uint8_t * {
            const uint32_t r = wrow(J, cc);
            return r < F ? gp + (uint64_t)r * (H / 2u) : up + (uint64_t)(r - F) * (H / 2u);
        };
        auto wr_scl = [&](int J, uint32_t cc) -> const uint8_t * {
            const uint32_t r = wrow(J, cc);
            return r < F ? gs + (uint64_t)r * (H / 32u) : us + (uint64_t)(r - F) * (H / 32u);
        };
        constexpr int W = C::NWV;
        L.mask = kinds_held<C>(wave);
#pragma unroll
        for (int q = 0; q < C::DA::per; q++) {
            const int ch = min(chunk_of<typename C::DA, W>(q, wave), C::A_CH - 1);
            const int h = ch & 1, i = (ch >> 1) % (C::BM / 16);
            const int t = (ch >> 1) / (C::BM / 16) % C::TERMS, ks = (ch >> 1) / (C::BM / 16) / C::TERMS;
            L.a[q] = a_row(t, 16u * i + a_dma_row(lane, h)) + 128u * ks + 16u * a_dma_piece(lane, h);
        }
#pragma unroll
        for (int q = 0; q < C::DB::per; q++) {
            const int ch = min(chunk_of<typename C::DB, W>(q, wave), C::B_CH - 1);
            if constexpr (C::KS == 2) {
                const uint32_t h = (uint32_t)ch & 1u;
                L.b[q] = wr_codes(ch >> 1, a_dma_row(lane, h)) + 16u * a_dma_piece(lane, h);
            } else {
                L.b[q] = wr_codes(ch, c) + 16u * g;
            }
        }
#pragma unroll
        for (int q = 0; q < C::DSB::per; q++) { /* 64 rows = 4 subtiles per chunk */
            const int ch = min(chunk_of<typename C::DSB, W>(q, wave), C::SB_CH - 1);
            L.sb[q] = wr_scl(ch * 4 + (int)g, c);
        }
        static_assert(C::AROW, "gate/up takes per-row activation scales");
        L.sa_stride = 0u;
        L.sb_recs = H / 512u;
    }
    RowScales<C> rs; /* lane row c of each of the wave's row blocks */
#pragma unroll
    for (int i = 0; i < C::WM; i++) {
        const uint32_t tk = tok(16u * (wm * (uint32_t)C::WM + (uint32_t)i) + c);
#pragma unroll
        for (int t = 0; t < C::TERMS; t++) rs.v[t][i] = A.B.xs[t][tk];
    }
    f32x4 acc[C::WM][C::WN];
#pragma unroll
    for (int i = 0; i < C::WM; i++)
#pragma unroll
        for (int j = 0; j < C::WN; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    mfma_pipeline<C>(acc, L, b0, b1, b2, sbuf0, sbuf1, H, wm, wn, live_blocks<C>(rows, wm), rs);

    const uint32_t fw0 = f0 + (uint32_t)FW * wn;
    gateup_epilogue<C, KIND>(acc, A, row0, rows, fw0, wm, g, c);
}

/* ---------------------------------------------------------------------- */
/* down                                                                    */
/* ---------------------------------------------------------------------- */

struct DownArgs {
    MfmaBuffers B;
    const uint32_t *tiles;
    const uint32_t *tile_count;
    const uint32_t *route_index;
    const k3_moe_expert *experts;
    uint16_t *y;
    uint32_t H, F;
};

/* One down block of class C: y[route] rows d0 .. d0 + BN. */
template <class C>
__device__ __forceinline__ void down_block(const DownArgs &A, uint32_t blk, uint8_t *b0,
                                           uint8_t *b1, uint8_t *b2, uint8_t *sbuf0,
                                           uint8_t *sbuf1) {
    uint32_t tile, colb;
    if (!xcd_work(blk, *A.tile_count, A.H / (uint32_t)C::BN, tile, colb)) return;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t g = lane >> 4, c = lane & 15u;
    const uint32_t wm = wave / C::NW, wn = wave % C::NW;
    const uint32_t e = A.tiles[3u * tile], row0 = A.tiles[3u * tile + 1u];
    const uint32_t rows = A.tiles[3u * tile + 2u];
    const uint32_t H = A.H, F = A.F;
    const k3_moe_expert ex = A.experts[e];
    const uint32_t d0 = colb * (uint32_t)C::BN;
    const uint8_t *wp = (const uint8_t *)ex.down_packed, *ws = (const uint8_t *)ex.down_scales;
    auto prow = [&](uint32_t r) -> uint64_t { return (uint64_t)row0 + (r < rows ? r : 0u); };
    /* output column of block subtile J, lane row cc: lane row cc of wave
     * column w's subtile j takes column 16 WN w + WN cc + j, so each lane
     * holds WN consecutive columns of every row (one store per row) */
    auto dcol = [&](int J, uint32_t cc) -> uint32_t {
        return d0 + (uint32_t)(16 * C::WN * (J / C::WN)) + (uint32_t)C::WN * cc + (uint32_t)(J % C::WN);
    };
    Loader<C> L;
    constexpr int W = C::NWV;
    L.mask = kinds_held<C>(wave);
#pragma unroll
    for (int q = 0; q < C::DA::per; q++) {
        const int ch = min(chunk_of<typename C::DA, W>(q, wave), C::A_CH - 1);
        const int h = ch & 1, i = (ch >> 1) % (C::BM / 16);
        const int t = (ch >> 1) / (C::BM / 16) % C::TERMS, ks = (ch >> 1) / (C::BM / 16) / C::TERMS;
        L.a[q] = A.B.aq[t] + prow(16u * i + a_dma_row(lane, h)) * F + 128u * ks +
                 16u * a_dma_piece(lane, h);
    }
#pragma unroll
    for (int q = 0; q < C::DB::per; q++) {
        const int ch = min(chunk_of<typename C::DB, W>(q, wave), C::B_CH - 1);
        if constexpr (C::KS == 2) {
            const uint32_t h = (uint32_t)ch & 1u;
            L.b[q] = wp + (uint64_t)dcol(ch >> 1, a_dma_row(lane, h)) * (F / 2u) +
                     16u * a_dma_piece(lane, h);
        } else {
            L.b[q] = wp + (uint64_t)dcol(ch, c) * (F / 2u) + 16u * g;
        }
    }
#pragma unroll
    for (int q = 0; q < C::DSB::per; q++) {
        const int ch = min(chunk_of<typename C::DSB, W>(q, wave), C::SB_CH - 1);
        L.sb[q] = ws + (uint64_t)dcol(4 * ch + (int)g, c) * (F / 32u);
    }
#pragma unroll
    for (int q = 0; q < C::DSA::per; q++) {
        const int ch = min(chunk_of<typename C::DSA, W>(q, wave), C::SA_CH - 1);
        const int t = ch / (C::SA_ROWS / 64);
        const uint32_t r = (uint32_t)((ch % (C::SA_ROWS / 64)) * 64) + lane;
        L.sa[q] = A.B.as[t] + prow(r) * 16u;
    }
    L.sa_stride = 16u * A.B.routes; /* scale block b of every row at + b 16 routes */
    L.sb_recs = F / 512u;
    f32x4 acc[C::WM][C::WN];
#pragma unroll
    for (int i = 0; i < C::WM; i++)
#pragma unroll
        for (int j = 0; j < C::WN; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    static_assert(!C::AROW, "down stages the activation's block scales");
    const RowScales<C> rs{};
    mfma_pipeline<C>(acc, L, b0, b1, b2, sbuf0, sbuf1, F, wm, wn, live_blocks<C>(rows, wm), rs);
#pragma unroll
    for (int i = 0; i < C::WM; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t lr = 16u * (wm * C::WM + (uint32_t)i) + 4u * g + (uint32_t)r;
            if (lr >= rows) continue;
            const uint64_t route = A.route_index[row0 + lr];
            static_assert(C::WN == 2 || C::WN == 4 || C::WN == 8, "2, 4 or 8 columns per lane");
            uint32_t pk[C::WN / 2];
#pragma unroll
            for (int j = 0; j < C::WN / 2; j++)
                pk[j] = (uint32_t)f32_to_bf16(acc[i][2 * j][r]) |
                        ((uint32_t)f32_to_bf16(acc[i][2 * j + 1][r]) << 16);
            uint16_t *dst = A.y + route * H + d0 + 16u * C::WN * wn + (uint32_t)C::WN * c;
            if constexpr (C::WN == 8)
                *(uint4 *)dst = make_uint4(pk[0], pk[1], pk[2], pk[3]);
            else if constexpr (C::WN == 4)
                *(uint2 *)dst = make_uint2(pk[0], pk[1]);
            else
                *(uint32_t *)dst = pk[0];
        }
}

/* Tile classes (rows per tile): 16, 64, 96, 128. One-term class 0 computes
 * 32 rows so that its A chunks still split over the waves. Class 0's
 * gate/up takes 128-row weight blocks of two waves (80 KB of LDS: two
 * blocks per CU; cfg2 gate/up 1.68 -> 1.60 ms, cfg3 level); its down
 * takes 256-row blocks of eight waves of 16 x 32 (two per SIMD: against
 * four waves of 16 x 64, cfg2 down -11%, cfg3 -5%). */
template <int TERMS>
using Cls0 = TileCfg<1, 8, TERMS == 2 ? 1 : 2, 2, TERMS, 3, 2, 2>;
template <int TERMS>
using Cls0G = TileCfg<1, 2, TERMS == 2 ? 1 : 2, 4, TERMS, 3, 2, 2>;
/* 64 x 256 blocks of eight waves (32 x 64 each, two per SIMD): against four
 * waves of 64 x 64, cfg4 -1.4%, cfg3 -0.8%; the same block size as the
 * 96- and 128-row classes, so gate/up launches the three together */
template <int TERMS>
using Cls1 = TileCfg<2, 4, 2, 4, TERMS, 2, 2, 2>;
/* 128 x 512 blocks: eight waves, two per SIMD, each 64 activation rows x
 * 128 weight rows; halves the activation re-reads of a 256-wide block, two
 * stage buffers */
template <int TERMS>
using Cls3 = TileCfg<2, 4, 4, 8, TERMS, 2>;
/* 96 x 512 blocks for experts of 65-96 rows, one tile each (most experts
 * of a Zipf batch's 128-row range): a quarter less activation staging per
 * K step than a padded 128-row tile, 48 rows per wave. One term stages
 * 12 activation chunks, which do not split over 8 waves: it keeps the
 * 128-row blocks. */
template <int TERMS>
using Cls2 = std::conditional_t<TERMS == 2, TileCfg<2, 4, 3, 8, 2, 2, 1, 0>, Cls3<TERMS>>;

/* LDS of a block running C or D: the ring and scale buffers are distinct
 * arrays (the pipeline names each buffer statically). */
template <class C, class D = C, class E = C>
struct RingSmem {
    static constexpr int max3(int a, int b, int c) { return a > b ? (a > c ? a : c) : (b > c ? b : c); }
    static constexpr int STAGE = max3(C::STAGE, D::STAGE, E::STAGE);
    static constexpr int SBUF = max3(C::SBUF, D::SBUF, E::SBUF);
    static constexpr bool THREE = C::STAGES == 3 || D::STAGES == 3 || E::STAGES == 3;
};

#define K3_RING_SMEM(R)                                                                      \
    __shared__ __attribute__((aligned(16))) uint8_t b0[R::STAGE], b1[R::STAGE];              \
    __shared__ __attribute__((aligned(16))) uint8_t sbuf0[R::SBUF], sbuf1[R::SBUF];          \
    __shared__ __attribute__((aligned(16))) uint8_t b2[R::THREE ? R::STAGE : 16]

/*
 * gate/up: grid xcd_grid(tile cap, F / (BN / 2)), block C::THREADS. The
 * block's BN weight rows are BN / 2 gate rows and the same up rows (see
 * gateup_block).
 */
template <class C, uint32_t KIND>
__global__ __launch_bounds__(C::THREADS) void gateup_mfma_kernel(GateUpArgs A) {
    using R = RingSmem<C>;
    K3_RING_SMEM(R);
    gateup_block<C, KIND>(A, blockIdx.x, b0, b1, b2, sbuf0, sbuf1);
}

/* Three tile classes of one block size in one launch: blocks [0, na) run
 * class C on A's list, [na, nb) class D on B's, the rest class E on E's.
 * Each class's blocks start while the previous one's last blocks still run,
 * so the launch has one tail instead of three (the 96- and 128-row gate/up
 * blocks run ~150 us; two classes in one launch: cfg4 gate/up -2%). */
template <class C, class D, class E, uint32_t KIND>
__global__ __launch_bounds__(C::THREADS) void gateup_mfma3_kernel(GateUpArgs A, GateUpArgs B,
                                                                  GateUpArgs Ea, uint32_t na,
                                                                  uint32_t nb) {
    static_assert(C::THREADS == D::THREADS && C::THREADS == E::THREADS, "one block size");
    using R = RingSmem<C, D, E>;
    K3_RING_SMEM(R);
    if (blockIdx.x < na)
        gateup_block<C, KIND>(A, blockIdx.x, b0, b1, b2, sbuf0, sbuf1);
    else if (blockIdx.x < nb)
        gateup_block<D, KIND>(B, blockIdx.x - na, b0, b1, b2, sbuf0, sbuf1);
    else
        gateup_block<E, KIND>(Ea, blockIdx.x - nb, b0, b1, b2, sbuf0, sbuf1);
}

/* down: grid xcd_grid(tile cap, H / BN), block C::THREADS. */
template <class C>
__global__ __launch_bounds__(C::THREADS) void down_mfma_kernel(DownArgs A) {
    using R = RingSmem<C>;
    K3_RING_SMEM(R);
    down_block<C>(A, blockIdx.x, b0, b1, b2, sbuf0, sbuf1);
}

/* Three down classes of one block size in one launch (as gateup_mfma3_kernel;
 * level with separate launches at cfg4, one launch where they are empty). */
template <class C, class D, class E>
__global__ __launch_bounds__(C::THREADS) void down_mfma3_kernel(DownArgs A, DownArgs B,
                                                                DownArgs Ea, uint32_t na,
                                                                uint32_t nb) {
    static_assert(C::THREADS == D::THREADS && C::THREADS == E::THREADS, "one block size");
    using R = RingSmem<C, D, E>;
    K3_RING_SMEM(R);
    if (blockIdx.x < na)
        down_block<C>(A, blockIdx.x, b0, b1, b2, sbuf0, sbuf1);
    else if (blockIdx.x < nb)
        down_block<D>(B, blockIdx.x - na, b0, b1, b2, sbuf0, sbuf1);
    else
        down_block<E>(Ea, blockIdx.x - nb, b0, b1, b2, sbuf0, sbuf1);
}


template <class C>
void launch_gateup(const GateUpArgs &a, uint32_t cap, hipStream_t st) {
    /* one kernel per activation kind: a kernel holding both epilogues runs
     * out of registers in the 128-row class */
    const dim3 grid(xcd_grid(cap, a.F / (C::BN / 2))), block(C::THREADS);
    if (a.kind == 1u)
        hipLaunchKernelGGL(HIP_KERNEL_NAME(gateup_mfma_kernel<C, 1u>), grid, block, 0, st, a);
    else
        hipLaunchKernelGGL(HIP_KERNEL_NAME(gateup_mfma_kernel<C, 0u>), grid, block, 0, st, a);
}

template <class C>
void launch_down(const DownArgs &a, uint32_t cap, hipStream_t st) {
    hipLaunchKernelGGL(HIP_KERNEL_NAME(down_mfma_kernel<C>), dim3(xcd_grid(cap, a.H / C::BN)),
                       dim3(C::THREADS), 0, st, a);
}

template <class C, class D, class E>
void launch_down3(const DownArgs &a, uint32_t cap_a, const DownArgs &b, uint32_t cap_b,
                  const DownArgs &e, uint32_t cap_e, hipStream_t st) {
    const uint32_t na = xcd_grid(cap_a, a.H / C::BN);
    const uint32_t nb = na + xcd_grid(cap_b, b.H / D::BN);
    hipLaunchKernelGGL(HIP_KERNEL_NAME(down_mfma3_kernel<C, D, E>),
                       dim3(nb + xcd_grid(cap_e, e.H / E::BN)), dim3(C::THREADS), 0, st, a, b, e,
                       na, nb);
}

template <class C, class D, class E>
void launch_gateup3(const GateUpArgs &a, uint32_t cap_a, const GateUpArgs &b, uint32_t cap_b,
                    const GateUpArgs &e, uint32_t cap_e, hipStream_t st) {
    const uint32_t na = xcd_grid(cap_a, a.F / (C::BN / 2));
    const uint32_t nb = na + xcd_grid(cap_b, b.F / (D::BN / 2));
    const dim3 grid(nb + xcd_grid(cap_e, e.F / (E::BN / 2))), block(C::THREADS);
    if (a.kind == 1u)
        hipLaunchKernelGGL(HIP_KERNEL_NAME(gateup_mfma3_kernel<C, D, E, 1u>), grid, block, 0, st,
                           a, b, e, na, nb);
    else
        hipLaunchKernelGGL(HIP_KERNEL_NAME(gateup_mfma3_kernel<C, D, E, 0u>), grid, block, 0, st,
                           a, b, e, na, nb);
}


template <int TERMS>
bool launch_terms(const MfmaBuffers &B, uint16_t *y, const uint16_t *hidden,
                  const uint32_t *counts, const uint32_t *offsets, const uint32_t *token_index,
                  const uint32_t *route_index, const k3_moe_expert *experts, const k3_moe_shape &s,
                  uint32_t T, hipStream_t st, const StageMarker &mark) {
    const uint32_t H = s.hidden, F = s.ffn;
    launch_split_rows<TERMS>(B, hidden, T, H, st);
    hipLaunchKernelGGL(tile_build_kernel, dim3(1), dim3(1024), 0, st, B, counts, offsets,
                       experts, s.expert_count, 0u);
    mark(K3_MOE_STAGE_GATE_UP);
    GateUpArgs ga{B, nullptr, nullptr, token_index, experts, H, F, s.activation,
                  s.activation == 1u ? 1.0f : s.beta, s.activation == 1u ? 1.0f : s.linear_beta};
    DownArgs da{B, nullptr, nullptr, route_index, experts, y, H, F};
    uint32_t base = 0u;
    const uint32_t *tl[kTileClasses];
    for (int c = 0; c < kTileClasses; c++) {
        tl[c] = B.tiles + 3u * base;
        base += B.tile_cap[c];
    }
    for (int c = 0; c < kTileClasses; c++) {
        if (!B.tile_cap[c]) continue;
        ga.tiles = tl[c];
        ga.tile_count = B.tile_count + c;
        if (c == 0) launch_gateup<RowScaled<Cls0G<TERMS>>>(ga, B.tile_cap[c], st);
    }
    /* classes 3, 2 and 1 (one block size) in one launch: one tail */
    if (B.tile_cap[3] || B.tile_cap[2] || B.tile_cap[1]) {
        GateUpArgs g[kTileClasses];
        for (int c = 1; c < kTileClasses; c++) {
            g[c] = ga;
            g[c].tiles = tl[c];
            g[c].tile_count = B.tile_count + c;
        }
        launch_gateup3<RowScaled<Cls3<TERMS>>, RowScaled<Cls2<TERMS>>, RowScaled<Cls1<TERMS>>>(
            g[3], B.tile_cap[3], g[2], B.tile_cap[2], g[1], B.tile_cap[1], st);
    }
    mark(K3_MOE_STAGE_DOWN);
    for (int c = 0; c < kTileClasses; c++) {
        if (!B.tile_cap[c]) continue;
        da.tiles = tl[c];
        da.tile_count = B.tile_count + c;
        if (c == 0) launch_down<Cls0<TERMS>>(da, B.tile_cap[c], st);
    }
    if (B.tile_cap[3] || B.tile_cap[2] || B.tile_cap[1]) {
        DownArgs d[kTileClasses];
        for (int c = 1; c < kTileClasses; c++) {
            d[c] = da;
            d[c].tiles = tl[c];
            d[c].tile_count = B.tile_count + c;
        }
        launch_down3<Cls3<TERMS>, Cls2<TERMS>, Cls1<TERMS>>(d[3], B.tile_cap[3], d[2],
                                                            B.tile_cap[2], d[1], B.tile_cap[1], st);
    }
    return hipGetLastError() == hipSuccess;
}

}  // namespace

void mfma_tile_caps(uint32_t T, uint32_t k, uint32_t E, uint32_t caps[kTileClasses]) {
    const uint64_t R = (uint64_t)T * k;
    auto upto = [&](uint64_t v) { return (uint32_t)(v < E ? v : E); };
    caps[0] = upto(R);         /* experts with 1-16 rows */
    caps[1] = upto(R / 17u);   /* 17-64 */
    caps[2] = upto(R / 65u);   /* 65-96 */
    /* > 96 rows: ceil(n / 128) <= n / 128 + 1 tiles each */
    caps[3] = (uint32_t)(R / 128u) + upto(R / 97u);
}

bool build_tiles_all(const MfmaBuffers &B, const uint32_t *counts, const uint32_t *offsets,
                     const k3_moe_expert *experts, uint32_t E, hipStream_t st) {
    if (E > 1024u) return false;
    hipLaunchKernelGGL(tile_build_kernel, dim3(1), dim3(1024), 0, st, B, counts, offsets, experts,
                       E, 1u);
    return hipGetLastError() == hipSuccess;
}

bool mfma_supported(const k3_moe_shape &s) {
    /* 16-byte scale records: whole ones per row of every weight tensor */
    return s.hidden % 512u == 0u && s.ffn % 512u == 0u && s.expert_count <= 1024u;
}

bool mfma_launch_experts(const MfmaBuffers &B, uint16_t *y, const uint16_t *hidden,
                         const uint32_t *counts, const uint32_t *offsets,
                         const uint32_t *token_index, const uint32_t *route_index,
                         const k3_moe_expert *experts, const k3_moe_shape &s, uint32_t T,
                         uint32_t terms, hipStream_t st, const StageMarker &mark) {
    if (!mfma_supported(s)) return false;
    if (terms == 2u)
        return launch_terms<2>(B, y, hidden, counts, offsets, token_index, route_index, experts, s,
                               T, st, mark);
    if (terms == 1u)
        return launch_terms<1>(B, y, hidden, counts, offsets, token_index, route_index, experts, s,
                               T, st, mark);
    return false;
}

}  // namespace k3

extern "C" bool k3_moe_mx8_quantize_bf16(uint8_t *hi_codes, uint8_t *hi_scales, uint8_t *lo_codes,
                                         uint8_t *lo_scales, const void *src, uint64_t count,
                                         void *stream) {
    using namespace k3;
    if (!hi_codes || !hi_scales || !src || count == 0u || count % 32u != 0u ||
        ((uintptr_t)src % 16u) != 0u || ((uintptr_t)hi_codes % 16u) != 0u ||
        ((lo_codes == nullptr) != (lo_scales == nullptr)) ||
        (lo_codes && ((uintptr_t)lo_codes % 16u) != 0u))
        return false;
    MfmaBuffers B{};
    B.xq[0] = hi_codes; B.xs[0] = hi_scales;
    B.xq[1] = lo_codes; B.xs[1] = lo_scales;
    const uint64_t blocks = count / 32u;
    const dim3 grid((uint32_t)((blocks + 255u) / 256u));
    if (lo_codes)
        hipLaunchKernelGGL(HIP_KERNEL_NAME(x_split_kernel<2>), grid, dim3(256), 0,
                           (hipStream_t)stream, B, (const uint16_t *)src, blocks);
    else
        hipLaunchKernelGGL(HIP_KERNEL_NAME(x_split_kernel<1>), grid, dim3(256), 0,
                           (hipStream_t)stream, B, (const uint16_t *)src, blocks);
    return hipGetLastError() == hipSuccess;
}

extern "C" bool k3_moe_mx8_quantize_rows_bf16(uint8_t *hi_codes, uint8_t *hi_scales,
                                              uint8_t *lo_codes, uint8_t *lo_scales,
                                              const void *src, uint32_t rows, uint32_t cols,
                                              void *stream) {
    using namespace k3;
    if (!hi_codes || !hi_scales || !src || rows == 0u || cols == 0u || cols % 8u != 0u ||
        ((uintptr_t)src % 16u) != 0u || ((uintptr_t)hi_codes % 8u) != 0u ||
        ((lo_codes == nullptr) != (lo_scales == nullptr)) ||
        (lo_codes && ((uintptr_t)lo_codes % 8u) != 0u))
        return false;
    MfmaBuffers B{};
    B.xq[0] = hi_codes; B.xs[0] = hi_scales;
    B.xq[1] = lo_codes; B.xs[1] = lo_scales;
    if (lo_codes)
        launch_split_rows<2>(B, (const uint16_t *)src, rows, cols, (hipStream_t)stream);
    else
        launch_split_rows<1>(B, (const uint16_t *)src, rows, cols, (hipStream_t)stream);
    return hipGetLastError() == hipSuccess;
}
