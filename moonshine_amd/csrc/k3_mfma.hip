/*
 * Grouped MXFP4 expert products on gfx950 scaled MFMA (prefill and batched
 * tokens). Replaces the per-expert k3_rocm_mxfp4_gemm_tiled_bf16 calls of
 * launch_prefill_expert (k3_engine_prefill.inc:962-990): one launch per
 * tile-size class covers every selected expert of the layer.
 *
 *   x_split_kernel      hidden rows -> MXFP8 hi (and lo) codes + scales
 *   tile_build_kernel   plan -> per-class tile lists (16/32/64-row tiles)
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
 * Tiles: a block is 4 waves along the weight rows (each wave 4 x 16 rows)
 * sharing 16 * WM activation rows; K advances 128 per step.
 */
#include "k3_device.h"
#include "k3_mfma.h"
#include "../../include/k3_moe.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace k3 {
namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kTileRows[3] = {16u, 32u, 64u};

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
            uint32_t word = 0u;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t code = f32_to_e4m3(__fmul_rn(v[4 * q + i], inv));
                word |= code << (8 * i);
                if (TERMS == 2 && t == 0)
                    v[4 * q + i] = __fsub_rn(v[4 * q + i], __fmul_rn(e4m3_to_f32(code), sc));
            }
            w[q] = word;
        }
        uint4 *dst = (uint4 *)(B.xq[t] + 32u * b);
        dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
        dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
        B.xs[t][b] = (uint8_t)sb;
    }
}

/* ---------------------------------------------------------------------- */
/* tile lists                                                              */
/* ---------------------------------------------------------------------- */

/* One block of 1024 threads (thread e = expert e). Class 0: experts with
 * <= 16 rows (one 16-row tile), class 1: <= 32 rows (one 32-row tile),
 * class 2: 64-row tiles. Tiles are listed in expert order. */
__global__ __launch_bounds__(1024) void tile_build_kernel(MfmaBuffers B,
                                                          const uint32_t *__restrict__ counts,
                                                          const uint32_t *__restrict__ offsets,
                                                          uint32_t E) {
    __shared__ uint32_t wave_tot[3][16];
    const uint32_t e = threadIdx.x, lane = e & 63u, wave = e >> 6;
    const uint32_t n = e < E ? counts[e] : 0u;
    const int cls = n == 0u ? 3 : (n <= 16u ? 0 : (n <= 32u ? 1 : 2));
    uint32_t nt[3], inc[3];
#pragma unroll
    for (int c = 0; c < 3; c++) {
        nt[c] = cls == c ? (c == 2 ? (n + 63u) / 64u : 1u) : 0u;
        inc[c] = nt[c];
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1)
#pragma unroll
        for (int c = 0; c < 3; c++) {
            const uint32_t a = __shfl_up(inc[c], o, 64);
            if ((int)lane >= o) inc[c] += a;
        }
    if (lane == 63u)
        for (int c = 0; c < 3; c++) wave_tot[c][wave] = inc[c];
    __syncthreads();
    uint32_t base_idx = 0u;
    for (int c = 0; c < 3; c++) {
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
}

/* ---------------------------------------------------------------------- */
/* MFMA core                                                               */
/* ---------------------------------------------------------------------- */

__device__ __forceinline__ i32x8 load_fp8_frag(const uint8_t *row, uint32_t k0, uint32_t g) {
    const uint4 a = gload((const uint4 *)(row + k0 + 16u * g));
    const uint4 b = gload((const uint4 *)(row + k0 + 64u + 16u * g));
    i32x8 v;
    v[0] = (int)a.x; v[1] = (int)a.y; v[2] = (int)a.z; v[3] = (int)a.w;
    v[4] = (int)b.x; v[5] = (int)b.y; v[6] = (int)b.z; v[7] = (int)b.w;
    return v;
}

__device__ __forceinline__ i32x8 load_fp4_frag(const uint8_t *row, uint32_t k0, uint32_t g) {
    const uint4 a = gload((const uint4 *)(row + k0 / 2u + 16u * g));
    i32x8 v;
    v[0] = (int)a.x; v[1] = (int)a.y; v[2] = (int)a.z; v[3] = (int)a.w;
    v[4] = 0; v[5] = 0; v[6] = 0; v[7] = 0;
    return v;
}

/*
 * acc[i][j] += A_i . W_j^T over K for this wave: A_i = activation rows of
 * m-subtile i (TERMS MXFP8 terms), W_j = weight rows of n-subtile j.
 * a_row[t][i] / a_scl[t][i] point at the lane's activation row (codes,
 * scales); w_row[j] / w_scl[j] at the lane's weight row.
 */
template <int WM, int TERMS>
__device__ __forceinline__ void mfma_rows(f32x4 (&acc)[WM][4], const uint8_t *(&a_row)[TERMS][WM],
                                          const uint8_t *(&a_scl)[TERMS][WM],
                                          const uint8_t *(&w_row)[4], const uint8_t *(&w_scl)[4],
                                          uint32_t K, uint32_t g) {
    for (uint32_t k0 = 0; k0 < K; k0 += 128u) {
        const uint32_t kb = k0 / 32u + g;
        i32x8 wf[4];
        int ws[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            wf[j] = load_fp4_frag(w_row[j], k0, g);
            ws[j] = (int)gload(w_scl[j] + kb);
        }
        i32x8 af[TERMS][WM];
        int as[TERMS][WM];
#pragma unroll
        for (int t = 0; t < TERMS; t++)
#pragma unroll
            for (int i = 0; i < WM; i++) {
                af[t][i] = load_fp8_frag(a_row[t][i], k0, g);
                as[t][i] = (int)gload(a_scl[t][i] + kb);
            }
#pragma unroll
        for (int t = 0; t < TERMS; t++)
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        af[t][i], wf[j], acc[i][j], 0, 4, 0, as[t][i], 0, ws[j]);
    }
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

/* grid (F / 128, tile cap), block 256. Wave w: gate and up rows
 * f0 + 32 w .. + 32 (n-subtiles 0, 1 = gate, 2, 3 = up). */
template <int WM, int TERMS>
__global__ __launch_bounds__(256) void gateup_mfma_kernel(GateUpArgs A) {
    const uint32_t tile = blockIdx.y;
    if (tile >= *A.tile_count) return;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t g = lane >> 4, c = lane & 15u;
    const uint32_t e = A.tiles[3u * tile], row0 = A.tiles[3u * tile + 1u];
    const uint32_t rows = A.tiles[3u * tile + 2u];
    const uint32_t H = A.H, F = A.F;
    const k3_moe_expert ex = A.experts[e];
    const uint32_t f0 = blockIdx.x * 128u + 32u * wave;

    const uint8_t *w_row[4], *w_scl[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t f = f0 + 16u * (uint32_t)(j & 1) + c;
        const uint8_t *p = (const uint8_t *)(j < 2 ? ex.gate_packed : ex.up_packed);
        const uint8_t *s = (const uint8_t *)(j < 2 ? ex.gate_scales : ex.up_scales);
        w_row[j] = p + (uint64_t)f * (H / 2u);
        w_scl[j] = s + (uint64_t)f * (H / 32u);
    }
    const uint8_t *a_row[TERMS][WM], *a_scl[TERMS][WM];
#pragma unroll
    for (int i = 0; i < WM; i++) {
        const uint32_t r = 16u * i + c;
        const uint32_t tok = A.token_index[row0 + (r < rows ? r : 0u)];
#pragma unroll
        for (int t = 0; t < TERMS; t++) {
            a_row[t][i] = A.B.xq[t] + (uint64_t)tok * H;
            a_scl[t][i] = A.B.xs[t] + (uint64_t)tok * (H / 32u);
        }
    }
    f32x4 acc[WM][4];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    mfma_rows<WM, TERMS>(acc, a_row, a_scl, w_row, w_scl, H, g);

    /* epilogue: activation, then the MXFP8 split of each row's 32-column
     * block (columns f0 .. f0 + 31 live in the 16 lanes of this g, two
     * subtiles each) */
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t lr = 16u * i + 4u * g + (uint32_t)r;
            float v[2];
#pragma unroll
            for (int j = 0; j < 2; j++)
                v[j] = bf16r(gated_act(bf16r(acc[i][j][r]), bf16r(acc[i][j + 2][r]), A.kind,
                                       A.beta, A.lb));
            const uint64_t prow = (uint64_t)row0 + (lr < rows ? lr : 0u);
#pragma unroll
            for (int t = 0; t < TERMS; t++) {
                float amax = fmaxf(fabsf(v[0]), fabsf(v[1]));
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
                const uint32_t sb = mx8_scale_byte(amax);
                const float inv = mx8_inv_scale(sb), sc = e8m0_to_f32(sb);
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const uint32_t code = f32_to_e4m3(__fmul_rn(v[j], inv));
                    if (lr < rows) A.B.aq[t][prow * F + f0 + 16u * j + c] = (uint8_t)code;
                    if (TERMS == 2 && t == 0)
                        v[j] = __fsub_rn(v[j], __fmul_rn(e4m3_to_f32(code), sc));
                }
                if (lr < rows && c == 0u) A.B.as[t][prow * (F / 32u) + f0 / 32u] = (uint8_t)sb;
            }
        }
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

/* grid (H / 256, tile cap), block 256. Wave w: down rows d0 + 64 w .. + 64. */
template <int WM, int TERMS>
__global__ __launch_bounds__(256) void down_mfma_kernel(DownArgs A) {
    const uint32_t tile = blockIdx.y;
    if (tile >= *A.tile_count) return;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t g = lane >> 4, c = lane & 15u;
    const uint32_t e = A.tiles[3u * tile], row0 = A.tiles[3u * tile + 1u];
    const uint32_t rows = A.tiles[3u * tile + 2u];
    const uint32_t H = A.H, F = A.F;
    const k3_moe_expert ex = A.experts[e];
    const uint32_t d0 = blockIdx.x * 256u + 64u * wave;

    const uint8_t *w_row[4], *w_scl[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t d = d0 + 16u * j + c;
        w_row[j] = (const uint8_t *)ex.down_packed + (uint64_t)d * (F / 2u);
        w_scl[j] = (const uint8_t *)ex.down_scales + (uint64_t)d * (F / 32u);
    }
    const uint8_t *a_row[TERMS][WM], *a_scl[TERMS][WM];
#pragma unroll
    for (int i = 0; i < WM; i++) {
        const uint32_t r = 16u * i + c;
        const uint64_t prow = (uint64_t)row0 + (r < rows ? r : 0u);
#pragma unroll
        for (int t = 0; t < TERMS; t++) {
            a_row[t][i] = A.B.aq[t] + prow * F;
            a_scl[t][i] = A.B.as[t] + prow * (F / 32u);
        }
    }
    f32x4 acc[WM][4];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    mfma_rows<WM, TERMS>(acc, a_row, a_scl, w_row, w_scl, F, g);
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t lr = 16u * i + 4u * g + (uint32_t)r;
            if (lr >= rows) continue;
            const uint64_t route = A.route_index[row0 + lr];
#pragma unroll
            for (int j = 0; j < 4; j++)
                A.y[route * H + d0 + 16u * j + c] = f32_to_bf16(acc[i][j][r]);
        }
}

template <int TERMS>
bool launch_terms(const MfmaBuffers &B, uint16_t *y, const uint16_t *hidden,
                  const uint32_t *counts, const uint32_t *offsets, const uint32_t *token_index,
                  const uint32_t *route_index, const k3_moe_expert *experts, const k3_moe_shape &s,
                  uint32_t T, hipStream_t st, const StageMarker &mark) {
    const uint32_t H = s.hidden, F = s.ffn;
    const uint64_t blocks = (uint64_t)T * H / 32u;
    hipLaunchKernelGGL(HIP_KERNEL_NAME(x_split_kernel<TERMS>), dim3((uint32_t)((blocks + 255u) / 256u)),
                       dim3(256), 0, st, B, hidden, blocks);
    hipLaunchKernelGGL(tile_build_kernel, dim3(1), dim3(1024), 0, st, B, counts, offsets,
                       s.expert_count);
    mark(K3_MOE_STAGE_GATE_UP);
    GateUpArgs ga{B, nullptr, nullptr, token_index, experts, H, F, s.activation,
                  s.activation == 1u ? 1.0f : s.beta, s.activation == 1u ? 1.0f : s.linear_beta};
    DownArgs da{B, nullptr, nullptr, route_index, experts, y, H, F};
    uint32_t base = 0u;
    const uint32_t *tl[3];
    for (int c = 0; c < 3; c++) {
        tl[c] = B.tiles + 3u * base;
        base += B.tile_cap[c];
    }
    for (int c = 0; c < 3; c++) {
        if (!B.tile_cap[c]) continue;
        ga.tiles = tl[c];
        ga.tile_count = B.tile_count + c;
        const dim3 grid(F / 128u, B.tile_cap[c]);
        if (c == 0) hipLaunchKernelGGL(HIP_KERNEL_NAME(gateup_mfma_kernel<1, TERMS>), grid, dim3(256), 0, st, ga);
        if (c == 1) hipLaunchKernelGGL(HIP_KERNEL_NAME(gateup_mfma_kernel<2, TERMS>), grid, dim3(256), 0, st, ga);
        if (c == 2) hipLaunchKernelGGL(HIP_KERNEL_NAME(gateup_mfma_kernel<4, TERMS>), grid, dim3(256), 0, st, ga);
    }
    mark(K3_MOE_STAGE_DOWN);
    for (int c = 0; c < 3; c++) {
        if (!B.tile_cap[c]) continue;
        da.tiles = tl[c];
        da.tile_count = B.tile_count + c;
        const dim3 grid(H / 256u, B.tile_cap[c]);
        if (c == 0) hipLaunchKernelGGL(HIP_KERNEL_NAME(down_mfma_kernel<1, TERMS>), grid, dim3(256), 0, st, da);
        if (c == 1) hipLaunchKernelGGL(HIP_KERNEL_NAME(down_mfma_kernel<2, TERMS>), grid, dim3(256), 0, st, da);
        if (c == 2) hipLaunchKernelGGL(HIP_KERNEL_NAME(down_mfma_kernel<4, TERMS>), grid, dim3(256), 0, st, da);
    }
    return hipGetLastError() == hipSuccess;
}

}  // namespace

void mfma_tile_caps(uint32_t T, uint32_t k, uint32_t E, uint32_t caps[3]) {
    const uint64_t R = (uint64_t)T * k;
    caps[0] = (uint32_t)(R < E ? R : E);
    caps[1] = (uint32_t)(R / 17u < E ? R / 17u : E);
    caps[2] = (uint32_t)(R / 64u + (R / 33u < E ? R / 33u : E));
}

bool mfma_supported(const k3_moe_shape &s) {
    return s.hidden % 256u == 0u && s.ffn % 128u == 0u && s.expert_count <= 1024u;
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
