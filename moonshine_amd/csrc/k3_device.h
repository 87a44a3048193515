/*
 * Device helpers shared by the gfx950 kernels of libk3moe.
 *
 * Numerics contract: every floating-point step below is written out (fmaf,
 * separately rounded mul/add; the library is compiled with
 * -ffp-contract=off), so the fixed "w64" reduction orders produce the same
 * bits as the CPU oracle that restates them.
 */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace k3 {

constexpr uint32_t kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
    return __uint_as_float((uint32_t)v << 16);
}
__device__ __forceinline__ float bf16_lo(uint32_t w) {
    return __uint_as_float(w << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t w) {
    return __uint_as_float(w & 0xffff0000u);
}

/* Global-address-space view of a pointer that came from memory (expert
 * tables): lets the compiler emit global_load with a scalar base instead of
 * flat_load with 64-bit per-lane addresses. */
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 gload(const uint4 *p) {
    const u32x4_t v = *(const __attribute__((address_space(1))) u32x4_t *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
/* 16 packed bytes at p: one 16-byte load when p is 16-byte aligned, two
 * 8-byte loads for the 8-mod-16 starts of real checkpoint spans
 * (k3_rocm_ops.cu:207-223). a16 is block-uniform. */
__device__ __forceinline__ uint4 gload16(const uint8_t *p, bool a16) {
    if (a16) return gload((const uint4 *)p);
    const uint2 lo = ((const uint2 *)p)[0], hi = ((const uint2 *)p)[1];
    return make_uint4(lo.x, lo.y, hi.x, hi.y);
}
/* Streaming forms for weights read once per call (decode): the
 * non-temporal hint keeps a layer's ~0.4 GB expert stream from allocating
 * in the L2 and the last-level cache (measured: decode layer 84.6 -> 80.5
 * us). */
__device__ __forceinline__ uint4 gload_nt(const uint4 *p) {
    const u32x4_t v = __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4_t *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 gload16_nt(const uint8_t *p, bool a16) {
    if (a16) return gload_nt((const uint4 *)p);
    typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
    const __attribute__((address_space(1))) u32x2_t *q = (const __attribute__((address_space(1))) u32x2_t *)p;
    const u32x2_t lo = __builtin_nontemporal_load(q), hi = __builtin_nontemporal_load(q + 1);
    return make_uint4(lo.x, lo.y, hi.x, hi.y);
}
__device__ __forceinline__ uint32_t gload_nt(const uint32_t *p) {
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) uint32_t *)p);
}
__device__ __forceinline__ uint32_t gload(const uint8_t *p) {
    return *(const __attribute__((address_space(1))) uint8_t *)p;
}

/* Round to nearest even; NaN stays a quiet NaN (hip_bfloat16 semantics). */
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t nan = (u >> 16) | 0x40u, rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    return (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? nan : rne); /* a select, no branch */
}

/* OCP E8M0 as the reference decodes it: 2^(e-127); 0 -> 2^-127 (bit pattern
 * 0x00400000), 255 -> +inf. */
__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
    return __uint_as_float(e == 0u ? 0x00400000u : (e & 0xffu) << 23);
}

/*
 * Deterministic exp (Cody-Waite reduction with a two-part ln2, degree-7
 * Taylor polynomial by Horner with fmaf, exact two-step power-of-two
 * scaling). The CPU oracle evaluates the same sequence.
 */
__device__ __forceinline__ float det_expf(float x) {
    /* the polynomial runs on x clamped into range (x itself wherever its
     * value is used) and the special cases are selected at the end, so the
     * sequence has no branches */
    const float xc = fminf(fmaxf(x, -104.0f), 89.0f);
    const float n = rintf(__fmul_rn(xc, 1.44269502162933349609375f));
    float r = fmaf(-n, 0.693145751953125f, xc);
    r = fmaf(-n, 1.428606765330187045037746429443359375e-6f, r);
    float p = 1.9841270113736391067504882812e-4f;
    p = fmaf(p, r, 1.3888889225199818611145019531e-3f);
    p = fmaf(p, r, 8.3333337679505348205566406250e-3f);
    p = fmaf(p, r, 4.1666667908430099487304687500e-2f);
    p = fmaf(p, r, 1.6666667163372039794921875000e-1f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int ni = (int)n;
    const int a = ni / 2;
    const int b = ni - a;
    const float e = __fmul_rn(__fmul_rn(p, __uint_as_float((uint32_t)(a + 127) << 23)),
                              __uint_as_float((uint32_t)(b + 127) << 23));
    const float big = x > 88.72283935546875f ? __builtin_huge_valf() : e;
    const float out = x < -103.97208404541015625f ? 0.0f : big;
    return x != x ? x : out;
}

__device__ __forceinline__ float det_tanhf(float y) {
    if (y != y) return y;
    const float a = fabsf(y);
    float r;
    if (a < 0.5f) {
        const float z = __fmul_rn(a, a);
        float p = -1.4558343870513183e-3f;
        p = fmaf(p, z, 3.5921280365724811e-3f);
        p = fmaf(p, z, -8.8632355299021966e-3f);
        p = fmaf(p, z, 2.1869488536155203e-2f);
        p = fmaf(p, z, -5.3968253968253968e-2f);
        p = fmaf(p, z, 1.3333333333333333e-1f);
        p = fmaf(p, z, -3.3333333333333333e-1f);
        r = fmaf(__fmul_rn(a, z), p, a);
    } else if (a < 9.1f) {
        const float e = det_expf(__fadd_rn(a, a));
        r = __fsub_rn(1.0f, __fdiv_rn(2.0f, __fadd_rn(e, 1.0f)));
    } else {
        r = 1.0f;
    }
    return copysignf(r, y);
}

__device__ __forceinline__ float det_sigmoid(float x) {
    return __fdiv_rn(1.0f, __fadd_rn(1.0f, det_expf(-x)));
}

/*
 * The router's choice sigmoid, evaluated with exactly the operations the
 * reference's score = 1.0f / (1.0f + expf(-logit)) (k3_rocm_ops.cu:1386)
 * becomes for gfx950 under its -ffast-math -fno-finite-math-only build:
 * t = -logit * log2(e) rounded to fp32, e = v_exp_f32(t) (2^t), 1 + e
 * rounded, v_rcp_f32; for logit > 87.33654 (where 2^t would be subnormal)
 * the input is first lowered by 64 and e scaled back by e^-64 (0x114b4ea4).
 * The expert ids depend on these bits (choice = score + bias): the same
 * instructions give the reference's ids bit for bit, including its
 * near-ties. v_exp_f32 and v_rcp_f32 are within 1 ulp; the result is
 * within 3e-7 of the real sigmoid (pinned by an exhaustive sweep on the
 * part). Route weights use det_sigmoid instead (pinned bit for bit by the
 * CPU oracle; within 1e-6 of the reference's weights).
 */
__device__ __forceinline__ float router_sigmoid(float x) {
    const bool big = x > __uint_as_float(0x42aeac50u);          /* 87.33654 */
    const float t = big ? __fadd_rn(x, -64.0f) : x;
    float e = __builtin_amdgcn_exp2f(__fmul_rn(t, __uint_as_float(0xbfb8aa3bu)));  /* -log2 e */
    if (big) e = __fmul_rn(e, __uint_as_float(0x114b4ea4u));   /* e^-64 */
    return __builtin_amdgcn_rcpf(__fadd_rn(1.0f, e));
}

/* Gated activations on bf16-rounded gate/up values. kind 0 = SiTU(beta, lb)
 * (k3_rocm_ops.cu:66-83), kind 1 = SwiGLU g*sigmoid(g)*u. */
__device__ __forceinline__ float gated_act(float g, float u, uint32_t kind,
                                           float beta, float lb) {
    if (kind == 1u) return __fmul_rn(__fmul_rn(g, det_sigmoid(g)), u);
    const float bg = __fmul_rn(beta, det_tanhf(__fdiv_rn(g, beta)));
    const float bu = __fmul_rn(lb, det_tanhf(__fdiv_rn(u, lb)));
    return __fmul_rn(__fmul_rn(bg, det_sigmoid(g)), bu);
}

/* Two e2m1 values of byte `sel` of `w` as fp32, unscaled (exact). */
template <int Sel>
__device__ __forceinline__ float2 fp4x2(uint32_t w) {
    auto v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, Sel);
    return make_float2(v[0], v[1]);
}

/*
 * Sum of 8 e2m1*x products of one packed u32 (8 nibbles, low nibble = even
 * column) against 8 fp32 activations, accumulated into gs in column order.
 */
__device__ __forceinline__ float fp4_dot8(uint32_t w, const float *x, float gs) {
    float2 a = fp4x2<0>(w), b = fp4x2<1>(w), c = fp4x2<2>(w), d = fp4x2<3>(w);
    gs = fmaf(a.x, x[0], gs); gs = fmaf(a.y, x[1], gs);
    gs = fmaf(b.x, x[2], gs); gs = fmaf(b.y, x[3], gs);
    gs = fmaf(c.x, x[4], gs); gs = fmaf(c.y, x[5], gs);
    gs = fmaf(d.x, x[6], gs); gs = fmaf(d.y, x[7], gs);
    return gs;
}

/* Group partial of one 16-byte (32 column) MXFP4 group. */
__device__ __forceinline__ float fp4_group(uint4 w, const float *x) {
    float gs = 0.0f;
    gs = fp4_dot8(w.x, x, gs);
    gs = fp4_dot8(w.y, x + 8, gs);
    gs = fp4_dot8(w.z, x + 16, gs);
    gs = fp4_dot8(w.w, x + 24, gs);
    return gs;
}

/* Unpack 32 bf16 (four uint4) to fp32. */
__device__ __forceinline__ void bf16x32_to_f32(const uint4 *src, float *x) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const uint4 v = src[q];
        x[8 * q + 0] = bf16_lo(v.x); x[8 * q + 1] = bf16_hi(v.x);
        x[8 * q + 2] = bf16_lo(v.y); x[8 * q + 3] = bf16_hi(v.y);
        x[8 * q + 4] = bf16_lo(v.z); x[8 * q + 5] = bf16_hi(v.z);
        x[8 * q + 6] = bf16_lo(v.w); x[8 * q + 7] = bf16_hi(v.w);
    }
}

/* Wave64 butterfly: v = v + v(lane ^ o) for o = 32 .. 1 (all lanes end
 * with the same value). Matches the oracle's butterfly64. */
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = __fadd_rn(v, __shfl_xor(v, o, 64));
    return v;
}

/*
 * Reduce N per-lane partials (N a power of two, <= 64) over the wave in one
 * transpose-reduce: at stage o each lane keeps half of its rows and adds
 * the partner's copy. Every row ends up with exactly the butterfly64 value
 * (same pairings, fp32 add is commutative). Which row a lane holds at the
 * end is given by wave_rows_owner<N>(). All indices are compile-time.
 */
template <int N, int O>
struct RowReduce {
    static __device__ __forceinline__ float run(float *p, int lane) {
        if constexpr (O == 0) {
            return p[0];
        } else if constexpr (N > 1) {
            constexpr int H = N / 2;
            const bool upper = (lane & O) != 0;
#pragma unroll
            for (int i = 0; i < H; i++) {
                const float send = upper ? p[i] : p[i + H];
                const float keep = upper ? p[i + H] : p[i];
                p[i] = __fadd_rn(keep, __shfl_xor(send, O, 64));
            }
            return RowReduce<H, O / 2>::run(p, lane);
        } else {
            float v = p[0];
#pragma unroll
            for (int o = O; o >= 1; o >>= 1) v = __fadd_rn(v, __shfl_xor(v, o, 64));
            return v;
        }
    }
};

template <int N>
__device__ __forceinline__ float wave_sum_rows(float (&p)[N]) {
    static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "N must be a power of two <= 64");
    return RowReduce<N, 32>::run(p, (int)(threadIdx.x & 63u));
}

/* Which row of wave_sum_rows<N> a lane holds at the end. */
template <int N>
__device__ __forceinline__ int wave_rows_owner() {
    const int lane = threadIdx.x & 63;
    int row = 0;
    int n = N;
    for (int o = 32; n > 1; o >>= 1) {
        n /= 2;
        if (lane & o) row += n;
    }
    return row;
}

/* ---- router logits in the reference's order ------------------------------ */

/*
 * k3_bf16_gemv_kernel<float> and the tiled GEMM's quad path
 * (k3_rocm_ops.cu:359-425, 512-661): 256 threads, thread t sums the 4-element
 * quads t, t + 256, ... into its partial, then an LDS tree 128 -> 1. The
 * reference is built with -ffast-math; hipcc (ROCm 7.2, gfx950) turns the
 * quad expression into v_pk_mul_f32 (w2 x2, w3 x3), v_pk_fma_f32 (w1 x1 +
 * w2 x2, w0 x0 + w3 x3) and two adds, so a quad adds (p1 + p2) + (p0 + p3)
 * to the partial, every step rounded to fp32. The products are exact (bf16
 * x bf16), so each multiply here rounds nothing it does not round there.
 */
__device__ __forceinline__ float ref_quad(uint32_t wlo, uint32_t whi, uint32_t xlo,
                                          uint32_t xhi) {
    const float p2 = __fmul_rn(bf16_lo(whi), bf16_lo(xhi));
    const float p3 = __fmul_rn(bf16_hi(whi), bf16_hi(xhi));
    const float a = fmaf(bf16_hi(wlo), bf16_hi(xlo), p2);
    const float b = fmaf(bf16_lo(wlo), bf16_lo(xlo), p3);
    return __fadd_rn(a, b);
}

/* 16-byte chunk c = lane + 64 j of a row: its quads 2c and 2c + 1 belong to
 * the reference's partials 2 lane + 128 (j & 1) and that + 1 (the quads of
 * a partial arrive in j order, as its thread adds them), kept in
 * acc[2 (j & 1)] and acc[2 (j & 1) + 1]. */
__device__ __forceinline__ void ref_chunk(float (&acc)[4], int j, uint4 w, uint4 x) {
    const int s = 2 * (j & 1);
    acc[s] = __fadd_rn(acc[s], ref_quad(w.x, w.y, x.x, x.y));
    acc[s + 1] = __fadd_rn(acc[s + 1], ref_quad(w.z, w.w, x.z, x.w));
}

/* The reference's tree over the four partials of every lane (ref_chunk):
 * level 128 adds acc[0] + acc[2] and acc[1] + acc[3] (partials t and t +
 * 128) in the lane; levels 64 .. 2 pair partials 2 lane and 2 lane + 2^k,
 * i.e. lanes lane ^ 32 .. lane ^ 1 (a wave64 butterfly of each); level 1
 * adds the lane's two results. Every lane returns the logit. */
__device__ __forceinline__ float ref_logit_finish(const float (&acc)[4]) {
    const float r0 = wave_sum(__fadd_rn(acc[0], acc[2]));
    const float r1 = wave_sum(__fadd_rn(acc[1], acc[3]));
    return __fadd_rn(r0, r1);
}

/* ---- MXFP8 (E4M3 codes + E8M0 block scales) ------------------------------ */

/* floor(log2(a)) of a finite a > 0 (normal or subnormal). */
__device__ __forceinline__ int ilog2_pos(float a) {
    const uint32_t u = __float_as_uint(a);
    const int e = (int)((u >> 23) & 255u);
    if (e) return e - 127;
    return (31 - __clz((int)(u & 0x7fffffu))) - 149;
}

/* OCP E4M3 decode (bias 7, subnormal step 2^-9, S.1111.111 = NaN). */
__device__ __forceinline__ float e4m3_to_f32(uint32_t v) {
    const uint32_t e = (v >> 3) & 15u, m = v & 7u;
    float mag;
    if (e == 15u && m == 7u) mag = __uint_as_float(0x7fc00000u);
    else if (e) mag = __uint_as_float(((e + 120u) << 23) | (m << 20));
    else mag = __fmul_rn((float)m, 0.001953125f);
    return (v & 0x80u) ? -mag : mag;
}

/* fp32 -> E4M3, round to nearest even, magnitude clamped to 448, NaN ->
 * 0x7f (the same steps as the CPU oracle's conversion). */
__device__ __forceinline__ uint32_t f32_to_e4m3(float v) {
    if (v != v) return 0x7fu;
    const uint32_t sign = (__float_as_uint(v) >> 31) << 7;
    float a = fabsf(v);
    if (a > 448.0f) a = 448.0f;
    if (a < 0.015625f) return sign | (uint32_t)rintf(__fmul_rn(a, 512.0f));
    const int e = (int)((__float_as_uint(a) >> 23) & 255u) - 127;
    const float m = __fmul_rn(a, __uint_as_float((uint32_t)(127 - e) << 23));
    int mant = (int)rintf(__fmul_rn(__fsub_rn(m, 1.0f), 8.0f));
    int ee = e;
    if (mant == 8) { mant = 0; ee++; }
    return sign | (uint32_t)(((ee + 7) << 3) | mant);
}

/* Two values to E4M3 codes in bytes 2 Hi .. 2 Hi + 1 of `old` (the other
 * half kept), by the part's round-to-nearest-even conversion: f32_to_e4m3's
 * codes for every input. Magnitudes are clamped to 448 first (only +-inf
 * exceeds it after MXFP8 scaling) and NaN inputs are mapped to 0x7f, as
 * f32_to_e4m3 does; the conversion itself is pinned against the CPU
 * encoder over every bf16 value within +-448, which covers every input the
 * MXFP8 split produces (bf16 values scaled by powers of two, and their
 * residuals). */
template <bool Hi>
__device__ __forceinline__ uint32_t e4m3x2(float a, float b, uint32_t old) {
    const float ac = fminf(fmaxf(a, -448.0f), 448.0f), bc = fminf(fmaxf(b, -448.0f), 448.0f);
    uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ac, bc, (int)old, Hi);
    constexpr int sa = Hi ? 16 : 0;
    if (a != a) w = (w & ~(0xffu << sa)) | (0x7fu << sa);
    if (b != b) w = (w & ~(0xffu << (sa + 8))) | (0x7fu << (sa + 8));
    return w;
}

/* e4m3x2 without the clamp and the NaN mapping, for encoders whose inputs
 * are finite (within +-448 after scaling) or whose non-finite inputs only
 * need to decode as NaN (an E4M3 NaN code, 0x7f or 0xff, may result). */
template <bool Hi>
__device__ __forceinline__ uint32_t e4m3x2_raw(float a, float b, uint32_t old) {
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int)old, Hi);
}

/* Two values rounded to bf16 (nearest even) by the part's packed
 * conversion, back as fp32; f32_to_bf16's values except that a NaN's
 * payload is not specified. */
__device__ __forceinline__ float2 bf16r2(float a, float b) {
    typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
    typedef float f32x2_v __attribute__((ext_vector_type(2)));
    const uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_v{a, b}, bf16x2_v));
    return make_float2(__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u));
}

/* Byte Sel of w as E4M3, decoded exactly (e4m3_to_f32's values). */
template <int Sel>
__device__ __forceinline__ float e4m3_byte(uint32_t w) {
    return __builtin_amdgcn_cvt_f32_fp8((int)w, Sel);
}

/* DPP lane read within a 16-lane row (all lanes active). */
template <int Ctrl>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), Ctrl, 0xf, 0xf, false));
}

/* Maximum over each aligned group of N lanes (N = 8 or 16) of a 16-lane
 * row, returned to every lane of the group: swaps of neighbours and of
 * pairs, then the mirror inside 8 lanes and (N = 16) inside the row.
 * fmaxf ignores NaN, so the result does not depend on the order. */
template <int N>
__device__ __forceinline__ float row_group_max(float v) {
    static_assert(N == 8 || N == 16, "8- or 16-lane groups");
    v = fmaxf(v, dpp_f<0xb1>(v));  /* quad_perm [1,0,3,2] */
    v = fmaxf(v, dpp_f<0x4e>(v));  /* quad_perm [2,3,0,1] */
    v = fmaxf(v, dpp_f<0x141>(v)); /* row_half_mirror */
    if constexpr (N == 16) v = fmaxf(v, dpp_f<0x140>(v)); /* row_mirror */
    return v;
}

/* Block exponent for MXFP8: floor(log2(amax)) - 8, plus one when the
 * maximum would exceed 448 after scaling, clamped to >= -127; -127 for an
 * all-zero block. Returns the scale byte (X + 127). */
__device__ __forceinline__ uint32_t mx8_scale_byte(float amax) {
    /* for a normal amax = 1.m 2^(e - 127): X = e - 135, and amax 2^-X =
     * 256 x 1.m exceeds 448 exactly when 1.m > 1.75 (mantissa field above
     * 0x600000), or for +inf; zero, subnormal and amax < 2^-119 clamp to
     * X = -127, i.e. byte 0 (branch-free) */
    const uint32_t u = __float_as_uint(amax);
    const int e = (int)((u >> 23) & 255u);
    const int b = e - 8 + (((u & 0x7fffffu) > 0x600000u || e == 255) ? 1 : 0);
    return amax > 0.0f && b > 0 ? (uint32_t)b : 0u;
}

/* 2^-(byte - 127) as the multiplier applied before rounding to E4M3. */
__device__ __forceinline__ float mx8_inv_scale(uint32_t byte) {
    return __uint_as_float((254u - byte) << 23);
}

}  // namespace k3
