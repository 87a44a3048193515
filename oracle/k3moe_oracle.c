/*
 * k3moe_oracle.c — CPU restatement of Moonshine's routed-MoE layer.
 * TEST INFRASTRUCTURE ONLY (see k3moe_oracle.h). Built with
 * -ffp-contract=off and without -ffast-math so every rounding is the one
 * written here.
 */
#include "k3moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* scalars                                                                   */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* bf16 <-> f32: hip_bfloat16 semantics (round to nearest even, NaN kept
 * quiet), as used by the reference via k3_float_to_bf16 (k3_rocm_ops.cu:36-39). */
float k3o_bf16_to_f32(uint16_t v) { return u2f((uint32_t)v << 16); }

uint16_t k3o_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* e2m1: {0, .5, 1, 1.5, 2, 3, 4, 6}, bit 3 = sign (k3_rocm_ops.cu:185-191). */
float k3o_e2m1(uint8_t nibble) {
    static const float magnitude[8] = {0.0f, 0.5f, 1.0f, 1.5f,
                                       2.0f, 3.0f, 4.0f, 6.0f};
    const float v = magnitude[nibble & 7u];
    return (nibble & 8u) ? -v : v;
}

/* e8m0: 2^(e-127); e = 0 gives the bit pattern 0x00400000 (2^-127) and
 * e = 255 gives +inf, exactly as k3_rocm_ops.cu:179-183. */
float k3o_e8m0(uint8_t e) {
    return u2f(e == 0u ? 0x00400000u : (uint32_t)e << 23);
}

/*
 * Deterministic exp: Cody-Waite reduction x = n ln2 + r with a two-part ln2,
 * then the degree-7 Taylor polynomial of e^r on |r| <= ln2/2 evaluated by
 * Horner with fmaf, then an exact two-step power-of-two scaling. The HIP
 * kernels evaluate the identical sequence, so sigmoid scores (and therefore
 * routing) agree bit for bit. Accuracy vs glibc expf is pinned in tests.
 */
float k3o_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -103.97208404541015625f) return 0.0f;
    const float n = rintf(x * 1.44269502162933349609375f);
    float r = fmaf(-n, 0.693145751953125f, x);
    r = fmaf(-n, 1.428606765330187045037746429443359375e-6f, r);
    float p = 1.9841270113736391067504882812e-4f;        /* 1/7! */
    p = fmaf(p, r, 1.3888889225199818611145019531e-3f);  /* 1/6! */
    p = fmaf(p, r, 8.3333337679505348205566406250e-3f);  /* 1/5! */
    p = fmaf(p, r, 4.1666667908430099487304687500e-2f);  /* 1/4! */
    p = fmaf(p, r, 1.6666667163372039794921875000e-1f);  /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int ni = (int)n;
    const int a = ni / 2;
    const int b = ni - a;
    return (p * u2f((uint32_t)(a + 127) << 23)) * u2f((uint32_t)(b + 127) << 23);
}

/* Deterministic tanh: odd Taylor series through a^15 for |a| < 0.5, else
 * 1 - 2/(e^{2a}+1) with k3o_expf, saturating to 1 for |a| >= 9.1. */
float k3o_tanhf(float y) {
    if (y != y) return y;
    const float a = fabsf(y);
    float r;
    if (a < 0.5f) {
        const float z = a * a;
        float p = -1.4558343870513183e-3f;     /* -929569/638512875 */
        p = fmaf(p, z, 3.5921280365724811e-3f);  /*  21844/6081075 */
        p = fmaf(p, z, -8.8632355299021966e-3f); /* -1382/155925 */
        p = fmaf(p, z, 2.1869488536155203e-2f);  /*  62/2835 */
        p = fmaf(p, z, -5.3968253968253968e-2f); /* -17/315 */
        p = fmaf(p, z, 1.3333333333333333e-1f);  /*  2/15 */
        p = fmaf(p, z, -3.3333333333333333e-1f); /* -1/3 */
        r = fmaf(a * z, p, a);
    } else if (a < 9.1f) {
        const float e = k3o_expf(a + a);
        r = 1.0f - 2.0f / (e + 1.0f);
    } else {
        r = 1.0f;
    }
    return copysignf(r, y);
}

float k3o_sigmoid(float x, int use_libm) {
    return 1.0f / (1.0f + (use_libm ? expf(-x) : k3o_expf(-x)));
}

/*
 * The router's choice sigmoid: the reference's 1/(1 + expf(-x))
 * (k3_rocm_ops.cu:1386) as its -ffast-math build evaluates it on gfx950
 * (t = x * -log2(e) in fp32, 2^t, 1 + 2^t, reciprocal; inputs above
 * 87.33654 lowered by 64 first and 2^t scaled back by e^-64). The device
 * uses the hardware exp2 and reciprocal instructions, which are within 1 ulp
 * but not correctly rounded; this restatement rounds both correctly (fp64
 * then fp32), so it equals the device except where an instruction is off
 * by its ulp (measured on the part: about 1 in 70 exp2 and 1 in 9
 * reciprocal inputs). Choices, and therefore ids, agree except at near-ties
 * within those ulps; the route weights use k3o_sigmoid(x, 0), bit-exact.
 */
float k3o_router_sigmoid(float x) {
    const int big = x > u2f(0x42aeac50u);                 /* 87.33654 */
    const float t = big ? x + -64.0f : x;
    float e = (float)exp2((double)(t * u2f(0xbfb8aa3bu))); /* -log2 e */
    if (big) e = e * u2f(0x114b4ea4u);                    /* e^-64 */
    return (float)(1.0 / (double)(1.0f + e));
}

/* ------------------------------------------------------------------------ */
/* activations                                                               */
/* ------------------------------------------------------------------------ */

/* SiTU, k3_rocm_ops.cu:66-83: bf16((beta*tanh(g/beta) * sigmoid(g)) *
 * (lb*tanh(u/lb))), left to right. */
void k3o_situ(uint16_t *out, const uint16_t *gate, const uint16_t *up,
              uint64_t n, float beta, float lb, int use_libm) {
    for (uint64_t i = 0; i < n; i++) {
        const float g = k3o_bf16_to_f32(gate[i]);
        const float u = k3o_bf16_to_f32(up[i]);
        const float tg = use_libm ? tanhf(g / beta) : k3o_tanhf(g / beta);
        const float tu = use_libm ? tanhf(u / lb) : k3o_tanhf(u / lb);
        const float bounded_gate = beta * tg;
        const float sig = k3o_sigmoid(g, use_libm);
        const float bounded_up = lb * tu;
        out[i] = k3o_f32_to_bf16((bounded_gate * sig) * bounded_up);
    }
}

/* SwiGLU, the beta, lb -> inf limit of SiTU: bf16((g * sigmoid(g)) * u). */
void k3o_swiglu(uint16_t *out, const uint16_t *gate, const uint16_t *up,
                uint64_t n, int use_libm) {
    for (uint64_t i = 0; i < n; i++) {
        const float g = k3o_bf16_to_f32(gate[i]);
        const float u = k3o_bf16_to_f32(up[i]);
        out[i] = k3o_f32_to_bf16((g * k3o_sigmoid(g, use_libm)) * u);
    }
}

/* ------------------------------------------------------------------------ */
/* reductions                                                                */
/* ------------------------------------------------------------------------ */

/* Wave64 butterfly: stage o replaces lane l by lane[l] + lane[l ^ o] for
 * o = 32, 16, 8, 4, 2, 1 (what __shfl_xor does); returns lane 0. */
static float butterfly64(float lane[64]) {
    float next[64];
    for (int o = 32; o >= 1; o >>= 1) {
        for (int l = 0; l < 64; l++) next[l] = lane[l] + lane[l ^ o];
        memcpy(lane, next, sizeof(next));
    }
    return lane[0];
}

/* LDS tree of the reference kernels: width = n/2 .. 1, p[t] += p[t+width]. */
static float tree_reduce(float *p, uint32_t n) {
    for (uint32_t w = n / 2u; w > 0; w /= 2u)
        for (uint32_t t = 0; t < w; t++) p[t] += p[t + w];
    return p[0];
}

/* ---- router logits ------------------------------------------------------ */

/* w64 order: elements in chunks of 8; lane l owns chunks l, l+64, ...;
 * acc = fmaf(w, x, acc) over each chunk in column order; butterfly64. */
static float logit_w64(const uint16_t *w, const uint16_t *x, uint32_t h) {
    float lane[64];
    const uint32_t chunks = (h + 7u) / 8u;
    for (uint32_t l = 0; l < 64u; l++) {
        float acc = 0.0f;
        for (uint32_t c = l; c < chunks; c += 64u)
            for (uint32_t i = 8u * c; i < 8u * c + 8u && i < h; i++)
                acc = fmaf(k3o_bf16_to_f32(w[i]), k3o_bf16_to_f32(x[i]), acc);
        lane[l] = acc;
    }
    return butterfly64(lane);
}

/* Reference order, k3_rocm_ops.cu:359-425 (and the tiled GEMM's quad path,
 * :512-661, which has the same per-row order): 256 lanes, lane j sums quads
 * j, j+256, ...; then the LDS tree 128 -> 1. The reference is built with
 * -ffast-math, so the order inside a quad is the one its compiler chose;
 * hipcc (ROCm 7.2, gfx950) emits, for the quad expression at :381-392,
 * v_pk_mul_f32 of (w2 x2, w3 x3), v_pk_fma_f32 giving (w1 x1 + w2 x2,
 * w0 x0 + w3 x3), then two adds: partial + ((p1 + p2) + (p0 + p3)), each
 * step rounded to fp32. The pair path (:395-405) adds p1 then p0; the
 * scalar path (:407-411) is one fmaf per element. */
static float logit_ref256(const uint16_t *w, const uint16_t *x, uint32_t h) {
    float p[256];
#define BF(a, i) k3o_bf16_to_f32((a)[i])
    for (uint32_t t = 0; t < 256u; t++) {
        float s = 0.0f;
        if ((h & 3u) == 0u) {
            for (uint32_t q = t; q < h / 4u; q += 256u) {
                const uint32_t i = 4u * q;
                const float p2 = BF(w, i + 2) * BF(x, i + 2);
                const float p3 = BF(w, i + 3) * BF(x, i + 3);
                const float a = fmaf(BF(w, i + 1), BF(x, i + 1), p2);
                const float b = fmaf(BF(w, i), BF(x, i), p3);
                s = s + (a + b);
            }
        } else if ((h & 1u) == 0u) {
            for (uint32_t q = t; q < h / 2u; q += 256u) {
                const uint32_t i = 2u * q;
                s = s + BF(w, i + 1) * BF(x, i + 1);
                s = s + BF(w, i) * BF(x, i);
            }
        } else {
            for (uint32_t i = t; i < h; i += 256u) s = fmaf(BF(w, i), BF(x, i), s);
        }
#undef BF
        p[t] = s;
    }
    return tree_reduce(p, 256u);
}

static float logit_f64(const uint16_t *w, const uint16_t *x, uint32_t h) {
    double s = 0.0;
    for (uint32_t i = 0; i < h; i++)
        s += (double)k3o_bf16_to_f32(w[i]) * (double)k3o_bf16_to_f32(x[i]);
    return (float)s;
}

void k3o_router_logits(float *logits, const uint16_t *weights,
                       const uint16_t *input, uint32_t tokens,
                       uint32_t experts, uint32_t hidden, int order) {
    k3o_bf16_gemm_f32(logits, weights, input, tokens, experts, hidden, order);
}

void k3o_bf16_gemm_f32(float *out, const uint16_t *weights,
                       const uint16_t *input, uint32_t vectors,
                       uint32_t rows, uint32_t columns, int order) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t t = 0; t < (int64_t)vectors; t++) {
        for (int64_t r = 0; r < (int64_t)rows; r++) {
            const uint16_t *w = weights + (uint64_t)r * columns;
            const uint16_t *x = input + (uint64_t)t * columns;
            float v;
            if (order == 0) v = logit_w64(w, x, columns);
            else if (order == 1) v = logit_ref256(w, x, columns);
            else v = logit_f64(w, x, columns);
            out[(uint64_t)t * rows + r] = v;
        }
    }
}

/* ---- router top-k ------------------------------------------------------- */

/*
 * k3_rocm_ops.cu:1361-1450 restated as the insertion-sort oracle of
 * tests/test_k3_moe_smoke.cu:215-253: choice = sigmoid(logit) + bias;
 * order (choice desc, id asc); weight_r = score_r / (1e-20 + sum of the k
 * selected scores in rank order) * scale with score = sigmoid(logit).
 * use_libm = 0 (the device model): the choice sigmoid is
 * k3o_router_sigmoid, the score sigmoid k3o_sigmoid(x, 0); use_libm = 1
 * (the reference's CPU oracle): glibc expf for both.
 */
int k3o_router_topk(uint32_t *ids, float *weights, const float *logits,
                    const float *bias, uint32_t tokens, uint32_t experts,
                    uint32_t top_k, float scale, int use_libm) {
    if (top_k == 0u || top_k > experts || top_k > 64u) return -1;
    for (uint32_t t = 0; t < tokens; t++) {
        float choice[64], raw[64];
        uint32_t id[64];
        for (uint32_t r = 0; r < top_k; r++) {
            choice[r] = -INFINITY; raw[r] = 0.0f; id[r] = UINT32_MAX;
        }
        const float *lg = logits + (uint64_t)t * experts;
        for (uint32_t e = 0; e < experts; e++) {
            const float s = k3o_sigmoid(lg[e], use_libm);
            const float c = (use_libm ? s : k3o_router_sigmoid(lg[e])) + bias[e];
            uint32_t pos = top_k;
            for (uint32_t r = 0; r < top_k; r++) {
                if (c > choice[r] || (c == choice[r] && e < id[r])) {
                    pos = r;
                    break;
                }
            }
            if (pos == top_k) continue;
            for (uint32_t r = top_k - 1u; r > pos; r--) {
                choice[r] = choice[r - 1u]; raw[r] = raw[r - 1u]; id[r] = id[r - 1u];
            }
            choice[pos] = c; raw[pos] = s; id[pos] = e;
        }
        float denominator = 1e-20f;
        for (uint32_t r = 0; r < top_k; r++) denominator += raw[r];
        for (uint32_t r = 0; r < top_k; r++) {
            ids[(uint64_t)t * top_k + r] = id[r];
            weights[(uint64_t)t * top_k + r] = raw[r] / denominator * scale;
        }
    }
    return 0;
}

/* ---- routing plan -------------------------------------------------------- */

/*
 * Expert-major grouping of k3_engine_prefill.inc:1175-1194: for every
 * selected expert in ascending id (the physical order of a contiguous
 * expert store, :1019-1058), rows (token asc, rank asc) with
 * route = token * top_k + rank. Equivalent to a stable sort of the
 * flattened routes by expert id.
 */
int k3o_route_plan(uint32_t *counts, uint32_t *offsets, uint32_t *unique,
                   uint32_t *unique_count, uint32_t *token_index,
                   uint32_t *route_index, const uint32_t *ids,
                   uint32_t tokens, uint32_t top_k, uint32_t experts) {
    const uint64_t routes = (uint64_t)tokens * top_k;
    memset(counts, 0, sizeof(uint32_t) * experts);
    for (uint64_t i = 0; i < routes; i++) {
        if (ids[i] >= experts) return -1;
        counts[ids[i]]++;
    }
    uint32_t running = 0u, u = 0u;
    for (uint32_t e = 0; e < experts; e++) {
        offsets[e] = running;
        running += counts[e];
        if (counts[e] != 0u) unique[u++] = e;
    }
    offsets[experts] = running;
    *unique_count = u;
    uint32_t *cursor = (uint32_t *)malloc(sizeof(uint32_t) * experts);
    if (!cursor) return -2;
    memcpy(cursor, offsets, sizeof(uint32_t) * experts);
    for (uint64_t i = 0; i < routes; i++) {
        const uint32_t e = ids[i];
        token_index[cursor[e]] = (uint32_t)(i / top_k);
        route_index[cursor[e]] = (uint32_t)i;
        cursor[e]++;
    }
    free(cursor);
    return 0;
}

/* ---- MXFP4 --------------------------------------------------------------- */

static inline float nib(const uint8_t *packed_row, uint32_t col) {
    const uint8_t b = packed_row[col / 2u];
    return k3o_e2m1((col & 1u) ? (uint8_t)(b >> 4) : (uint8_t)(b & 15u));
}

/* w64 order: lane l owns 32-column groups l, l+64, ...; per group
 * gs = fmaf(e2m1, x, gs) over its 32 columns in order, then
 * acc = fmaf(gs, e8m0, acc); butterfly64. */
static float mx_row_w64(const uint8_t *p, const uint8_t *s,
                        const uint16_t *x, uint32_t cols) {
    float lane[64];
    const uint32_t groups = cols / 32u;
    for (uint32_t l = 0; l < 64u; l++) {
        float acc = 0.0f;
        for (uint32_t g = l; g < groups; g += 64u) {
            float gs = 0.0f;
            for (uint32_t c = 32u * g; c < 32u * g + 32u; c++)
                gs = fmaf(nib(p, c), k3o_bf16_to_f32(x[c]), gs);
            acc = fmaf(gs, k3o_e8m0(s[g]), acc);
        }
        lane[l] = acc;
    }
    return butterfly64(lane);
}

/* Reference order, k3_rocm_ops.cu:225-273: 128 lanes, lane j owns groups
 * j, j+128, ...; LDS tree 64 -> 1. The source sums four dot8 partials of
 * e2m1 * scale * x; under -ffast-math hipcc (ROCm 7.2, gfx950) factors the
 * group's scale out and emits one chain over the 32 products e2m1 * x
 * (each exact in fp32): a multiply of column 2, then fmaf in the column
 * order of kRefGroupOrder, then partial = fmaf(chain, 2^(s-127), partial). */
static const uint8_t kRefGroupOrder[32] = {
    2, 1, 0, 3, 4, 5, 6, 7, 9, 8, 10, 11, 12, 13, 14, 15,
    17, 16, 18, 19, 20, 21, 22, 23, 25, 24, 26, 27, 28, 29, 30, 31};

static float mx_row_ref128(const uint8_t *p, const uint8_t *s,
                           const uint16_t *x, uint32_t cols) {
    float part[128];
    const uint32_t groups = cols / 32u;
    for (uint32_t t = 0; t < 128u; t++) {
        float acc = 0.0f;
        for (uint32_t g = t; g < groups; g += 128u) {
            const uint32_t c0 = 32u * g;
            uint32_t c = c0 + kRefGroupOrder[0];
            float ch = nib(p, c) * k3o_bf16_to_f32(x[c]);
            for (uint32_t i = 1; i < 32u; i++) {
                c = c0 + kRefGroupOrder[i];
                ch = fmaf(nib(p, c), k3o_bf16_to_f32(x[c]), ch);
            }
            acc = fmaf(ch, k3o_e8m0(s[g]), acc);
        }
        part[t] = acc;
    }
    return tree_reduce(part, 128u);
}

static double mx_row_f64(const uint8_t *p, const uint8_t *s,
                         const uint16_t *x, uint32_t cols) {
    double acc = 0.0;
    for (uint32_t c = 0; c < cols; c++)
        acc += (double)nib(p, c) * (double)k3o_e8m0(s[c / 32u]) *
               (double)k3o_bf16_to_f32(x[c]);
    return acc;
}

/* ---- MX8 activations (MXFP8: OCP E4M3 codes + one E8M0 scale per 32) ---- */

/* OCP E4M3 ("fn") decode: bias 7, no infinities, S.1111.111 = NaN. */
float k3o_e4m3(uint8_t v) {
    const uint32_t e = (v >> 3) & 15u, m = v & 7u;
    if (e == 15u && m == 7u) return u2f(0x7fc00000u);
    const float mag = e ? ldexpf(1.0f + (float)m / 8.0f, (int)e - 7)
                        : ldexpf((float)m / 8.0f, -6);
    return (v & 0x80u) ? -mag : mag;
}

/* fp32 -> E4M3, round to nearest even, magnitude clamped to 448 (the
 * largest finite code), NaN -> 0x7f. Built from the value's own exponent so
 * host and device evaluate the same steps. */
uint8_t k3o_f32_to_e4m3(float v) {
    if (v != v) return 0x7fu;
    const uint8_t sign = (f2u(v) >> 31) ? 0x80u : 0u;
    float a = fabsf(v);
    if (a > 448.0f) a = 448.0f;
    if (a < 0.015625f) /* below 2^-6: subnormal step 2^-9 (code 8 = 2^-6) */
        return sign | (uint8_t)rintf(a * 512.0f);
    const int e = (int)((f2u(a) >> 23) & 255u) - 127; /* a is a normal fp32 */
    const float m = a * u2f((uint32_t)(127 - e) << 23);  /* [1, 2) exactly */
    int mant = (int)rintf((m - 1.0f) * 8.0f);
    int ee = e;
    if (mant == 8) { mant = 0; ee++; }
    return sign | (uint8_t)(((ee + 7) << 3) | mant);
}

/* floor(log2(a)) of a finite a > 0 (normal or subnormal fp32). */
static int ilog2f_pos(float a) {
    const uint32_t u = f2u(a);
    const int e = (int)((u >> 23) & 255u);
    if (e) return e - 127;
    return (31 - __builtin_clz(u & 0x7fffffu)) - 149;
}

/* MXFP8 quantization of a run of n fp32 values sharing one scale (a block
 * of 32, or a whole row): X = floor(log2(max |v|)) - 8, plus one when
 * max |v| * 2^-X exceeds 448 (E4M3's largest finite value, so nothing
 * saturates), clamped to >= -127 (X = -127 for an all-zero run); scale
 * byte = X + 127, q = E4M3(v * 2^-X) rounded to nearest even. The scaled
 * maximum lands in (224, 448]. */
static void mx8_run(uint8_t *q, uint8_t *scale, const float *v, uint64_t n) {
    float amax = 0.0f;
    for (uint64_t i = 0; i < n; i++) {
        const float a = fabsf(v[i]);
        amax = a > amax ? a : amax;
    }
    int X = -127;
    if (amax > 0.0f) {
        X = ilog2f_pos(amax) - 8;
        if (amax * u2f((uint32_t)(127 - X) << 23) > 448.0f) X++;
        if (X < -127) X = -127;
    }
    *scale = (uint8_t)(X + 127);
    const float inv = X == -127 ? u2f(0x7f000000u) : u2f((uint32_t)(127 - X) << 23);
    for (uint64_t i = 0; i < n; i++) q[i] = k3o_f32_to_e4m3(v[i] * inv);
}

static float mx8_value(uint8_t q, uint8_t scale) {
    return k3o_e4m3(q) * k3o_e8m0(scale);
}

void k3o_mx8_quantize(uint8_t *q, uint8_t *scales, const uint16_t *src, uint64_t n) {
    float v[32];
    for (uint64_t b = 0; b < n / 32u; b++) {
        for (int i = 0; i < 32; i++) v[i] = k3o_bf16_to_f32(src[32u * b + i]);
        mx8_run(q + 32u * b, scales + b, v, 32u);
    }
}

/* Two-term MXFP8 split of a run of n values with one scale per term: hi =
 * MXFP8(x), lo = MXFP8(x - hi) with its own scale (the difference is exact
 * in fp32). hi + lo reproduces every bf16 element within 2^6 of the run's
 * maximum exactly, and smaller ones to within 2^-22 of that maximum. v and
 * r are scratch of n floats. */
static void mx8_split_run(uint8_t *hi_q, uint8_t *hi_s, uint8_t *lo_q, uint8_t *lo_s,
                          const uint16_t *src, uint64_t n, float *v, float *r) {
    for (uint64_t i = 0; i < n; i++) v[i] = k3o_bf16_to_f32(src[i]);
    mx8_run(hi_q, hi_s, v, n);
    for (uint64_t i = 0; i < n; i++) r[i] = v[i] - mx8_value(hi_q[i], *hi_s);
    mx8_run(lo_q, lo_s, r, n);
}

/* Per 32-element block. */
void k3o_mx8_split(uint8_t *hi_q, uint8_t *hi_s, uint8_t *lo_q, uint8_t *lo_s,
                   const uint16_t *src, uint64_t n) {
    float v[32], r[32];
    for (uint64_t b = 0; b < n / 32u; b++)
        mx8_split_run(hi_q + 32u * b, hi_s + b, lo_q + 32u * b, lo_s + b, src + 32u * b, 32u, v, r);
}

/* One scale per row (and term) of a [rows, cols] matrix: the encoding of
 * the MFMA path's token rows, whose per-row scales stay in registers. */
void k3o_mx8_quantize_rows(uint8_t *q, uint8_t *scales, const uint16_t *src, uint64_t rows,
                           uint64_t cols) {
    float *v = (float *)malloc(4u * cols);
    for (uint64_t t = 0; t < rows; t++) {
        for (uint64_t i = 0; i < cols; i++) v[i] = k3o_bf16_to_f32(src[t * cols + i]);
        mx8_run(q + t * cols, scales + t, v, cols);
    }
    free(v);
}

void k3o_mx8_split_rows(uint8_t *hi_q, uint8_t *hi_s, uint8_t *lo_q, uint8_t *lo_s,
                        const uint16_t *src, uint64_t rows, uint64_t cols) {
    float *v = (float *)malloc(8u * cols);
    for (uint64_t t = 0; t < rows; t++)
        mx8_split_run(hi_q + t * cols, hi_s + t, lo_q + t * cols, lo_s + t, src + t * cols, cols,
                      v, v + cols);
    free(v);
}

/* bf16 bits of the split's reconstruction hi + lo, rounded to bf16 (it is
 * exactly x for every element that matters; used only to feed fp64). */
static double mx_row_split(const uint8_t *p, const uint8_t *s, const uint8_t *hq,
                           const uint8_t *hs, const uint8_t *lq, const uint8_t *ls,
                           uint32_t cols, uint32_t sblk) {
    double acc = 0.0;
    for (uint32_t c = 0; c < cols; c++) {
        const double xv = (double)mx8_value(hq[c], hs[c / sblk]) +
                          (double)mx8_value(lq[c], ls[c / sblk]);
        acc += (double)nib(p, c) * (double)k3o_e8m0(s[c / 32u]) * xv;
    }
    return acc;
}

/* fp64 dot of one MXFP4 row with MXFP8-quantized activations. */
static double mx_row_mx8(const uint8_t *p, const uint8_t *s, const uint8_t *xq,
                         const uint8_t *xs, uint32_t cols, uint32_t sblk) {
    double acc = 0.0;
    for (uint32_t c = 0; c < cols; c++)
        acc += (double)nib(p, c) * (double)k3o_e8m0(s[c / 32u]) *
               (double)k3o_e4m3(xq[c]) * (double)k3o_e8m0(xs[c / sblk]);
    return acc;
}

void k3o_mxfp4_gemm(uint16_t *out, float *out_f32, const uint8_t *packed,
                    const uint8_t *scales, const uint16_t *input,
                    uint32_t vectors, uint32_t rows, uint32_t columns,
                    int order) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t t = 0; t < (int64_t)vectors; t++) {
        for (int64_t r = 0; r < (int64_t)rows; r++) {
            const uint8_t *p = packed + (uint64_t)r * (columns / 2u);
            const uint8_t *s = scales + (uint64_t)r * (columns / 32u);
            const uint16_t *x = input + (uint64_t)t * columns;
            float v;
            if (order == 0) v = mx_row_w64(p, s, x, columns);
            else if (order == 1) v = mx_row_ref128(p, s, x, columns);
            else v = (float)mx_row_f64(p, s, x, columns);
            const uint64_t o = (uint64_t)t * rows + r;
            if (out) out[o] = k3o_f32_to_bf16(v);
            if (out_f32) out_f32[o] = v;
        }
    }
}

/* ---- Q8-128 static projections ------------------------------------------ */

/* k3_rocm_ops.cu:662-697: per 128-element block, scale = max|w| / 127 (1 for
 * an all-zero block), code = clamp(rint(w / scale), -127, 127). Division
 * here is IEEE (the reference builds with fast math); a NaN codes as 0. */
void k3o_q8_quantize(int8_t *q, float *scales, const uint16_t *w,
                     uint32_t rows, uint32_t cols) {
    const uint64_t blocks = (uint64_t)rows * (cols / 128u);
    for (uint64_t b = 0; b < blocks; b++) {
        const uint16_t *x = w + 128u * b;
        float m = 0.0f;
        for (uint32_t i = 0; i < 128u; i++) m = fmaxf(m, fabsf(k3o_bf16_to_f32(x[i])));
        const float sc = m > 0.0f ? m / 127.0f : 1.0f;
        scales[b] = sc;
        for (uint32_t i = 0; i < 128u; i++) {
            float r = rintf(k3o_bf16_to_f32(x[i]) / sc);
            if (r != r) r = 0.0f;
            r = fminf(fmaxf(r, -127.0f), 127.0f);
            q[128u * b + i] = (int8_t)(int)r;
        }
    }
}

/* k3_rocm_ops.cu:699-711: w = bf16(q * scale). */
void k3o_q8_dequantize(uint16_t *w, const int8_t *q, const float *scales,
                       uint32_t rows, uint32_t cols) {
    const uint64_t n = (uint64_t)rows * cols;
    for (uint64_t i = 0; i < n; i++)
        w[i] = k3o_f32_to_bf16((float)q[i] * scales[i / 128u]);
}

/* w64: lane l owns 32-column groups l, l+64, ...; gs = fmaf(q, x, gs) over
 * the group in column order (products exact), acc = fmaf(gs, scale, acc);
 * butterfly64. */
static float q8_row_w64(const int8_t *q, const float *s, const uint16_t *x, uint32_t cols) {
    float lane[64];
    const uint32_t groups = cols / 32u;
    for (uint32_t l = 0; l < 64u; l++) {
        float acc = 0.0f;
        for (uint32_t g = l; g < groups; g += 64u) {
            float gs = 0.0f;
            for (uint32_t i = 32u * g; i < 32u * g + 32u; i++)
                gs = fmaf((float)q[i], k3o_bf16_to_f32(x[i]), gs);
            acc = fmaf(gs, s[g / 4u], acc);
        }
        lane[l] = acc;
    }
    return butterfly64(lane);
}

/* Reference order, k3_rocm_ops.cu:713-751: 256 threads, thread t sums the
 * octets t, t+256, ... as partial += (q * scale) * x (as written), then the
 * LDS tree. Tolerance checks only (fast-math build). */
static float q8_row_ref256(const int8_t *q, const float *s, const uint16_t *x, uint32_t cols) {
    float p[256];
    const uint32_t octets = cols / 8u;
    for (uint32_t t = 0; t < 256u; t++) {
        float partial = 0.0f;
        for (uint32_t o = t; o < octets; o += 256u) {
            const float sc = s[o / 16u];
            for (uint32_t i = 8u * o; i < 8u * o + 8u; i++)
                partial += ((float)q[i] * sc) * k3o_bf16_to_f32(x[i]);
        }
        p[t] = partial;
    }
    return tree_reduce(p, 256u);
}

static double q8_row_f64(const int8_t *q, const float *s, const uint16_t *x, uint32_t cols) {
    double acc = 0.0;
    for (uint32_t i = 0; i < cols; i++)
        acc += (double)q[i] * (double)s[i / 128u] * (double)k3o_bf16_to_f32(x[i]);
    return acc;
}

void k3o_q8_gemm(uint16_t *out, float *out_f32, const int8_t *q,
                 const float *scales, const uint16_t *input, uint32_t vectors,
                 uint32_t rows, uint32_t cols, int order) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t t = 0; t < (int64_t)vectors; t++) {
        for (int64_t r = 0; r < (int64_t)rows; r++) {
            const int8_t *qr = q + (uint64_t)r * cols;
            const float *sr = scales + (uint64_t)r * (cols / 128u);
            const uint16_t *x = input + (uint64_t)t * cols;
            float v;
            if (order == 0) v = q8_row_w64(qr, sr, x, cols);
            else if (order == 1) v = q8_row_ref256(qr, sr, x, cols);
            else v = (float)q8_row_f64(qr, sr, x, cols);
            const uint64_t o = (uint64_t)t * rows + r;
            if (out) out[o] = k3o_f32_to_bf16(v);
            if (out_f32) out_f32[o] = v;
        }
    }
}

/* ---- RMSNorm (k3_rocm_ops.cu:837-867) ------------------------------------- */

void k3o_rms_norm(uint16_t *out, const uint16_t *in, const uint16_t *weight,
                  uint32_t vectors, uint32_t hidden, float eps, int order) {
    for (uint32_t v = 0; v < vectors; v++) {
        const uint16_t *x = in + (uint64_t)v * hidden;
        uint16_t *o = out + (uint64_t)v * hidden;
        float p[256];
        for (uint32_t t = 0; t < 256u; t++) {
            float acc = 0.0f;
            if (order == 0) { /* 8-element chunks t, t + 256, ... */
                for (uint32_t c = t; 8u * c < hidden; c += 256u)
                    for (uint32_t d = 8u * c; d < 8u * c + 8u && d < hidden; d++) {
                        const float e = k3o_bf16_to_f32(x[d]);
                        acc = fmaf(e, e, acc);
                    }
            } else { /* reference: elements t, t + 256, ... */
                for (uint32_t d = t; d < hidden; d += 256u) {
                    const float e = k3o_bf16_to_f32(x[d]);
                    acc = acc + e * e;
                }
            }
            p[t] = acc;
        }
        if (order == 2) {
            double ss = 0.0;
            for (uint32_t d = 0; d < hidden; d++) {
                const double e = k3o_bf16_to_f32(x[d]);
                ss += e * e;
            }
            const double inv = 1.0 / sqrt(ss / hidden + (double)eps);
            for (uint32_t d = 0; d < hidden; d++)
                o[d] = k3o_f32_to_bf16((float)((double)k3o_bf16_to_f32(x[d]) * inv *
                                               (double)k3o_bf16_to_f32(weight[d])));
            continue;
        }
        float total;
        if (order == 0) {
            float w[4];
            for (int q = 0; q < 4; q++) w[q] = butterfly64(p + 64 * q);
            total = (w[0] + w[1]) + (w[2] + w[3]);
        } else {
            total = tree_reduce(p, 256u);
        }
        const float inv = 1.0f / sqrtf(total / (float)hidden + eps);
        for (uint32_t d = 0; d < hidden; d++)
            o[d] = k3o_f32_to_bf16((k3o_bf16_to_f32(x[d]) * inv) * k3o_bf16_to_f32(weight[d]));
    }
}

/* ---- combine ------------------------------------------------------------- */

/* k3_rocm_ops.cu:1452-1474: sum starts at 0 and adds w[r] * y[r] in rank
 * order, product and sum each rounded to fp32 (as the source is written). */
void k3o_weighted_sum(uint16_t *out, const uint16_t *vectors,
                      const float *weights, uint32_t tokens,
                      uint32_t vector_count, uint32_t hidden) {
    for (uint32_t t = 0; t < tokens; t++) {
        const uint16_t *v = vectors + (uint64_t)t * vector_count * hidden;
        const float *w = weights + (uint64_t)t * vector_count;
        for (uint32_t d = 0; d < hidden; d++) {
            float sum = 0.0f;
            for (uint32_t r = 0; r < vector_count; r++) {
                const float prod = w[r] * k3o_bf16_to_f32(v[(uint64_t)r * hidden + d]);
                sum = sum + prod;
            }
            out[(uint64_t)t * hidden + d] = k3o_f32_to_bf16(sum);
        }
    }
}

/* k3_rocm_ops.cu:1499-1510. */
void k3o_add(uint16_t *out, const uint16_t *left, const uint16_t *right,
             uint64_t n) {
    for (uint64_t i = 0; i < n; i++)
        out[i] = k3o_f32_to_bf16(k3o_bf16_to_f32(left[i]) + k3o_bf16_to_f32(right[i]));
}

/* k3_rocm_ops.cu:1476-1497: gather out[i] = in[ids[i]]; scatter
 * out[ids[i]] = in[i]. */
void k3o_copy_rows(uint16_t *out, const uint16_t *in, const uint32_t *row_ids,
                   uint32_t row_count, uint32_t row_size, int scatter) {
    for (uint32_t i = 0; i < row_count; i++) {
        const uint64_t a = (uint64_t)i * row_size;
        const uint64_t b = (uint64_t)row_ids[i] * row_size;
        if (scatter) memcpy(out + b, in + a, (size_t)row_size * 2u);
        else memcpy(out + a, in + b, (size_t)row_size * 2u);
    }
}

/* ------------------------------------------------------------------------ */
/* whole layer                                                               */
/* ------------------------------------------------------------------------ */

/*
 * Per token t (config form, or K3-native expert stage when hidden = latent):
 *   logits = router(x_t)                      k3_engine.cu:1554-1557
 *   ids, w = topk(logits, bias, k, scale)     k3_engine.cu:1558-1563
 *   for rank r: e = ids[r]                    k3_engine.cu:1032-1066
 *     g = bf16(W1_e x), u = bf16(W3_e x), a = act(g, u), y_r = bf16(W2_e a)
 *   c = bf16(sum_r w_r y_r)                   k3_engine.cu:1851-1855
 *   out = bf16(residual + c)                  k3_engine.cu:1889-1897
 * (the K3-native RMSNorm / routed-up / shared-expert tail is not part of
 * this function).
 */
int k3o_layer(const k3o_shape *sh, uint32_t tokens,
              const uint16_t *hidden_in, const uint16_t *residual,
              const uint16_t *router_weight, const float *router_bias,
              const k3o_expert *experts,
              const uint32_t *ids_in, const float *weights_in,
              const uint32_t *token_list, uint32_t token_list_count,
              uint16_t *output, uint32_t *ids_out, float *weights_out,
              float *logits_out, uint16_t *expert_out, int gemv_order,
              int threads) {
    const uint32_t H = sh->hidden, E = sh->experts, K = sh->top_k, F = sh->ffn;
    const uint32_t n = token_list ? token_list_count : tokens;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
    int status = 0;
    float *logits = (float *)malloc(sizeof(float) * (uint64_t)E * (n ? n : 1));
    uint32_t *ids = (uint32_t *)malloc(sizeof(uint32_t) * (uint64_t)K * (n ? n : 1));
    float *wts = (float *)malloc(sizeof(float) * (uint64_t)K * (n ? n : 1));
    uint16_t *ys = (uint16_t *)malloc(sizeof(uint16_t) * (uint64_t)K * H * (n ? n : 1));
    if (!logits || !ids || !wts || !ys) { status = -2; goto done; }

    for (uint32_t i = 0; i < n; i++) {
        const uint32_t t = token_list ? token_list[i] : i;
        const uint16_t *x = hidden_in + (uint64_t)t * H;
        if (ids_in) {
            memcpy(ids + (uint64_t)i * K, ids_in + (uint64_t)t * K, 4u * K);
            memcpy(wts + (uint64_t)i * K, weights_in + (uint64_t)t * K, 4u * K);
        } else {
            /* the router's logits in the reference's order (every router
             * path of the library computes them that way) */
            k3o_bf16_gemm_f32(logits + (uint64_t)i * E, router_weight, x, 1u, E, H, 1);
            k3o_router_topk(ids + (uint64_t)i * K, wts + (uint64_t)i * K,
                            logits + (uint64_t)i * E, router_bias, 1u, E, K,
                            sh->scale, 0);
        }
        for (uint32_t r = 0; r < K; r++) {
            const uint32_t e = ids[(uint64_t)i * K + r];
            if (e >= E || !experts[e].w1_packed) { status = -1; goto done; }
        }
    }

    {
        /* (route, 64-row block) work items, so every core has work even at
         * one token; each output row is computed exactly as before. */
        const uint64_t J = (uint64_t)n * K, RB = 64u;
        const uint64_t nb_f = (F + RB - 1u) / RB, nb_h = (H + RB - 1u) / RB;
        const int ord = gemv_order, mx = (ord == 3 || ord == 4);
        uint16_t *g = (uint16_t *)malloc(2u * J * F), *u = (uint16_t *)malloc(2u * J * F);
        uint16_t *a = (uint16_t *)malloc(2u * J * F);
        uint8_t *xq = NULL, *xs = NULL, *xq2 = NULL, *xs2 = NULL;
        uint8_t *aq = NULL, *as = NULL, *aq2 = NULL, *as2 = NULL;
        if (mx) {
            xq = (uint8_t *)malloc((uint64_t)n * H); xs = (uint8_t *)malloc((uint64_t)n * H / 32u);
            xq2 = (uint8_t *)malloc((uint64_t)n * H); xs2 = (uint8_t *)malloc((uint64_t)n * H / 32u);
            aq = (uint8_t *)malloc(J * F); as = (uint8_t *)malloc(J * F / 32u);
            aq2 = (uint8_t *)malloc(J * F); as2 = (uint8_t *)malloc(J * F / 32u);
        }
        if (!g || !u || !a || (mx && (!xq || !xs || !xq2 || !xs2 || !aq || !as || !aq2 || !as2))) {
            status = -2;
        } else {
            if (mx) {
#pragma omp parallel for schedule(static)
                for (int64_t i = 0; i < (int64_t)n; i++) {
                    const uint32_t t = token_list ? token_list[i] : (uint32_t)i;
                    const uint16_t *x = hidden_in + (uint64_t)t * H;
                    const uint64_t o = (uint64_t)i * H;
                    if (ord == 3) k3o_mx8_quantize_rows(xq + o, xs + i, x, 1u, H);
                    else k3o_mx8_split_rows(xq + o, xs + i, xq2 + o, xs2 + i, x, 1u, H);
                }
            }
#pragma omp parallel for schedule(dynamic, 1)
            for (int64_t item = 0; item < (int64_t)(J * nb_f); item++) {
                const uint64_t job = (uint64_t)item / nb_f, r0 = ((uint64_t)item % nb_f) * RB;
                const uint32_t i = (uint32_t)(job / K);
                const uint32_t t = token_list ? token_list[i] : i;
                const uint16_t *x = hidden_in + (uint64_t)t * H;
                const k3o_expert *ex = &experts[ids[job]];
                const uint64_t xo = (uint64_t)i * H;
                for (uint64_t row = r0; row < r0 + RB && row < F; row++) {
                    const uint64_t po = row * (H / 2u), so = row * (H / 32u);
                    float vg, vu;
                    if (ord == 0) {
                        vg = mx_row_w64(ex->w1_packed + po, ex->w1_scales + so, x, H);
                        vu = mx_row_w64(ex->w3_packed + po, ex->w3_scales + so, x, H);
                    } else if (ord == 1) {
                        vg = mx_row_ref128(ex->w1_packed + po, ex->w1_scales + so, x, H);
                        vu = mx_row_ref128(ex->w3_packed + po, ex->w3_scales + so, x, H);
                    } else if (ord == 3) {
                        vg = (float)mx_row_mx8(ex->w1_packed + po, ex->w1_scales + so, xq + xo, xs + i, H, H);
                        vu = (float)mx_row_mx8(ex->w3_packed + po, ex->w3_scales + so, xq + xo, xs + i, H, H);
                    } else if (ord == 4) {
                        vg = (float)mx_row_split(ex->w1_packed + po, ex->w1_scales + so, xq + xo, xs + i,
                                                 xq2 + xo, xs2 + i, H, H);
                        vu = (float)mx_row_split(ex->w3_packed + po, ex->w3_scales + so, xq + xo, xs + i,
                                                 xq2 + xo, xs2 + i, H, H);
                    } else {
                        vg = (float)mx_row_f64(ex->w1_packed + po, ex->w1_scales + so, x, H);
                        vu = (float)mx_row_f64(ex->w3_packed + po, ex->w3_scales + so, x, H);
                    }
                    g[job * F + row] = k3o_f32_to_bf16(vg);
                    u[job * F + row] = k3o_f32_to_bf16(vu);
                }
            }
#pragma omp parallel for schedule(static)
            for (int64_t job = 0; job < (int64_t)J; job++) {
                const uint64_t o = (uint64_t)job * F;
                if (sh->activation == 1u) k3o_swiglu(a + o, g + o, u + o, F, 0);
                else k3o_situ(a + o, g + o, u + o, F, sh->beta, sh->linear_beta, 0);
                if (ord == 3) k3o_mx8_quantize(aq + o, as + o / 32u, a + o, F);
                if (ord == 4) k3o_mx8_split(aq + o, as + o / 32u, aq2 + o, as2 + o / 32u, a + o, F);
            }
#pragma omp parallel for schedule(dynamic, 1)
            for (int64_t item = 0; item < (int64_t)(J * nb_h); item++) {
                const uint64_t job = (uint64_t)item / nb_h, r0 = ((uint64_t)item % nb_h) * RB;
                const k3o_expert *ex = &experts[ids[job]];
                const uint64_t ao = job * F;
                uint16_t *y = ys + job * H;
                for (uint64_t row = r0; row < r0 + RB && row < H; row++) {
                    const uint64_t po = row * (F / 2u), so = row * (F / 32u);
                    float v;
                    if (ord == 0) v = mx_row_w64(ex->w2_packed + po, ex->w2_scales + so, a + ao, F);
                    else if (ord == 1) v = mx_row_ref128(ex->w2_packed + po, ex->w2_scales + so, a + ao, F);
                    else if (ord == 3) v = (float)mx_row_mx8(ex->w2_packed + po, ex->w2_scales + so, aq + ao, as + ao / 32u, F, 32u);
                    else if (ord == 4) v = (float)mx_row_split(ex->w2_packed + po, ex->w2_scales + so, aq + ao, as + ao / 32u,
                                                               aq2 + ao, as2 + ao / 32u, F, 32u);
                    else v = (float)mx_row_f64(ex->w2_packed + po, ex->w2_scales + so, a + ao, F);
                    y[row] = k3o_f32_to_bf16(v);
                }
            }
        }
        free(g); free(u); free(a); free(xq); free(xs); free(xq2); free(xs2);
        free(aq); free(as); free(aq2); free(as2);
        if (status) goto done;
    }

    for (uint32_t i = 0; i < n; i++) {
        const uint32_t t = token_list ? token_list[i] : i;
        uint16_t *c = (uint16_t *)malloc(2u * H);
        k3o_weighted_sum(c, ys + (uint64_t)i * K * H, wts + (uint64_t)i * K, 1u, K, H);
        if (residual) k3o_add(output + (uint64_t)i * H, residual + (uint64_t)t * H, c, H);
        else memcpy(output + (uint64_t)i * H, c, 2u * H);
        free(c);
        if (ids_out) memcpy(ids_out + (uint64_t)i * K, ids + (uint64_t)i * K, 4u * K);
        if (weights_out) memcpy(weights_out + (uint64_t)i * K, wts + (uint64_t)i * K, 4u * K);
        if (logits_out && !ids_in) memcpy(logits_out + (uint64_t)i * E, logits + (uint64_t)i * E, 4u * E);
        if (expert_out) memcpy(expert_out + (uint64_t)i * K * H, ys + (uint64_t)i * K * H, 2u * K * H);
    }
done:
    free(logits); free(ids); free(wts); free(ys);
    return status;
}

/* ------------------------------------------------------------------------ */
/* prefill workspace ledger                                                  */
/* ------------------------------------------------------------------------ */

/* k3_prefill.c:136-234 per-token byte counts for the K3 shape
 * (hidden 7168, KDA inner 12288, head dim 128, dense 33792, latent 3584,
 * expert hidden 3072, shared 6144, top-k 16, 896 experts, 96 heads, MLA
 * q-lora 1536, q 96*192, cache dim 576, 24 MLA layers). */
int k3o_prefill_workspace(uint32_t chunk, k3o_workspace *o) {
    const uint64_t b = 2u;
    const uint64_t hidden = 7168u * b, inner = 12288u * b, dense = 33792u * b;
    const uint64_t main_t = 5u * hidden + 10u * inner + 128u * b + 96u * b + 3u * dense;
    const uint64_t hid_t = 2u * hidden, attn_t = 8u * hidden;
    const uint64_t moe_t = 896u * 4u +
        (3584u + 3u * 3072u + 16u * 3584u + 2u * 3584u + 7168u + 3u * 6144u + 7168u) * b;
    const uint64_t mla_t = (2u * 1536u + 96u * 192u + 576u + 96u * 576u + 3u * 12288u) * b;
    const uint64_t route_t = 16u * 8u, index_t = 8u;
    o->hidden_row_bytes = hid_t * chunk;
    o->attn_res_row_bytes = attn_t * chunk;
    o->main_scratch_bytes = main_t * chunk;
    o->moe_scratch_bytes = moe_t * chunk;
    o->mla_scratch_bytes = mla_t * chunk;
    o->route_bytes = route_t * chunk;
    o->expert_index_bytes = index_t * chunk;
    o->batch_workspace_bytes = o->hidden_row_bytes + o->attn_res_row_bytes +
        o->main_scratch_bytes + o->moe_scratch_bytes + o->mla_scratch_bytes +
        o->route_bytes + o->expert_index_bytes;
    const uint64_t one = hid_t + attn_t + main_t + moe_t + mla_t + route_t + index_t;
    o->incremental_workspace_bytes =
        o->batch_workspace_bytes > one ? o->batch_workspace_bytes - one : 0u;
    o->mla_append_bytes = (uint64_t)chunk * 24u * 576u * b;
    return 0;
}
