/*
 * Grouped expert products on CDNA4 scaled MFMA (prefill / batched tokens).
 *
 * Activations enter the MFMA as E4M3 codes with E8M0 scales against the
 * experts' native MXFP4 weights, through V_MFMA_SCALE_F32_16X16X128_F8F6F4:
 * the token rows x with one scale per row (and term), the gate/up
 * activation with one per 32 columns (MXFP8). In the split precision every
 * bf16 value is carried as two terms hi + lo (lo quantizes x - hi), which
 * reproduces it exactly except for elements more than 2^6 below the
 * maximum of their scale run (error <= 2^-22 of that maximum), so the
 * products are those of the bf16 inputs and only the fp32 accumulation
 * order differs from the exact path.
 */
#pragma once

#include "k3_decode.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "k3_moe.h"

namespace k3 {

/* Tile classes by an expert's row count: one 16-row tile (<= 16 rows), one
 * 64-row tile (<= 64), one 96-row tile (<= 96), or 128-row tiles. */
constexpr int kTileClasses = 4;

struct MfmaBuffers {
    uint8_t *xq[2], *xs[2];     /* [T, H] codes, [T] row scales: hi, lo */
    uint8_t *aq[2], *as[2];     /* [routes, F] codes; scales [F / 512][routes][16]
                                   (16 scale bytes = 512 columns of a row) */
    uint32_t routes;            /* rows of aq / as */
    uint32_t *tiles;            /* kTileClasses x tile_cap x {expert, row0, rows} */
    uint32_t *tile_count;       /* [kTileClasses] */
    uint32_t *unaligned;        /* [E + 1]: count, then the selected experts with a
                                   tensor that is not 8-byte aligned (any order) */
    uint32_t tile_cap[kTileClasses];
};

/* Per-class tile lists of every selected expert (counts/offsets of the plan
 * on the stream already), for the exact grouped kernels: tiles of at most
 * 128 rows spread a heavy expert's rows over many workgroups. E <= 1024. */
bool build_tiles_all(const MfmaBuffers &B, const uint32_t *counts, const uint32_t *offsets,
                     const k3_moe_expert *experts, uint32_t E, hipStream_t st);

/* Device tile bounds for T tokens, per tile class. */
void mfma_tile_caps(uint32_t T, uint32_t k, uint32_t E, uint32_t caps[kTileClasses]);

/* Plan (counts/offsets/unique/token_index/route_index) must be on the
 * stream already. Writes y [routes, H] bf16 in route order. terms: 1 or 2. */
bool mfma_supported(const k3_moe_shape &s);

bool mfma_launch_experts(const MfmaBuffers &B, uint16_t *y, const uint16_t *hidden,
                         const uint32_t *counts, const uint32_t *offsets,
                         const uint32_t *token_index, const uint32_t *route_index,
                         const k3_moe_expert *experts, const k3_moe_shape &s, uint32_t T,
                         uint32_t terms, hipStream_t st, const StageMarker &mark);

}  // namespace k3
