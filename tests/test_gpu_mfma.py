"""GPU parity of the scaled-MFMA expert path (K3_MOE_MFMA / K3_MOE_MFMA_FP8).

- The MXFP8 activation encoding (k3_moe_mx8_quantize_bf16) is bit-exact to
  the oracle's k3o_mx8_quantize / k3o_mx8_split.
- Routing (ids, weights, plan) is the exact path's, so ids match bit for bit.
- Layer outputs: the MFMA accumulation order differs from the w64 order, so
  outputs are compared at a stated tolerance, against the oracle's fp64
  layer on the same (split) inputs and against the GPU's own exact path on
  every token of the K3-shape batches (T = 64, 512 and the 8192-token Zipf
  prefill, which exercises all three tile classes).

Tolerance for K3_MOE_MFMA (bf16-faithful): relative L2 <= 2e-3 of the
layer output, and every |difference| <= 4 bf16 ulps at max(|element|,
output RMS). Each output element is a weighted sum of k expert outputs that
were rounded to bf16 at their own (RMS-sized) magnitude, after two more bf16
roundings (gate/up, activation) whose boundaries the fp32 order can cross;
so an element that cancels to near zero still carries errors of a few
RMS-sized ulps. The bound allows that and nothing more.
"""
import ctypes
import dataclasses

import numpy as np
import pytest
import torch

import _oracle as O
from moonshine_amd import layer as L
from moonshine_amd._lib import lib
from moonshine_amd.synth import (CONFIGS, EXACT, MFMA, MFMA_FP8, bf16_bits_to_f32,
                                 f32_to_bf16_bits, make_inputs)

pytestmark = pytest.mark.gpu

REL_L2 = 2e-3
ULPS = 4

_stores = {}


def get_layer(cfg, inputs, cuda):
    key = (cfg.experts, cfg.hidden, cfg.ffn, cfg.seed)
    if key not in _stores:
        _stores.clear()
        torch.cuda.empty_cache()
        _stores[key] = L.ExpertStore(cfg.experts, cfg.hidden, cfg.ffn, seed=cfg.seed, device=cuda)
    return L.build_layer(cfg, inputs, device=cuda, store=_stores[key])


def forward(moe, inputs, cuda, precision):
    x = L.bf16_tensor(inputs.hidden, cuda)
    r = L.bf16_tensor(inputs.residual, cuda)
    T, k = x.shape[0], moe.shape.top_k
    ids = torch.zeros((T, k), dtype=torch.int32, device=cuda)
    w = torch.zeros((T, k), dtype=torch.float32, device=cuda)
    out = moe.forward(x, r, ids=ids, weights=w, precision=precision)
    torch.cuda.synchronize()
    return L.bf16_bits(out), ids.cpu().numpy().view(np.uint32), w.cpu().numpy()


def assert_close(got_bits, want_bits, what):
    got = bf16_bits_to_f32(got_bits).astype(np.float64)
    want = bf16_bits_to_f32(want_bits).astype(np.float64)
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    rms = np.sqrt(np.mean(want ** 2))
    # bf16 ulp at max(|element|, rms)
    ulp = np.ldexp(1.0, np.frexp(np.maximum(np.abs(want), rms))[1] - 8)
    d = np.abs(got - want)
    worst = (d / ulp).max()
    print(f"{what}: rel-L2 {rel:.3g}, max |d| {d.max():.4g}, worst {worst:.2f} ulp "
          f"(rms {rms:.4g}), elements differing {np.mean(got != want):.3%}")
    assert rel <= REL_L2, f"{what}: relative L2 {rel:.3g} > {REL_L2}"
    assert worst <= ULPS, f"{what}: an element differs by {worst:.2f} > {ULPS} ulp"


def test_mx8_quantize_bitexact(cuda):
    rng = np.random.default_rng(21)
    n = 32 * 4096
    x = rng.standard_normal(n).astype(np.float32) * np.repeat(
        np.ldexp(1.0, rng.integers(-60, 60, n // 32)), 32)
    x[:32] = 0.0
    x[32:64] = 1e-39
    x[64:96] = np.float32(6.5e4) * rng.standard_normal(32).astype(np.float32)
    x[96:128] = rng.standard_normal(32).astype(np.float32)   # +-inf among finite values
    x[100], x[113] = np.inf, -np.inf
    x[128:160] = rng.standard_normal(32).astype(np.float32)  # NaN among finite values
    x[130] = np.nan
    x[160:192] = np.float32(2.0 ** -133)                      # amax below 2^-119: scale byte 0
    xb = f32_to_bf16_bits(x)
    # every bf16 value within +-448, 31 to a block behind a 448 marker (block
    # scale 2^0, so each value is encoded as itself): every input the split
    # can hand the E4M3 conversion is such a value times a power of two
    pos = np.arange(0x0000, 0x43E1, dtype=np.uint32)
    sweep = np.concatenate([pos, pos | 0x8000]).astype(np.uint16)
    pad = (-sweep.size) % 31
    sweep = np.concatenate([sweep, np.zeros(pad, np.uint16)]).reshape(-1, 31)
    marker = np.full((sweep.shape[0], 1), 0x43E0, np.uint16)
    xb = np.concatenate([xb, np.concatenate([marker, sweep], axis=1).ravel()])
    n = xb.size
    src = torch.from_numpy(xb.view(np.int16)).to(cuda)
    hq = torch.empty(n, dtype=torch.uint8, device=cuda)
    lq = torch.empty(n, dtype=torch.uint8, device=cuda)
    hs = torch.empty(n // 32, dtype=torch.uint8, device=cuda)
    ls = torch.empty(n // 32, dtype=torch.uint8, device=cuda)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib().k3_moe_mx8_quantize_bf16(P(hq), P(hs), P(lq), P(ls), P(src), n, st)
    torch.cuda.synchronize()
    want = O.mx8_split(xb)
    for got, exp in zip((hq, hs, lq, ls), want):
        np.testing.assert_array_equal(got.cpu().numpy(), exp)
    assert lib().k3_moe_mx8_quantize_bf16(P(hq), P(hs), None, None, P(src), n, st)
    torch.cuda.synchronize()
    q1, s1 = O.mx8_quantize(xb)
    np.testing.assert_array_equal(hq.cpu().numpy(), q1)
    np.testing.assert_array_equal(hs.cpu().numpy(), s1)
    # argument checks
    assert not lib().k3_moe_mx8_quantize_bf16(P(hq), P(hs), None, None, P(src), 33, st)
    assert not lib().k3_moe_mx8_quantize_bf16(P(hq), P(hs), P(lq), None, P(src), n, st)


@pytest.mark.parametrize("cols", [7168, 2048, 520, 2056, 9000])
def test_mx8_quantize_rows_bitexact(cuda, cols):
    """Per-row scales (the token rows of the gate/up products) against the
    oracle's k3o_mx8_split_rows / k3o_mx8_quantize_rows."""
    rng = np.random.default_rng(22 + cols)
    rows = 96
    x = rng.standard_normal((rows, cols)).astype(np.float32) * np.ldexp(
        1.0, rng.integers(-60, 60, (rows, 1)))
    x[:, ::5] *= np.ldexp(1.0, rng.integers(-30, 0, (rows, (cols + 4) // 5)))
    x[0] = 0.0
    x[1] = 1e-39
    x[2] *= np.float32(6.5e4)
    x[3, 100], x[3, 7] = np.inf, -np.inf        # +-inf among finite values
    x[4, 17] = np.nan                           # NaN among finite values
    x[5] = np.float32(2.0 ** -133)              # maximum below 2^-119: scale byte 0
    xb = f32_to_bf16_bits(x)
    # rows of every bf16 value within +-448 behind a 448 marker (row scale
    # 2^0: each value encoded as itself)
    pos = np.arange(0x0000, 0x43E1, dtype=np.uint32)
    sweep = np.concatenate([pos, pos | 0x8000]).astype(np.uint16)
    per = cols - 1
    sweep = np.concatenate([sweep, np.zeros((-sweep.size) % per, np.uint16)]).reshape(-1, per)
    marker = np.full((sweep.shape[0], 1), 0x43E0, np.uint16)
    xb = np.concatenate([xb, np.concatenate([marker, sweep], axis=1)])
    rows = xb.shape[0]
    src = torch.from_numpy(xb.view(np.int16)).to(cuda)
    hq = torch.empty((rows, cols), dtype=torch.uint8, device=cuda)
    lq = torch.empty_like(hq)
    hs = torch.empty(rows, dtype=torch.uint8, device=cuda)
    ls = torch.empty_like(hs)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib().k3_moe_mx8_quantize_rows_bf16(P(hq), P(hs), P(lq), P(ls), P(src), rows, cols, st)
    torch.cuda.synchronize()
    for got, exp in zip((hq, hs, lq, ls), O.mx8_split_rows(xb)):
        np.testing.assert_array_equal(got.cpu().numpy(), exp)
    assert lib().k3_moe_mx8_quantize_rows_bf16(P(hq), P(hs), None, None, P(src), rows, cols, st)
    torch.cuda.synchronize()
    q1, s1 = O.mx8_quantize_rows(xb)
    np.testing.assert_array_equal(hq.cpu().numpy(), q1)
    np.testing.assert_array_equal(hs.cpu().numpy(), s1)
    assert not lib().k3_moe_mx8_quantize_rows_bf16(P(hq), P(hs), None, None, P(src), rows, 12, st)
    assert not lib().k3_moe_mx8_quantize_rows_bf16(P(hq), P(hs), P(lq), None, P(src), rows, cols,
                                                   st)


def small_cfg(tokens):
    """Config 0's shape (H 2048, 64 experts, top-4, F 512) with a batch."""
    return dataclasses.replace(CONFIGS[0], name=f"cfg0x{tokens}", tokens=tokens)


@pytest.mark.parametrize("shape", [(2048, 512), (1536, 1536)], ids=["h2048", "h1536"])
@pytest.mark.parametrize("precision,order", [(MFMA, O.ORDER_SPLIT), (MFMA_FP8, O.ORDER_MX8)],
                         ids=["mfma", "mfma_fp8"])
def test_small_batch_vs_oracle(cuda, precision, order, shape):
    """H 1536: an odd count of 16-byte scale records per gate/up row (the
    last two-record scale block holds one)."""
    cfg = dataclasses.replace(small_cfg(72), hidden=shape[0], ffn=shape[1])
    inputs = make_inputs(cfg, tokens=cfg.tokens)
    moe = get_layer(cfg, inputs, cuda)
    out, ids, w = forward(moe, inputs, cuda, precision)
    want_ids, want_w = O.router_topk(O.router_logits(inputs.router_weight, inputs.hidden),
                                     inputs.router_bias, cfg.top_k, cfg.scale)
    np.testing.assert_array_equal(ids, want_ids)
    np.testing.assert_array_equal(w, want_w)
    experts = {int(e): moe.store.host_expert(int(e)) for e in np.unique(ids)}
    want = O.layer(cfg, inputs, experts, order=order)
    assert_close(out, want["output"], f"precision {precision} vs oracle order {order}")
    if precision == MFMA:
        exact, _, _ = forward(moe, inputs, cuda, EXACT)
        assert_close(out, exact, "mfma vs exact (GPU)")


def rel_and_ulps(got_bits, want_bits):
    got = bf16_bits_to_f32(got_bits).astype(np.float64)
    want = bf16_bits_to_f32(want_bits).astype(np.float64)
    rms = np.sqrt(np.mean(want ** 2))
    ulp = np.ldexp(1.0, np.frexp(np.maximum(np.abs(want), rms))[1] - 8)
    return np.linalg.norm(got - want) / np.linalg.norm(want), (np.abs(got - want) / ulp).max()


def test_outlier_channels_vs_exact(cuda):
    """Massive-activation rows: two channels per token at about 1e3 times the
    row RMS (as in real post-norm hidden states). Two effects add error
    here. The gate/up input has one E8M0 scale per token row, so the
    outliers set the scale of the whole row and the two-term encoding
    keeps about 2^-8 of a small element rather than all its bits (the
    oracle's split order against the exact order on CPU, this input:
    rel-L2 4.2e-4). And inside one fp8 MFMA the 128 products are aligned
    to the largest, so an outlier's product truncates the others (about
    2^-15 of the sum of |products| per instruction); that dominates. The
    per-element bar stays 4 bf16 ulp of max(|element|, RMS); the rel-L2
    bar for such rows is 4e-3 (measured 2.5e-3, 39% of elements 1 ulp
    apart), against 2e-3 for ordinary rows. The one-term MFMA_FP8 precision
    is measured and reported (not bf16-faithful; no default uses it); its
    bound only catches breakage."""
    cfg = CONFIGS[2]
    T = 64
    inputs = make_inputs(cfg, tokens=T)
    rng = np.random.default_rng(404)
    x = bf16_bits_to_f32(inputs.hidden).copy()
    for t in range(T):
        ch = rng.choice(cfg.hidden, 2, replace=False)
        x[t, ch] = rng.choice([-1.0, 1.0], 2) * rng.uniform(800.0, 1200.0, 2)
    inputs.hidden = f32_to_bf16_bits(x)
    moe = get_layer(cfg, inputs, cuda)
    exact, ids0, w0 = forward(moe, inputs, cuda, EXACT)
    mfma, ids1, w1 = forward(moe, inputs, cuda, MFMA)
    fp8, ids2, w2 = forward(moe, inputs, cuda, MFMA_FP8)
    for ids, w in ((ids1, w1), (ids2, w2)):
        np.testing.assert_array_equal(ids, ids0)
        np.testing.assert_array_equal(w, w0)
    rel, worst = rel_and_ulps(mfma, exact)
    print(f"outlier rows: mfma vs exact: rel-L2 {rel:.3g}, worst {worst:.2f} ulp")
    assert rel <= 4e-3 and worst <= ULPS
    rel, worst = rel_and_ulps(fp8, exact)
    print(f"outlier rows: mfma_fp8 (one term) vs exact: rel-L2 {rel:.3g}, worst {worst:.1f} ulp")
    assert np.isfinite(rel) and rel < 0.5


@pytest.mark.parametrize("cfg_index", [2, 3, 4])
def test_k3_batches_vs_exact(cuda, cfg_index):
    cfg = CONFIGS[cfg_index]
    inputs = make_inputs(cfg, tokens=cfg.tokens)
    moe = get_layer(cfg, inputs, cuda)
    print(f"{cfg.name}: T={cfg.tokens}", flush=True)
    out, ids, w = forward(moe, inputs, cuda, MFMA)
    exact, ids_e, w_e = forward(moe, inputs, cuda, EXACT)
    np.testing.assert_array_equal(ids, ids_e)
    np.testing.assert_array_equal(w, w_e)
    assert_close(out, exact, f"{cfg.name} mfma vs exact")
    # repeat: same bits (no state carried between calls)
    again, _, _ = forward(moe, inputs, cuda, MFMA)
    np.testing.assert_array_equal(again, out)


def test_unsupported_shape_rejected(cuda):
    cfg = dataclasses.replace(CONFIGS[0], name="odd", tokens=4, hidden=2080, experts=16, top_k=2,
                              seed=3)
    inputs = make_inputs(cfg, tokens=4)
    moe = L.build_layer(cfg, inputs, device=cuda)
    with pytest.raises(RuntimeError):
        forward(moe, inputs, cuda, MFMA)
    forward(moe, inputs, cuda, EXACT)  # the exact path takes any H % 32 == 0


def test_tile_class_edges_vs_exact(cuda):
    """Experts routed exactly 16, 17, 64, 65, 80, 96, 97, 128, 129 and 200
    rows (every tile class and its edges, including the 96-row class and a
    partial last 128-row tile), through k3_moe_experts_bf16 with given
    routes: MFMA against the exact path (itself bit-exact to the oracle)."""
    cfg = small_cfg(260)
    inputs = make_inputs(cfg, tokens=cfg.tokens)
    moe = get_layer(cfg, inputs, cuda)
    T, k = cfg.tokens, cfg.top_k
    counts = {0: 65, 1: 80, 2: 96, 3: 97, 4: 128, 5: 129, 6: 16, 7: 17, 8: 64, 9: 200}
    ids = np.full((T, k), 0xFFFFFFFF, np.uint32)  # unused slots: no route
    used = np.zeros(T, np.int64)
    for e, n in counts.items():
        order = np.argsort(used, kind="stable")[:n]  # the tokens with the fewest routes
        for t in order:
            ids[t, used[t]] = e
            used[t] += 1
    assert used.max() <= k
    rng = np.random.default_rng(7)
    w = (rng.random((T, k)) * 0.5 + 0.1).astype(np.float32)
    x = L.bf16_tensor(inputs.hidden, cuda)
    r = L.bf16_tensor(inputs.residual, cuda)
    ids_d = torch.from_numpy(ids.view(np.int32)).to(cuda)
    w_d = torch.from_numpy(w).to(cuda)
    out = moe.experts_only(x, ids_d, w_d, residual=r, precision=MFMA)
    exact = moe.experts_only(x, ids_d, w_d, residual=r, precision=EXACT)
    torch.cuda.synchronize()
    assert_close(L.bf16_bits(out), L.bf16_bits(exact), "tile class edges mfma vs exact")


@pytest.mark.parametrize("T,k,rows", [(70, 1, {7: 70}), (100, 1, {7: 100}),
                                       (200, 1, {7: 130, 8: 70}), (100, 2, {7: 100, 8: 80})],
                         ids=["96only", "128only", "128x2+96", "top2"])
def test_paired_class_launch_edges(cuda, T, k, rows):
    """The 96- and 128-row classes run in one launch, either part of which
    may be empty (with R = T k routes the 128-row tile cap is 0 below 97
    routes): experts routed exactly the listed row counts (rank r of the
    first tokens), MFMA against the exact path."""
    cfg = dataclasses.replace(small_cfg(T), top_k=k)
    inputs = make_inputs(cfg, tokens=T)
    moe = get_layer(cfg, inputs, cuda)
    ids = np.full((T, k), 0xFFFFFFFF, np.uint32)
    used = np.zeros(T, np.int64)
    for e, n in rows.items():
        order = np.argsort(used, kind="stable")[:n]  # the tokens with the fewest routes
        for t in order:
            ids[t, used[t]] = e
            used[t] += 1
    assert used.max() <= k
    w = np.full(ids.shape, 0.5, np.float32)
    x = L.bf16_tensor(inputs.hidden, cuda)
    r = L.bf16_tensor(inputs.residual, cuda)
    ids_d = torch.from_numpy(ids.view(np.int32)).to(cuda)
    w_d = torch.from_numpy(w).to(cuda)
    out = moe.experts_only(x, ids_d, w_d, residual=r, precision=MFMA)
    exact = moe.experts_only(x, ids_d, w_d, residual=r, precision=EXACT)
    torch.cuda.synchronize()
    assert_close(L.bf16_bits(out), L.bf16_bits(exact), f"paired classes {rows}")


@pytest.mark.parametrize("T,H,F,E,k", [(33, 1024, 1024, 300, 2), (2, 3584, 1024, 300, 8),
                                       (300, 1536, 1536, 64, 4), (100, 3584, 3072, 300, 8),
                                       (257, 2560, 512, 8, 2), (180, 512, 3072, 16, 1)])
def test_shapes_vs_exact(cuda, T, H, F, E, k):
    """Shapes across the MFMA path's domain (hidden, ffn % 512; odd and even
    scale-record counts; top-k 1..8; 2 to 300 tokens; few experts, so
    every tile class fills): MFMA against the exact path, routes
    identical."""
    cfg = dataclasses.replace(CONFIGS[0], name=f"s{T}x{H}x{F}x{E}x{k}", tokens=T, hidden=H, ffn=F,
                              experts=E, top_k=k, seed=800 + T + E)
    inputs = make_inputs(cfg, tokens=T)
    moe = get_layer(cfg, inputs, cuda)
    out, ids, w = forward(moe, inputs, cuda, MFMA)
    exact, ids_e, w_e = forward(moe, inputs, cuda, EXACT)
    np.testing.assert_array_equal(ids, ids_e)
    np.testing.assert_array_equal(w, w_e)
    assert_close(out, exact, f"{cfg.name} mfma vs exact")


def test_k3_shape_mixed_alignment_bitexact(cuda):
    """The K3 shape (hidden 7168, ffn 2048, 896 experts, top-16) at 300
    tokens, every tile class populated, with the odd experts' tensors at 8
    mod 16 (real checkpoint spans): the MFMA path stages them by the same
    16-byte direct-to-LDS loads and gives the bits of the aligned store."""
    cfg = dataclasses.replace(CONFIGS[1], name="k3-300-mixed", tokens=300)
    inputs = make_inputs(cfg, tokens=300)
    ref, ids_a, w_a = forward(get_layer(cfg, inputs, cuda), inputs, cuda, MFMA)
    mixed = L.ExpertStore(cfg.experts, cfg.hidden, cfg.ffn, seed=cfg.seed, device=cuda,
                          misalign=8, misalign_odd=True)
    try:
        got, ids_m, w_m = forward(L.build_layer(cfg, inputs, device=cuda, store=mixed), inputs,
                                  cuda, MFMA)
    finally:
        del mixed
        torch.cuda.empty_cache()
    np.testing.assert_array_equal(ids_m, ids_a)
    np.testing.assert_array_equal(w_m, w_a)
    np.testing.assert_array_equal(got, ref)
