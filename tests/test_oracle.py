"""Pins the CPU oracle (test infrastructure) against independent facts:
library routines (glibc via numpy/math, torch's bf16 cast), closed forms,
brute force on small inputs and the reference's own literal constants.
"""
import math

import numpy as np
import pytest
import torch

import _oracle as O
from moonshine_amd.synth import CONFIGS, bf16_bits_to_f32, f32_to_bf16_bits, make_inputs

L = O.lib()


def ulp_diff(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


def test_bf16_round_trip_and_rne_against_torch():
    rng = np.random.default_rng(0)
    f = np.concatenate([rng.normal(0, 10, 20000), rng.normal(0, 1e-30, 2000),
                        [0.0, -0.0, 1.0, 65504.0, 3.4e38, -3.4e38, np.inf, -np.inf]]).astype(np.float32)
    ties = (np.arange(1000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    f = np.concatenate([f, ties])
    want = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([L.k3o_f32_to_bf16(float(v)) for v in f], np.uint16)
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(f32_to_bf16_bits(f), want)
    for b in range(0, 65536, 97):
        v = L.k3o_bf16_to_f32(b)
        if not math.isnan(v):
            assert L.k3o_f32_to_bf16(v) == b
    assert math.isnan(L.k3o_bf16_to_f32(L.k3o_f32_to_bf16(float("nan"))))


def test_e2m1_e8m0_tables_exhaustive():
    for n in range(16):
        s, e, m = n >> 3, (n >> 1) & 3, n & 1
        mag = m * 0.5 if e == 0 else (1 + m / 2) * 2.0 ** (e - 1)  # OCP MX e2m1
        v = L.k3o_e2m1(n)
        assert v == (-mag if s else mag) and math.copysign(1, v) == (-1 if s else 1)
    for e in range(1, 255):
        assert L.k3o_e8m0(e) == 2.0 ** (e - 127)
    assert L.k3o_e8m0(0) == 2.0 ** -127  # reference bit pattern 0x00400000
    assert L.k3o_e8m0(255) == math.inf


def test_expf_and_tanhf_accuracy():
    x = np.concatenate([np.linspace(-103.9, 88.7, 200001), np.linspace(-1, 1, 20001)]).astype(np.float32)
    got = np.array([L.k3o_expf(float(v)) for v in x[::7]], np.float32)
    want = np.exp(x[::7].astype(np.float64)).astype(np.float32)
    normal = want > 1.2e-38
    assert ulp_diff(got[normal], want[normal]).max() <= 2
    assert np.all(np.abs(got[~normal] - want[~normal]) <= 2.0 ** -148)
    assert L.k3o_expf(0.0) == 1.0 and L.k3o_expf(100.0) == math.inf and L.k3o_expf(-110.0) == 0.0
    y = np.linspace(-12, 12, 100001).astype(np.float32)
    got = np.array([L.k3o_tanhf(float(v)) for v in y[::3]], np.float32)
    want = np.tanh(y[::3].astype(np.float64)).astype(np.float32)
    assert ulp_diff(got, want).max() <= 4
    assert L.k3o_tanhf(0.0) == 0.0 and L.k3o_tanhf(20.0) == 1.0 and L.k3o_tanhf(-20.0) == -1.0


def test_logits_orders_vs_fp64_and_kat():
    rng = np.random.default_rng(1)
    E, H, T = 37, 7168, 3
    w = f32_to_bf16_bits(rng.normal(0, 0.02, (E, H)).astype(np.float32))
    x = f32_to_bf16_bits(rng.normal(0, 1, (T, H)).astype(np.float32))
    exact = bf16_bits_to_f32(x).astype(np.float64) @ bf16_bits_to_f32(w).astype(np.float64).T
    bound = (np.abs(bf16_bits_to_f32(x)).astype(np.float64) @ np.abs(bf16_bits_to_f32(w)).T) * H * 2.0 ** -24
    for order in (O.ORDER_W64, O.ORDER_REF, O.ORDER_F64):
        got = O.router_logits(w, x, order)
        assert np.all(np.abs(got - exact) <= bound + 1e-30)
    # single nonzero product: exact in every order
    w1 = np.zeros((2, 100), np.uint16)
    x1 = np.zeros((1, 100), np.uint16)
    w1[0, 77] = f32_to_bf16_bits(np.float32(1.5))
    w1[1, 3] = f32_to_bf16_bits(np.float32(-0.375))
    x1[0, 77] = f32_to_bf16_bits(np.float32(3.0))
    x1[0, 3] = f32_to_bf16_bits(np.float32(2.0))
    for order in (O.ORDER_W64, O.ORDER_REF):
        np.testing.assert_array_equal(O.router_logits(w1, x1, order), [[4.5, -0.75]])
    # batch == sequential
    full = O.router_logits(w, x)
    for t in range(T):
        np.testing.assert_array_equal(O.router_logits(w, x[t:t + 1])[0], full[t])


def test_topk_special_cases_and_brute_force():
    E, k = 896, 16
    logits = np.zeros((1, E), np.float32)
    bias = np.zeros(E, np.float32)
    ids, w = O.router_topk(logits, bias, k, 2.5)
    np.testing.assert_array_equal(ids[0], np.arange(k))  # ties -> lower id
    np.testing.assert_allclose(w[0], 2.5 / k, rtol=1e-6)
    rng = np.random.default_rng(2)
    bias = rng.normal(0, 10, E).astype(np.float32)  # bias dominates
    ids, _ = O.router_topk(logits, bias, k, 1.0)
    np.testing.assert_array_equal(ids[0], np.argsort(-bias, kind="stable")[:k])
    for trial in range(20):
        logits = rng.normal(0, 1.7, (1, E)).astype(np.float32)
        if trial % 2:
            logits[0, ::5] = logits[0, 1]
        bias = rng.normal(0, 0.01, E).astype(np.float32)
        ids, w = O.router_topk(logits, bias, k, 2.5)
        score = np.array([L.k3o_sigmoid(float(v), 0) for v in logits[0]], np.float32)
        choice = (score + bias).astype(np.float32)
        brute = sorted(range(E), key=lambda e: (-float(choice[e]), e))[:k]
        np.testing.assert_array_equal(ids[0], brute)
        np.testing.assert_allclose(w[0].sum(dtype=np.float64), 2.5, rtol=1e-6)
        np.testing.assert_allclose(w[0], score[brute] / score[brute].sum() * 2.5, rtol=2e-6)


@pytest.mark.parametrize("T,k,E", [(1, 16, 896), (50, 4, 64), (300, 16, 896)])
def test_route_plan_brute_force(T, k, E):
    rng = np.random.default_rng(T)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32)
    counts, offsets, unique, tok, route = O.route_plan(ids, E)
    flat = ids.reshape(-1)
    order = sorted(range(T * k), key=lambda i: (int(flat[i]), i))
    np.testing.assert_array_equal(route, order)
    np.testing.assert_array_equal(tok, np.array(order) // k)
    np.testing.assert_array_equal(counts, np.bincount(flat, minlength=E))
    np.testing.assert_array_equal(unique, np.nonzero(counts)[0])
    assert offsets[-1] == T * k and sorted(route.tolist()) == list(range(T * k))
    # the reference's own loop (k3_engine_prefill.inc:1175-1194), literally
    for e in unique[:5]:
        lst = [(t, t * k + r) for t in range(T) for r in range(k) if ids[t, r] == e]
        a, b = offsets[e], offsets[e + 1]
        assert list(zip(tok[a:b], route[a:b])) == lst


def test_mxfp4_orders_vs_fp64_envelope_and_kat():
    rng = np.random.default_rng(4)
    for rows, cols in ((512, 3584), (512, 3072), (64, 7168)):
        p = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
        s = rng.integers(121, 126, (rows, cols // 32), dtype=np.uint8)
        x = f32_to_bf16_bits(rng.normal(0, 1, (2, cols)).astype(np.float32))
        _, f64 = O.mxfp4_gemm(p, s, x, rows, cols, O.ORDER_F64)
        for order in (O.ORDER_W64, O.ORDER_REF):
            got, f = O.mxfp4_gemm(p, s, x, rows, cols, order)
            # reference envelope: <= 0.25 abs or <= 1% rel vs fp64
            # (tests/test_k3_mxfp4_envelope.cu:334-341), here much tighter
            err = np.abs(bf16_bits_to_f32(got) - f64)
            assert np.all((err <= 0.25) | (err <= 0.01 * np.abs(f64)))
            assert np.all(np.abs(f - f64) <= 1e-5 * np.maximum(1, np.abs(f64)))
    # single nonzero weight: exact power-of-two product
    p = np.zeros((1, 32), np.uint8)
    s = np.full((1, 2), 127, np.uint8)
    p[0, 20] = 0x70  # column 41 = +6.0
    s[0, 1] = 130   # x 8
    x = np.zeros((1, 64), np.uint16)
    x[0, 41] = f32_to_bf16_bits(np.float32(-1.25))
    got, _ = O.mxfp4_gemm(p, s, x, 1, 64)
    assert bf16_bits_to_f32(got)[0, 0] == -60.0


def test_weighted_sum_add_by_hand():
    v = f32_to_bf16_bits(np.array([[[1.0, 2.0], [3.0, -4.0], [0.5, 8.0]]], np.float32))
    w = np.array([[0.5, 0.25, 2.0]], np.float32)
    got = bf16_bits_to_f32(O.weighted_sum(v, w))
    np.testing.assert_array_equal(got, [[0.5 + 0.75 + 1.0, 1.0 - 1.0 + 16.0]])
    a = f32_to_bf16_bits(np.array([1.0, 256.0], np.float32))
    b = f32_to_bf16_bits(np.array([2.0 ** -9, 1.0], np.float32))
    np.testing.assert_array_equal(bf16_bits_to_f32(O.add(a, b)), [1.0, 257.0 if False else 256.0])


def test_activations_vs_libm():
    rng = np.random.default_rng(5)
    g = f32_to_bf16_bits(rng.normal(0, 5, 20000).astype(np.float32))
    u = f32_to_bf16_bits(rng.normal(0, 40, 20000).astype(np.float32))
    for fn, kw in ((O.situ, {}), (O.swiglu, {})):
        det = bf16_bits_to_f32(fn(g, u, **kw))
        lib = bf16_bits_to_f32(fn(g, u, use_libm=True, **kw))
        # same bf16 except at rounding boundaries (<= 1 bf16 ulp)
        assert np.max(np.abs(det - lib) / np.maximum(np.abs(lib), 1e-30)) <= 2.0 ** -7
        assert np.mean(det == lib) > 0.99
    gf, uf = bf16_bits_to_f32(g).astype(np.float64), bf16_bits_to_f32(u).astype(np.float64)
    ref = 4 * np.tanh(gf / 4) / (1 + np.exp(-gf)) * 25 * np.tanh(uf / 25)
    got = bf16_bits_to_f32(O.situ(g, u))
    assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-30)


def test_reduced_layer_orders_agree_and_golden():
    cfg = CONFIGS[0]
    inputs = make_inputs(cfg)
    rng = np.random.default_rng(cfg.seed)
    ids = O.router_topk(O.router_logits(inputs.router_weight, inputs.hidden), inputs.router_bias,
                        cfg.top_k, cfg.scale)[0]
    sizes = (cfg.ffn * cfg.hidden // 2, cfg.ffn * cfg.hidden // 32) * 3
    experts = {}
    for e in ids[0]:
        experts[int(e)] = [rng.integers(0, 256, n, dtype=np.uint8) if j % 2 == 0 else
                           rng.integers(121, 126, n, dtype=np.uint8) for j, n in enumerate(sizes)]
    a = O.layer(cfg, inputs, experts, order=O.ORDER_W64)
    b = O.layer(cfg, inputs, experts, order=O.ORDER_F64)
    c = O.layer(cfg, inputs, experts, order=O.ORDER_REF)
    np.testing.assert_array_equal(a["ids"], b["ids"])
    fa, fb, fc = (bf16_bits_to_f32(z["output"]).astype(np.float64) for z in (a, b, c))
    assert np.linalg.norm(fa - fb) / np.linalg.norm(fb) < 5e-3
    assert np.linalg.norm(fc - fb) / np.linalg.norm(fb) < 5e-3


def test_prefill_workspace_ledger_reference_constants():
    w = O.Workspace()
    for chunk in (1, 512, 8192):
        assert L.k3o_prefill_workspace(chunk, w) == 0
        # tests/test_k3_prefill_plan.c:24,69-76 (K3_ONE_TOKEN_WORKSPACE)
        assert w.batch_workspace_bytes == 1116360 * chunk
        assert w.incremental_workspace_bytes == 1116360 * (chunk - 1)
        assert w.mla_append_bytes == chunk * 24 * 576 * 2
