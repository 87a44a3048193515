"""CPU checks of what the certified MFMA router (k3_router.hip) relies on:

1. the choice sigmoid is within 3e-7 of the real sigmoid everywhere. The
   device evaluates the reference's hardware exp2/reciprocal sequence
   (router_sigmoid; pinned on the part by an exhaustive sweep in
   test_gpu_router.py); its CPU restatement k3o_router_sigmoid is checked
   here. The 2e-6 absolute slack of the choice bound covers the error of
   both the approximate and the exact choice twice over;
2. the candidate rule keeps every expert of the exact top-k: with exact
   logits l, approximate logits a anywhere within |a - l| <= err, choices
   c = sigmoid + bias, ce = s'(max(0, |a| - err)) err + 2e-6 + 2^-21 |c|,
   T_k the k-th largest approximate choice and E_k the largest ce at or
   above it, the exact top-k (ties towards the lower id) satisfies
   c~ + ce >= T_k - E_k. Brute force over random and adversarial cases
   (errors pushed to the bound against the true order, exact ties), with
   the slope and ce formed in fp32 in the kernel's order
   (sigmoid_slope_bound: e = 2^(-m log2 e), slope = e / (1 + e)^2, every
   step relative-accurate).
"""
import numpy as np

import _oracle as O

L = O.lib()


def sig64(z):
    return 1.0 / (1.0 + np.exp(-z))


def test_deterministic_sigmoid_error():
    z = np.concatenate([np.linspace(-90, 90, 400001), np.linspace(-4, 4, 100001)]).astype(np.float32)
    want = sig64(z[::5].astype(np.float64))
    for fn in (lambda v: L.k3o_sigmoid(v, 0), L.k3o_router_sigmoid):
        got = np.array([fn(float(v)) for v in z[::5]], np.float64)
        assert np.abs(got - want).max() <= 3e-7


def f32(v):
    return np.float32(v)


def fmaf(a, b, c):
    """fp32 fused multiply-add: the fp32 product is exact in fp64."""
    return f32(np.float64(a) * np.float64(b) + np.float64(c))


def det_sigmoid_f32(z, rng):
    """The real sigmoid rounded to f32, off by up to 3e-7 (the pinned bound)."""
    s = sig64(z.astype(np.float64))
    return (s + rng.uniform(-3e-7, 3e-7, s.shape)).astype(np.float32)


def candidates(a, err, bias, k, rng):
    s = det_sigmoid_f32(a, rng)
    ch = (s + bias).astype(np.float32)
    # the kernel's fp32 sequence (sigmoid_slope_bound): m = max(0, |a| - err);
    # e = 2^(min(m, 88) * -log2 e); r = 1 / (1 + e); slope = ((e r) r) (1 + 2^-10);
    # ce = fma(slope, err, fma(2^-21, |c|, 2e-6))
    m = np.maximum(np.float32(0), (np.abs(a) - err).astype(np.float32)).astype(np.float32)
    tt = (np.minimum(m, np.float32(88)) * np.float32(-1.44269502162933349609375)).astype(np.float32)
    e = np.exp2(tt.astype(np.float64)).astype(np.float32)
    r = (1.0 / (np.float64(1) + e).astype(np.float32).astype(np.float64)).astype(np.float32)
    slope = ((e * r).astype(np.float32) * r).astype(np.float32)
    slope = (slope * np.float32(1.0 + 2.0 ** -10)).astype(np.float32)
    ce = np.array([fmaf(slope[i], err[i], fmaf(4.76837158203125e-7, abs(ch[i]), 2e-6))
                   for i in range(len(ch))], np.float32)
    order = np.lexsort((np.arange(len(ch)), -ch.astype(np.float64)))
    tk = ch[order[k - 1]]
    ek = ce[ch >= tk].max()
    lim = np.float32(tk - ek)
    lim = np.float32(lim - abs(lim) * 2.384185791015625e-7)
    return (ch + ce).astype(np.float32) >= lim


def exact_topk(l, bias, k, rng):
    s = det_sigmoid_f32(l, rng)
    ch = (s + bias).astype(np.float32).astype(np.float64)
    order = np.lexsort((np.arange(len(ch)), -ch))
    return order[:k]


def test_candidate_rule_keeps_exact_topk():
    rng = np.random.default_rng(11)
    for trial in range(3000):
        E = int(rng.choice([16, 64, 300, 896, 1024]))
        k = int(rng.integers(1, min(E, 32) + 1))
        spread = float(rng.choice([0.1, 1.0, 3.0, 20.0]))
        l = rng.normal(0, spread, E).astype(np.float32)
        if trial % 7 == 0:  # exact ties
            l[1::2] = l[0::2][: len(l[1::2])]
        bias = (rng.normal(0, float(rng.choice([0.0, 0.01, 0.5, 5.0])), E)).astype(np.float32)
        if trial % 11 == 0:
            bias[:] = bias[0]
        if trial % 5 == 0:  # logits out in the sigmoid's tail, small and large errors
            l = (rng.choice([-1.0, 1.0], E) * rng.uniform(8.0, 17.0, E)).astype(np.float32)
        err = (np.abs(rng.normal(0, 0.01, E)) * float(rng.choice([0.01, 1.0, 30.0]))).astype(np.float32)
        if trial % 13 == 0:
            err = rng.uniform(10.0, 100.0, E).astype(np.float32)
        # approximate logits: random within the bound, or pushed to the bound
        # against the exact order (top experts down, the rest up)
        if trial % 2:
            a = l + err * rng.uniform(-1, 1, E).astype(np.float32)
        else:
            top = exact_topk(l, bias, k, rng)
            sgn = np.ones(E, np.float32)
            sgn[top] = -1.0
            a = l + sgn * err
        a = a.astype(np.float32)
        cand = candidates(a, err, bias, k, rng)
        want = exact_topk(l, bias, k, rng)
        assert cand[want].all(), (trial, E, k)
        assert cand.sum() >= k


def test_slope_bound_covers_the_sigmoid_slope():
    """The kernel's slope (sigmoid_slope_bound: e = 2^(-m log2 e), slope =
    ((e r) r)(1 + 2^-10), r = 1 / (1 + e)) is at least the real slope
    s(m)(1 - s(m)) over [0, 88), with 4 ulp of slack for the hardware exp2
    and reciprocal (each within 1 ulp), and the real slope is below 2^-126
    past 88, where the kernel returns 0."""
    m = np.concatenate([np.linspace(0, 88, 2_000_001), np.geomspace(1e-8, 88, 200_001)])
    m = m.astype(np.float32)
    tt = (np.minimum(m, np.float32(88)) * np.float32(-1.44269502162933349609375)).astype(np.float32)
    e = np.exp2(tt.astype(np.float64)).astype(np.float32)
    r = (1.0 / (np.float64(1) + e).astype(np.float32).astype(np.float64)).astype(np.float32)
    slope = ((e * r).astype(np.float32) * r).astype(np.float32)
    slope = (slope * np.float32(1.0 + 2.0 ** -10)).astype(np.float64)
    md = m.astype(np.float64)
    real = np.exp(-md) / (1.0 + np.exp(-md)) ** 2
    assert (slope * (1.0 - 4 * 2.0 ** -23) >= real).all()
    assert np.exp(-88.0) < 2.0 ** -126
