"""GPU parity of the certified MFMA router (k3_moe_router_bf16) against the
exact prefill router pair k3_rocm_bf16_gemm_f32 + k3_rocm_router_topk_f32_batch
(k3_engine_prefill.inc:1448-1460): ids and weights bit-identical on every
token, including exact ties, all-zero, huge, tiny and non-finite tokens."""
import ctypes

import numpy as np
import pytest
import torch

import _ops as ops
from moonshine_amd._lib import lib
from moonshine_amd.synth import CONFIGS, f32_to_bf16_bits, make_inputs

pytestmark = pytest.mark.gpu


def dev(a, cuda):
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def exact_routes(w, b, x, T, E, H, k, scale, cuda):
    logits = torch.empty((T, E), dtype=torch.float32, device=cuda)
    ids = torch.empty((T, k), dtype=torch.int32, device=cuda)
    wts = torch.empty((T, k), dtype=torch.float32, device=cuda)
    assert ops.k3_rocm_bf16_gemm_f32(logits, w, x, T, E, H)
    assert ops.k3_rocm_router_topk_f32_batch(ids, wts, logits, b, T, E, k, scale)
    torch.cuda.synchronize()
    return ids.cpu().numpy(), wts.cpu().numpy(), logits.cpu().numpy()


def certified_routes(w, b, x, T, E, H, k, scale, cuda):
    need = lib().k3_moe_router_scratch_bytes(T, E)
    assert need > 0
    scratch = torch.empty(need, dtype=torch.uint8, device=cuda)
    ids = torch.full((T, k), -7, dtype=torch.int32, device=cuda)
    wts = torch.full((T, k), -7.0, dtype=torch.float32, device=cuda)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    assert lib().k3_moe_router_bf16(P(ids), P(wts), P(x), P(w), P(b), T, E, H, k, scale,
                                    P(scratch), need,
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    approx = scratch[:4 * T * E].view(torch.float32).view(T, E).cpu().numpy()
    return ids.cpu().numpy(), wts.cpu().numpy(), approx


def check(w_bits, bias, x_bits, k, scale, cuda, bound_rows=None):
    T, H = x_bits.shape
    E = w_bits.shape[0]
    w = dev(w_bits.view(np.int16), cuda)
    b = dev(bias.astype(np.float32), cuda)
    x = dev(x_bits.view(np.int16), cuda)
    want_ids, want_w, logits = exact_routes(w, b, x, T, E, H, k, scale, cuda)
    got_ids, got_w, approx = certified_routes(w, b, x, T, E, H, k, scale, cuda)
    np.testing.assert_array_equal(got_ids, want_ids)
    np.testing.assert_array_equal(got_w.view(np.uint32), want_w.view(np.uint32))
    if bound_rows is not None and T >= 32:
        # the MFMA logits sit inside the error bound the candidates rely on:
        # |a - l| <= (H / 32 + 270) u ||w_e|| ||x_t||, u = 2^-24 (both sums'
        # rounding)
        wf = (w_bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        xf = (x_bits[bound_rows].astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        scale_ = np.linalg.norm(xf, axis=1)[:, None] * np.linalg.norm(wf, axis=1)[None, :]
        diff = np.abs(approx[bound_rows].astype(np.float64) - logits[bound_rows])
        bound = (H // 32 + 270) * 2.0 ** -24 * scale_
        assert (diff <= bound).all(), float((diff / bound).max())
    return got_ids


def bf16(a):
    return f32_to_bf16_bits(np.asarray(a, dtype=np.float32))


def test_certified_router_k3_prefill(cuda):
    """The cfg4 batch: 8192 tokens, 896 experts, hidden 7168, top-16."""
    cfg = CONFIGS[4]
    inp = make_inputs(cfg)
    check(inp.router_weight, inp.router_bias, inp.hidden, cfg.top_k, cfg.scale, cuda,
          bound_rows=np.arange(0, cfg.tokens, 97))


@pytest.mark.parametrize("T,E,H,k", [(128, 64, 512, 4), (300, 200, 1024, 8), (517, 896, 7168, 16),
                                     (1000, 1024, 8192, 32), (130, 40, 64, 1), (33, 896, 7168, 16),
                                     (64, 256, 2048, 8), (31, 64, 512, 4), (129, 896, 7168, 16),
                                     (257, 1000, 1024, 8), (1024, 896, 7168, 16),
                                     (1500, 300, 1024, 8), (2048, 64, 512, 32)])
def test_certified_router_shapes(cuda, T, E, H, k):
    rng = np.random.default_rng(T * 7 + E)
    w = bf16(rng.normal(0, 0.02, (E, H)))
    b = (rng.normal(0, 0.01, E)).astype(np.float32)
    x = bf16(rng.normal(0, 1, (T, H)))
    check(w, b, x, k, 2.5, cuda, bound_rows=np.arange(T))


@pytest.mark.parametrize("T", [256, 1100])
def test_certified_router_adversarial(cuda, T):
    """Exact logit ties (duplicated router rows, equal biases), all-zero
    tokens (every choice equal), huge, tiny and non-finite tokens, and a
    bias that dominates the logits; at 1100 tokens (one wave per token)
    also one bias for every expert, so the all-zero token's 256 keys tie
    (more than 64 at the threshold: the full bitwise search)."""
    rng = np.random.default_rng(5)
    E, H, k = 256, 1024, 8
    wf = rng.normal(0, 0.02, (E, H)).astype(np.float32)
    wf[1::2] = wf[0::2]  # rows 2j and 2j + 1 equal
    w = bf16(wf)
    b = np.repeat(rng.normal(0, 0.01, E // 2), 2).astype(np.float32)
    xf = rng.normal(0, 1, (T, H)).astype(np.float32)
    xf[0] = 0.0
    xf[1] *= 1e30
    xf[2] *= 1e-30
    xf[3, 7] = np.nan
    xf[4, 9] = np.inf
    xf[5, 11] = -np.inf
    xf[6] = 3e38  # logits overflow
    xf[7] = xf[8]
    x = bf16(xf)
    ids = check(w, b, x, k, 1.0, cuda)
    # ties resolved towards the lower id, like the exact router
    assert (ids[9:] >= 0).all()
    big_bias = rng.normal(0, 10.0, E).astype(np.float32)
    check(w, big_bias, x, k, 1.0, cuda)
    if T > 1000:
        check(w, np.full(E, 0.25, np.float32), x, k, 1.0, cuda)


def test_router_sigmoid_exhaustive_bound(cuda):
    """The router's choice sigmoid (the reference's hardware exp2/reciprocal
    sequence, k3_moe_router_choices_f32 with no bias) on EVERY fp32 logit in
    [-100, 100]: within 3e-7 of the real sigmoid, the bound the certified
    router's choice error (k3_router.hip) assumes. Also the share of inputs
    where the CPU restatement k3o_router_sigmoid (correctly rounded exp2 and
    reciprocal) equals the device bits, on a random sample."""
    import _oracle as O
    worst = 0.0
    top = np.float32(100.0).view(np.int32)
    step = 1 << 27
    for sign in (0, 1 << 31):
        for lo in range(0, int(top) + 1, step):
            hi = min(lo + step, int(top) + 1)
            bits = torch.arange(lo, hi, dtype=torch.int64, device=cuda)
            bits = (bits | sign).to(torch.int64)
            bits = torch.where(bits >= 1 << 31, bits - (1 << 32), bits).to(torch.int32)
            x = bits.view(torch.float32)
            out = torch.empty_like(x)
            assert lib().k3_moe_router_choices_f32(ctypes.c_void_p(out.data_ptr()),
                                                   ctypes.c_void_p(x.data_ptr()), None, 1,
                                                   x.numel(), None)
            ref = torch.sigmoid(x.double())
            worst = max(worst, float((out.double() - ref).abs().max()))
            del bits, x, out, ref
    print(f"\nrouter sigmoid: worst |s - sigmoid| over all fp32 in [-100, 100] = {worst:.3g}")
    assert worst <= 3e-7
    rng = np.random.default_rng(3)
    xs = np.concatenate([rng.normal(0, 3, 100000), rng.uniform(-40, 40, 100000)]).astype(np.float32)
    out = torch.empty(xs.size, dtype=torch.float32, device=cuda)
    assert lib().k3_moe_router_choices_f32(ctypes.c_void_p(out.data_ptr()),
                                           ctypes.c_void_p(dev(xs, cuda).data_ptr()), None, 1,
                                           xs.size, None)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    emu = np.array([O.lib().k3o_router_sigmoid(float(v)) for v in xs], np.float32)
    same = float((got.view(np.uint32) == emu.view(np.uint32)).mean())
    ulps = np.abs(got.view(np.int32).astype(np.int64) - emu.view(np.int32).astype(np.int64))
    i = int(np.argmax(ulps))
    print(f"router sigmoid: CPU restatement equals the device on {same:.4%} of "
          f"{xs.size} inputs, max {ulps.max()} ulp apart (at x = {xs[i]!r})")
    assert same >= 0.8
    assert np.abs(got.astype(np.float64) - emu).max() <= 4 * 2.0 ** -24


def test_router_choices_with_bias(cuda):
    rng = np.random.default_rng(5)
    T, E = 3, 896
    lg = rng.normal(0, 2, (T, E)).astype(np.float32)
    b = rng.normal(0, 0.1, E).astype(np.float32)
    out = torch.empty((T, E), dtype=torch.float32, device=cuda)
    s = torch.empty((T, E), dtype=torch.float32, device=cuda)
    dl = dev(lg, cuda)
    assert lib().k3_moe_router_choices_f32(ctypes.c_void_p(out.data_ptr()),
                                           ctypes.c_void_p(dl.data_ptr()),
                                           ctypes.c_void_p(dev(b, cuda).data_ptr()), T, E, None)
    assert lib().k3_moe_router_choices_f32(ctypes.c_void_p(s.data_ptr()),
                                           ctypes.c_void_p(dl.data_ptr()), None, T, E, None)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), (s.cpu().numpy() + b).astype(np.float32))
