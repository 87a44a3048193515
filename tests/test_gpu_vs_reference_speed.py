"""Speed of the layer against the reference's OWN kernels on the same MI355X
(oracle/_ref/libk3ref_ops.so: the reference's k3_rocm_ops.cu built for gfx950
from its own source with its own flags).

Both sides run from HIP graphs, so only device time is compared (the
reference engine launches from C; a Python launch loop would time Python).
The reference composition is the one test_gpu_refparity checks for
parity: decode as k3_engine.cu:1554-1563, 1032-1066, 1889-1897 (router GEMV,
top-k, per route gate/up/down MXFP4 GEMVs and activation, weighted sum,
add); prefill as k3_engine_prefill.inc:1448-1460, 938-997, 1557-1609
(router GEMM, top-k, per expert gather, gate/up GEMMs, activation, down
GEMM, scatter, weighted sum, add). Its routes and expert plan are fixed
from an eager run first -- the reference engine reads its routes on the
host before it launches the experts (k3_engine.cu:1569-1598) and builds
the prefill plan on the host (k3_engine_prefill.inc:1175-1194) -- and its
graph still replays the router and top-k kernels. The SwiGLU step is this
library's k3_rocm_swiglu_bf16 (the reference ABI has no SwiGLU).

Prints both device times per call and asserts only that the layer is not
slower than the reference on its own headline shapes.
"""
import ctypes
import time

import numpy as np
import pytest
import torch

import _oracle as O
from moonshine_amd import layer as L
import _ops as ops
from moonshine_amd._lib import SIGNATURES
from moonshine_amd.synth import CONFIGS, EXACT, MFMA, make_inputs

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not O.REF_OPS.exists(), reason="reference not built (oracle/_ref)")]


class Ref:
    """The reference's k3_rocm_* launchers on torch's current stream."""

    NAMES = ("k3_rocm_mxfp4_gemv_bf16", "k3_rocm_mxfp4_gemm_bf16", "k3_rocm_bf16_gemv_f32",
             "k3_rocm_bf16_gemm_f32", "k3_rocm_router_topk_f32", "k3_rocm_router_topk_f32_batch",
             "k3_rocm_weighted_sum_bf16", "k3_rocm_weighted_sum_bf16_batch", "k3_rocm_add_bf16",
             "k3_rocm_gather_rows_bf16", "k3_rocm_scatter_rows_bf16")

    def __init__(self):
        self.h = ctypes.CDLL(str(O.REF_OPS))
        for name in self.NAMES:
            res, args = SIGNATURES[name]
            fn = getattr(self.h, name)
            fn.restype, fn.argtypes = res, args

    def __getattr__(self, name):
        fn = getattr(self.h, "k3_rocm_" + name)

        def call(*a):
            conv = [ctypes.c_void_p(x.data_ptr()) if isinstance(x, torch.Tensor) else x for x in a]
            assert fn(*conv, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        return call


def graph_ms(fn, reps):
    """Device time per call of fn() replayed from a HIP graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        fn()
    g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / reps


def u32(t):
    return t.cpu().numpy().view(np.uint32)


def test_decode_speed_vs_reference(cuda):
    cfg = CONFIGS[1]
    inputs = make_inputs(cfg, tokens=1)
    store = L.ExpertStore(cfg.experts, cfg.hidden, cfg.ffn, seed=cfg.seed, device=cuda)
    moe = L.build_layer(cfg, inputs, device=cuda, store=store)
    R = Ref()
    E, k, H, F = cfg.experts, cfg.top_k, cfg.hidden, cfg.ffn
    x = L.bf16_tensor(inputs.hidden, cuda)
    r = L.bf16_tensor(inputs.residual, cuda)
    logits = torch.zeros(E, dtype=torch.float32, device=cuda)
    ids = torch.zeros(k, dtype=torch.int32, device=cuda)
    w = torch.zeros(k, dtype=torch.float32, device=cuda)
    R.bf16_gemv_f32(logits, moe.router_weight, x[0], E, H)
    R.router_topk_f32(ids, w, logits, moe.router_bias, E, k, ctypes.c_float(cfg.scale))
    torch.cuda.synchronize()
    experts = [store.device_expert(int(e)) for e in u32(ids)]
    g = torch.zeros(F, dtype=torch.bfloat16, device=cuda)
    u, a = torch.zeros_like(g), torch.zeros_like(g)
    y = torch.zeros((k, H), dtype=torch.bfloat16, device=cuda)
    c = torch.zeros(H, dtype=torch.bfloat16, device=cuda)
    out_ref = torch.zeros(H, dtype=torch.bfloat16, device=cuda)

    def reference():
        R.bf16_gemv_f32(logits, moe.router_weight, x[0], E, H)
        R.router_topk_f32(ids, w, logits, moe.router_bias, E, k, ctypes.c_float(cfg.scale))
        for rank, (gp, gs, dp, ds, up, us) in enumerate(experts):
            R.mxfp4_gemv_bf16(g, gp, gs, x[0], F, H)
            R.mxfp4_gemv_bf16(u, up, us, x[0], F, H)
            assert ops.k3_rocm_swiglu_bf16(a, g, u, F)
            R.mxfp4_gemv_bf16(y[rank], dp, ds, a, H, F)
        R.weighted_sum_bf16(c, y, w, k, H)
        R.add_bf16(out_ref, r[0], c, H)

    out = torch.empty_like(x)
    ids_o = torch.zeros((1, k), dtype=torch.int32, device=cuda)
    w_o = torch.zeros((1, k), dtype=torch.float32, device=cuda)

    def ours():
        moe.forward(x, r, out=out, ids=ids_o, weights=w_o)

    t_ref = graph_ms(reference, 50)
    t_ours = graph_ms(ours, 50)
    np.testing.assert_array_equal(u32(ids_o)[0], u32(ids))
    print(f"\ncfg1 decode, device time per token: reference kernels {t_ref * 1e3:.1f} us, "
          f"this layer {t_ours * 1e3:.1f} us ({t_ref / t_ours:.2f}x)")
    assert t_ours < t_ref


@pytest.mark.timeout(900)
@pytest.mark.parametrize("cfg_index", [3, 4])
def test_prefill_speed_vs_reference(cuda, cfg_index):
    cfg = CONFIGS[cfg_index]
    T = cfg.tokens
    inputs = make_inputs(cfg, tokens=T)
    store = L.ExpertStore(cfg.experts, cfg.hidden, cfg.ffn, seed=cfg.seed, device=cuda)
    moe = L.build_layer(cfg, inputs, device=cuda, store=store)
    R = Ref()
    E, k, H, F = cfg.experts, cfg.top_k, cfg.hidden, cfg.ffn
    x = L.bf16_tensor(inputs.hidden, cuda)
    r = L.bf16_tensor(inputs.residual, cuda)
    logits = torch.zeros((T, E), dtype=torch.float32, device=cuda)
    ids = torch.zeros((T, k), dtype=torch.int32, device=cuda)
    w = torch.zeros((T, k), dtype=torch.float32, device=cuda)
    R.bf16_gemm_f32(logits, moe.router_weight, x, T, E, H)
    R.router_topk_f32_batch(ids, w, logits, moe.router_bias, T, E, k, ctypes.c_float(cfg.scale))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    counts, offsets, unique, tok, route = O.route_plan(u32(ids), E)
    plan_s = time.perf_counter() - t0
    tok_d = torch.from_numpy(tok.view(np.int32)).to(cuda)
    route_d = torch.from_numpy(route.view(np.int32)).to(cuda)
    nmax = int(counts.max())
    xg = torch.zeros((nmax, H), dtype=torch.bfloat16, device=cuda)
    g = torch.zeros((nmax, F), dtype=torch.bfloat16, device=cuda)
    u, a = torch.zeros_like(g), torch.zeros_like(g)
    yo = torch.zeros((nmax, H), dtype=torch.bfloat16, device=cuda)
    slots = torch.zeros((T * k, H), dtype=torch.bfloat16, device=cuda)
    c = torch.zeros((T, H), dtype=torch.bfloat16, device=cuda)
    out_ref = torch.zeros_like(c)
    plan = [(int(counts[e]), int(offsets[e]), store.device_expert(int(e))) for e in unique]

    def reference():
        R.bf16_gemm_f32(logits, moe.router_weight, x, T, E, H)
        R.router_topk_f32_batch(ids, w, logits, moe.router_bias, T, E, k, ctypes.c_float(cfg.scale))
        for n, o, (gp, gs, dp, ds, up, us) in plan:
            R.gather_rows_bf16(xg, x, tok_d[o:o + n], n, H)
            R.mxfp4_gemm_bf16(g, gp, gs, xg, n, F, H)
            R.mxfp4_gemm_bf16(u, up, us, xg, n, F, H)
            assert ops.k3_rocm_swiglu_bf16(a, g, u, n * F)
            R.mxfp4_gemm_bf16(yo, dp, ds, a, n, H, F)
            R.scatter_rows_bf16(slots, yo, route_d[o:o + n], n, H)
        R.weighted_sum_bf16_batch(c, slots, w, T, k, H)
        R.add_bf16(out_ref, r, c, T * H)

    out = torch.empty_like(x)
    ids_o = torch.zeros((T, k), dtype=torch.int32, device=cuda)
    w_o = torch.zeros((T, k), dtype=torch.float32, device=cuda)
    times = {}
    for name, prec in (("mfma", MFMA), ("exact", EXACT)):
        def ours(prec=prec):
            moe.forward(x, r, out=out, ids=ids_o, weights=w_o, precision=prec)
        times[name] = graph_ms(ours, 3 if cfg_index == 4 else 10)
    t_ref = graph_ms(reference, 1 if cfg_index == 4 else 3)
    print(f"\n{cfg.name} T={T}, device time per layer: reference kernels {t_ref:.2f} ms "
          f"(+ {plan_s * 1e3:.0f} ms host plan), this layer MFMA {times['mfma']:.2f} ms "
          f"({t_ref / times['mfma']:.1f}x), exact {times['exact']:.2f} ms "
          f"({t_ref / times['exact']:.1f}x)")
    assert times["mfma"] < t_ref
