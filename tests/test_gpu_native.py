"""GPU parity of the K3-native MoE layer (k3_moe_native_forward_bf16)
against the oracle composed from its pinned pieces (router, Q8-128 / bf16
static projections, routed experts on the latent, RMSNorm, SiTU shared
expert, adds). Exact precision is bit-identical end to end."""
import numpy as np
import pytest
import torch

import _oracle as O
from moonshine_amd import native as N
from moonshine_amd.layer import bf16_bits, bf16_tensor
from moonshine_amd.synth import f32_to_bf16_bits

pytestmark = pytest.mark.gpu

SMALL = N.NativeConfig("native-small", 1, 1024, 512, 64, 4, 256, 768, seed=2001)


def host_statics(layer):
    return {name: w.host() for name, w in layer.statics().items()}


def run_and_check(cfg, T, cuda, layer=None, residual=True, precision=0):
    layer = layer or N.NativeLayer(cfg, device=cuda)
    rng = np.random.default_rng(cfg.seed + T)
    x = f32_to_bf16_bits(rng.normal(0, 1, (T, cfg.hidden)).astype(np.float32))
    r = f32_to_bf16_bits(rng.normal(0, 1, (T, cfg.hidden)).astype(np.float32)) if residual else None
    ids = torch.zeros((T, cfg.top_k), dtype=torch.int32, device=cuda)
    w = torch.zeros((T, cfg.top_k), dtype=torch.float32, device=cuda)
    out = layer.forward(bf16_tensor(x, cuda), None if r is None else bf16_tensor(r, cuda),
                        ids=ids, weights=w, precision=precision)
    torch.cuda.synchronize()
    got = bf16_bits(out)
    got_ids = ids.cpu().numpy().view(np.uint32)
    experts = {int(e): layer.store.host_expert(int(e)) for e in np.unique(got_ids)}
    want = O.native_layer(cfg, layer.router_weight_bits, layer.router_bias, layer.norm_bits,
                          host_statics(layer), x, r, experts)
    np.testing.assert_array_equal(got_ids, want["ids"])
    np.testing.assert_array_equal(w.cpu().numpy(), want["weights"])
    return got, want, layer


@pytest.mark.parametrize("kind", [N.STATIC_Q8, N.STATIC_BF16])
@pytest.mark.parametrize("T", [1, 5, 160])  # 160: the certified MFMA router
def test_native_small_bitexact(cuda, kind, T):
    cfg = N.NativeConfig(SMALL.name, T, SMALL.hidden, SMALL.latent, SMALL.experts, SMALL.top_k,
                         SMALL.ffn, SMALL.shared, static_kind=kind, seed=SMALL.seed + kind)
    got, want, _ = run_and_check(cfg, T, cuda)
    np.testing.assert_array_equal(got, want["output"])


def test_native_without_residual(cuda):
    got, want, _ = run_and_check(SMALL, 3, cuda, residual=False)
    np.testing.assert_array_equal(got, want["output"])


def test_native_k3_decode_bitexact(cuda):
    """The K3 layer at its real size, one token, Q8-128 static projections."""
    got, want, _ = run_and_check(N.K3_NATIVE_LAYER, 1, cuda)
    np.testing.assert_array_equal(got, want["output"])


@pytest.mark.timeout(600)
def test_native_k3_mfma_batch_close_to_exact(cuda):
    """The K3 layer at its real size (latent 3584: an odd count of 16-byte
    scale records per gate/up weight row; F 3072), 64 tokens under the
    MXFP8 precision against the exact precision of the same layer: the
    same routes and weights, outputs within the MFMA bound."""
    cfg = N.K3_NATIVE_LAYER
    T = 64
    layer = N.NativeLayer(cfg, device=cuda)
    rng = np.random.default_rng(cfg.seed + T)
    x = bf16_tensor(f32_to_bf16_bits(rng.normal(0, 1, (T, cfg.hidden)).astype(np.float32)), cuda)
    r = bf16_tensor(f32_to_bf16_bits(rng.normal(0, 1, (T, cfg.hidden)).astype(np.float32)), cuda)
    res = []
    for precision in (0, 1):
        ids = torch.zeros((T, cfg.top_k), dtype=torch.int32, device=cuda)
        w = torch.zeros((T, cfg.top_k), dtype=torch.float32, device=cuda)
        out = layer.forward(x, r, ids=ids, weights=w, precision=precision)
        torch.cuda.synchronize()
        res.append((bf16_bits(out), ids.cpu().numpy(), w.cpu().numpy()))
    (ge, ie, we), (gm, im, wm) = res
    np.testing.assert_array_equal(im, ie)
    np.testing.assert_array_equal(wm, we)
    gf = (gm.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    wf = (ge.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    rel = np.linalg.norm(gf - wf) / np.linalg.norm(wf)
    print(f"\nK3-native T={T}: MFMA vs exact rel-L2 {rel:.3g}")
    assert rel <= 2e-3, rel


def test_native_mfma_close_to_exact(cuda):
    """MFMA expert products inside the native layer: routes stay exact; the
    output is within the MFMA precision's stated bound of the exact one."""
    cfg = N.NativeConfig("native-mfma", 40, 1024, 512, 64, 4, 512, 768, seed=2003)
    layer = N.NativeLayer(cfg, device=cuda)
    got, want, _ = run_and_check(cfg, 40, cuda, layer=layer, precision=1, residual=False)
    gf = (got.astype(np.uint32) << 16).view(np.float32)
    wf = (want["output"].astype(np.uint32) << 16).view(np.float32)
    rel = np.linalg.norm(gf - wf) / np.linalg.norm(wf)
    assert rel <= 2e-3, rel


@pytest.mark.parametrize("kind", [N.STATIC_Q8, N.STATIC_BF16])
def test_native_mfma_projections_close_to_exact(cuda, kind):
    """A batch under the MXFP8 precision: the static projections run on
    bf16 MFMA too (exact products, another fp32 summation order). Routes
    stay exact; the output is within the MFMA precision's bound."""
    T = 300
    cfg = N.NativeConfig("native-proj", T, 1024, 512, 64, 4, 512, 768, static_kind=kind,
                         seed=2100 + kind)
    got, want, _ = run_and_check(cfg, T, cuda, precision=1)
    gf = (got.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    wf = (want["output"].astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    rel = np.linalg.norm(gf - wf) / np.linalg.norm(wf)
    assert rel <= 2e-3, rel


@pytest.mark.parametrize("T", [1, 5])
def test_native_shared_stream_same_bits(cuda, T):
    """The shared-stream form (latent projection and shared gate/up on a
    second stream, joined by events) gives the same bits, call after call."""
    layer = N.NativeLayer(SMALL, device=cuda)
    side = torch.cuda.Stream()
    rng = np.random.default_rng(77 + T)
    xs = [f32_to_bf16_bits(rng.normal(0, 1, (T, SMALL.hidden)).astype(np.float32)) for _ in range(2)]
    rs = [f32_to_bf16_bits(rng.normal(0, 1, (T, SMALL.hidden)).astype(np.float32)) for _ in range(2)]
    statics = host_statics(layer)
    want = []
    for x, r in zip(xs, rs):
        ids = O.router_topk(O.router_logits(layer.router_weight_bits, x), layer.router_bias,
                            SMALL.top_k, SMALL.scale)[0]
        experts = {int(e): layer.store.host_expert(int(e)) for e in np.unique(ids)}
        want.append(O.native_layer(SMALL, layer.router_weight_bits, layer.router_bias,
                                   layer.norm_bits, statics, x, r, experts)["output"])
    dx = [bf16_tensor(x, cuda) for x in xs]
    dr = [bf16_tensor(r, cuda) for r in rs]
    for rep in range(6):
        i = rep % 2
        out = layer.forward(dx[i], dr[i], shared_stream=side.cuda_stream)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bf16_bits(out), want[i])


@pytest.mark.parametrize("streams", [1, 2])
def test_native_graph_replay_same_bits(cuda, streams):
    """One-token calls captured in a HIP graph (with and without the shared
    stream) give the oracle's bits on every replay, with eager calls that
    reuse the workspace between the replays."""
    layer = N.NativeLayer(SMALL, device=cuda)
    side = torch.cuda.Stream()
    rng = np.random.default_rng(91 + streams)
    xs = [f32_to_bf16_bits(rng.normal(0, 1, (1, SMALL.hidden)).astype(np.float32)) for _ in range(3)]
    rs = [f32_to_bf16_bits(rng.normal(0, 1, (1, SMALL.hidden)).astype(np.float32)) for _ in range(3)]
    statics = host_statics(layer)
    want = []
    for x, r in zip(xs, rs):
        ids = O.router_topk(O.router_logits(layer.router_weight_bits, x), layer.router_bias,
                            SMALL.top_k, SMALL.scale)[0]
        experts = {int(e): layer.store.host_expert(int(e)) for e in np.unique(ids)}
        want.append(O.native_layer(SMALL, layer.router_weight_bits, layer.router_bias,
                                   layer.norm_bits, statics, x, r, experts)["output"])
    dx = [bf16_tensor(x, cuda) for x in xs]
    dr = [bf16_tensor(r, cuda) for r in rs]
    outs = [torch.zeros_like(dx[0]) for _ in range(2)]
    shared = side.cuda_stream if streams == 2 else None
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap):
        layer.forward(dx[0], dr[0], out=outs[0], stream=cap.cuda_stream, shared_stream=shared)
        cap.synchronize()
        with torch.cuda.graph(g, stream=cap):
            for i in range(2):
                layer.forward(dx[i], dr[i], out=outs[i], stream=cap.cuda_stream,
                              shared_stream=shared)
    torch.cuda.synchronize()
    for rep in range(4):
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i in range(2):
            np.testing.assert_array_equal(bf16_bits(outs[i]), want[i], err_msg=f"replay {rep}")
        eager = layer.forward(dx[2], dr[2])  # eager work on the same workspace
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bf16_bits(eager), want[2])


@pytest.mark.parametrize("q8", [True, False])
@pytest.mark.parametrize("T,rows,cols", [(1, 200, 384), (33, 200, 384), (130, 129, 1024),
                                         (256, 256, 512)])
def test_proj_mfma_ragged_vs_row_kernels(cuda, q8, T, rows, cols):
    """k3_moe_proj_mfma_bf16 at ragged token and row counts (partial
    128 x 128 tiles, clamped rows) against the exact row kernels. Each
    output may differ from the row kernel's by the two fp32 summation
    orders' error (at most 2 K u sum |products| between them, u = 2^-24)
    plus one bf16 rounding step of the larger value; most elements are
    identical."""
    import ctypes
    import _ops as ops
    from moonshine_amd._lib import lib
    rng = np.random.default_rng(T * 1000 + rows + cols + q8)
    x = f32_to_bf16_bits(rng.normal(0, 1, (T, cols)).astype(np.float32))
    xd = torch.from_numpy(x.view(np.int16)).to(cuda)
    if q8:
        q = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
        s = (rng.random((rows, cols // 128)) * 1e-2 + 1e-3).astype(np.float32)
        wd, sd = torch.from_numpy(q).to(cuda), torch.from_numpy(s).to(cuda)
        wf = q.astype(np.float64) * np.repeat(s.astype(np.float64), 128, axis=1)
    else:
        w = f32_to_bf16_bits(rng.normal(0, 0.05, (rows, cols)).astype(np.float32))
        wd, sd = torch.from_numpy(w.view(np.int16)).to(cuda), None
        wf = (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    want = torch.zeros((T, rows), dtype=torch.int16, device=cuda)
    got = torch.full((T, rows), -1, dtype=torch.int16, device=cuda)
    if q8:
        assert ops.k3_rocm_q8_128_gemm_bf16(want, wd, sd, xd, T, rows, cols)
    else:
        assert ops.k3_rocm_bf16_gemm_bf16(want, wd, xd, T, rows, cols)
    P = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib().k3_moe_proj_mfma_bf16(P(got), P(wd), P(sd), P(xd), T, rows, cols, q8, st)
    torch.cuda.synchronize()
    g = (got.cpu().numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    e = (want.cpu().numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    xf = (x.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    absum = np.abs(xf) @ np.abs(wf).T                      # sum |products| per output
    exact = xf @ wf.T
    m = np.maximum(np.abs(g), np.abs(e))
    ulp = np.ldexp(1.0, np.floor(np.log2(np.maximum(m, 1e-30))).astype(int) - 7)
    bound = 2.0 * cols * 2.0 ** -24 * absum + ulp
    d = np.abs(g - e)
    assert np.all(d <= bound), f"worst excess {np.max(d - bound):.3g}"
    # both near the fp64 value (a wrong row, scale or clamp is far outside)
    assert np.all(np.abs(g - exact) <= bound + np.abs(exact) * 2.0 ** -8)
    same = np.mean(d == 0)
    print(f"T={T} rows={rows} cols={cols} q8={q8}: identical {same:.1%}, worst |d|/ulp {np.max(d / ulp):.2f}")
    assert same >= 0.5
    # argument checks
    assert not lib().k3_moe_proj_mfma_bf16(P(got), P(wd), P(sd), P(xd), T, rows, cols - 32, q8, st)
    if q8:
        assert not lib().k3_moe_proj_mfma_bf16(P(got), P(wd), None, P(xd), T, rows, cols, q8, st)
