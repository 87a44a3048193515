"""GPU parity of the fused routed-MoE layer (k3_moe_forward_bf16) against the
CPU oracle on the seeded benchmark configurations.

Exact precision is bit-identical to the oracle: router logits (the
reference's own order), expert ids, route weights, the routing plan and the
layer output (expert GEMVs in the w64 order).
"""
import ctypes

import numpy as np
import pytest
import torch

import _oracle as O
from moonshine_amd import layer as L
from moonshine_amd._lib import lib
from moonshine_amd.synth import CONFIGS, K3_NATIVE, Config, bf16_bits_to_f32, make_inputs

pytestmark = pytest.mark.gpu

_stores = {}


def get_layer(cfg, inputs, cuda):
    key = (cfg.experts, cfg.hidden, cfg.ffn, cfg.seed)
    if key not in _stores:
        _stores.clear()
        torch.cuda.empty_cache()
        _stores[key] = L.ExpertStore(cfg.experts, cfg.hidden, cfg.ffn, seed=cfg.seed, device=cuda)
    return L.build_layer(cfg, inputs, device=cuda, store=_stores[key])


def run(cfg, inputs, moe, cuda):
    x = L.bf16_tensor(inputs.hidden, cuda)
    r = L.bf16_tensor(inputs.residual, cuda)
    T, k = x.shape[0], cfg.top_k
    ids = torch.zeros((T, k), dtype=torch.int32, device=cuda)
    w = torch.zeros((T, k), dtype=torch.float32, device=cuda)
    out = moe.forward(x, r, ids=ids, weights=w)
    torch.cuda.synchronize()
    return (L.bf16_bits(out), ids.cpu().numpy().view(np.uint32), w.cpu().numpy())


def run_profiled(cfg, inputs, moe, cuda):
    """k3_moe_forward_profiled_bf16 with every stage event set."""
    from moonshine_amd._lib import K3MoeProfile
    x = L.bf16_tensor(inputs.hidden, cuda)
    r = L.bf16_tensor(inputs.residual, cuda)
    T = x.shape[0]
    out = torch.empty_like(x)
    ws = moe.workspace(T)
    prof = K3MoeProfile()
    hip = ctypes.CDLL("libamdhip64.so")
    events = []
    for i in range(7):
        e = ctypes.c_void_p()
        assert hip.hipEventCreate(ctypes.byref(e)) == 0
        prof.stage_events[i] = e.value
        events.append(e)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    assert lib().k3_moe_forward_profiled_bf16(
        P(out), P(x), P(r), P(moe.router_weight), P(moe.router_bias), P(moe.store.table),
        ctypes.byref(moe.shape), T, 0, None, None, P(ws), ws.numel(), ctypes.byref(prof),
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return L.bf16_bits(out)


def host_experts(store, ids):
    """The selected experts' six tensors, copied from the device store
    (test_synth_store_host_matches_device pins them to the host generator)."""
    return {int(e): [t.cpu().numpy() for t in store.device_expert(int(e))]
            for e in np.unique(ids) if e < store.experts}


def check_tokens(cfg, inputs, store, got_out, got_ids, got_w, tokens):
    """Output bits of the listed tokens against the oracle layer run on the
    device's routes (the routes themselves are checked by the caller)."""
    tokens = np.asarray(tokens, dtype=np.uint32)
    want = O.layer(cfg, inputs, host_experts(store, got_ids[tokens]), tokens=tokens,
                   ids=np.ascontiguousarray(got_ids), weights=np.ascontiguousarray(got_w))
    np.testing.assert_array_equal(got_out[tokens], want["output"])


def test_synth_store_host_matches_device(cuda):
    cfg = CONFIGS[0]
    store = L.ExpertStore(cfg.experts, cfg.hidden, cfg.ffn, seed=cfg.seed, device=cuda)
    for e in (0, 17, cfg.experts - 1):
        for d, h in zip(store.device_expert(e), store.host_expert(e)):
            np.testing.assert_array_equal(d.cpu().numpy(), h)
    s = store.host_expert(3)[1]
    assert s.min() >= 121 and s.max() <= 125


# decode shapes beyond the BASELINE configs: a hidden size that is not a
# multiple of the larger kernels' row tiles (6208 = 97 x 64), and top_k > 16
DECODE_RAGGED = Config("decode-ragged-rows", 1, 6208, 128, 8, 1024, seed=1006)
DECODE_TOPK20 = Config("decode-topk20", 1, 2048, 128, 20, 512, seed=1007)
# hidden = 33 x 32: odd group count (byte-wise scale loads in gate/up)
DECODE_ODD_GROUPS = Config("decode-odd-groups", 1, 1056, 64, 4, 512, seed=1008)


@pytest.mark.parametrize("cfg", [CONFIGS[0], CONFIGS[1], K3_NATIVE, DECODE_RAGGED, DECODE_TOPK20,
                                 DECODE_ODD_GROUPS],
                         ids=lambda c: c.name)
def test_decode_layer_bitexact(cuda, cfg):
    inputs = make_inputs(cfg)
    moe = get_layer(cfg, inputs, cuda)
    out, ids, w = run(cfg, inputs, moe, cuda)
    want = O.layer(cfg, inputs, host_experts(moe.store, ids))
    # logits bit-exact too (the reference's order)
    logits = torch.zeros((1, cfg.experts), dtype=torch.float32, device=cuda)
    import _ops as ops
    assert ops.k3_rocm_bf16_gemv_f32(logits, moe.router_weight, L.bf16_tensor(inputs.hidden, cuda),
                                     cfg.experts, cfg.hidden)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(logits.cpu().numpy(), want["logits"])
    np.testing.assert_array_equal(ids, want["ids"])
    np.testing.assert_array_equal(w, want["weights"])
    np.testing.assert_array_equal(out, want["output"])
    assert len(set(ids[0].tolist())) == cfg.top_k
    np.testing.assert_allclose(w.sum(), cfg.scale, rtol=1e-6)
    # the profiled entry point (stage events recorded) gives the same bits
    np.testing.assert_array_equal(run_profiled(cfg, inputs, moe, cuda), want["output"])
    # repeated calls reuse the workspace; alternate with a second token so
    # stale routes or activations would show
    other = make_inputs(cfg, seed=cfg.seed + 77)
    want2 = O.layer(cfg, other, host_experts(moe.store, O.router_topk(
        O.router_logits(other.router_weight, other.hidden), other.router_bias, cfg.top_k,
        cfg.scale)[0]))
    moe2 = L.build_layer(cfg, other, device=cuda, store=moe.store)
    for _ in range(3):
        o2, i2, _ = run(cfg, inputs, moe, cuda)
        np.testing.assert_array_equal(o2, out)
        o3, i3, _ = run(cfg, other, moe2, cuda)
        np.testing.assert_array_equal(o3, want2["output"])



def test_decode_graph_replay_same_bits(cuda):
    """Decode calls captured in a HIP graph give the oracle's bits on every
    replay, with eager calls on the same workspace between the replays."""
    import dataclasses
    cfg = CONFIGS[1]
    a = make_inputs(cfg)
    other = make_inputs(cfg, seed=cfg.seed + 5)
    b = dataclasses.replace(a, hidden=other.hidden, residual=other.residual)
    moe = get_layer(cfg, a, cuda)
    wants = []
    for inp in (a, b):
        ids = O.router_topk(O.router_logits(inp.router_weight, inp.hidden), inp.router_bias,
                            cfg.top_k, cfg.scale)[0]
        wants.append(O.layer(cfg, inp, host_experts(moe.store, ids))["output"])
    xa, ra = L.bf16_tensor(a.hidden, cuda), L.bf16_tensor(a.residual, cuda)
    out = torch.zeros_like(xa)
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap):
        moe.forward(xa, ra, out=out, stream=cap.cuda_stream)
        cap.synchronize()
        with torch.cuda.graph(g, stream=cap):
            moe.forward(xa, ra, out=out, stream=cap.cuda_stream)
    torch.cuda.synchronize()
    for rep in range(4):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(L.bf16_bits(out), wants[0], err_msg=f"replay {rep}")
        o2, _, _ = run(cfg, b, moe, cuda)  # eager, same layer and workspace
        np.testing.assert_array_equal(o2, wants[1])


@pytest.mark.parametrize("T", [1, 5])
def test_missing_routes(cuda, T):
    """Only two experts selectable (NaN bias elsewhere) with top_k = 4: the
    last two slots of every token are missing (id UINT32_MAX, weight 0) and
    contribute nothing. Decode (T = 1, whose top-k resolves descriptors
    itself) and the batched path must both match the oracle run on the
    two live routes with the top-k's own weights (the combine adds live
    routes in rank order, so this is bit-exact)."""
    import dataclasses
    cfg = CONFIGS[0]
    inputs = make_inputs(cfg, tokens=T, seed=cfg.seed + 5)
    bias = np.full(cfg.experts, np.nan, np.float32)
    bias[5], bias[40] = 0.01, -0.02
    inputs = dataclasses.replace(inputs, router_bias=bias)
    moe = get_layer(cfg, inputs, cuda)
    out, ids, w = run(cfg, inputs, moe, cuda)
    want_ids, want_w = O.router_topk(O.router_logits(inputs.router_weight, inputs.hidden), bias,
                                     cfg.top_k, cfg.scale)
    assert set(want_ids[:, :2].ravel().tolist()) <= {5, 40}
    assert (want_ids[:, 2:] == 0xFFFFFFFF).all() and (want_w[:, 2:] == 0).all()
    np.testing.assert_array_equal(ids, want_ids)
    np.testing.assert_array_equal(w, want_w)
    live = dataclasses.replace(cfg, top_k=2)
    want = O.layer(live, inputs, host_experts(moe.store, want_ids[:, :2]),
                   ids=np.ascontiguousarray(want_ids[:, :2]),
                   weights=np.ascontiguousarray(want_w[:, :2]))
    np.testing.assert_array_equal(out, want["output"])


@pytest.mark.parametrize("cfg_index,check", [(0, None), (2, 16), (3, 32)])
def test_batched_layer_bitexact(cuda, cfg_index, check):
    cfg = CONFIGS[cfg_index]
    T = cfg.tokens if cfg_index else 40
    inputs = make_inputs(cfg, tokens=T)
    moe = get_layer(cfg, inputs, cuda)
    out, ids, w = run(cfg, inputs, moe, cuda)
    # routing of every token is checked against the oracle router
    want_logits = O.router_logits(inputs.router_weight, inputs.hidden)
    bad = O.check_routes(ids, w, want_logits, inputs.router_bias, cfg.top_k, cfg.scale)
    assert bad.size <= max(1, T // 1000)
    rng = np.random.default_rng(5)
    tokens = np.arange(T) if check is None else np.sort(rng.choice(T, check, replace=False))
    check_tokens(cfg, inputs, moe.store, out, ids, w, tokens)
    # a token alone (decode path) gives the same bits as inside the batch
    t = int(tokens[-1])
    one = make_inputs(cfg, tokens=T)
    one.hidden, one.residual = one.hidden[t:t + 1].copy(), one.residual[t:t + 1].copy()
    o1, i1, w1 = run(cfg, one, moe, cuda)
    np.testing.assert_array_equal(i1[0], ids[t])
    np.testing.assert_array_equal(o1[0], out[t])


def plan_of(ids, E, cuda):
    """k3_moe_route_plan (the plan kernels the layer runs) on given routes."""
    T, k = ids.shape
    d_ids = torch.from_numpy(np.ascontiguousarray(ids).view(np.int32)).to(cuda)
    counts = torch.zeros(E, dtype=torch.int32, device=cuda)
    offsets = torch.zeros(E + 1, dtype=torch.int32, device=cuda)
    unique = torch.zeros(E, dtype=torch.int32, device=cuda)
    summary = torch.zeros(4, dtype=torch.int32, device=cuda)
    tok = torch.zeros(T * k, dtype=torch.int32, device=cuda)
    route = torch.zeros(T * k, dtype=torch.int32, device=cuda)
    nscratch = lib().k3_moe_plan_scratch_bytes(T, E)
    scratch = torch.zeros(nscratch, dtype=torch.uint8, device=cuda)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    assert lib().k3_moe_route_plan(P(counts), P(offsets), P(unique), P(summary), P(tok), P(route),
                                   P(d_ids), T, k, E, P(scratch), nscratch,
                                   ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    h = lambda t: t.cpu().numpy().view(np.uint32)
    n = int(h(summary)[0])
    return h(counts), h(offsets), h(unique)[:n], h(tok), h(route)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("precision", [0, 1], ids=["exact", "mfma"])
def test_cfg4_full_routes_and_sample_vs_oracle(cuda, precision):
    """BASELINE config 4 at full size (8192 tokens, Zipf bias): every
    token's ids equal to the C oracle router's or a near-tie of it within
    the ulps of its sigmoid restatement (O.check_routes), and every weight
    bit-equal to the oracle's formula on those ids; the plan of
    the layer's routes equal to the oracle's stable-sort plan; output bits
    of 24 tokens (up to 9 of them routed to the three heaviest experts, and
    every near-tie token) equal to
    the oracle on the exact path, and inside the MFMA tolerance (rel-L2
    <= 2e-3, 4 bf16 ulp of max(|v|, RMS)) on the MFMA path."""
    cfg = CONFIGS[4]
    T = cfg.tokens
    inputs = make_inputs(cfg)
    moe = get_layer(cfg, inputs, cuda)
    x = L.bf16_tensor(inputs.hidden, cuda)
    r = L.bf16_tensor(inputs.residual, cuda)
    ids_d = torch.zeros((T, cfg.top_k), dtype=torch.int32, device=cuda)
    w_d = torch.zeros((T, cfg.top_k), dtype=torch.float32, device=cuda)
    out_d = moe.forward(x, r, ids=ids_d, weights=w_d, precision=precision)
    torch.cuda.synchronize()
    out, ids, w = L.bf16_bits(out_d), ids_d.cpu().numpy().view(np.uint32), w_d.cpu().numpy()
    logits = O.router_logits(inputs.router_weight, inputs.hidden)
    bad = O.check_routes(ids, w, logits, inputs.router_bias, cfg.top_k, cfg.scale)
    print(f"\ncfg4: {bad.size}/{T} tokens' ids differ from the oracle router, all near-ties "
          f"within the ulps of its sigmoid restatement")
    assert bad.size <= 4
    c, o, u, t_i, r_i = O.route_plan(ids, cfg.experts)
    gc, go, gu, gt, gr = plan_of(ids, cfg.experts, cuda)
    for a, b in ((gc, c), (go, o), (gu, u), (gt, t_i), (gr, r_i)):
        np.testing.assert_array_equal(a, b)
    heavy = np.argsort(-c, kind="stable")[:3]
    print(f"\ncfg4: U = {u.size}, heaviest experts {heavy.tolist()} with {c[heavy].tolist()} rows")
    rng = np.random.default_rng(44)
    picks = set()
    for e in heavy:
        rows = t_i[o[e]:o[e + 1]]
        picks.update(rng.choice(rows, min(3, rows.size), replace=False).tolist())
    picks.update(int(t) for t in bad)
    picks.update(rng.choice(T, 24 - len(picks), replace=False).tolist())
    tokens = np.array(sorted(picks), dtype=np.uint32)
    assert tokens.size >= 16
    if precision == 0:
        check_tokens(cfg, inputs, moe.store, out, ids, w, tokens)
    else:
        want = O.layer(cfg, inputs, host_experts(moe.store, ids[tokens]), tokens=tokens, ids=ids,
                       weights=w)
        g = bf16_bits_to_f32(out[tokens]).astype(np.float64)
        f = bf16_bits_to_f32(want["output"]).astype(np.float64)
        rel = np.linalg.norm(g - f) / np.linalg.norm(f)
        rms = np.sqrt(np.mean(f * f))
        lim = 4 * 2.0 ** (np.floor(np.log2(np.maximum(np.abs(f), rms))) - 7)
        print(f"cfg4 MFMA vs oracle on {tokens.size} tokens: rel-L2 {rel:.3g}")
        assert rel <= 2e-3
        assert (np.abs(g - f) <= lim).all()


@pytest.mark.timeout(900)
@pytest.mark.parametrize("precision", [0, 1], ids=["exact", "mfma"])
def test_max_tokens_k3(cuda, precision):
    """The largest batch the layer takes, 65535 tokens (the entry points'
    limit; the combine's grid is one row of blocks per token, 65535 the
    largest grid dimension), at the K3 shape with config 4's Zipf routing:
    1,048,560 routes, per-route outputs past 2^32 elements, every tile
    class full. The plan of all routes equals the oracle's stable-sort
    plan; 512 sampled tokens' ids match the oracle router (near-ties as
    O.check_routes allows) with bit-equal weights; 24 of them (some on the
    heaviest experts) match the oracle layer bit for bit on the exact path
    and within the MFMA tolerance on the MFMA path."""
    cfg = CONFIGS[4]
    T = 65535
    inputs = make_inputs(cfg, tokens=T)
    moe = get_layer(cfg, inputs, cuda)
    x = L.bf16_tensor(inputs.hidden, cuda)
    r = L.bf16_tensor(inputs.residual, cuda)
    ids_d = torch.zeros((T, cfg.top_k), dtype=torch.int32, device=cuda)
    w_d = torch.zeros((T, cfg.top_k), dtype=torch.float32, device=cuda)
    out_d = moe.forward(x, r, ids=ids_d, weights=w_d, precision=precision)
    torch.cuda.synchronize()
    out, ids, w = L.bf16_bits(out_d), ids_d.cpu().numpy().view(np.uint32), w_d.cpu().numpy()
    del out_d, x, r
    c, o, u, t_i, r_i = O.route_plan(ids, cfg.experts)
    gc, go, gu, gt, gr = plan_of(ids, cfg.experts, cuda)
    for a, b in ((gc, c), (go, o), (gu, u), (gt, t_i), (gr, r_i)):
        np.testing.assert_array_equal(a, b)
    rng = np.random.default_rng(65535)
    sample = np.sort(rng.choice(T, 512, replace=False))
    sample[-1] = T - 1  # the last grid row
    logits = O.router_logits(inputs.router_weight, inputs.hidden[sample])
    bad = O.check_routes(ids[sample], w[sample], logits, inputs.router_bias, cfg.top_k, cfg.scale)
    heavy = np.argsort(-c, kind="stable")[:3]
    print(f"\nT={T}: U = {u.size}, heaviest experts {heavy.tolist()} with {c[heavy].tolist()} rows; "
          f"{bad.size}/512 sampled tokens near-ties")
    picks = {int(T - 1), 0}
    for e in heavy:
        rows = t_i[o[e]:o[e + 1]]
        picks.update(rng.choice(rows, 3, replace=False).tolist())
    picks.update(int(sample[t]) for t in bad)
    picks.update(rng.choice(sample, 24 - len(picks), replace=False).tolist())
    tokens = np.array(sorted(picks), dtype=np.uint32)
    if precision == 0:
        check_tokens(cfg, inputs, moe.store, out, ids, w, tokens)
    else:
        want = O.layer(cfg, inputs, host_experts(moe.store, ids[tokens]), tokens=tokens, ids=ids,
                       weights=w)
        g = bf16_bits_to_f32(out[tokens]).astype(np.float64)
        f = bf16_bits_to_f32(want["output"]).astype(np.float64)
        rel = np.linalg.norm(g - f) / np.linalg.norm(f)
        rms = np.sqrt(np.mean(f * f))
        lim = 4 * 2.0 ** (np.floor(np.log2(np.maximum(np.abs(f), rms))) - 7)
        print(f"T={T} MFMA vs oracle on {tokens.size} tokens: rel-L2 {rel:.3g}")
        assert rel <= 2e-3
        assert (np.abs(g - f) <= lim).all()


def test_expert_stage_on_given_routes(cuda):
    cfg = CONFIGS[0]
    T = 9
    inputs = make_inputs(cfg, tokens=T)
    moe = get_layer(cfg, inputs, cuda)
    rng = np.random.default_rng(9)
    ids = np.stack([rng.choice(cfg.experts, cfg.top_k, replace=False) for _ in range(T)]).astype(np.uint32)
    ids[3] = [5, 5, 6, 7]  # duplicate route within a token: second one dropped
    w = rng.random((T, cfg.top_k)).astype(np.float32)
    x = L.bf16_tensor(inputs.hidden, cuda)
    r = L.bf16_tensor(inputs.residual, cuda)
    out = moe.experts_only(x, torch.from_numpy(ids.view(np.int32)).to(cuda), torch.from_numpy(w).to(cuda), r)
    torch.cuda.synchronize()
    got = L.bf16_bits(out)
    keep = np.array([0, 1, 2, 4, 5, 6, 7, 8])
    want = O.layer(cfg, inputs, host_experts(moe.store, ids), ids=ids, weights=w, tokens=keep)
    np.testing.assert_array_equal(got[keep], want["output"])


@pytest.mark.parametrize("T,E,k,zipf", [(1, 896, 16, False), (300, 64, 4, False), (8192, 896, 16, True),
                                        (777, 1024, 32, False)])
def test_route_plan_bitexact(cuda, T, E, k, zipf):
    rng = np.random.default_rng(T + E)
    if zipf:
        p = (np.arange(1, E + 1) ** -1.1)
        p /= p.sum()
        ids = np.stack([rng.choice(E, k, replace=False, p=p) for _ in range(T)]).astype(np.uint32)
    else:
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32)
    d_ids = torch.from_numpy(ids.view(np.int32)).to(cuda)
    counts = torch.zeros(E, dtype=torch.int32, device=cuda)
    offsets = torch.zeros(E + 1, dtype=torch.int32, device=cuda)
    unique = torch.zeros(E, dtype=torch.int32, device=cuda)
    summary = torch.zeros(4, dtype=torch.int32, device=cuda)
    tok = torch.zeros(T * k, dtype=torch.int32, device=cuda)
    route = torch.zeros(T * k, dtype=torch.int32, device=cuda)
    nscratch = lib().k3_moe_plan_scratch_bytes(T, E)
    scratch = torch.zeros(nscratch, dtype=torch.uint8, device=cuda)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    assert lib().k3_moe_route_plan(P(counts), P(offsets), P(unique), P(summary), P(tok), P(route),
                                   P(d_ids), T, k, E, P(scratch), nscratch,
                                   ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    c, o, u, t_i, r_i = O.route_plan(ids, E)
    h = lambda t: t.cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(h(counts), c)
    np.testing.assert_array_equal(h(offsets), o)
    s = h(summary)
    assert s[0] == u.size and s[1] == 0 and s[2] == c.max()
    np.testing.assert_array_equal(h(unique)[:u.size], u)
    np.testing.assert_array_equal(h(tok), t_i)
    np.testing.assert_array_equal(h(route), r_i)


class MappedHost:
    """hipHostMalloc'd, device-mapped host memory (the reference engine's
    route outputs, k3_engine.cu:623-640); freed on close()."""

    def __init__(self, nbytes):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t,
                                           ctypes.c_uint]
        self.hip.hipHostGetDevicePointer.argtypes = [ctypes.POINTER(ctypes.c_void_p),
                                                     ctypes.c_void_p, ctypes.c_uint]
        self.hip.hipHostFree.argtypes = [ctypes.c_void_p]
        self.host = ctypes.c_void_p()
        assert self.hip.hipHostMalloc(ctypes.byref(self.host), nbytes, 0x2) == 0  # mapped
        self.dev = ctypes.c_void_p()
        assert self.hip.hipHostGetDevicePointer(ctypes.byref(self.dev), self.host, 0) == 0
        self.nbytes = nbytes

    def array(self, dtype, count):
        buf = (ctypes.c_char * self.nbytes).from_address(self.host.value)
        return np.frombuffer(buf, dtype=dtype, count=count)

    def close(self):
        self.hip.hipHostFree(self.host)


@pytest.mark.parametrize("T", [1, 5, 40])  # 40: the certified MFMA router
def test_routes_into_mapped_host_memory(cuda, T):
    """The layer's optional route copies written straight into host-mapped
    memory, as the reference engine reads them."""
    cfg = CONFIGS[0]
    inputs = make_inputs(cfg, tokens=T, seed=cfg.seed + 9)
    moe = get_layer(cfg, inputs, cuda)
    n = T * cfg.top_k
    mi, mw = MappedHost(4 * n), MappedHost(4 * n)
    try:
        mi.array(np.uint32, n)[:] = 0xDEADBEEF
        mw.array(np.float32, n)[:] = -1.0
        x = L.bf16_tensor(inputs.hidden, cuda)
        r = L.bf16_tensor(inputs.residual, cuda)
        ws = moe.workspace(T)
        out = torch.empty_like(x)
        P = lambda t: ctypes.c_void_p(t.data_ptr())
        assert lib().k3_moe_forward_bf16(P(out), P(x), P(r), P(moe.router_weight),
                                         P(moe.router_bias), P(moe.store.table),
                                         ctypes.byref(moe.shape), T, 0, mi.dev, mw.dev, P(ws),
                                         ws.numel(),
                                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        want = O.layer(cfg, inputs, host_experts(moe.store, np.arange(cfg.experts)))
        np.testing.assert_array_equal(mi.array(np.uint32, n).reshape(T, -1), want["ids"])
        np.testing.assert_array_equal(mw.array(np.float32, n).reshape(T, -1), want["weights"])
        np.testing.assert_array_equal(L.bf16_bits(out), want["output"])
        # the single-vector router ABI into the same mapped buffers
        import _ops as ops
        logits = torch.from_numpy(O.router_logits(inputs.router_weight, inputs.hidden)[0]).to(cuda)
        mi.array(np.uint32, n)[:] = 0
        assert ops.lib().k3_rocm_router_topk_f32(mi.dev, mw.dev, P(logits), P(moe.router_bias),
                                                 cfg.experts, cfg.top_k, cfg.scale, None)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(mi.array(np.uint32, cfg.top_k), want["ids"][0])
    finally:
        mi.close()
        mw.close()


def test_unaligned_expert_tensors(cuda):
    """Expert tensors starting 8 bytes past a 16-byte boundary (real
    checkpoint spans): the decode and exact kernels load them as 8-byte
    pairs and the MFMA kernels' 16-byte direct-to-LDS loads take them as
    they are, so every path gives the same bits as on an aligned copy
    (every expert shifted, or only the odd ones). Tensors that are not even
    8-byte aligned (4 past a 16-byte boundary) leave the MFMA path for the
    exact kernels: the layer then equals the exact path bit for bit."""
    cfg = CONFIGS[0]
    aligned = L.ExpertStore(cfg.experts, cfg.hidden, cfg.ffn, seed=cfg.seed, device=cuda)
    shifted = L.ExpertStore(cfg.experts, cfg.hidden, cfg.ffn, seed=cfg.seed, device=cuda,
                            misalign=8)
    mixed = L.ExpertStore(cfg.experts, cfg.hidden, cfg.ffn, seed=cfg.seed, device=cuda,
                          misalign=8, misalign_odd=True)
    odd4 = L.ExpertStore(cfg.experts, cfg.hidden, cfg.ffn, seed=cfg.seed, device=cuda,
                         misalign=4)
    assert (shifted.table.cpu().numpy().view(np.uint64) % 16 == 8).all()
    assert (odd4.table.cpu().numpy().view(np.uint64) % 16 == 4).all()
    for T in (1, 5):
        inputs = make_inputs(cfg, tokens=T, seed=cfg.seed + 31)
        ref = run(cfg, inputs, L.build_layer(cfg, inputs, device=cuda, store=aligned), cuda)
        got = run(cfg, inputs, L.build_layer(cfg, inputs, device=cuda, store=shifted), cuda)
        for a, b in zip(got, ref):
            np.testing.assert_array_equal(a, b)
        if T == 1:
            want = O.layer(cfg, inputs, host_experts(aligned, ref[1]))
            np.testing.assert_array_equal(ref[0], want["output"])
    for T in (40, 300):
        inputs = make_inputs(cfg, tokens=T, seed=cfg.seed + 32)
        x = L.bf16_tensor(inputs.hidden, cuda)
        r = L.bf16_tensor(inputs.residual, cuda)
        fwd = lambda store, precision: L.bf16_bits(
            L.build_layer(cfg, inputs, device=cuda, store=store).forward(x, r, precision=precision))
        mfma = fwd(aligned, 1)
        np.testing.assert_array_equal(fwd(shifted, 1), mfma)
        np.testing.assert_array_equal(fwd(mixed, 1), mfma)
        np.testing.assert_array_equal(fwd(odd4, 1), fwd(aligned, 0))


def test_c_harness():
    """The C caller of the ABI (tests/c/k3_moe_harness.c): decode and
    batched layers through k3_moe_forward_bf16 from C, routes into mapped
    host memory, a 4-layer decode chain on one stream with one sync, and
    the prefill router entry point, bit-exact against the C oracle."""
    import pathlib
    import subprocess
    exe = pathlib.Path(__file__).resolve().parent / "c" / "k3_moe_harness"
    assert exe.exists(), "tests/c/k3_moe_harness not built (make -C tests/c)"
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count("output match, ids match, weights match") == 2
    assert "4-layer decode chain (one stream, one sync) match" in r.stdout
    assert "router entry point, 40 tokens: ids and weights match" in r.stdout
