"""ctypes bridge to oracle/libk3moe_oracle.so (the CPU checker).

Test infrastructure only: the product never imports this module.
"""
import ctypes
import pathlib

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[1]
ORACLE = ROOT / "oracle" / "libk3moe_oracle.so"
REF_OPS = ROOT / "oracle" / "_ref" / "libk3ref_ops.so"
REF_PREFILL = ROOT / "oracle" / "_ref" / "libk3ref_prefill.so"

ORDER_W64, ORDER_REF, ORDER_F64, ORDER_MX8, ORDER_SPLIT = 0, 1, 2, 3, 4

_p = ctypes.c_void_p
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64
_f = ctypes.c_float
_i = ctypes.c_int


class Expert(ctypes.Structure):
    _fields_ = [(n, _p) for n in ("w1p", "w1s", "w2p", "w2s", "w3p", "w3s")]


class Shape(ctypes.Structure):
    _fields_ = [("hidden", _u32), ("experts", _u32), ("top_k", _u32), ("ffn", _u32),
                ("scale", _f), ("activation", _u32), ("beta", _f), ("linear_beta", _f)]


class Workspace(ctypes.Structure):
    _fields_ = [(n, _u64) for n in (
        "hidden_row_bytes", "attn_res_row_bytes", "main_scratch_bytes", "moe_scratch_bytes",
        "mla_scratch_bytes", "route_bytes", "expert_index_bytes", "batch_workspace_bytes",
        "incremental_workspace_bytes", "mla_append_bytes")]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not ORACLE.exists():
            raise RuntimeError(f"{ORACLE} not built (make -C oracle)")
        L = ctypes.CDLL(str(ORACLE))
        sig = {
            "k3o_bf16_to_f32": (_f, [ctypes.c_uint16]),
            "k3o_f32_to_bf16": (ctypes.c_uint16, [_f]),
            "k3o_e2m1": (_f, [ctypes.c_uint8]),
            "k3o_e8m0": (_f, [ctypes.c_uint8]),
            "k3o_expf": (_f, [_f]),
            "k3o_tanhf": (_f, [_f]),
            "k3o_sigmoid": (_f, [_f, _i]),
            "k3o_router_sigmoid": (_f, [_f]),
            "k3o_situ": (None, [_p, _p, _p, _u64, _f, _f, _i]),
            "k3o_swiglu": (None, [_p, _p, _p, _u64, _i]),
            "k3o_router_logits": (None, [_p, _p, _p, _u32, _u32, _u32, _i]),
            "k3o_router_topk": (_i, [_p, _p, _p, _p, _u32, _u32, _u32, _f, _i]),
            "k3o_route_plan": (_i, [_p, _p, _p, _p, _p, _p, _p, _u32, _u32, _u32]),
            "k3o_mxfp4_gemm": (None, [_p, _p, _p, _p, _p, _u32, _u32, _u32, _i]),
            "k3o_bf16_gemm_f32": (None, [_p, _p, _p, _u32, _u32, _u32, _i]),
            "k3o_weighted_sum": (None, [_p, _p, _p, _u32, _u32, _u32]),
            "k3o_add": (None, [_p, _p, _p, _u64]),
            "k3o_copy_rows": (None, [_p, _p, _p, _u32, _u32, _i]),
            "k3o_layer": (_i, [ctypes.POINTER(Shape), _u32, _p, _p, _p, _p, ctypes.POINTER(Expert),
                              _p, _p, _p, _u32, _p, _p, _p, _p, _p, _i, _i]),
            "k3o_prefill_workspace": (_i, [_u32, ctypes.POINTER(Workspace)]),
            "k3o_e4m3": (_f, [ctypes.c_uint8]),
            "k3o_f32_to_e4m3": (ctypes.c_uint8, [_f]),
            "k3o_mx8_quantize": (None, [_p, _p, _p, _u64]),
            "k3o_mx8_split": (None, [_p, _p, _p, _p, _p, _u64]),
            "k3o_mx8_quantize_rows": (None, [_p, _p, _p, _u64, _u64]),
            "k3o_mx8_split_rows": (None, [_p, _p, _p, _p, _p, _u64, _u64]),
            "k3o_q8_quantize": (None, [_p, _p, _p, _u32, _u32]),
            "k3o_q8_dequantize": (None, [_p, _p, _p, _u32, _u32]),
            "k3o_q8_gemm": (None, [_p, _p, _p, _p, _p, _u32, _u32, _u32, _i]),
            "k3o_rms_norm": (None, [_p, _p, _p, _u32, _u32, _f, _i]),
        }
        for n, (r, a) in sig.items():
            fn = getattr(L, n)
            fn.restype, fn.argtypes = r, a
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_p)


def router_logits(w, x, order=ORDER_REF):
    """Router logits; by default in the reference's order, which every
    router path of the library computes (k3_rocm_ops.cu:359-425)."""
    E, H = w.shape
    T = x.shape[0]
    out = np.empty((T, E), np.float32)
    lib().k3o_router_logits(_ptr(out), _ptr(w), _ptr(x), T, E, H, order)
    return out


def router_topk(logits, bias, k, scale, use_libm=False):
    T, E = logits.shape
    ids = np.empty((T, k), np.uint32)
    w = np.empty((T, k), np.float32)
    assert lib().k3o_router_topk(_ptr(ids), _ptr(w), _ptr(np.ascontiguousarray(logits)),
                                 _ptr(bias), T, E, k, scale, int(use_libm)) == 0
    return ids, w


def router_choices(logits, bias):
    """The router's choices as the oracle models the device: router_sigmoid
    (correctly rounded restatement of the hardware sequence) + bias, fp32."""
    f = lib().k3o_router_sigmoid
    s = np.array([f(float(v)) for v in np.ravel(logits)], np.float32).reshape(np.shape(logits))
    return (s + np.asarray(bias, np.float32)).astype(np.float32)


def route_weights(ids, logits, scale):
    """weight_r = s_r / (1e-20 + sum of the selected s in rank order) * scale
    with s = k3o_sigmoid(logit, 0), fp32 left to right, for given ids (the
    top-k's weight formula, k3_rocm_ops.cu:1440-1448)."""
    f = lib().k3o_sigmoid
    out = np.zeros(ids.shape, np.float32)
    for t in range(ids.shape[0]):
        live = [int(e) for e in ids[t] if e < logits.shape[1]]
        sc = [np.float32(f(float(logits[t, e]), 0)) for e in live]
        den = np.float32(1e-20)
        for v in sc:
            den = np.float32(den + v)
        for r, v in enumerate(sc):
            out[t, r] = np.float32(np.float32(v / den) * np.float32(scale))
    return out


def check_routes(got_ids, got_w, logits, bias, k, scale, max_bad=None):
    """Device routes against the oracle router on the same logits.

    The device orders experts by the hardware sigmoid the reference kernel
    uses (bit-identical to the reference's ids, tested against it on the
    GPU); the oracle's restatement of that sigmoid rounds exp2 and the
    reciprocal correctly, so it can sit up to a few ulp from the device. ids
    must therefore equal the oracle's except at near-ties: every token whose
    ids differ must hold a top-k of the oracle's choices when each choice may
    be off by 4 ulp of the sigmoid plus one rounding of the bias add.
    Weights are bit-exact to the oracle's formula on the device's own ids.
    At most max_bad tokens (default max(1, T // 1000)) may differ, so a
    change that moves many tokens onto near-tie alternatives fails.
    Returns the indices of the tokens whose ids differ."""
    want_ids, want_w = router_topk(logits, bias, k, scale)
    bad = np.nonzero((np.asarray(got_ids) != want_ids).any(axis=1))[0]
    T = np.asarray(got_ids).shape[0]
    limit = max(1, T // 1000) if max_bad is None else max_bad
    assert bad.size <= limit, f"{bad.size} of {T} tokens route differently from the oracle"
    for t in bad:
        c = router_choices(logits[t], bias).astype(np.float64)
        tol = 4 * 2.0 ** -24 + 2.0 ** -23 * np.abs(c)
        sel = np.asarray(got_ids[t], np.int64)
        live = sel[sel < c.size]
        for a, b in zip(live[:-1], live[1:]):
            assert c[a] >= c[b] - (tol[a] + tol[b]), f"token {t}: ranks out of order"
        rest = np.setdiff1d(np.arange(c.size), live)
        if rest.size and live.size:
            assert (c[live] + tol[live]).min() >= (c[rest] - tol[rest]).max(), \
                f"token {t}: routes are not a near-tie of the oracle's top-k"
        want_w[t] = route_weights(np.asarray(got_ids[t:t + 1]), logits[t:t + 1], scale)[0]
    np.testing.assert_array_equal(np.asarray(got_w), want_w)
    return bad


def route_plan(ids, experts):
    T, k = ids.shape
    counts = np.empty(experts, np.uint32)
    offsets = np.empty(experts + 1, np.uint32)
    unique = np.zeros(experts, np.uint32)
    ucount = np.zeros(1, np.uint32)
    tok = np.empty(T * k, np.uint32)
    route = np.empty(T * k, np.uint32)
    assert lib().k3o_route_plan(_ptr(counts), _ptr(offsets), _ptr(unique), _ptr(ucount),
                                _ptr(tok), _ptr(route), _ptr(np.ascontiguousarray(ids)), T, k,
                                experts) == 0
    return counts, offsets, unique[:ucount[0]], tok, route


def mxfp4_gemm(packed, scales, x, rows, cols, order=ORDER_W64):
    T = x.shape[0]
    out = np.empty((T, rows), np.uint16)
    f = np.empty((T, rows), np.float32)
    lib().k3o_mxfp4_gemm(_ptr(out), _ptr(f), _ptr(packed), _ptr(scales), _ptr(x), T, rows, cols,
                         order)
    return out, f


def bf16_gemm_f32(w, x, order=ORDER_REF):
    rows, cols = w.shape
    T = x.shape[0]
    out = np.empty((T, rows), np.float32)
    lib().k3o_bf16_gemm_f32(_ptr(out), _ptr(w), _ptr(x), T, rows, cols, order)
    return out


def bf16_gemm_bf16(w, x, order=ORDER_W64):
    """bf16 output of the bf16 -> f32 sum (the library's bf16 projections
    use the w64 order), rounded once."""
    from moonshine_amd.synth import f32_to_bf16_bits
    return f32_to_bf16_bits(bf16_gemm_f32(w, x, order))


def q8_quantize(w):
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty((rows, cols // 128), np.float32)
    lib().k3o_q8_quantize(_ptr(q), _ptr(s), _ptr(np.ascontiguousarray(w)), rows, cols)
    return q, s


def q8_dequantize(q, s):
    rows, cols = q.shape
    w = np.empty((rows, cols), np.uint16)
    lib().k3o_q8_dequantize(_ptr(w), _ptr(np.ascontiguousarray(q)), _ptr(np.ascontiguousarray(s)),
                            rows, cols)
    return w


def q8_gemm(q, s, x, order=ORDER_W64):
    rows, cols = q.shape
    T = x.shape[0]
    out = np.empty((T, rows), np.uint16)
    f = np.empty((T, rows), np.float32)
    lib().k3o_q8_gemm(_ptr(out), _ptr(f), _ptr(np.ascontiguousarray(q)),
                      _ptr(np.ascontiguousarray(s)), _ptr(np.ascontiguousarray(x)), T, rows, cols,
                      order)
    return out, f


def rms_norm(x, w, eps=1e-5, order=ORDER_W64):
    T, H = x.shape
    out = np.empty((T, H), np.uint16)
    lib().k3o_rms_norm(_ptr(out), _ptr(np.ascontiguousarray(x)), _ptr(np.ascontiguousarray(w)), T,
                       H, eps, order)
    return out


def situ(g, u, beta=4.0, lb=25.0, use_libm=False):
    out = np.empty_like(g)
    lib().k3o_situ(_ptr(out), _ptr(g), _ptr(u), g.size, beta, lb, int(use_libm))
    return out


def swiglu(g, u, use_libm=False):
    out = np.empty_like(g)
    lib().k3o_swiglu(_ptr(out), _ptr(g), _ptr(u), g.size, int(use_libm))
    return out


def weighted_sum(v, w):
    T, K, H = v.shape
    out = np.empty((T, H), np.uint16)
    lib().k3o_weighted_sum(_ptr(out), _ptr(v), _ptr(w), T, K, H)
    return out


def add(a, b):
    out = np.empty_like(a)
    lib().k3o_add(_ptr(out), _ptr(a), _ptr(b), a.size)
    return out


def e4m3_table():
    return np.array([lib().k3o_e4m3(c) for c in range(256)], np.float32)


def f32_to_e4m3(v):
    v = np.asarray(v, np.float32).ravel()
    return np.array([lib().k3o_f32_to_e4m3(float(x)) for x in v], np.uint8)


def mx8_quantize(x_bf16):
    """bf16 bits [..., n] (n % 32 == 0) -> (E4M3 codes, E8M0 scales per 32)."""
    x = np.ascontiguousarray(x_bf16, np.uint16)
    q = np.empty(x.shape, np.uint8)
    s = np.empty(x.shape[:-1] + (x.shape[-1] // 32,), np.uint8)
    lib().k3o_mx8_quantize(_ptr(q), _ptr(s), _ptr(x), x.size)
    return q, s


def mx8_split(x_bf16):
    """bf16 bits [..., n] -> (hi codes, hi scales, lo codes, lo scales)."""
    x = np.ascontiguousarray(x_bf16, np.uint16)
    hq, lq = np.empty(x.shape, np.uint8), np.empty(x.shape, np.uint8)
    sh = x.shape[:-1] + (x.shape[-1] // 32,)
    hs, ls = np.empty(sh, np.uint8), np.empty(sh, np.uint8)
    lib().k3o_mx8_split(_ptr(hq), _ptr(hs), _ptr(lq), _ptr(ls), _ptr(x), x.size)
    return hq, hs, lq, ls


def mx8_quantize_rows(x_bf16):
    """bf16 bits [rows, cols] -> (E4M3 codes, one E8M0 scale per row)."""
    x = np.ascontiguousarray(x_bf16, np.uint16)
    q = np.empty(x.shape, np.uint8)
    s = np.empty(x.shape[0], np.uint8)
    lib().k3o_mx8_quantize_rows(_ptr(q), _ptr(s), _ptr(x), x.shape[0], x.shape[1])
    return q, s


def mx8_split_rows(x_bf16):
    """bf16 bits [rows, cols] -> (hi codes, hi row scales, lo codes, lo row scales)."""
    x = np.ascontiguousarray(x_bf16, np.uint16)
    hq, lq = np.empty(x.shape, np.uint8), np.empty(x.shape, np.uint8)
    hs, ls = np.empty(x.shape[0], np.uint8), np.empty(x.shape[0], np.uint8)
    lib().k3o_mx8_split_rows(_ptr(hq), _ptr(hs), _ptr(lq), _ptr(ls), _ptr(x), x.shape[0],
                             x.shape[1])
    return hq, hs, lq, ls


def mx8_dequantize_rows(q, s):
    t = e4m3_table().astype(np.float64)
    return t[q] * np.ldexp(1.0, s.astype(np.int64) - 127)[:, None]


def mx8_dequantize(q, s):
    t = e4m3_table().astype(np.float64)
    v = t[q].reshape(q.shape[:-1] + (q.shape[-1] // 32, 32))
    sc = np.ldexp(1.0, s.astype(np.int64) - 127)
    sc = np.where(s == 0, 2.0 ** -127, sc)
    return (v * sc[..., None]).reshape(q.shape)


def layer(cfg, inputs, experts, tokens=None, ids=None, weights=None, order=ORDER_W64,
          threads=0):
    """experts: dict e -> list of six uint8 arrays (w1p, w1s, w2p, w2s, w3p, w3s)."""
    T = inputs.hidden.shape[0]
    shape = Shape(cfg.hidden, cfg.experts, cfg.top_k, cfg.ffn, cfg.scale, cfg.activation,
                  cfg.beta, cfg.linear_beta)
    table = (Expert * cfg.experts)()
    keep = []
    for e, tensors in experts.items():
        arrs = [np.ascontiguousarray(t) for t in tensors]
        keep.append(arrs)
        table[e] = Expert(*[a.ctypes.data for a in arrs])
    tl = None if tokens is None else np.ascontiguousarray(tokens, dtype=np.uint32)
    n = T if tl is None else tl.size
    out = np.empty((n, cfg.hidden), np.uint16)
    ids_out = np.empty((n, cfg.top_k), np.uint32)
    w_out = np.empty((n, cfg.top_k), np.float32)
    logits = np.empty((n, cfg.experts), np.float32)
    yout = np.empty((n, cfg.top_k, cfg.hidden), np.uint16)
    rc = lib().k3o_layer(ctypes.byref(shape), T, _ptr(inputs.hidden), _ptr(inputs.residual),
                         _ptr(inputs.router_weight), _ptr(inputs.router_bias), table,
                         _ptr(ids), _ptr(weights), _ptr(tl), 0 if tl is None else tl.size,
                         _ptr(out), _ptr(ids_out), _ptr(w_out), _ptr(logits), _ptr(yout), order,
                         threads)
    if rc != 0:
        raise RuntimeError(f"k3o_layer failed ({rc})")
    return dict(output=out, ids=ids_out, weights=w_out, logits=logits, expert_out=yout)


def native_layer(ncfg, router_weight, router_bias, norm, statics, x, residual, experts):
    """K3-native MoE layer from the oracle's pieces, in the order of
    k3_engine.cu:1549-1563, 1668-1689, 1851-1897 (include/k3_moe.h).
    statics: name -> (kind, data, scales) with kind 0 = bf16 bits, 1 = Q8-128."""
    from moonshine_amd.synth import Config, HostInputs
    T = x.shape[0]

    def proj(name, inp):
        kind, data, scales = statics[name]
        if kind == 0:
            return bf16_gemm_bf16(data, inp)
        return q8_gemm(data, scales, inp)[0]

    logits = router_logits(router_weight, x)
    ids, w = router_topk(logits, router_bias, ncfg.top_k, ncfg.scale)
    latent = proj("routed_down", x)
    rcfg = Config("routed", T, ncfg.latent, ncfg.experts, ncfg.top_k, ncfg.ffn, ncfg.scale,
                  ncfg.activation, ncfg.beta, ncfg.linear_beta)
    rin = HostInputs(np.zeros((ncfg.experts, ncfg.latent), np.uint16), router_bias, latent, None)
    routed = layer(rcfg, rin, experts, ids=ids, weights=w)["output"]
    normed = rms_norm(routed, norm, ncfg.eps)
    full = proj("routed_up", normed)
    g, u = proj("shared_gate", x), proj("shared_up", x)
    a = swiglu(g, u) if ncfg.activation == 1 else situ(g, u, ncfg.beta, ncfg.linear_beta)
    shared = proj("shared_down", a)
    total = add(full, shared)
    out = add(residual, total) if residual is not None else total
    return dict(output=out, ids=ids, weights=w, latent=latent, routed=routed, normed=normed,
                full=full, shared=shared)
