"""The engine-side binding of libk3moe (tests/engine_link/k3_engine_moe.inc),
compiled into the reference engine's own translation unit (k3_engine.cu +
k3_engine_prefill.inc, engine_with_moe.cu) and linked with libk3moe.so
(tests/engine_link/Makefile), driven at the real K3 shape: the router on
the 7168-wide post-norm hidden state (k3_engine.cu:1554-1557), the experts
on the 3584-wide latent with F 3072 (:1668-1672), SiTU(4, 25) (:1056),
routed scale 1.0 (:1563), 896 experts, top-16. Checked against the oracle
composed from its pinned pieces: routes of the router input, experts on the
latent, rank-order combine. The engine library is built here from the
reference sources; a box without it skips."""
import ctypes
import pathlib

import numpy as np
import pytest
import torch

import _oracle as O
from moonshine_amd import native as N
from moonshine_amd.layer import bf16_bits, bf16_tensor
from moonshine_amd.synth import Config, HostInputs, f32_to_bf16_bits

ROOT = pathlib.Path(__file__).resolve().parents[1]
ENGINE = ROOT / "tests" / "engine_link" / "lib" / "libk3engine_on_k3moe.so"

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not ENGINE.exists(), reason="engine binding not built "
                                 "(make -C tests/engine_link, needs the reference sources)")]

_p, _u32, _sz = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_size_t


class EngineExpertLayout(ctypes.Structure):
    """k3_engine_expert_layout (k3_engine.cu:105-111)."""
    _fields_ = [("relative", ctypes.c_uint64 * 6), ("physical_start", ctypes.c_uint64),
                ("aligned_start", ctypes.c_uint64), ("aligned_bytes", ctypes.c_uint32),
                ("shard", ctypes.c_uint16)]


class StTensor(ctypes.Structure):
    """k3_st_tensor (k3_safetensors.h:21-29)."""
    _fields_ = [("name", ctypes.c_char_p), ("physical_offset", ctypes.c_uint64),
                ("byte_length", ctypes.c_uint64), ("shape", ctypes.c_uint64 * 8),
                ("shard", ctypes.c_uint16), ("ndim", ctypes.c_uint8), ("dtype", ctypes.c_int)]


class StaticWeight(ctypes.Structure):
    """k3_static_weight (k3_static_store.h:20-26); kind 1 = BF16, 2 = Q8_128."""
    _fields_ = [("tensor", ctypes.POINTER(StTensor)), ("data", _p), ("scales", _p),
                ("resident_bytes", ctypes.c_uint64), ("kind", ctypes.c_int)]


_lib = None


def engine():
    global _lib
    if _lib is None:
        h = ctypes.CDLL(str(ENGINE), mode=ctypes.RTLD_GLOBAL)
        h.k3_engine_moe_workspace_bytes.restype = _sz
        h.k3_engine_moe_workspace_bytes.argtypes = [_u32]
        h.k3_engine_moe_native_workspace_bytes.restype = _sz
        h.k3_engine_moe_native_workspace_bytes.argtypes = [_u32]
        h.k3_engine_moe_descriptors.restype = ctypes.c_bool
        h.k3_engine_moe_descriptors.argtypes = [_p, ctypes.POINTER(_p),
                                                ctypes.POINTER(EngineExpertLayout), _u32]
        h.k3_engine_moe_decode.restype = ctypes.c_bool
        h.k3_engine_moe_decode.argtypes = [_p] * 9 + [_sz, _p]
        h.k3_engine_moe_prefill.restype = ctypes.c_bool
        h.k3_engine_moe_prefill.argtypes = [_p] * 6 + [_u32, _u32, _p, _p, _p, _sz, _p]
        h.k3_engine_moe_native_block.restype = ctypes.c_bool
        h.k3_engine_moe_native_block.argtypes = (
            [_p, _p, _p, _p, _p, ctypes.POINTER(StaticWeight), _p, ctypes.POINTER(StaticWeight),
             ctypes.POINTER(StaticWeight), ctypes.POINTER(StaticWeight),
             ctypes.POINTER(StaticWeight), _p, _u32, _u32, _p, _p, _p, _sz, _p, _p])
        _lib = h
    return _lib


_layer = {}


def k3_layer(cuda):
    """The K3 layer at its real size: router [896, 7168], 896 resident
    experts on the latent (3584 / 3072), Q8-128 static projections."""
    if "k3" not in _layer:
        _layer["k3"] = N.NativeLayer(N.K3_NATIVE_LAYER, device=cuda)
    return _layer["k3"]


def engine_table(layer, cuda):
    """The descriptor table through the binding, from the engine's layouts:
    each expert's span base and the six relative offsets of its tensors."""
    st = layer.store
    E = st.experts
    bases = (_p * E)(*[st.buffer.data_ptr() + e * st.span + st.shifts[e] for e in range(E)])
    lays = (EngineExpertLayout * E)()
    for e in range(E):
        for j in range(6):
            lays[e].relative[j] = st.offsets[j]
        lays[e].aligned_bytes = st.span
    table = torch.zeros((E, 6), dtype=torch.int64, device=cuda)
    assert engine().k3_engine_moe_descriptors(_p(table.data_ptr()), bases, lays, E)
    assert torch.equal(table, st.table), "binding descriptors differ from the store's"
    return table


def routed_cfg(cfg, T):
    return Config("routed", T, cfg.latent, cfg.experts, cfg.top_k, cfg.ffn, cfg.scale,
                  cfg.activation, cfg.beta, cfg.linear_beta)


def composed(layer, x_bits, latent_bits, tokens=None):
    """Oracle: routes from the router input, experts on the latent, the
    rank-order combine without residual."""
    cfg = layer.cfg
    logits = O.router_logits(layer.router_weight_bits, x_bits)
    ids, w = O.router_topk(logits, layer.router_bias, cfg.top_k, cfg.scale)
    T = x_bits.shape[0]
    experts = {int(e): layer.store.host_expert(int(e)) for e in np.unique(ids if tokens is None
                                                                         else ids[tokens])}
    rin = HostInputs(np.zeros((cfg.experts, cfg.latent), np.uint16), layer.router_bias,
                     latent_bits, None)
    out = O.layer(routed_cfg(cfg, T), rin, experts, tokens=tokens, ids=ids, weights=w)["output"]
    return ids, w, out


def rand_bits(rng, shape):
    return f32_to_bf16_bits(rng.normal(0, 1, shape).astype(np.float32))


def test_decode_binding_k3(cuda):
    """k3_engine_moe_decode, one token at a time (3 tokens), routes into
    host-mapped memory as the engine's route_ids_host: ids, weights and the
    routed combine bit-identical to the composed oracle."""
    from test_gpu_layer import MappedHost
    layer = k3_layer(cuda)
    cfg = layer.cfg
    table = engine_table(layer, cuda)
    rng = np.random.default_rng(77)
    T = 3
    x = rand_bits(rng, (T, cfg.hidden))
    lat = rand_bits(rng, (T, cfg.latent))
    xd, ld = bf16_tensor(x, cuda), bf16_tensor(lat, cuda)
    nbytes = engine().k3_engine_moe_workspace_bytes(1)
    assert nbytes > 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=cuda)
    mids, mw = MappedHost(4 * cfg.top_k), MappedHost(4 * cfg.top_k)
    want_ids, want_w, want = composed(layer, x, lat)
    try:
        for t in range(T):
            out = torch.empty((1, cfg.latent), dtype=torch.int16, device=cuda)
            assert engine().k3_engine_moe_decode(
                _p(out.data_ptr()), _p(xd[t].data_ptr()), _p(ld[t].data_ptr()),
                _p(layer.router_weight.data_ptr()), _p(layer.router_bias_d.data_ptr()),
                _p(table.data_ptr()), mids.dev, mw.dev, _p(ws.data_ptr()), nbytes,
                _p(torch.cuda.current_stream().cuda_stream))
            torch.cuda.synchronize()
            np.testing.assert_array_equal(mids.array(np.uint32, cfg.top_k), want_ids[t])
            np.testing.assert_array_equal(mw.array(np.float32, cfg.top_k), want_w[t])
            np.testing.assert_array_equal(bf16_bits(out)[0], want[t])
    finally:
        mids.close()
        mw.close()


@pytest.mark.timeout(600)
def test_prefill_binding_k3(cuda):
    """k3_engine_moe_prefill on 64 tokens: K3_MOE_EXACT bit-identical to
    the composed oracle (routes of every token; outputs of 8 sampled
    tokens), K3_MOE_MFMA the same routes and within the MFMA path's stated
    tolerance of the exact output (rel-L2 <= 2e-3, <= 4 bf16 ulp of
    max(|element|, RMS))."""
    layer = k3_layer(cuda)
    cfg = layer.cfg
    table = engine_table(layer, cuda)
    rng = np.random.default_rng(78)
    T = 64
    x = rand_bits(rng, (T, cfg.hidden))
    lat = rand_bits(rng, (T, cfg.latent))
    xd, ld = bf16_tensor(x, cuda), bf16_tensor(lat, cuda)
    nbytes = engine().k3_engine_moe_workspace_bytes(T)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=cuda)
    outs = []
    for precision in (0, 1):
        out = torch.empty((T, cfg.latent), dtype=torch.int16, device=cuda)
        ids = torch.zeros((T, cfg.top_k), dtype=torch.int32, device=cuda)
        w = torch.zeros((T, cfg.top_k), dtype=torch.float32, device=cuda)
        assert engine().k3_engine_moe_prefill(
            _p(out.data_ptr()), _p(xd.data_ptr()), _p(ld.data_ptr()),
            _p(layer.router_weight.data_ptr()), _p(layer.router_bias_d.data_ptr()),
            _p(table.data_ptr()), T, precision, _p(ids.data_ptr()), _p(w.data_ptr()),
            _p(ws.data_ptr()), nbytes, _p(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        outs.append((bf16_bits(out), ids.cpu().numpy().view(np.uint32), w.cpu().numpy()))
    sample = np.sort(rng.choice(T, 8, replace=False)).astype(np.uint32)
    want_ids, want_w, want = composed(layer, x, lat, tokens=sample)
    for got, ids, w in outs:
        np.testing.assert_array_equal(ids, want_ids)
        np.testing.assert_array_equal(w, want_w)
    np.testing.assert_array_equal(outs[0][0][sample], want)
    from moonshine_amd.synth import bf16_bits_to_f32
    e = bf16_bits_to_f32(outs[0][0]).astype(np.float64)
    m = bf16_bits_to_f32(outs[1][0]).astype(np.float64)
    rel = np.linalg.norm(m - e) / np.linalg.norm(e)
    rms = float(np.sqrt(np.mean(e * e)))
    ulp = np.ldexp(1.0, np.frexp(np.maximum(np.abs(e), rms))[1] - 8)
    worst = float((np.abs(m - e) / ulp).max())
    print(f"\nengine prefill binding, K3 latent, 64 tokens: MFMA vs exact rel-L2 {rel:.3g}, "
          f"worst {worst:.2f} ulp")
    assert rel <= 2e-3 and worst <= 4


def test_native_block_binding_k3(cuda):
    """k3_engine_moe_native_block from the engine's own k3_static_weight
    structs (kind, tensor shape, data, scales): bit-identical to the
    library's native block on the same weights (itself bit-exact to the
    composed oracle at this size, test_gpu_native.py), so the mapping of
    each engine weight to its role is right."""
    layer = k3_layer(cuda)
    cfg = layer.cfg
    table = engine_table(layer, cuda)
    rng = np.random.default_rng(79)
    x = bf16_tensor(rand_bits(rng, (1, cfg.hidden)), cuda)
    r = bf16_tensor(rand_bits(rng, (1, cfg.hidden)), cuda)
    keep = []

    def sw(w):
        t = StTensor()
        t.shape[0], t.shape[1], t.ndim = w.rows, w.cols, 2
        keep.append(t)
        s = StaticWeight(ctypes.pointer(t), w.data.data_ptr(),
                         None if w.scales is None else w.scales.data_ptr(), w.nbytes,
                         2 if w.kind == N.STATIC_Q8 else 1)
        keep.append(s)
        return ctypes.byref(s)

    nbytes = engine().k3_engine_moe_native_workspace_bytes(1)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=cuda)
    out = torch.empty_like(x)
    ids = torch.zeros((1, cfg.top_k), dtype=torch.int32, device=cuda)
    w = torch.zeros((1, cfg.top_k), dtype=torch.float32, device=cuda)
    assert engine().k3_engine_moe_native_block(
        _p(out.data_ptr()), _p(x.data_ptr()), _p(r.data_ptr()),
        _p(layer.router_weight.data_ptr()), _p(layer.router_bias_d.data_ptr()),
        sw(layer.routed_down), _p(layer.norm.data_ptr()), sw(layer.routed_up),
        sw(layer.shared_gate), sw(layer.shared_up), sw(layer.shared_down),
        _p(table.data_ptr()), 1, 0, _p(ids.data_ptr()), _p(w.data_ptr()), _p(ws.data_ptr()),
        nbytes, _p(torch.cuda.current_stream().cuda_stream), None)
    ids2 = torch.zeros_like(ids)
    w2 = torch.zeros_like(w)
    want = layer.forward(x, r, ids=ids2, weights=w2)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids2) and torch.equal(w, w2)
    np.testing.assert_array_equal(bf16_bits(out), bf16_bits(want))
