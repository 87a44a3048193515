"""k3_moe_forward_static_bf16 (the entry point with no caller workspace)
against k3_moe_forward_bf16 on the same inputs: identical bits for the
output, the ids and the weights, on two calls in a row with the second one
smaller (so a stale workspace from the first would show), at the K3
config; and the static maximum rejected cleanly."""
import ctypes

import numpy as np
import pytest
import torch

from moonshine_amd import layer as L
from moonshine_amd._lib import lib
from moonshine_amd.synth import CONFIGS, make_inputs

pytestmark = pytest.mark.gpu

_store = {}


def call_static(moe, x, r, precision):
    T, k = x.shape[0], moe.cfg.top_k
    out = torch.empty_like(x)
    ids = torch.zeros((T, k), dtype=torch.int32, device=x.device)
    w = torch.zeros((T, k), dtype=torch.float32, device=x.device)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    ok = lib().k3_moe_forward_static_bf16(
        P(out), P(x), P(r), P(moe.router_weight), P(moe.router_bias), P(moe.store.table),
        ctypes.byref(moe.shape), T, precision, P(ids), P(w),
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    return ok, out, ids, w


def call_ref(moe, x, r, precision):
    T, k = x.shape[0], moe.cfg.top_k
    ids = torch.zeros((T, k), dtype=torch.int32, device=x.device)
    w = torch.zeros((T, k), dtype=torch.float32, device=x.device)
    out = moe.forward(x, r, ids=ids, weights=w, precision=precision)
    return out, ids, w


@pytest.mark.parametrize("cfg_index,sizes,precision", [(1, (48, 1), 0), (1, (64, 5), 1),
                                                        (0, (40, 1), 0)])
def test_static_matches_workspace_entry(cuda, cfg_index, sizes, precision):
    cfg = CONFIGS[cfg_index]
    inputs = make_inputs(cfg, tokens=max(sizes))
    key = (cfg.experts, cfg.hidden, cfg.ffn, cfg.seed)
    if key not in _store:
        _store.clear()
        torch.cuda.empty_cache()
        _store[key] = L.ExpertStore(cfg.experts, cfg.hidden, cfg.ffn, seed=cfg.seed, device=cuda)
    moe = L.build_layer(cfg, inputs, device=cuda, store=_store[key])
    X = L.bf16_tensor(inputs.hidden, cuda)
    R = L.bf16_tensor(inputs.residual, cuda)
    for n, T in enumerate(sizes):
        # a different slice of tokens on each call
        x = X[n:n + T].contiguous()
        r = R[n:n + T].contiguous()
        print(f"static entry: {cfg.name} call {n} T={T} precision={precision}", flush=True)
        ok, o_s, i_s, w_s = call_static(moe, x, r, precision)
        assert ok
        o_r, i_r, w_r = call_ref(moe, x, r, precision)
        torch.cuda.synchronize()
        assert torch.equal(i_s, i_r)
        assert torch.equal(w_s, w_r)
        assert torch.equal(o_s.view(torch.int16), o_r.view(torch.int16))


def test_static_rejects_oversize(cuda):
    cfg = CONFIGS[1]
    shape = L.make_shape(cfg)
    cap = 32 << 20
    T = 1
    while lib().k3_moe_workspace_bytes(ctypes.byref(shape), T) <= cap:
        T += 1
    assert T > 64
    # rejected before any pointer is touched: nothing is launched
    dummy = torch.zeros(16, dtype=torch.int16, device=cuda)
    P = ctypes.c_void_p(dummy.data_ptr())
    assert not lib().k3_moe_forward_static_bf16(P, P, None, P, P, P, ctypes.byref(shape), T, 0,
                                                None, None, None)
