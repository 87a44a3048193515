"""GPU parity of k3_moe_routed_bf16 (router on one input, experts on another,
the K3 engine's form) against the oracle composed from its pinned pieces:
reference-order router logits on the router input, the reference top-k, and
the routed experts + combine on the expert input. Bit-identical ids,
weights and output."""
import ctypes

import numpy as np
import pytest
import torch

import _oracle as O
from moonshine_amd._lib import lib
from moonshine_amd.layer import ExpertStore, RoutedMoE, bf16_bits, bf16_tensor
from moonshine_amd.synth import Config, HostInputs, f32_to_bf16_bits

pytestmark = pytest.mark.gpu

_p = ctypes.c_void_p


def run_routed(cuda, T, R, residual=True, seed=0):
    cfg = Config("routed-small", T, 512, 64, 4, 256, seed=3100 + seed)
    rng = np.random.default_rng(cfg.seed + 7 * T + R)
    rw = f32_to_bf16_bits(rng.normal(0, 0.02, (cfg.experts, R)).astype(np.float32))
    bias = rng.normal(0, 0.01, cfg.experts).astype(np.float32)
    rx = f32_to_bf16_bits(rng.normal(0, 1, (T, R)).astype(np.float32))
    ex = f32_to_bf16_bits(rng.normal(0, 1, (T, cfg.hidden)).astype(np.float32))
    res = f32_to_bf16_bits(rng.normal(0, 1, (T, cfg.hidden)).astype(np.float32)) if residual else None
    store = ExpertStore(cfg.experts, cfg.hidden, cfg.ffn, seed=cfg.seed, device=cuda)
    moe = RoutedMoE(cfg, bf16_tensor(rw, cuda), torch.from_numpy(bias).to(cuda), store)
    ws = moe.workspace(T)
    d_rx, d_ex = bf16_tensor(rx, cuda), bf16_tensor(ex, cuda)
    d_res = None if res is None else bf16_tensor(res, cuda)
    out = torch.empty_like(d_ex)
    ids = torch.zeros((T, cfg.top_k), dtype=torch.int32, device=cuda)
    w = torch.zeros((T, cfg.top_k), dtype=torch.float32, device=cuda)
    st = torch.cuda.current_stream().cuda_stream
    print(f"\nk3_moe_routed_bf16 T={T} router_columns={R} residual={residual}", flush=True)
    ok = lib().k3_moe_routed_bf16(
        _p(out.data_ptr()), _p(d_rx.data_ptr()), R, _p(d_ex.data_ptr()),
        None if d_res is None else _p(d_res.data_ptr()), _p(moe.router_weight.data_ptr()),
        _p(moe.router_bias.data_ptr()), _p(store.table.data_ptr()), ctypes.byref(moe.shape), T,
        0, _p(ids.data_ptr()), _p(w.data_ptr()), _p(ws.data_ptr()), ws.numel(), _p(st))
    assert ok
    torch.cuda.synchronize()
    got_ids = ids.cpu().numpy().view(np.uint32)

    logits = O.router_logits(rw, rx)
    want_ids, want_w = O.router_topk(logits, bias, cfg.top_k, cfg.scale)
    np.testing.assert_array_equal(got_ids, want_ids)
    np.testing.assert_array_equal(w.cpu().numpy(), want_w)
    experts = {int(e): store.host_expert(int(e)) for e in np.unique(want_ids)}
    rin = HostInputs(np.zeros((cfg.experts, cfg.hidden), np.uint16), bias, ex, res)
    want = O.layer(cfg, rin, experts, ids=want_ids, weights=want_w)["output"]
    np.testing.assert_array_equal(bf16_bits(out), want)


# (1, 1024) and (1, 8192): the decode kernels with a router wider than the
# experts; (1, 8200): one token past the decode router's width, through the
# batched router; 3 and 40 tokens: the batched router (40: its MFMA form).
@pytest.mark.parametrize("T,R", [(1, 1024), (1, 8192), (1, 8200), (3, 1024), (40, 2048)])
def test_routed_bitexact(cuda, T, R):
    run_routed(cuda, T, R)


def test_routed_without_residual(cuda):
    run_routed(cuda, 1, 1024, residual=False, seed=1)
    run_routed(cuda, 5, 1024, residual=False, seed=2)


def test_routed_rejects_bad_router_width(cuda):
    """router_columns must be a multiple of 8 (16-byte router rows)."""
    cfg = Config("routed-small", 1, 512, 64, 4, 256)
    store = ExpertStore(cfg.experts, cfg.hidden, cfg.ffn, seed=1, device=cuda)
    R = 1020
    moe = RoutedMoE(cfg, torch.zeros((cfg.experts, R), dtype=torch.bfloat16, device=cuda),
                    torch.zeros(cfg.experts, dtype=torch.float32, device=cuda), store)
    ws = moe.workspace(1)
    rx = torch.zeros((1, R), dtype=torch.bfloat16, device=cuda)
    ex = torch.zeros((1, cfg.hidden), dtype=torch.bfloat16, device=cuda)
    out = torch.empty_like(ex)
    st = torch.cuda.current_stream().cuda_stream
    assert not lib().k3_moe_routed_bf16(
        _p(out.data_ptr()), _p(rx.data_ptr()), R, _p(ex.data_ptr()), None,
        _p(moe.router_weight.data_ptr()), _p(moe.router_bias.data_ptr()),
        _p(store.table.data_ptr()), ctypes.byref(moe.shape), 1, 0, None, None,
        _p(ws.data_ptr()), ws.numel(), _p(st))
