"""Host-side driver of the K3-native MoE layer (k3_moe_native_forward_bf16).

The routed experts (ExpertStore, MXFP4) run on a latent of width D between
two static projections (routed_down [D, H], routed_up [H, D]) with an RMSNorm
in between, beside a dense shared expert (gate/up [S, H], down [H, S]); see
include/k3_moe.h. Static weights are bf16 or Q8-128. Synthetic weights are
generated on the device from a seeded torch generator (N(0, 0.02) static
projections, N(1, 0.1) norm weight); Q8-128 codes come from the library's
own quantizer. torch is used only for device memory and streams.
"""
import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from ._lib import K3MoeNativeShape, K3MoeNativeWeights, K3MoeShape, K3MoeStaticWeight, lib
from .layer import ExpertStore, bf16_bits
from .synth import ACT_SITU, EXACT, f32_to_bf16_bits

STATIC_BF16, STATIC_Q8 = 0, 1


@dataclass(frozen=True)
class NativeConfig:
    name: str
    tokens: int
    hidden: int          # H: router columns, layer width
    latent: int          # D: expert input/output width
    experts: int
    top_k: int
    ffn: int             # F: expert intermediate width
    shared: int          # shared expert intermediate width
    scale: float = 1.0
    activation: int = ACT_SITU
    beta: float = 4.0
    linear_beta: float = 25.0
    eps: float = 1e-5
    static_kind: int = STATIC_Q8
    seed: int = 0


# The K3 layer as the reference engine runs it (k3_engine.cu:35-45): H 7168,
# latent 3584, 896 experts of F 3072, top-16, shared expert 6144, SiTU(4, 25),
# routed scale 1, Q8-128 static projections.
K3_NATIVE_LAYER = NativeConfig("k3-native-layer", 1, 7168, 3584, 896, 16, 3072, 6144, seed=1006)


def routed_shape(cfg: NativeConfig) -> K3MoeShape:
    return K3MoeShape(cfg.latent, cfg.experts, cfg.top_k, cfg.ffn, cfg.scale, cfg.activation,
                      cfg.beta, cfg.linear_beta)


class StaticWeight:
    """One static projection [rows, columns] on the device."""

    def __init__(self, rows, cols, kind, gen, device):
        self.rows, self.cols, self.kind = rows, cols, kind
        w = (torch.randn((rows, cols), generator=gen, device=device) * 0.02).to(torch.bfloat16)
        if kind == STATIC_BF16:
            self.data, self.scales = w, None
        else:
            self.data = torch.empty((rows, cols), dtype=torch.int8, device=device)
            self.scales = torch.empty((rows, cols // 128), dtype=torch.float32, device=device)
            st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            if not lib().k3_rocm_bf16_quantize_q8_128(ctypes.c_void_p(self.data.data_ptr()),
                                                      ctypes.c_void_p(self.scales.data_ptr()),
                                                      ctypes.c_void_p(w.data_ptr()), rows, cols,
                                                      st):
                raise RuntimeError("k3_rocm_bf16_quantize_q8_128 failed")
            del w

    def c_struct(self):
        return K3MoeStaticWeight(self.kind, self.rows, self.cols, self.data.data_ptr(),
                                 None if self.scales is None else self.scales.data_ptr())

    def host(self):
        """(kind, data, scales) as numpy (bf16 bits or int8 codes + f32)."""
        if self.kind == STATIC_BF16:
            return self.kind, bf16_bits(self.data), None
        return self.kind, self.data.cpu().numpy(), self.scales.cpu().numpy()

    @property
    def nbytes(self):
        return self.data.numel() * self.data.element_size() + (
            0 if self.scales is None else self.scales.numel() * 4)


class NativeLayer:
    """One K3-native MoE layer with synthetic weights resident on the device."""

    def __init__(self, cfg: NativeConfig, device="cuda", store=None):
        self.cfg = cfg
        gen = torch.Generator(device=device)
        gen.manual_seed(cfg.seed)
        H, D, S, E = cfg.hidden, cfg.latent, cfg.shared, cfg.experts
        rng = np.random.default_rng(cfg.seed)
        self.router_weight_bits = f32_to_bf16_bits(rng.normal(0, 0.02, (E, H)).astype(np.float32))
        self.router_bias = rng.normal(0, 0.01, E).astype(np.float32)
        self.norm_bits = f32_to_bf16_bits(rng.normal(1.0, 0.1, D).astype(np.float32))
        self.router_weight = torch.from_numpy(self.router_weight_bits.view(np.int16)).to(device)
        self.router_bias_d = torch.from_numpy(self.router_bias).to(device)
        self.norm = torch.from_numpy(self.norm_bits.view(np.int16)).to(device)
        k = cfg.static_kind
        self.routed_down = StaticWeight(D, H, k, gen, device)
        self.routed_up = StaticWeight(H, D, k, gen, device)
        self.shared_gate = StaticWeight(S, H, k, gen, device)
        self.shared_up = StaticWeight(S, H, k, gen, device)
        self.shared_down = StaticWeight(H, S, k, gen, device)
        self.store = store if store is not None else ExpertStore(E, D, cfg.ffn, seed=cfg.seed,
                                                                 device=device)
        self.shape = K3MoeNativeShape(routed_shape(cfg), H, S, cfg.eps)
        self.weights = K3MoeNativeWeights(
            self.router_weight.data_ptr(), self.router_bias_d.data_ptr(),
            self.routed_down.c_struct(), self.norm.data_ptr(), self.routed_up.c_struct(),
            self.shared_gate.c_struct(), self.shared_up.c_struct(), self.shared_down.c_struct(),
            self.store.table.data_ptr())
        self._ws = None

    def statics(self):
        return dict(routed_down=self.routed_down, routed_up=self.routed_up,
                    shared_gate=self.shared_gate, shared_up=self.shared_up,
                    shared_down=self.shared_down)

    def static_bytes(self):
        return sum(w.nbytes for w in self.statics().values())

    def workspace(self, tokens):
        need = lib().k3_moe_native_workspace_bytes(ctypes.byref(self.shape), tokens)
        if need == 0:
            raise ValueError("unsupported native shape or token count")
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.router_weight.device)
        return self._ws

    def forward(self, hidden, residual=None, out=None, ids=None, weights=None, precision=EXACT,
                stream=None, shared_stream=None):
        T = hidden.shape[0]
        ws = self.workspace(T)
        if out is None:
            out = torch.empty_like(hidden)
        st = torch.cuda.current_stream().cuda_stream if stream is None else stream
        P = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
        ok = lib().k3_moe_native_forward_bf16(P(out), P(hidden), P(residual),
                                              ctypes.byref(self.weights), ctypes.byref(self.shape),
                                              T, precision, P(ids), P(weights), P(ws), ws.numel(),
                                              ctypes.c_void_p(st),
                                              None if shared_stream is None
                                              else ctypes.c_void_p(shared_stream))
        if not ok:
            raise RuntimeError("k3_moe_native_forward_bf16 rejected its arguments or failed")
        return out


__all__ = ["NativeConfig", "NativeLayer", "K3_NATIVE_LAYER", "STATIC_BF16", "STATIC_Q8"]
