"""Host-side driver of the fused routed-MoE layer (libk3moe.so).

ExpertStore keeps every routed expert of a layer resident in HBM in the
checkpoint-native MXFP4 layout, one contiguous span per expert with the
six tensors in the reference's order (w1 packed/scale, w2 packed/scale,
w3 packed/scale; k3_prefill.c:71-108), and a device table of k3_moe_expert
descriptors. RoutedMoE runs k3_moe_forward_bf16 on it.

torch is used only for device memory and the stream handle.
"""
import ctypes

import numpy as np
import torch

from ._lib import K3MoeExpert, K3MoeShape, lib
from .synth import ACT_SWIGLU, EXACT, Config

_ALIGN = 256


def _align(n):
    return (n + _ALIGN - 1) // _ALIGN * _ALIGN


def expert_tensor_sizes(hidden, ffn):
    """Byte sizes of (gate_p, gate_s, down_p, down_s, up_p, up_s)."""
    return (ffn * hidden // 2, ffn * hidden // 32, hidden * ffn // 2, hidden * ffn // 32,
            ffn * hidden // 2, ffn * hidden // 32)


class ExpertStore:
    """All experts of one layer resident on the device, synthetic contents.

    Tensor j of expert e is generated from stream id e * 8 + j of the
    counter-based generator (k3_moe_synth_fill); scale tensors (j odd) hold
    E8M0 exponents 121..125.
    """

    def __init__(self, experts, hidden, ffn, seed, device="cuda", misalign=0, misalign_odd=False):
        """misalign (0, 4 or 8): start every tensor that many bytes past a
        16-byte boundary (8: as real checkpoint spans do,
        k3_rocm_ops.cu:207-223); misalign_odd: only the tensors of odd
        experts."""
        self.experts, self.hidden, self.ffn, self.seed = experts, hidden, ffn, seed
        self.sizes = expert_tensor_sizes(hidden, ffn)
        self.offsets = []
        off = 0
        for s in self.sizes:
            self.offsets.append(off)
            off += _align(s + misalign)
        self.span = off
        self.payload_bytes = sum(self.sizes)
        self.buffer = torch.empty(experts * self.span, dtype=torch.uint8, device=device)
        base = self.buffer.data_ptr()
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        table = np.zeros((experts, 6), dtype=np.uint64)
        self.shifts = []
        for e in range(experts):
            shift = misalign if (not misalign_odd or e % 2 == 1) else 0
            self.shifts.append(shift)
            for j, (o, s) in enumerate(zip(self.offsets, self.sizes)):
                start = e * self.span + o + shift
                ptr = base + start
                table[e, j] = ptr
                # the generator writes from 8-byte aligned starts: other
                # shifts are filled aligned and copied into place
                tmp = None if shift % 8 == 0 else torch.empty(s, dtype=torch.uint8, device=device)
                dst = ptr if tmp is None else tmp.data_ptr()
                if not lib().k3_moe_synth_fill(ctypes.c_void_p(dst), s, seed, e * 8 + j, j & 1,
                                               stream):
                    raise RuntimeError("k3_moe_synth_fill failed")
                if tmp is not None:
                    self.buffer[start:start + s].copy_(tmp)
        self.table = torch.from_numpy(table.view(np.int64)).to(device)

    def host_expert(self, e):
        """The six tensors of expert e regenerated on the host (numpy uint8)."""
        out = []
        for j, s in enumerate(self.sizes):
            a = np.empty(s, dtype=np.uint8)
            lib().k3_moe_synth_fill_host(a.ctypes.data_as(ctypes.c_void_p), s, self.seed,
                                         e * 8 + j, j & 1)
            out.append(a)
        return out

    def device_expert(self, e):
        """Views of expert e's six tensors in the device buffer."""
        b = e * self.span + self.shifts[e]
        return [self.buffer[b + o: b + o + s] for o, s in zip(self.offsets, self.sizes)]


def make_shape(cfg: Config) -> K3MoeShape:
    return K3MoeShape(cfg.hidden, cfg.experts, cfg.top_k, cfg.ffn, cfg.scale, cfg.activation,
                      cfg.beta, cfg.linear_beta)


class RoutedMoE:
    """One routed-MoE layer: bf16 router + resident MXFP4 experts."""

    def __init__(self, cfg: Config, router_weight, router_bias, store: ExpertStore):
        self.cfg = cfg
        self.shape = make_shape(cfg)
        self.router_weight = router_weight  # torch bf16 [E, H] on device
        self.router_bias = router_bias      # torch f32 [E] on device
        self.store = store
        self._ws = None

    def workspace(self, tokens):
        need = lib().k3_moe_workspace_bytes(ctypes.byref(self.shape), tokens)
        if need == 0:
            raise ValueError("unsupported shape or token count")
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.router_weight.device)
            st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            if not lib().k3_moe_workspace_init(ctypes.c_void_p(self._ws.data_ptr()), need, st):
                raise RuntimeError("k3_moe_workspace_init failed")
        return self._ws

    def forward(self, hidden, residual=None, out=None, ids=None, weights=None,
                precision=EXACT, stream=None):
        T = hidden.shape[0]
        ws = self.workspace(T)
        if out is None:
            out = torch.empty_like(hidden)
        st = torch.cuda.current_stream().cuda_stream if stream is None else stream
        ok = lib().k3_moe_forward_bf16(
            ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(hidden.data_ptr()),
            None if residual is None else ctypes.c_void_p(residual.data_ptr()),
            ctypes.c_void_p(self.router_weight.data_ptr()),
            ctypes.c_void_p(self.router_bias.data_ptr()),
            ctypes.c_void_p(self.store.table.data_ptr()), ctypes.byref(self.shape), T, precision,
            None if ids is None else ctypes.c_void_p(ids.data_ptr()),
            None if weights is None else ctypes.c_void_p(weights.data_ptr()),
            ctypes.c_void_p(ws.data_ptr()), ws.numel(), ctypes.c_void_p(st))
        if not ok:
            raise RuntimeError("k3_moe_forward_bf16 rejected its arguments or failed to launch")
        return out

    def experts_only(self, hidden, ids, weights, residual=None, out=None, precision=EXACT,
                     stream=None):
        T = hidden.shape[0]
        ws = self.workspace(T)
        if out is None:
            out = torch.empty_like(hidden)
        st = torch.cuda.current_stream().cuda_stream if stream is None else stream
        ok = lib().k3_moe_experts_bf16(
            ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(hidden.data_ptr()),
            None if residual is None else ctypes.c_void_p(residual.data_ptr()),
            ctypes.c_void_p(ids.data_ptr()), ctypes.c_void_p(weights.data_ptr()),
            ctypes.c_void_p(self.store.table.data_ptr()), ctypes.byref(self.shape), T, precision,
            ctypes.c_void_p(ws.data_ptr()), ws.numel(), ctypes.c_void_p(st))
        if not ok:
            raise RuntimeError("k3_moe_experts_bf16 rejected its arguments or failed to launch")
        return out


def bf16_tensor(bits, device="cuda"):
    """uint16 bf16 bit array -> torch.bfloat16 device tensor."""
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def bf16_bits(t):
    """torch.bfloat16 tensor -> numpy uint16 bit array (host)."""
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def build_layer(cfg: Config, inputs, device="cuda", store=None):
    if store is None:
        store = ExpertStore(cfg.experts, cfg.hidden, cfg.ffn, seed=cfg.seed, device=device)
    w = bf16_tensor(inputs.router_weight, device)
    b = torch.from_numpy(inputs.router_bias).to(device)
    return RoutedMoE(cfg, w, b, store)


__all__ = ["ExpertStore", "RoutedMoE", "build_layer", "bf16_tensor", "bf16_bits",
           "ACT_SWIGLU", "EXACT"]
