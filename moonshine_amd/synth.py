"""Seeded synthetic inputs of the benchmark configurations (numpy, host).

Normal tensors (router weight, bias, hidden state, residual) come from
numpy's PCG64 generator and are rounded to bf16 (RNE) on the host. The big
MXFP4 expert store is generated on the device by k3_moe_synth_fill
(layer.ExpertStore).
"""
from dataclasses import dataclass

import numpy as np

EXACT = 0
MFMA = 1      # two-term MXFP8 activations on scaled MFMA (bf16 tolerance)
MFMA_FP8 = 2  # one-term MXFP8 activations (approximate)
ACT_SITU = 0
ACT_SWIGLU = 1


@dataclass(frozen=True)
class Config:
    name: str
    tokens: int
    hidden: int
    experts: int
    top_k: int
    ffn: int
    scale: float = 2.5
    activation: int = ACT_SWIGLU
    beta: float = 4.0
    linear_beta: float = 25.0
    zipf: bool = False
    seed: int = 0


# BASELINE.json configs (index = position in "configs"). Config 0 names no
# routed scale; 2.5 is used, as for the others.
CONFIGS = [
    Config("cfg0-reduced", 1, 2048, 64, 4, 512, seed=1000),
    Config("cfg1-k3-decode", 1, 7168, 896, 16, 2048, seed=1001),
    Config("cfg2-k3-batched-decode", 64, 7168, 896, 16, 2048, seed=1002),
    Config("cfg3-k3-prefill-512", 512, 7168, 896, 16, 2048, seed=1003),
    Config("cfg4-k3-prefill-8192-zipf", 8192, 7168, 896, 16, 2048, zipf=True, seed=1004),
]
# K3-native expert stage (latent 3584, expert hidden 3072, SiTU(4,25), scale 1).
K3_NATIVE = Config("k3-native", 1, 3584, 896, 16, 3072, scale=1.0, activation=ACT_SITU,
                   seed=1005)


def f32_to_bf16_bits(a):
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.asarray(a, dtype=np.float32, order="C").view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = np.where(nan, (u >> 16) | 0x40, (u + 0x7FFF + ((u >> 16) & 1)) >> 16)
    return np.asarray(r, dtype=np.uint16)


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


@dataclass
class HostInputs:
    router_weight: np.ndarray  # uint16 bf16 bits [E, H]
    router_bias: np.ndarray    # float32 [E]
    hidden: np.ndarray         # uint16 bf16 bits [T, H]
    residual: np.ndarray       # uint16 bf16 bits [T, H]


def make_inputs(cfg: Config, tokens: int | None = None, seed: int | None = None) -> HostInputs:
    T = cfg.tokens if tokens is None else tokens
    rng = np.random.default_rng(cfg.seed if seed is None else seed)
    w = f32_to_bf16_bits(rng.normal(0.0, 0.02, (cfg.experts, cfg.hidden)).astype(np.float32))
    if cfg.zipf:
        rank = rng.permutation(cfg.experts) + 1
        bias = (2.0 * rank.astype(np.float64) ** -1.1).astype(np.float32)
    else:
        bias = rng.normal(0.0, 0.01, cfg.experts).astype(np.float32)
    x = f32_to_bf16_bits(rng.normal(0.0, 1.0, (T, cfg.hidden)).astype(np.float32))
    r = f32_to_bf16_bits(rng.normal(0.0, 1.0, (T, cfg.hidden)).astype(np.float32))
    return HostInputs(w, bias, x, r)
