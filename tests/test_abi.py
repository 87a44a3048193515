"""The C ABI (CPU): libk3moe.so loads and exports every function that
include/*.h declares, the ctypes table covers them, and the host-only entry
points (sizes, argument validation) behave without a GPU."""
import ctypes
import pathlib
import re

import pytest

from moonshine_amd import _lib
from moonshine_amd.synth import CONFIGS

ROOT = pathlib.Path(__file__).resolve().parents[1]
DECL = re.compile(r"^(?:bool|size_t|void|uint\w+_t|int)\s+\**(k3_\w+)\s*\(", re.M)


def declared():
    out = {}
    for h in sorted((ROOT / "include").glob("*.h")):
        for name in DECL.findall(h.read_text()):
            out[name] = h.name
    return out


def test_headers_declare_entry_points():
    d = declared()
    assert "k3_moe_forward_bf16" in d and "k3_rocm_mxfp4_gemv_bf16" in d
    assert "k3_prefill_plan_build" in d and "k3_prefill_plan_build_with_aux_workspace" in d
    assert len(d) >= 28


@pytest.mark.parametrize("name", sorted(declared()))
def test_library_exports(name):
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    assert hasattr(lib, name), f"{name} ({declared()[name]}) is not exported"


def test_ctypes_table_covers_moe_and_ops_headers():
    missing = [n for n, h in declared().items()
               if h in ("k3_moe.h", "k3_rocm_ops.h") and n not in _lib.SIGNATURES]
    assert not missing, missing


def shape(cfg):
    return _lib.K3MoeShape(cfg.hidden, cfg.experts, cfg.top_k, cfg.ffn, cfg.scale, cfg.activation,
                           cfg.beta, cfg.linear_beta)


def test_workspace_sizes_and_validation():
    L = _lib.lib()
    s1 = L.k3_moe_workspace_bytes(ctypes.byref(shape(CONFIGS[1])), 1)
    s4 = L.k3_moe_workspace_bytes(ctypes.byref(shape(CONFIGS[4])), 8192)
    assert 0 < s1 < (1 << 24) and s4 > 8192 * 16 * 7168 * 2
    assert s1 % 256 == 0 and s4 % 256 == 0
    assert L.k3_moe_workspace_bytes(ctypes.byref(shape(CONFIGS[1])), 0) == 0
    assert L.k3_moe_workspace_bytes(ctypes.byref(shape(CONFIGS[1])), 65536) == 0
    bad = shape(CONFIGS[1])
    bad.top_k = 33
    assert L.k3_moe_workspace_bytes(ctypes.byref(bad), 4) == 0
    assert L.k3_moe_plan_scratch_bytes(8192, 896) >= 4 * 896 * 32
    # argument checks return false before touching a device
    assert not L.k3_moe_forward_bf16(None, None, None, None, None, None,
                                     ctypes.byref(shape(CONFIGS[1])), 1, 0, None, None, None, 0,
                                     None)
    assert not L.k3_rocm_mxfp4_gemv_bf16(None, None, None, None, 16, 64, None)
    assert not L.k3_moe_mx8_quantize_bf16(None, None, None, None, None, 32, None)
    assert not L.k3_moe_mx8_quantize_rows_bf16(None, None, None, None, None, 1, 32, None)


def test_router_scratch_sizes_and_validation():
    """k3_moe_router_bf16: scratch sized for the K-sliced approximate logits
    of small batches (at most 16 slices, about 512 tile-slice works), one
    slice at large batches; bad arguments return false before any launch."""
    L = _lib.lib()
    T, E = 8192, 896
    big = L.k3_moe_router_scratch_bytes(T, E)
    assert big >= 4 * T * E + 4 * E and big < 2 * 4 * T * E  # one slice at T = 8192
    small = L.k3_moe_router_scratch_bytes(64, E)
    assert small >= 16 * 4 * 64 * E  # 7 tiles: 16 slices
    assert L.k3_moe_router_scratch_bytes(0, E) == 0
    assert L.k3_moe_router_scratch_bytes(65536, E) == 0
    assert L.k3_moe_router_scratch_bytes(64, 1025) == 0
    p = ctypes.c_void_p(256)  # never dereferenced: the checks fail first
    assert not L.k3_moe_router_bf16(p, p, p, p, p, 64, E, 7168, 16, 1.0, p, small - 1, None)
    assert not L.k3_moe_router_bf16(p, p, p, p, p, 64, E, 7168, 33, 1.0, p, small, None)
    assert not L.k3_moe_router_bf16(p, p, p, p, p, 64, E, 0, 16, 1.0, p, small, None)
    assert not L.k3_moe_router_bf16(p, p, p, p, p, 64, 8, 7168, 16, 1.0, p, small, None)
    assert not L.k3_moe_router_bf16(None, p, p, p, p, 64, E, 7168, 16, 1.0, p, small, None)
    assert not L.k3_moe_router_bf16(p, p, p, p, p, 64, E, 7168, 16, 1.0,
                                    ctypes.c_void_p(264), small, None)  # scratch not 256-aligned


def test_row_alignment_is_validated_before_launch():
    """output / hidden / residual rows move 16 bytes at a time: a pointer
    that is not 16-byte aligned is refused (false, nothing launched)."""
    L = _lib.lib()
    s = ctypes.byref(shape(CONFIGS[1]))
    buf = (ctypes.c_uint8 * 4096)()
    base = (ctypes.addressof(buf) + 255) & ~255
    ok, off = ctypes.c_void_p(base), ctypes.c_void_p(base + 8)
    for out, hid, res in ((off, ok, ok), (ok, off, ok), (ok, ok, off)):
        assert not L.k3_moe_forward_bf16(out, hid, res, ok, ok, ok, s, 1, 0, None, None, ok,
                                         1 << 40, None)
        assert not L.k3_moe_experts_bf16(out, hid, res, ok, ok, ok, s, 1, 0, ok, 1 << 40, None)
