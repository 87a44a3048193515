"""ctypes binding of libk3moe.so, the gfx950 routed-MoE library.

The shared library is the product; this module only declares its C ABI
(include/k3_rocm_ops.h, include/k3_moe.h). There is no fallback: if the
library is missing, importing an op raises.
"""
import ctypes
import pathlib

LIB_PATH = pathlib.Path(__file__).resolve().with_name("libk3moe.so")

_b = ctypes.c_bool
_p = ctypes.c_void_p
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64
_f = ctypes.c_float
_sz = ctypes.c_size_t


class K3MoeShape(ctypes.Structure):
    """k3_moe_shape (include/k3_moe.h)."""

    _fields_ = [
        ("hidden", _u32),
        ("expert_count", _u32),
        ("top_k", _u32),
        ("ffn", _u32),
        ("scaling_factor", _f),
        ("activation", _u32),
        ("beta", _f),
        ("linear_beta", _f),
    ]


class K3MoeExpert(ctypes.Structure):
    """k3_moe_expert (include/k3_moe.h): six device pointers."""

    _fields_ = [
        ("gate_packed", _p),
        ("gate_scales", _p),
        ("down_packed", _p),
        ("down_scales", _p),
        ("up_packed", _p),
        ("up_scales", _p),
    ]


class K3MoeStaticWeight(ctypes.Structure):
    """k3_moe_static_weight (include/k3_moe.h)."""

    _fields_ = [("kind", _u32), ("rows", _u32), ("columns", _u32), ("data", _p),
                ("scales", _p)]


class K3MoeNativeShape(ctypes.Structure):
    """k3_moe_native_shape (include/k3_moe.h)."""

    _fields_ = [("routed", K3MoeShape), ("model_hidden", _u32), ("shared_hidden", _u32),
                ("norm_epsilon", _f)]


class K3MoeNativeWeights(ctypes.Structure):
    """k3_moe_native_weights (include/k3_moe.h)."""

    _fields_ = [("router_weight", _p), ("router_bias", _p), ("routed_down", K3MoeStaticWeight),
                ("routed_norm", _p), ("routed_up", K3MoeStaticWeight),
                ("shared_gate", K3MoeStaticWeight), ("shared_up", K3MoeStaticWeight),
                ("shared_down", K3MoeStaticWeight), ("experts", _p)]


STAGES = ("router", "topk", "plan", "gate_up", "down", "combine", "end")


class K3MoeProfile(ctypes.Structure):
    """k3_moe_profile: hipEvent_t recorded before each stage."""

    _fields_ = [("stage_events", _p * len(STAGES))]


# name -> (restype, argtypes); every symbol declared in include/*.h.
SIGNATURES = {
    "k3_rocm_situ_bf16": (_b, [_p, _p, _p, _u64, _f, _f, _p]),
    "k3_rocm_swiglu_bf16": (_b, [_p, _p, _p, _u64, _p]),
    "k3_rocm_mxfp4_gemv_bf16": (_b, [_p, _p, _p, _p, _u32, _u32, _p]),
    "k3_rocm_mxfp4_gemm_bf16": (_b, [_p, _p, _p, _p, _u32, _u32, _u32, _p]),
    "k3_rocm_mxfp4_gemm_tiled_bf16": (_b, [_p, _p, _p, _p, _u32, _u32, _u32, _u32, _p]),
    "k3_rocm_bf16_gemv_f32": (_b, [_p, _p, _p, _u32, _u32, _p]),
    "k3_rocm_bf16_gemm_f32": (_b, [_p, _p, _p, _u32, _u32, _u32, _p]),
    "k3_rocm_bf16_gemm_tiled_f32": (_b, [_p, _p, _p, _u32, _u32, _u32, _u32, _p]),
    "k3_rocm_rms_norm_bf16": (_b, [_p, _p, _p, _u32, _u32, _f, _p]),
    "k3_rocm_bf16_gemv_bf16": (_b, [_p, _p, _p, _u32, _u32, _p]),
    "k3_rocm_bf16_gemm_bf16": (_b, [_p, _p, _p, _u32, _u32, _u32, _p]),
    "k3_rocm_bf16_gemm_tiled_bf16": (_b, [_p, _p, _p, _u32, _u32, _u32, _u32, _p]),
    "k3_rocm_bf16_quantize_q8_128": (_b, [_p, _p, _p, _u32, _u32, _p]),
    "k3_rocm_q8_128_dequantize_bf16": (_b, [_p, _p, _p, _u32, _u32, _p]),
    "k3_rocm_q8_128_gemv_bf16": (_b, [_p, _p, _p, _p, _u32, _u32, _p]),
    "k3_rocm_q8_128_gemm_bf16": (_b, [_p, _p, _p, _p, _u32, _u32, _u32, _p]),
    "k3_rocm_q8_128_gemm_tiled_bf16": (_b, [_p, _p, _p, _p, _u32, _u32, _u32, _u32, _p]),
    "k3_rocm_router_topk_f32": (_b, [_p, _p, _p, _p, _u32, _u32, _f, _p]),
    "k3_rocm_router_topk_f32_batch": (_b, [_p, _p, _p, _p, _u32, _u32, _u32, _f, _p]),
    "k3_rocm_weighted_sum_bf16": (_b, [_p, _p, _p, _u32, _u32, _p]),
    "k3_rocm_weighted_sum_bf16_batch": (_b, [_p, _p, _p, _u32, _u32, _u32, _p]),
    "k3_rocm_gather_rows_bf16": (_b, [_p, _p, _p, _u32, _u32, _p]),
    "k3_rocm_scatter_rows_bf16": (_b, [_p, _p, _p, _u32, _u32, _p]),
    "k3_rocm_add_bf16": (_b, [_p, _p, _p, _u64, _p]),
    "k3_moe_workspace_bytes": (_sz, [ctypes.POINTER(K3MoeShape), _u32]),
    "k3_moe_native_workspace_bytes": (_sz, [ctypes.POINTER(K3MoeNativeShape), _u32]),
    "k3_moe_native_forward_bf16": (_b, [_p, _p, _p, ctypes.POINTER(K3MoeNativeWeights),
                                        ctypes.POINTER(K3MoeNativeShape), _u32, _u32, _p, _p,
                                        _p, _sz, _p, _p]),
    "k3_moe_workspace_init": (_b, [_p, _sz, _p]),
    "k3_moe_plan_scratch_bytes": (_sz, [_u32, _u32]),
    "k3_moe_router_scratch_bytes": (_sz, [_u32, _u32]),
    "k3_moe_router_bf16": (_b, [_p, _p, _p, _p, _p, _u32, _u32, _u32, _u32, _f, _p, _sz, _p]),
    "k3_moe_route_plan": (_b, [_p, _p, _p, _p, _p, _p, _p, _u32, _u32, _u32, _p, _sz, _p]),
    "k3_moe_forward_bf16": (_b, [_p, _p, _p, _p, _p, _p, ctypes.POINTER(K3MoeShape), _u32,
                                 _u32, _p, _p, _p, _sz, _p]),
    "k3_moe_forward_profiled_bf16": (_b, [_p, _p, _p, _p, _p, _p, ctypes.POINTER(K3MoeShape),
                                          _u32, _u32, _p, _p, _p, _sz, _p, _p]),
    "k3_moe_forward_static_bf16": (_b, [_p, _p, _p, _p, _p, _p, ctypes.POINTER(K3MoeShape),
                                        _u32, _u32, _p, _p, _p]),
    "k3_moe_routed_bf16": (_b, [_p, _p, _u32, _p, _p, _p, _p, _p, ctypes.POINTER(K3MoeShape),
                                _u32, _u32, _p, _p, _p, _sz, _p]),
    "k3_moe_router_choices_f32": (_b, [_p, _p, _p, _u32, _u32, _p]),
    "k3_moe_experts_bf16": (_b, [_p, _p, _p, _p, _p, _p, ctypes.POINTER(K3MoeShape), _u32,
                                 _u32, _p, _sz, _p]),
    "k3_moe_proj_mfma_bf16": (_b, [_p, _p, _p, _p, _u32, _u32, _u32, ctypes.c_bool, _p]),
    "k3_moe_synth_fill": (_b, [_p, _u64, _u64, _u64, _u32, _p]),
    "k3_moe_synth_fill_host": (None, [_p, _u64, _u64, _u64, _u32]),
    "k3_moe_mx8_quantize_bf16": (_b, [_p, _p, _p, _p, _p, _u64, _p]),
    "k3_moe_mx8_quantize_rows_bf16": (_b, [_p, _p, _p, _p, _p, _u32, _u32, _p]),
}

_lib = None


def lib():
    """Load libk3moe.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `make -C moonshine_amd` "
                "(or __graft_entry__.build()); there is no fallback path")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib
