"""Link-level drop-in (CPU): the reference engine's routed-MoE callers
(/root/reference/k3_engine.cu with k3_engine_prefill.inc:938-997,
1448-1614 and k3_engine.cu:1032-1066, 1554-1563, 1851-1897) built from
their own sources against include/ and linked with libk3moe.so in place of
k3_rocm_ops.o's routed-MoE functions and k3_prefill.o
(tests/engine_link/Makefile). Needs the reference sources, so it runs in
the build container only."""
import ctypes
import pathlib
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
REF = pathlib.Path("/root/reference")
D = ROOT / "tests" / "engine_link"
B = D / "_build"
LIB = ROOT / "moonshine_amd" / "libk3moe.so"

pytestmark = pytest.mark.skipif(not (REF / "k3_engine.cu").exists() or not LIB.exists(),
                                reason="needs the reference sources and a built libk3moe.so")


def nm(path, *flags):
    out = subprocess.run(["nm", "-D", *flags, str(path)], capture_output=True, text=True,
                         check=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if ln.split()}


@pytest.fixture(scope="module")
def built():
    r = subprocess.run(["make", "-j8", "-C", str(D)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    return D / "lib" / "libk3engine_on_k3moe.so"


def test_headers_declare_the_reference_signatures(built):
    # header_compat.c compiled as C and C++ with -Werror (Makefile)
    assert (B / "header_compat_c.o").exists() and (B / "header_compat_cpp.o").exists()
    # the engine was compiled with include/k3_prefill.h standing in for the reference's
    assert int((B / "overlay_used.txt").read_text().split()[0]) >= 1


def test_engine_links_against_libk3moe(built):
    ours = {s for s in nm(LIB, "--defined-only") if s.startswith("k3_")}
    eng_defined = nm(built, "--defined-only")
    eng_undefined = nm(built, "--undefined-only")
    # no symbol defined twice: nothing libk3moe exports is also exported by the engine side
    assert not (ours & eng_defined), sorted(ours & eng_defined)
    # the routed-MoE entry points the engine calls resolve to libk3moe
    moe = {"k3_rocm_mxfp4_gemv_bf16", "k3_rocm_mxfp4_gemm_bf16", "k3_rocm_bf16_gemv_f32",
           "k3_rocm_bf16_gemm_f32", "k3_rocm_router_topk_f32", "k3_rocm_router_topk_f32_batch",
           "k3_rocm_situ_bf16", "k3_rocm_gather_rows_bf16", "k3_rocm_scatter_rows_bf16",
           "k3_rocm_weighted_sum_bf16", "k3_rocm_weighted_sum_bf16_batch", "k3_rocm_add_bf16",
           "k3_prefill_plan_build_with_aux_workspace"}
    assert moe <= eng_undefined, sorted(moe - eng_undefined)
    assert moe <= ours
    needed = subprocess.run(["readelf", "-d", str(built)], capture_output=True, text=True,
                            check=True).stdout
    assert "libk3moe.so" in needed
    # the reference's own kernels outside the path stay with the engine
    assert {"k3_rocm_argmax_bf16", "k3_rocm_kda_recurrent_bf16_f32_state"} <= eng_defined
    # every symbol resolves at load time (RTLD_NOW), linked with --no-undefined
    ctypes.CDLL(str(built), mode=ctypes.RTLD_GLOBAL | 2)
