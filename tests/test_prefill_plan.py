"""k3_prefill_plan_build(_with_aux_workspace) on synthetic checkpoint
directories (CPU: the planner is host code in libk3moe.so).

Pinned by the reference's locked constants (tests/test_k3_prefill_plan.c:
15-26: expert/layer/store payload bytes, 1,116,360 workspace bytes per
token, the Q8/32 decode cache, the 176,160,768-byte auxiliary workspace),
by closed forms of the read ledger and segment count of each synthetic
layout, and -- where the reference's own k3_prefill.c has been built from
its sources into oracle/_ref -- by field-for-field equality with it on
every case, failures included.
"""
import ctypes

import numpy as np
import pytest

import _oracle as O
import _st_model as S
from moonshine_amd._lib import LIB_PATH

K3_EXPERT_BYTES = 17547264
K3_LAYER_BYTES = 15722348544
K3_ROUTED_BYTES = 1446456066048
K3_CACHE_32_BYTES = 51659145216
K3_ONE_TOKEN = 1116360
K3_KDA_DEQUANT = 176160768
STAGING = 17551360

ours = S.bind(ctypes.CDLL(str(LIB_PATH)))
ref = S.bind(ctypes.CDLL(str(O.REF_PREFILL))) if O.REF_PREFILL.exists() else None


@pytest.fixture(scope="module")
def numeric():
    return S.layout(shards=4, order="numeric")


@pytest.fixture(scope="module")
def shuffled():
    return S.layout(shards=7, order="shuffled", gap=4096 + 123, seed=3)


def both(directory, *args, **kw):
    got = S.build(ours, directory, *args, **kw)
    if ref is not None:
        want = S.build(ref, directory, *args, **kw)
        assert got[0] == want[0], (got[2], want[2])
        if got[0]:
            assert got[1] == want[1]
    return got


@pytest.mark.parametrize("chunk", [2, 8, 512, 8192, 16384, 32768])
def test_retain_ledger_constants(numeric, chunk):
    ok, p, err = both(numeric, chunk, max(chunk, 8192), 32, 16, 0)
    assert ok, err
    assert p["chunk_tokens"] == chunk
    assert p["routed_layers"] == 92 and p["routed_layer_sweeps"] == 92
    assert p["expert_read_requests"] == 92 * 896
    assert p["shard_segments"] == 92  # one contiguous segment per layer
    assert p["routed_layer_payload_bytes"] == K3_LAYER_BYTES == 896 * K3_EXPERT_BYTES
    assert p["routed_store_payload_bytes"] == K3_ROUTED_BYTES
    assert p["decode_cache_bytes"] == K3_CACHE_32_BYTES
    assert p["batch_workspace_bytes"] == K3_ONE_TOKEN * chunk
    assert p["incremental_workspace_bytes"] == K3_ONE_TOKEN * (chunk - 1)
    assert p["auxiliary_workspace_bytes"] == 0
    assert p["mla_append_bytes"] == chunk * 24 * 576 * 2
    assert p["staging_window_bytes"] == 2 * STAGING
    assert p["registered_staging_bytes"] == 16 * STAGING
    assert p["new_layer_buffer_bytes"] == 0
    assert p["retained_cache_bytes"] == K3_CACHE_32_BYTES
    assert p["borrowed_cache_bytes"] == 0
    assert p["new_device_bytes"] == p["batch_workspace_bytes"]
    # the read ledger of this layout in closed form: each layer's experts
    # are back to back from a 40-byte offset past a page boundary
    req = phys = 0
    ends = [0] * 4
    for layer in range(1, 93):
        s = layer % 4
        pos = max(ends[s], 8 * 4096 + 40)
        for _ in range(896):
            a0, a1 = pos // 4096 * 4096, -(-(pos + K3_EXPERT_BYTES) // 4096) * 4096
            req += a1 - a0
            pos += K3_EXPERT_BYTES
            phys += a1 - a0
        ends[s] = pos
    # the last expert of each shard's final layer is clipped to the file
    # (file = end + 4096 * 3 + 17, so nothing is clipped here)
    assert p["routed_store_requested_read_bytes"] == req
    assert p["routed_store_physical_read_bytes"] == phys


def test_segments_follow_physical_order(shuffled):
    ok, p, err = both(shuffled, 2, 8192, 32, 16, 0)
    assert ok, err
    # 896 experts per layer with a gap after every 7th in physical order
    # (after positions 6, 13, ..., 895): 127 breaks inside the layer, the
    # last gap follows its final expert -> 128 segments per layer
    assert p["shard_segments"] == 92 * 128
    assert p["routed_store_payload_bytes"] == K3_ROUTED_BYTES


def test_leases(numeric):
    ok, p, err = both(numeric, 8, 8192, 32, 16, 1)  # borrow cold
    assert ok, err
    assert p["borrowed_cache_bytes"] == p["batch_workspace_bytes"]
    assert p["retained_cache_bytes"] == K3_CACHE_32_BYTES - p["batch_workspace_bytes"]
    assert p["new_device_bytes"] == 0
    ok, p, err = both(numeric, 3905, 8192, 32, 16, 2)  # borrow warm: whole expert slots
    assert ok, err
    slots = -(-p["batch_workspace_bytes"] // K3_EXPERT_BYTES)
    assert p["borrowed_cache_bytes"] == slots * K3_EXPERT_BYTES
    assert p["retained_cache_bytes"] == K3_CACHE_32_BYTES - slots * K3_EXPERT_BYTES
    ok, p, err = both(numeric, 65536, 131072, 30, 16, 2)  # too big to lend
    assert not ok and "cannot lend" in err
    for chunk in (16384, 32768):
        ok, p, err = both(numeric, chunk, chunk, 32, 16, 1)
        assert ok, err


def test_auxiliary_workspace(numeric):
    ok, p, err = both(numeric, 8192, 8192, 32, 16, 1, aux=K3_KDA_DEQUANT)
    assert ok, err
    assert p["auxiliary_workspace_bytes"] == K3_KDA_DEQUANT
    assert p["batch_workspace_bytes"] == K3_ONE_TOKEN * 8192 + K3_KDA_DEQUANT
    assert p["incremental_workspace_bytes"] == K3_ONE_TOKEN * 8191
    assert p["borrowed_cache_bytes"] == p["batch_workspace_bytes"] and p["new_device_bytes"] == 0
    ok, p, err = both(numeric, 512, 8192, 32, 16, 0, aux=K3_KDA_DEQUANT)
    assert ok, err
    assert p["retained_cache_bytes"] == K3_CACHE_32_BYTES
    assert p["new_device_bytes"] == p["batch_workspace_bytes"] == K3_ONE_TOKEN * 512 + K3_KDA_DEQUANT


def test_argument_checks(numeric):
    for args in [(2, 1048577), (0, 8192), (9000, 8192)]:
        ok, p, err = both(numeric, *args, 32, 16, 0)
        assert not ok and err
        assert all(v == 0 for v in p.values())  # *plan zeroed
    assert not both(numeric, 2, 8192, 0, 16, 0)[0]   # no decode-cache experts
    assert not both(numeric, 2, 8192, 32, 1, 0)[0]   # fewer than 2 staging slots
    assert not both(numeric, 2, 8192, 32, 16, 3)[0]  # unknown lease
    ok, p, err = both(numeric, 2, 131072, 32, 16, 0)
    assert ok and p["context_remaining"] == 131072


def _drop(name):
    def f(entries):
        entries[:] = [e for e in entries if e[0] != name]
    return f


def _edit(name, **kw):
    cols = {"shard": 1, "offset": 2, "length": 3, "dtype": 4}

    def f(entries):
        for e in entries:
            if e[0] == name:
                for k, v in kw.items():
                    e[cols[k]] = v(e[cols[k]]) if callable(v) else v
    return f


@pytest.mark.parametrize("mutate,needle", [
    (_drop(S.expert_name(40, 7, "w2.weight_scale")), "missing"),
    (_edit(S.expert_name(3, 100, "w3.weight_packed"), dtype=S.DTYPE_BF16), "contiguous"),
    (_edit(S.expert_name(92, 0, "w2.weight_packed"), offset=lambda o: o + 64), "contiguous"),
    (_edit(S.expert_name(5, 9, "w1.weight_scale"), shard=lambda s: (s + 1) % 4), "contiguous"),
], ids=["missing", "dtype", "hole", "split-shard"])
def test_directory_errors(mutate, needle):
    d = S.layout(shards=4, order="numeric", mutate=mutate)
    ok, _, err = both(d, 2, 8192, 32, 16, 0)
    assert not ok and needle in err, err


def test_overlap_and_short_file_rejected():
    def overlap(entries):
        # move layer 7's expert 300 onto expert 299's bytes
        delta = -K3_EXPERT_BYTES // 2
        for e in entries:
            if e[0].startswith("language_model.model.layers.7.block_sparse_moe.experts.300."):
                e[2] += delta
    ok, _, err = both(S.layout(shards=4, mutate=overlap), 2, 8192, 32, 16, 0)
    assert not ok and "overlap" in err, err
    ok, _, err = both(S.layout(shards=4, tail=-100), 2, 8192, 32, 16, 0)
    assert not ok and "ledger" in err, err


@pytest.mark.skipif(ref is None, reason="reference planner not built (oracle/_ref)")
def test_reference_built_from_source_is_loaded():
    assert ref is not None and hasattr(ref, "k3_prefill_plan_build")
