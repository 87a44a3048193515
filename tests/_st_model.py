"""In-memory k3_st_model tensor directories for the prefill planner tests.

Builds the C structs of k3_safetensors.h (tensor names sorted by strcmp, as
k3_st_model_open leaves them) over numpy buffers, so the planner can be
called through ctypes on synthetic checkpoint layouts. Test infrastructure.
"""
import ctypes

import numpy as np

LAYERS, EXPERTS = 92, 896
PARTS = ("w1.weight_packed", "w1.weight_scale", "w2.weight_packed", "w2.weight_scale",
         "w3.weight_packed", "w3.weight_scale")
# K3 expert tensors: w1/w3 [3072, 3584] and w2 [3584, 3072] MXFP4
PART_BYTES = (3072 * 3584 // 2, 3072 * 3584 // 32, 3584 * 3072 // 2, 3584 * 3072 // 32,
              3072 * 3584 // 2, 3072 * 3584 // 32)
EXPERT_BYTES = sum(PART_BYTES)
assert EXPERT_BYTES == 17547264
DTYPE_U8, DTYPE_BF16 = 3, 1

TENSOR = np.dtype({"names": ["name", "offset", "length", "shape", "shard", "ndim", "dtype"],
                   "formats": [np.uint64, np.uint64, np.uint64, (np.uint64, 8), np.uint16,
                               np.uint8, np.int32],
                   "offsets": [0, 8, 16, 24, 88, 90, 92], "itemsize": 96})
SHARD = np.dtype({"names": ["path", "fd", "direct_fd", "file_bytes", "data_offset"],
                  "formats": [np.uint64, np.int32, np.int32, np.uint64, np.uint64],
                  "offsets": [0, 8, 12, 16, 24], "itemsize": 32})


class Model(ctypes.Structure):
    _fields_ = [("shards", ctypes.c_void_p), ("shard_count", ctypes.c_size_t),
                ("tensors", ctypes.c_void_p), ("tensor_count", ctypes.c_size_t),
                ("tensor_capacity", ctypes.c_size_t)]


class Plan(ctypes.Structure):
    _fields_ = ([(n, ctypes.c_uint32) for n in (
        "chunk_tokens", "context_remaining", "routed_layers", "routed_layer_sweeps",
        "expert_read_requests", "shard_segments")] +
        [(n, ctypes.c_uint64) for n in (
            "hidden_row_bytes", "attn_res_row_bytes", "main_scratch_bytes", "moe_scratch_bytes",
            "mla_scratch_bytes", "route_bytes", "expert_index_bytes",
            "auxiliary_workspace_bytes", "batch_workspace_bytes",
            "incremental_workspace_bytes", "mla_append_bytes", "routed_layer_payload_bytes",
            "routed_store_payload_bytes", "routed_store_requested_read_bytes",
            "routed_store_physical_read_bytes", "staging_window_bytes",
            "registered_staging_bytes", "decode_cache_bytes", "retained_cache_bytes",
            "borrowed_cache_bytes", "new_layer_buffer_bytes", "new_device_bytes")])

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}


def expert_name(layer, expert, part):
    return f"language_model.model.layers.{layer}.block_sparse_moe.experts.{expert}.{part}"


class Directory:
    """entries: list of (name, shard, offset, length, dtype)."""

    def __init__(self, entries, shard_bytes):
        entries = sorted(entries, key=lambda e: e[0].encode())
        blob = b"".join(e[0].encode() + b"\0" for e in entries)
        self._names = np.frombuffer(blob, np.uint8).copy()
        starts = np.zeros(len(entries), np.uint64)
        if entries:
            lens = np.array([len(e[0]) + 1 for e in entries], np.uint64)
            starts[1:] = np.cumsum(lens)[:-1]
        self._t = np.zeros(max(len(entries), 1), TENSOR)
        base = self._names.ctypes.data
        self._t["name"][:len(entries)] = base + starts
        self._t["shard"][:len(entries)] = [e[1] for e in entries]
        self._t["offset"][:len(entries)] = [e[2] for e in entries]
        self._t["length"][:len(entries)] = [e[3] for e in entries]
        self._t["dtype"][:len(entries)] = [e[4] for e in entries]
        self._t["ndim"][:len(entries)] = 1
        self._t["shape"][:len(entries), 0] = [e[3] for e in entries]
        self._s = np.zeros(len(shard_bytes), SHARD)
        self._s["file_bytes"] = shard_bytes
        self._s["fd"] = -1
        self._s["direct_fd"] = -1
        self.model = Model(self._s.ctypes.data, len(shard_bytes), self._t.ctypes.data,
                           len(entries), len(entries))


def layout(shards=4, order="numeric", gap=0, base=8 * 4096 + 40, tail=4096 * 3 + 17, seed=0,
           mutate=None):
    """Routed experts of all 92 layers. Layer l lives in shard l % shards;
    within a layer experts are laid out in `order` ("numeric" or "shuffled")
    with `gap` bytes between experts (every 7th expert only, so runs and
    breaks both occur). mutate(entries) may edit the list before it is
    frozen. Returns a Directory."""
    rng = np.random.default_rng(seed)
    entries, ends = [], [0] * shards
    for layer in range(1, LAYERS + 1):
        s = layer % shards
        pos = max(ends[s], base)
        perm = np.arange(EXPERTS) if order == "numeric" else rng.permutation(EXPERTS)
        for i, e in enumerate(perm):
            for part, nbytes in zip(PARTS, PART_BYTES):
                entries.append([expert_name(layer, int(e), part), s, pos, nbytes, DTYPE_U8])
                pos += nbytes
            if gap and i % 7 == 6:
                pos += gap
        ends[s] = pos
    if mutate:
        mutate(entries)
    return Directory([tuple(e) for e in entries], [end + tail for end in ends])


def build(lib, directory, chunk, context, experts=32, slots=16, lease=0, aux=None):
    plan = Plan()
    err = ctypes.create_string_buffer(512)
    m = ctypes.byref(directory.model)
    if aux is None:
        ok = lib.k3_prefill_plan_build(m, chunk, context, experts, slots, lease,
                                       ctypes.byref(plan), err, 512)
    else:
        ok = lib.k3_prefill_plan_build_with_aux_workspace(m, chunk, context, experts, slots,
                                                          lease, ctypes.c_uint64(aux),
                                                          ctypes.byref(plan), err, 512)
    return bool(ok), plan.as_dict(), err.value.decode()


def bind(lib):
    for n in ("k3_prefill_plan_build", "k3_prefill_plan_build_with_aux_workspace"):
        f = getattr(lib, n)
        f.restype = ctypes.c_bool
    lib.k3_prefill_plan_build.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                          ctypes.c_uint16, ctypes.c_uint16, ctypes.c_int,
                                          ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]
    lib.k3_prefill_plan_build_with_aux_workspace.argtypes = [
        ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint16, ctypes.c_uint16,
        ctypes.c_int, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]
    return lib
