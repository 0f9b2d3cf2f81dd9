"""ctypes access to the CPU restatement in oracle/ (test infrastructure only)."""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE_PATH = ROOT / "oracle" / "build" / "liboracle.so"

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float

SIGNATURES = {
    "orc_f32_to_f16": (None, [_P, _P, ctypes.c_size_t]),
    "orc_f16_to_f32": (None, [_P, _P, ctypes.c_size_t]),
    "orc_rope_table": (_I, [_I, _F, _F, _I, _I, _P, _P]),
    "orc_rope_apply": (None, [_P, _I, _I, _P, _P]),
    "orc_next_capacity": (_I, [_I, _I, _I, _I]),
    "orc_dense_create": (_P, [_I, _I, _I, _I]),
    "orc_dense_destroy": (None, [_P]),
    "orc_dense_store": (_I, [_P, _I, _I, _P, _P, _I]),
    "orc_dense_reserve": (_I, [_P, _I]),
    "orc_dense_release": (None, [_P]),
    "orc_dense_allocated": (_I, [_P]),
    "orc_dense_bytes": (ctypes.c_longlong, [_P]),
    "orc_dense_get": (_I, [_P, _I, _I, _I, _I, _I, _P]),
    "orc_paged_create": (_P, [_I] * 11),
    "orc_paged_destroy": (None, [_P]),
    "orc_paged_reserve": (_I, [_P, _I, _I]),
    "orc_paged_release": (_I, [_P, _I]),
    "orc_paged_truncate": (_I, [_P, _I, _I]),
    "orc_paged_fork": (_I, [_P, _I, _I]),
    "orc_paged_step": (_I, [_P, _P, _I]),
    "orc_paged_append_rope": (_I, [_P, _I, _P, _I, _P, _P]),
    "orc_paged_gather": (_I, [_P, _I, _I, _I, _I, _P, _P, _I]),
    "orc_paged_slot": (_I, [_P, _I, _P, _P, _P]),
    "orc_paged_table": (_I, [_P, _I, _P]),
    "orc_paged_refcounts": (None, [_P, _P]),
    "orc_paged_free_list": (_I, [_P, _P]),
    "orc_paged_kv_bytes": (ctypes.c_longlong, [_P]),
    "orc_attention_scalar": (None, [_P, _P, _P, _I, _I, _I, _I, _P]),
    "orc_attention_managed": (None, [_P, _P, _P, _I, _I, _I, _I, _P]),
    "orc_attention_fp64": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _F, _P]),
    "orc_attention_split": (None, [_P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "orc_paged_attention": (ctypes.c_double, [_P, _I, _P, _I, _P, _I, _I]),
    "orc_paged_attention_pages": (ctypes.c_double, [_P, _I, _P, _I, _P, _I, _I, _P, _I, _P]),
    "orc_dotnet_random": (None, [ctypes.c_int32, _I, ctypes.c_int32, ctypes.c_int32, _P]),
    "orc_page_bound": (_F, [_P, _I, _I, _P, _I, _I]),
    "orc_page_select": (None, [_I, _I, _I, _I, _P, _I, _I, _P, _I, ctypes.c_int32, _P]),
    "orc_decoder_create": (_P, [_P, _P, _P, _P, _F, _P, _P]),
    "orc_decoder_destroy": (None, [_P]),
    "orc_decoder_cache": (_P, [_P]),
    "orc_decoder_forward": (_I, [_P, _P, _I, _P, _I]),
    "orc_plan_attention": (_I, [_P, _I, _I, _I, _P, _I, _P]),
    "orc_prefix_create": (_P, [_I]),
    "orc_prefix_destroy": (None, [_P]),
    "orc_prefix_claim": (_I, [_P, _P, _I]),
    "orc_prefix_remember": (None, [_P, _P, _I, _P, _I]),
    "orc_prefix_clear": (None, [_P]),
    "orc_q8_project_f32": (ctypes.c_double, [_P, _P, _P, _P, _I, _I, _I, _P, _I, _P, _I, _I, _I]),
    "orc_q8_project_f64": (None, [_P, _P, _P, _P, _I, _I, _I, _P, _I, _P, _I, _I, _P]),
}


def load() -> ctypes.CDLL:
    if not ORACLE_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
    library = ctypes.CDLL(str(ORACLE_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        function = getattr(library, name)
        function.restype = restype
        function.argtypes = argtypes
    return library


ORACLE = load()


def ptr(array: np.ndarray) -> int:
    assert array.flags["C_CONTIGUOUS"]
    return array.ctypes.data


def f32_to_f16(values) -> np.ndarray:
    source = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(source.shape, dtype=np.uint16)
    ORACLE.orc_f32_to_f16(ptr(source), ptr(out), source.size)
    return out


def f16_to_f32(bits) -> np.ndarray:
    source = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(source.shape, dtype=np.float32)
    ORACLE.orc_f16_to_f32(ptr(source), ptr(out), source.size)
    return out


def rope_table(head_dim, theta, positions, yarn_factor=0.0, yarn_original=0):
    half = head_dim // 2
    cos = np.empty((positions, half), dtype=np.float32)
    sin = np.empty((positions, half), dtype=np.float32)
    status = ORACLE.orc_rope_table(head_dim, theta, yarn_factor, yarn_original, positions, ptr(cos), ptr(sin))
    assert status == 0, status
    return cos, sin


def rope_apply(values, heads, head_dim, cos_row, sin_row) -> np.ndarray:
    out = np.ascontiguousarray(values, dtype=np.float32).copy()
    c = np.ascontiguousarray(cos_row, dtype=np.float32)
    s = np.ascontiguousarray(sin_row, dtype=np.float32)
    ORACLE.orc_rope_apply(ptr(out), heads, head_dim, ptr(c), ptr(s))
    return out


def attention(kind, query, keys, values, heads, kv_heads, head_dim, position, split_keys=None):
    """Attention of one query position over dense [positions][kv_heads][head_dim] K/V (fp32)."""
    q = np.ascontiguousarray(query, dtype=np.float32)
    k = np.ascontiguousarray(keys, dtype=np.float32)
    v = np.ascontiguousarray(values, dtype=np.float32)
    out = np.zeros(heads * head_dim, dtype=np.float32)
    if kind == "scalar":
        ORACLE.orc_attention_scalar(ptr(q), ptr(k), ptr(v), heads, kv_heads, head_dim, position, ptr(out))
    elif kind == "managed":
        ORACLE.orc_attention_managed(ptr(q), ptr(k), ptr(v), heads, kv_heads, head_dim, position, ptr(out))
    elif kind == "split":
        ORACLE.orc_attention_split(ptr(q), ptr(k), ptr(v), heads, kv_heads, head_dim, position, split_keys, ptr(out))
    elif kind == "fp64":
        scale = np.float32(1.0) / np.sqrt(np.float32(head_dim))
        status = ORACLE.orc_attention_fp64(ptr(q), ptr(k), ptr(v), None, heads, kv_heads, head_dim, position,
                                           float(scale), ptr(out))
        assert status == 0, status
    else:
        raise ValueError(kind)
    return out


class DenseCache:
    """Qwen2KvCache restatement."""

    def __init__(self, layers, maximum, kv_width, growth):
        self.handle = ORACLE.orc_dense_create(layers, maximum, kv_width, growth)
        assert self.handle
        self.kv_width = kv_width

    def __del__(self):
        ORACLE.orc_dense_destroy(self.handle)

    def store(self, layer, position, key, value):
        k = np.ascontiguousarray(key, dtype=np.float32)
        v = np.ascontiguousarray(value, dtype=np.float32)
        return ORACLE.orc_dense_store(self.handle, layer, position, ptr(k), ptr(v), k.size)

    def reserve(self, positions):
        return ORACLE.orc_dense_reserve(self.handle, positions)

    def release(self):
        ORACLE.orc_dense_release(self.handle)

    @property
    def allocated(self):
        return ORACLE.orc_dense_allocated(self.handle)

    @property
    def allocated_bytes(self):
        return ORACLE.orc_dense_bytes(self.handle)

    def get(self, layer, position, head, head_dim, value=False):
        out = np.empty(head_dim, dtype=np.float32)
        status = ORACLE.orc_dense_get(self.handle, layer, position, head, head_dim, 1 if value else 0, ptr(out))
        return status, out


class PagedCache:
    """The paged restatement (the specification the GPU table kernels follow)."""

    def __init__(self, layers, heads, kv_heads, head_dim, maximum, growth, page_tokens, precision, slots,
                 max_pages, step_tokens):
        self.handle = ORACLE.orc_paged_create(layers, heads, kv_heads, head_dim, maximum, growth, page_tokens,
                                              precision, slots, max_pages, step_tokens)
        assert self.handle
        self.heads, self.kv_heads, self.head_dim = heads, kv_heads, head_dim
        self.precision = precision
        self.max_pages = max_pages
        self.pages_per_slot = -(-maximum // page_tokens)

    def __del__(self):
        ORACLE.orc_paged_destroy(self.handle)

    def reserve(self, slot, positions):
        return ORACLE.orc_paged_reserve(self.handle, slot, positions)

    def release(self, slot):
        return ORACLE.orc_paged_release(self.handle, slot)

    def truncate(self, slot, length):
        return ORACLE.orc_paged_truncate(self.handle, slot, length)

    def fork(self, source, target):
        return ORACLE.orc_paged_fork(self.handle, source, target)

    def step(self, tokens):
        array = np.ascontiguousarray(tokens, dtype=np.int32)
        if array.shape[1] == 2:
            full = np.zeros((array.shape[0], 4), dtype=np.int32)
            full[:, 0], full[:, 2], full[:, 3] = array[:, 0], array[:, 1], -1
            array = full
        return ORACLE.orc_paged_step(self.handle, ptr(array), array.shape[0])

    def append_rope(self, layer, qkv, cos, sin):
        assert qkv.dtype == np.float32 and qkv.flags["C_CONTIGUOUS"]
        return ORACLE.orc_paged_append_rope(self.handle, layer, ptr(qkv), qkv.shape[1], ptr(cos), ptr(sin))

    def gather(self, slot, layer, first, count, raw=False):
        dtype = np.uint16 if (raw and self.precision == 1) else np.float32
        k = np.zeros((count, self.kv_heads, self.head_dim), dtype=dtype)
        v = np.zeros_like(k)
        status = ORACLE.orc_paged_gather(self.handle, slot, layer, first, count, ptr(k), ptr(v), 1 if raw else 0)
        assert status == 0, status
        return k, v

    def slot(self, slot):
        cap, length, pages = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        status = ORACLE.orc_paged_slot(self.handle, slot, ctypes.byref(cap), ctypes.byref(length),
                                       ctypes.byref(pages))
        assert status == 0
        return {"capacity": cap.value, "length": length.value, "pages": pages.value}

    def table(self, slot):
        out = np.empty(self.pages_per_slot, dtype=np.int32)
        assert ORACLE.orc_paged_table(self.handle, slot, ptr(out)) == 0
        return out

    def refcounts(self):
        out = np.empty(self.max_pages, dtype=np.int32)
        ORACLE.orc_paged_refcounts(self.handle, ptr(out))
        return out

    def free_list(self):
        out = np.empty(self.max_pages, dtype=np.int32)
        count = ORACLE.orc_paged_free_list(self.handle, ptr(out))
        return out[:count]

    @property
    def kv_bytes(self):
        return ORACLE.orc_paged_kv_bytes(self.handle)

    def attention(self, layer, qkv, out, threads=1, activation=None, prompt_start=None, maximum=None):
        """Step attention for one layer. With ``activation`` = (budget, window, page_tokens, selection, seed) the
        decode units attend their selected pages; then returns the masks [tokens][kv_heads][maximum] (bool)."""
        if activation is None:
            return ORACLE.orc_paged_attention(self.handle, layer, ptr(qkv), qkv.shape[1], ptr(out), out.shape[1],
                                              threads)
        parameters = np.asarray(activation, dtype=np.int32)
        tokens = qkv.shape[0]
        start = tokens if prompt_start is None else prompt_start
        masks = np.zeros((tokens, self.kv_heads, maximum), dtype=np.uint8)
        ORACLE.orc_paged_attention_pages(self.handle, layer, ptr(qkv), qkv.shape[1], ptr(out), out.shape[1], threads,
                                         ptr(parameters), start, ptr(masks))
        return masks.astype(bool)


def plan_attention(tokens, kv_heads, run_tokens):
    array = np.ascontiguousarray(tokens, dtype=np.int32)
    capacity = max(1, array.shape[0] * kv_heads)
    blocks = np.zeros((capacity, 8), dtype=np.uint32)
    summary = np.zeros(4, dtype=np.uint32)
    count = ORACLE.orc_plan_attention(ptr(array), array.shape[0], kv_heads, run_tokens, ptr(blocks), capacity,
                                      ptr(summary))
    assert count >= 0
    return blocks[:count], {"run_blocks": int(summary[0]), "single_blocks": int(summary[1]),
                            "split_keys": int(summary[2]), "splits": int(summary[3])}


class Prefix:
    def __init__(self, enabled=True):
        self.handle = ORACLE.orc_prefix_create(1 if enabled else 0)

    def __del__(self):
        ORACLE.orc_prefix_destroy(self.handle)

    def claim(self, prompt):
        array = np.ascontiguousarray(prompt, dtype=np.int32)
        return ORACLE.orc_prefix_claim(self.handle, ptr(array), array.size)

    def remember(self, prompt, generated):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        g = np.ascontiguousarray(generated, dtype=np.int32)
        ORACLE.orc_prefix_remember(self.handle, ptr(p), p.size, ptr(g), g.size)

    def clear(self):
        ORACLE.orc_prefix_clear(self.handle)


def q8_project(segments, inputs, output, accumulate=False, exact=False, threads=1):
    """A Q8_0 projection on the restatement. ``segments``: [(blocks uint8 [rows][columns / 32 * 34], bias float32
    [rows] or None, out_column)]; ``inputs`` float32 [tokens][>= columns]; ``output`` float32 [tokens][stride],
    updated in place. ``exact``: the FP64 anchor, returning sum |terms| per element; otherwise the reference's FP32
    matrix-vector order, returning the wall time in seconds."""
    count = len(segments)
    blocks = [np.ascontiguousarray(b, dtype=np.uint8) for b, _, _ in segments]
    biases = [None if bias is None else np.ascontiguousarray(bias, dtype=np.float32) for _, bias, _ in segments]
    weights = (ctypes.c_void_p * count)(*[b.ctypes.data for b in blocks])
    bias_pointers = (ctypes.c_void_p * count)(*[None if b is None else b.ctypes.data for b in biases])
    rows = (ctypes.c_int * count)(*[b.shape[0] for b in blocks])
    columns = blocks[0].shape[1] // 34 * 32
    out_columns = (ctypes.c_int * count)(*[int(column) for _, _, column in segments])
    inputs = np.ascontiguousarray(inputs, dtype=np.float32)
    assert output.dtype == np.float32 and output.flags["C_CONTIGUOUS"]
    tokens = inputs.shape[0]
    if exact:
        magnitude = np.zeros(output.shape, dtype=np.float64)
        ORACLE.orc_q8_project_f64(weights, bias_pointers, rows, out_columns, count, columns, tokens, ptr(inputs),
                                  inputs.shape[1], ptr(output), output.shape[1], int(accumulate), ptr(magnitude))
        return magnitude
    return ORACLE.orc_q8_project_f32(weights, bias_pointers, rows, out_columns, count, columns, tokens, ptr(inputs),
                                     inputs.shape[1], ptr(output), output.shape[1], int(accumulate), threads)


def dotnet_random(seed, count, low=0, high=0):
    """System.Random(seed): Next() (low == high == 0) or Next(low, high), ``count`` times."""
    out = np.zeros(count, dtype=np.int32)
    ORACLE.orc_dotnet_random(seed, count, low, high, ptr(out))
    return out


def page_bound(queries, group, head_dim, keys, first, last):
    q = np.ascontiguousarray(queries, dtype=np.float32)
    k = np.ascontiguousarray(keys, dtype=np.float32)
    return float(ORACLE.orc_page_bound(ptr(q), group, head_dim, ptr(k), first, last))


def page_select(budget, window, queries, group, head_dim, keys, position, seed=0, page_tokens=64, random=False):
    """KvPageSelector.Select: the selected positions 0..position (bool)."""
    q = np.ascontiguousarray(queries, dtype=np.float32)
    k = np.ascontiguousarray(keys, dtype=np.float32)
    selected = np.zeros(position + 1, dtype=np.uint8)
    ORACLE.orc_page_select(budget, window, page_tokens, 1 if random else 0, ptr(q), group, head_dim, ptr(k), position,
                           seed, ptr(selected))
    return selected.astype(bool)


LAYER_FIELDS = ("attention_norm", "query", "key", "value", "query_bias", "key_bias", "value_bias", "query_norm",
                "key_norm", "attention_output", "feed_forward_norm", "gate", "up", "down", "encodings")


class DecoderOracle:
    """The decoder step restated on the CPU (orc_decoder_*), over a model file and its layout."""

    def __init__(self, blob, layout, shape, cosines, sines, page_tokens=64, max_pages=None):
        self.blob = np.ascontiguousarray(blob, dtype=np.uint8)
        self.shape = shape
        self.cosines = np.ascontiguousarray(cosines, dtype=np.float32)
        self.sines = np.ascontiguousarray(sines, dtype=np.float32)
        self.layers = np.array([[int(layer[name]) for name in LAYER_FIELDS] for layer in layout["layers"]],
                               dtype=np.uint64)
        self.top = np.array([layout["token_embedding"], layout["output_norm"], layout["output"],
                             layout.get("embedding_encoding", 8), layout.get("output_encoding", 8)], dtype=np.uint64)
        pages = max_pages or shape.session_slots * -(-shape.context // page_tokens)
        precision = 1 if shape.kv_precision in ("f16", "fp16") else 0
        self.dims = np.array([shape.layers, shape.hidden, shape.feed_forward, shape.heads, shape.kv_heads,
                              shape.head_dim, shape.vocabulary, shape.context, shape.session_slots, shape.step_tokens,
                              precision, shape.growth, page_tokens, pages], dtype=np.int32)
        self.handle = ORACLE.orc_decoder_create(ptr(self.blob), ptr(self.layers), ptr(self.top), ptr(self.dims),
                                                shape.rms_epsilon, ptr(self.cosines), ptr(self.sines))
        assert self.handle

    def __del__(self):
        if getattr(self, "handle", None):
            ORACLE.orc_decoder_destroy(self.handle)

    def forward(self, tokens, threads=8):
        array = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1, 4)
        rows = int((array[:, 3] >= 0).sum())
        logits = np.zeros((max(rows, 1), self.shape.vocabulary), dtype=np.float32)
        status = ORACLE.orc_decoder_forward(self.handle, ptr(array), array.shape[0], ptr(logits), threads)
        assert status == 0, status
        return logits[:rows]
