"""The dense decoder step over libsynapse_kv (libsynapse_gpu's model API).

``Decoder`` mirrors what the reference's managed executor does with a GPU model
(src/Synapse.Runtime/Features/GpuKernels/GpuDecoderExecutor.cs; native/synapse-gpu/src/Features/GpuKernels/
ffi.rs:106-271): it describes the mapped weights by byte offset (``DecoderDesc`` / ``DecoderLayerOffsets``,
decoder.rs:60-116), hands over the RoPE tables, and runs batched steps of ``BatchToken`` rows that return the
logits of the tokens that ask for them. There is no CPU fallback: without the HIP library every call raises.

``synthetic_model`` writes a model file of a given shape with Q8_0 (or, per matrix, Q4_K / Q6_K) matrices and FP32
norms and biases (random values of sane magnitude, for tests and benchmarks; there is no network for real
checkpoints).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from .kv_cache import batch_tokens, rope_table
from .projection import Q4_K_BYTES, Q6_K_BYTES, dequantize_q4_k, dequantize_q6_k, matrix_bytes
from .native import (
    ENCODING_Q4_K,
    ENCODING_Q6_K,
    ENCODING_Q8_0,
    KV_F16,
    KV_F32,
    NO_TENSOR,
    DecoderDesc,
    LayerOffsets,
    NativeKvLibrary,
    PageActivation,
    SELECT_KEY_BOUND,
    SELECT_RANDOM,
)

BLOCK_ELEMENTS = 32
BLOCK_BYTES = 34


@dataclass
class DecoderShape:
    layers: int
    hidden: int
    feed_forward: int
    heads: int
    kv_heads: int
    head_dim: int
    vocabulary: int
    context: int
    session_slots: int = 4
    step_tokens: int = 512
    logits_rows: int = 16
    rms_epsilon: float = 1e-6
    kv_precision: str = "f32"
    growth: int = 256
    theta: float = 1_000_000.0

    @property
    def kv_width(self) -> int:
        return self.kv_heads * self.head_dim


def q8_bytes(rows: int, columns: int) -> int:
    return rows * (columns // BLOCK_ELEMENTS) * BLOCK_BYTES


# The packing order of DecoderLayerOffsets.encodings (decoder/encoding.rs:75-85) by GGUF tensor name.
LAYER_MATRICES = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")


def q4_k_m(tensor: str) -> int:
    """The Q4_K_M mix of the reference's K-quant tests (KQuantWeightTests.Q4KM): Q6_K for V, the feed-forward down
    projection and the output matrix, Q4_K for the rest (the token embedding included)."""
    return ENCODING_Q6_K if tensor in ("attn_v", "ffn_down", "output") else ENCODING_Q4_K


def _random_kquant(rng, encoding: int, rows: int, columns: int, spread: float) -> np.ndarray:
    """Random K-quant super-blocks with weights of standard deviation about `spread`: random code and scale bytes,
    d (and dmin = 7.5 d for Q4_K, centring the sub-blocks on average) fitted on a sample of the blocks."""
    per = Q4_K_BYTES if encoding == ENCODING_Q4_K else Q6_K_BYTES
    count = rows * (columns // 256)
    blocks = np.frombuffer(rng.bytes(count * per), dtype=np.uint8).reshape(count, per).copy()
    def half(value: float) -> np.ndarray:
        return np.array([value], dtype=np.float16).view(np.uint8)

    one = half(1.0)
    sample = min(count, 2048)
    if encoding == ENCODING_Q4_K:
        blocks[:, 0:2] = one
        blocks[:, 2:4] = half(7.5)
        unit = dequantize_q4_k(blocks[:sample], 256).std()
        factor = spread / max(float(unit), 1e-30)
        blocks[:, 0:2] = half(factor)
        blocks[:, 2:4] = half(7.5 * factor)
    else:
        blocks[:, 208:210] = one
        unit = dequantize_q6_k(blocks[:sample], 256).std()
        blocks[:, 208:210] = half(spread / max(float(unit), 1e-30))
    return blocks.reshape(-1)


def synthetic_model(shape: DecoderShape, seed: int = 0, biases: bool = True, encodings=None) -> tuple[np.ndarray, dict]:
    """A model file: Q8_0 matrices (random codes, FP16 scales giving weights of standard deviation about
    1/sqrt(columns)), FP32 norms near 1 and small FP32 biases. ``encodings`` (a function of the GGUF tensor name:
    token_embd, attn_q, ..., ffn_down, output; e.g. ``q4_k_m``) picks another encoding per matrix, whose rows are
    random K-quant super-blocks of the same spread. Returns (bytes, layout) where layout holds the byte offsets in
    DecoderDesc / DecoderLayerOffsets terms."""
    choose = encodings or (lambda name: ENCODING_Q8_0)
    rng = np.random.default_rng(seed)
    parts: list[tuple[str, int, object]] = []
    offset = 0

    def place(size: int, alignment: int) -> int:
        nonlocal offset
        offset = (offset + alignment - 1) // alignment * alignment
        start = offset
        offset += size
        return start

    def matrix(rows: int, columns: int, spread: float, name: str) -> int:
        encoding = choose(name)
        start = place(matrix_bytes(encoding, rows, columns), 4)
        parts.append(("q8" if encoding == ENCODING_Q8_0 else encoding, start, (rows, columns, spread)))
        return start

    def vector(values: int, center: float, spread: float) -> int:
        start = place(values * 4, 4)
        parts.append(("f32", start, (values, center, spread)))
        return start

    s = shape
    layout = {"token_embedding": matrix(s.vocabulary, s.hidden, 1.0, "token_embd"), "layers": [],
              "embedding_encoding": choose("token_embd"), "output_encoding": choose("output")}
    packed = sum(choose(name) << (4 * index) for index, name in enumerate(LAYER_MATRICES))
    for _ in range(s.layers):
        layer = {
            "attention_norm": vector(s.hidden, 1.0, 0.2),
            "query": matrix(s.hidden, s.hidden, s.hidden ** -0.5, "attn_q"),
            "key": matrix(s.kv_width, s.hidden, s.hidden ** -0.5, "attn_k"),
            "value": matrix(s.kv_width, s.hidden, s.hidden ** -0.5, "attn_v"),
            "query_bias": vector(s.hidden, 0.0, 0.1) if biases else NO_TENSOR,
            "key_bias": vector(s.kv_width, 0.0, 0.1) if biases else NO_TENSOR,
            "value_bias": vector(s.kv_width, 0.0, 0.1) if biases else NO_TENSOR,
            "query_norm": NO_TENSOR,
            "key_norm": NO_TENSOR,
            "attention_output": matrix(s.hidden, s.hidden, s.hidden ** -0.5, "attn_output"),
            "feed_forward_norm": vector(s.hidden, 1.0, 0.2),
            "gate": matrix(s.feed_forward, s.hidden, s.hidden ** -0.5, "ffn_gate"),
            "up": matrix(s.feed_forward, s.hidden, s.hidden ** -0.5, "ffn_up"),
            "down": matrix(s.hidden, s.feed_forward, s.feed_forward ** -0.5, "ffn_down"),
            "encodings": packed,
        }
        layout["layers"].append(layer)
    layout["output_norm"] = vector(s.hidden, 1.0, 0.2)
    layout["output"] = matrix(s.vocabulary, s.hidden, s.hidden ** -0.5, "output")
    blob = np.zeros(offset, dtype=np.uint8)
    for kind, start, spec in parts:
        if kind == "f32":
            values, center, spread = spec
            data = (center + spread * (rng.random(values, dtype=np.float32) * 2 - 1)).astype(np.float32)
            blob[start:start + values * 4] = data.view(np.uint8)
        elif kind != "q8":
            rows, columns, spread = spec
            data = _random_kquant(rng, kind, rows, columns, spread)
            blob[start:start + data.size] = data
        else:
            rows, columns, spread = spec
            blocks = rows * (columns // BLOCK_ELEMENTS)
            view = blob[start:start + blocks * BLOCK_BYTES].reshape(blocks, BLOCK_BYTES)
            view[:, 2:] = np.frombuffer(rng.bytes(blocks * BLOCK_ELEMENTS), dtype=np.uint8).reshape(blocks, 32)
            # Uniform int8 codes have a standard deviation of about 74: scales around spread / 74, varied per block.
            scales = (spread / 74.0) * (0.5 + rng.random(blocks, dtype=np.float32))
            view[:, :2] = scales.astype(np.float16).view(np.uint8).reshape(blocks, 2)
    return blob, layout


class Decoder:
    """A dense decoder on the device: ``forward(tokens)`` returns the logits rows the tokens ask for."""

    def __init__(self, blob: np.ndarray, layout: dict, shape: DecoderShape, device: int = 0,
                 library: NativeKvLibrary | None = None, abi: str = "kv"):
        """``abi`` "gpu" creates and steps the model through libsynapse_gpu's ABI version 3 (synapse_gpu_*, backend
        3 on the current device) instead of synapse_kv_decoder_*: the reference loader's own calls."""
        self.library = library or NativeKvLibrary.load()
        self.shape = shape
        self.blob = np.ascontiguousarray(blob, dtype=np.uint8)
        self.cosines, self.sines = rope_table(shape.head_dim, shape.theta, shape.context, library=self.library)
        self.layers = (LayerOffsets * shape.layers)()
        for index, layer in enumerate(layout["layers"]):
            for name, _ in LayerOffsets._fields_:
                setattr(self.layers[index], name, int(layer[name]))
        desc = DecoderDesc()
        desc.weights = self.blob.ctypes.data
        desc.weights_length = self.blob.nbytes
        desc.layers = self.layers
        desc.rope_cosines = self.cosines.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
        desc.rope_sines = self.sines.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
        desc.token_embedding = int(layout["token_embedding"])
        desc.output_norm = int(layout["output_norm"])
        desc.output = int(layout["output"])
        desc.layer_count = shape.layers
        desc.hidden = shape.hidden
        desc.feed_forward = shape.feed_forward
        desc.heads = shape.heads
        desc.kv_heads = shape.kv_heads
        desc.head_dim = shape.head_dim
        desc.vocabulary = shape.vocabulary
        desc.context = shape.context
        desc.session_slots = shape.session_slots
        desc.step_tokens = shape.step_tokens
        desc.logits_rows = shape.logits_rows
        desc.rms_epsilon = shape.rms_epsilon
        desc.embedding_encoding = layout.get("embedding_encoding", ENCODING_Q8_0)
        desc.rope_layout = layout.get("rope_layout", 0)
        desc.activation = layout.get("activation", 0)
        desc.kv_precision = KV_F16 if shape.kv_precision in ("f16", "fp16") else KV_F32
        desc.kv_growth_positions = shape.growth
        desc.output_encoding = layout.get("output_encoding", ENCODING_Q8_0)
        self.desc = desc
        handle = ctypes.c_void_p()
        self.abi = abi
        if abi == "gpu":
            from .native import GPU_BACKEND_HIP

            self.library.check(self.library.g_decoder_create(GPU_BACKEND_HIP, ctypes.byref(desc), ctypes.byref(handle)))
        else:
            self.library.check(self.library.c_decoder_create(ctypes.byref(desc), device, ctypes.byref(handle)))
        self.handle = handle
        cache = ctypes.c_void_p()
        self.library.check(self.library.c_decoder_cache(self.handle, ctypes.byref(cache)))
        self.cache = cache

    def close(self) -> None:
        if getattr(self, "handle", None) is not None and self.handle.value:
            if getattr(self, "abi", "kv") == "gpu":
                self.library.g_decoder_destroy(self.handle)
            else:
                self.library.c_decoder_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_stream(self, stream) -> None:
        address = stream if isinstance(stream, int) else int(getattr(stream, "cuda_stream", 0) or 0)
        self.library.check(self.library.c_decoder_set_stream(self.handle, address))

    def reserve(self, slot: int, positions: int) -> None:
        self.library.check(self.library.c_decoder_reserve(self.handle, slot, positions))

    @property
    def kv_bytes(self) -> int:
        return int(self.library.c_decoder_kv_bytes(self.handle))

    def forward(self, tokens, prompt_start: int | None = None, out: np.ndarray | None = None) -> np.ndarray:
        """One step of (slot, token, position, logits_row) rows; returns [k][vocabulary] FP32 logits, written into
        `out` when given (a reusable, ideally pinned, host buffer of at least k rows)."""
        buffer = tokens if isinstance(tokens, ctypes.Array) else batch_tokens(tokens)
        rows = sum(1 for token in buffer if token.logits_row >= 0)
        if out is not None:
            if out.dtype != np.float32 or not out.flags["C_CONTIGUOUS"] or out.size < rows * self.shape.vocabulary:
                raise ValueError("out must be a contiguous float32 buffer of at least k x vocabulary values")
            logits = out.reshape(-1)[:max(rows, 1) * self.shape.vocabulary].reshape(max(rows, 1), -1)
        else:
            logits = np.zeros((max(rows, 1), self.shape.vocabulary), dtype=np.float32)
        if prompt_start is None and self.abi == "gpu":
            status = self.library.g_decoder_forward(self.handle, buffer, len(buffer), logits.ctypes.data, logits.size)
        elif prompt_start is None:
            status = self.library.c_decoder_forward(self.handle, buffer, len(buffer), logits.ctypes.data, logits.size)
        else:
            status = self.library.c_decoder_forward_prompt(self.handle, buffer, len(buffer), prompt_start,
                                                           logits.ctypes.data, logits.size)
        self.library.check(status)
        return logits[:rows]

    def set_option(self, option: int, value: int) -> None:
        self.library.check(self.library.c_set_option(self.cache, option, value))

    def set_page_activation(self, budget_pages: int | None, window_tokens: int = 0, selection: str = "key_bound",
                            seed: int = 0) -> None:
        """KV page activation on the model's cache (ModelLoadOptions.KvPageActivation); None: dense."""
        if budget_pages is None:
            activation = PageActivation(0, 0, 0, 64, SELECT_KEY_BOUND, 0)
        else:
            kind = {"key_bound": SELECT_KEY_BOUND, "random": SELECT_RANDOM}[selection]
            activation = PageActivation(1, budget_pages, window_tokens, 64, kind, seed)
        self.library.check(self.library.c_set_page_activation(self.cache, ctypes.byref(activation)))
