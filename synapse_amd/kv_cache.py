"""Host-side mirror of Synapse's KV-cache contract over libsynapse_kv.

``PagedKvCache`` offers the operations the reference exposes for this path, with the same argument meaning
and error behaviour:

* ``reserve(slot, positions)`` -- ``IBatchDecoder.Reserve`` / ``synapse_gpu_decoder_reserve``
  (src/Synapse.Runtime/Features/TextGeneration/BatchDecoding.cs:10-33; ffi.rs:250-263) with the
  ``Qwen2KvCache.Reserve`` policy (Qwen2KvCache.cs:56-72); positions beyond the context raise
  :class:`InvalidOperationError` (ArgumentOutOfRange on the managed side);
* ``release(slot)`` -- ``Qwen2KvCache.Release`` (Qwen2KvCache.cs:75-84);
* ``allocated_bytes`` -- ``AllocatedKvBytes`` / ``synapse_gpu_decoder_kv_bytes`` (ffi.rs:229-248);
* ``step`` + ``append_rope`` + ``attention`` -- one layer of ``IBatchDecoder.Forward``'s attention half
  (step/layers.rs:62-148, step/attention.rs:9-145) for a batch of ``BatchToken`` (decoder.rs:133-141);
* ``step(tokens, prompt_start)`` -- ``Forward(tokens, promptStart)``: tokens from ``prompt_start`` on are prompt
  tokens;
* ``set_page_activation(budget_pages, window_tokens, ...)`` -- ``ModelLoadOptions.KvPageActivation`` (ADR-016,
  KvPageActivation.cs, KvPageSelector.cs, Qwen2KvPageMasks.cs): decode units attend the sink page, the recent
  window and the budgeted pages;
* ``fork`` / ``truncate`` -- prefix reuse (DirectSessionPrefix.cs:16-41) as copy-on-write page sharing, and
  rollback (native/synapse-core/src/Features/SessionState/kv_pages.rs:158-177).

Device buffers are torch tensors on the cache's device (or raw device addresses). The HIP library is the only
implementation: without it every call raises :class:`NotSupportedError`.
"""

from __future__ import annotations

import ctypes

import numpy as np

from .native import (
    KV_F16,
    KV_F32,
    OPTION_PREFILL_RUNS,
    OPTION_PREFILL_SPLIT_KEYS,
    OPTION_SPLIT_KEYS,
    SELECT_KEY_BOUND,
    SELECT_RANDOM,
    BatchToken,
    PageActivation,
    CacheDesc,
    NativeKvLibrary,
    KERNEL_KINDS,
    PageStats,
    Profile,
)

PRECISIONS = {"f32": KV_F32, "fp32": KV_F32, "float32": KV_F32, "f16": KV_F16, "fp16": KV_F16, "float16": KV_F16}


def _address(buffer) -> int:
    if isinstance(buffer, int):
        return buffer
    if hasattr(buffer, "data_ptr"):
        return int(buffer.data_ptr())
    raise TypeError("expected a device tensor or a device address")


def rope_table(
    head_dim: int,
    theta: float,
    positions: int,
    yarn_factor: float = 0.0,
    yarn_original: int = 0,
    library: NativeKvLibrary | None = None,
) -> tuple[np.ndarray, np.ndarray]:
    """RopeFrequencies tables (RopeFrequencies.cs:20-81): [positions][head_dim / 2] cosines and sines."""
    library = library or NativeKvLibrary.load()
    half = head_dim // 2
    cosines = np.empty((positions, half), dtype=np.float32)
    sines = np.empty((positions, half), dtype=np.float32)
    library.check(
        library.c_rope_table(
            head_dim, theta, yarn_factor, yarn_original, positions, cosines.ctypes.data, sines.ctypes.data
        )
    )
    return cosines, sines


def batch_tokens(tokens) -> ctypes.Array:
    """BatchToken array from (slot, position) pairs, (slot, token, position, logits_row) rows, or BatchTokens."""
    array = np.asarray(tokens, dtype=np.int32)
    if array.ndim != 2 or array.shape[1] not in (2, 4):
        raise ValueError("tokens must be (slot, position) pairs or (slot, token, position, logits_row) rows")
    if array.shape[1] == 2:
        full = np.zeros((array.shape[0], 4), dtype=np.int32)
        full[:, 0] = array[:, 0]
        full[:, 2] = array[:, 1]
        full[:, 3] = -1
        array = full
    array = np.ascontiguousarray(array)
    buffer = (BatchToken * array.shape[0])()
    ctypes.memmove(buffer, array.ctypes.data, array.nbytes)
    return buffer


class PagedKvCache:
    """A growable paged KV cache with GQA attention on one MI355X.

    Shape arguments follow DecoderDesc (decoder.rs:95-128): ``layers`` counts executed layers (dropped layers
    are never allocated), ``heads``/``kv_heads``/``head_dim`` the attention shape, ``max_positions`` the
    context, ``growth_positions`` the ADR-017 growth unit, ``session_slots`` the KV slots and ``step_tokens``
    the largest step. ``page_tokens`` positions of every layer share one page; ``max_pages`` sizes the pool.
    """

    def __init__(
        self,
        *,
        layers: int,
        heads: int,
        kv_heads: int,
        head_dim: int,
        max_positions: int,
        growth_positions: int = 1024,
        page_tokens: int = 256,
        precision: str = "f16",
        session_slots: int = 1,
        step_tokens: int = 512,
        max_pages: int | None = None,
        rope_theta: float = 1_000_000.0,
        rope_cosines: np.ndarray | None = None,
        rope_sines: np.ndarray | None = None,
        device: int = 0,
        library: NativeKvLibrary | None = None,
    ):
        self.library = library or NativeKvLibrary.load()
        self.layers = layers
        self.heads = heads
        self.kv_heads = kv_heads
        self.head_dim = head_dim
        self.max_positions = max_positions
        self.page_tokens = page_tokens
        self.precision = PRECISIONS[precision]
        self.session_slots = session_slots
        self.pages_per_slot = -(-max_positions // page_tokens)
        if max_pages is None:
            max_pages = session_slots * self.pages_per_slot
        self.max_pages = max_pages
        if rope_cosines is None or rope_sines is None:
            rope_cosines, rope_sines = rope_table(head_dim, rope_theta, max_positions, library=self.library)
        self.rope_cosines = np.ascontiguousarray(rope_cosines, dtype=np.float32)
        self.rope_sines = np.ascontiguousarray(rope_sines, dtype=np.float32)
        expected = (max_positions, head_dim // 2)
        if self.rope_cosines.shape != expected or self.rope_sines.shape != expected:
            raise ValueError(f"RoPE tables must be {expected}")
        desc = CacheDesc(
            self.rope_cosines.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
            self.rope_sines.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
            layers,
            heads,
            kv_heads,
            head_dim,
            max_positions,
            growth_positions,
            page_tokens,
            self.precision,
            session_slots,
            step_tokens,
            max_pages,
            device,
        )
        handle = ctypes.c_void_p()
        self.library.check(self.library.c_cache_create(ctypes.byref(desc), ctypes.byref(handle)))
        self.handle = handle
        self.qkv_width = (heads + 2 * kv_heads) * head_dim

    # -- lifetime ------------------------------------------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "handle", None) is not None and self.handle.value:
            self.library.c_cache_destroy(self.handle)
            self.handle = None

    def __enter__(self) -> "PagedKvCache":
        return self

    def __exit__(self, *_exc) -> None:
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- configuration -------------------------------------------------------------------------------------
    def set_stream(self, stream) -> None:
        address = stream if isinstance(stream, int) else int(getattr(stream, "cuda_stream", 0) or 0)
        self.library.check(self.library.c_set_stream(self.handle, address))

    def set_option(self, option: int, value: int) -> None:
        self.library.check(self.library.c_set_option(self.handle, option, value))

    def set_split_keys(self, keys: int) -> None:
        self.set_option(OPTION_SPLIT_KEYS, keys)

    def set_prefill_runs(self, enabled: bool) -> None:
        self.set_option(OPTION_PREFILL_RUNS, 1 if enabled else 0)

    def set_prefill_split_keys(self, keys: int) -> None:
        self.set_option(OPTION_PREFILL_SPLIT_KEYS, keys)

    # -- capacity (ADR-017) --------------------------------------------------------------------------------
    def reserve(self, slot: int, positions: int) -> None:
        if slot < 0 or positions < 0:
            raise ValueError("slot and positions must be non-negative")
        self.library.check(self.library.c_reserve(self.handle, slot, positions))

    def release(self, slot: int) -> None:
        self.library.check(self.library.c_release(self.handle, slot))

    def truncate(self, slot: int, length: int) -> None:
        self.library.check(self.library.c_truncate(self.handle, slot, length))

    def fork(self, source: int, target: int) -> None:
        self.library.check(self.library.c_fork(self.handle, source, target))

    @property
    def allocated_bytes(self) -> int:
        return int(self.library.c_bytes(self.handle))

    def slot_info(self, slot: int) -> dict:
        capacity, length, pages = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
        self.library.check(
            self.library.c_slot_info(self.handle, slot, ctypes.byref(capacity), ctypes.byref(length), ctypes.byref(pages))
        )
        return {"capacity": capacity.value, "length": length.value, "pages": pages.value}

    # -- the step ------------------------------------------------------------------------------------------
    def step(self, tokens, prompt_start: int | None = None) -> None:
        """Prepares a step; tokens from ``prompt_start`` on (default: none) are prompt tokens."""
        buffer = tokens if isinstance(tokens, ctypes.Array) else batch_tokens(tokens)
        if prompt_start is None:
            self.library.check(self.library.c_step(self.handle, buffer, len(buffer)))
        else:
            if prompt_start < 0:
                raise ValueError("prompt_start must be non-negative")
            self.library.check(self.library.c_step_prompt(self.handle, buffer, len(buffer), prompt_start))

    def set_page_activation(self, budget_pages: int | None, window_tokens: int = 0, page_tokens: int = 64,
                            selection: str = "key_bound", seed: int = 0) -> None:
        """KV page activation (``KvPageActivation(BudgetPages, WindowTokens)``); ``None`` restores dense attention.

        ``selection`` is ``"key_bound"`` (KvPageSelection.KeyBound) or ``"random"`` (the control). Negative budgets
        or windows raise ValueError (ArgumentOutOfRangeException in KvPageActivation.Validate).
        """
        if budget_pages is None:
            activation = PageActivation(0, 0, 0, 64, SELECT_KEY_BOUND, 0)
        else:
            if budget_pages < 0 or window_tokens < 0:
                raise ValueError("budget_pages and window_tokens must be non-negative")
            kinds = {"key_bound": SELECT_KEY_BOUND, "random": SELECT_RANDOM}
            if selection not in kinds:
                raise ValueError(f"unknown KV page selection {selection!r}")
            activation = PageActivation(1, budget_pages, window_tokens, page_tokens, kinds[selection], seed)
        self.library.check(self.library.c_set_page_activation(self.handle, ctypes.byref(activation)))

    def append_rope(self, layer: int, qkv, qkv_stride: int | None = None) -> None:
        stride = self.qkv_width if qkv_stride is None else qkv_stride
        self.library.check(self.library.c_append_rope(self.handle, layer, _address(qkv), stride))

    def attention(self, layer: int, qkv, output, qkv_stride: int | None = None, out_stride: int | None = None) -> None:
        q_stride = self.qkv_width if qkv_stride is None else qkv_stride
        o_stride = self.heads * self.head_dim if out_stride is None else out_stride
        self.library.check(
            self.library.c_attention(self.handle, layer, _address(qkv), q_stride, _address(output), o_stride)
        )

    def append_attention(self, layer: int, qkv, output, qkv_stride: int | None = None,
                         out_stride: int | None = None) -> None:
        """append_rope + attention in one call (one launch when every token owns its slot); qkv is read only."""
        q_stride = self.qkv_width if qkv_stride is None else qkv_stride
        o_stride = self.heads * self.head_dim if out_stride is None else out_stride
        self.library.check(
            self.library.c_append_attention(self.handle, layer, _address(qkv), q_stride, _address(output), o_stride)
        )

    def profile_begin(self) -> None:
        """Starts per-kernel GPU timing (events recorded by each dispatch on the cache's stream)."""
        self.library.check(self.library.c_profile_begin(self.handle))

    def profile_end(self) -> dict:
        """Waits for the stream; returns {kind: (launches, milliseconds)} for the kinds that ran."""
        profile = Profile()
        self.library.check(self.library.c_profile_end(self.handle, ctypes.byref(profile)))
        return {kind: (int(profile.launches[index]), float(profile.milliseconds[index]))
                for index, kind in enumerate(KERNEL_KINDS) if profile.launches[index]}

    def synchronize(self) -> None:
        self.library.check(self.library.c_synchronize(self.handle))

    # -- read-back for checks ------------------------------------------------------------------------------
    def block_table(self, slot: int) -> np.ndarray:
        out = np.empty(self.pages_per_slot, dtype=np.int32)
        count = ctypes.c_size_t()
        self.library.check(
            self.library.c_read_block_table(self.handle, slot, out.ctypes.data, out.size, ctypes.byref(count))
        )
        return out[: count.value]

    def refcounts(self) -> np.ndarray:
        out = np.empty(self.max_pages, dtype=np.int32)
        self.library.check(self.library.c_read_refcounts(self.handle, out.ctypes.data, out.size))
        return out

    def free_list(self) -> np.ndarray:
        out = np.empty(self.max_pages, dtype=np.int32)
        count = ctypes.c_size_t()
        self.library.check(self.library.c_read_free_list(self.handle, out.ctypes.data, out.size, ctypes.byref(count)))
        return out[: count.value]

    def page_stats(self) -> dict:
        stats = PageStats()
        self.library.check(self.library.c_page_stats(self.handle, ctypes.byref(stats)))
        return {name: getattr(stats, name) for name, _ in PageStats._fields_ if name != "reserved"}

    def export_prefix(self, slot: int, length: int, key) -> bytes:
        """Positions 0..length-1 of `slot` as a persistent prefix payload keyed by `key` (a PrefixKey or a
        (model, tokenizer, rope, prefix) tuple): synapse_kv_export_prefix."""
        from .native import PrefixKey

        key = key if isinstance(key, PrefixKey) else PrefixKey(*key)
        size = ctypes.c_uint64()
        self.library.check(self.library.c_export_prefix(self.handle, slot, length, ctypes.byref(key), None, 0,
                                                        ctypes.byref(size)))
        payload = (ctypes.c_uint8 * size.value)()
        self.library.check(self.library.c_export_prefix(self.handle, slot, length, ctypes.byref(key), payload,
                                                        size.value, ctypes.byref(size)))
        return bytes(payload)

    def import_prefix(self, slot: int, key, payload: bytes) -> int:
        """Loads a payload into the empty `slot`; returns the positions it holds (synapse_kv_import_prefix)."""
        from .native import PrefixKey

        key = key if isinstance(key, PrefixKey) else PrefixKey(*key)
        buffer = (ctypes.c_uint8 * len(payload)).from_buffer_copy(payload)
        length = ctypes.c_uint32()
        self.library.check(self.library.c_import_prefix(self.handle, slot, ctypes.byref(key), buffer, len(payload),
                                                        ctypes.byref(length)))
        return int(length.value)

    def prefix_hash(self, tokens) -> int:
        """FNV-1a 64 of the token ids as little-endian int32 (synapse_kv_prefix_hash)."""
        data = np.ascontiguousarray(tokens, dtype="<i4").tobytes()
        buffer = (ctypes.c_uint8 * max(1, len(data))).from_buffer_copy(data or b"\0")
        return int(self.library.c_prefix_hash(buffer, len(data)))

    def read_kv(self, slot: int, layer: int, first: int, count: int) -> tuple[np.ndarray, np.ndarray]:
        """K and V of positions [first, first + count) as [count][kv_heads][head_dim] in the storage type
        (float32, or uint16 FP16 bit patterns)."""
        dtype = np.uint16 if self.precision == KV_F16 else np.float32
        keys = np.zeros((count, self.kv_heads, self.head_dim), dtype=dtype)
        values = np.zeros_like(keys)
        self.library.check(
            self.library.c_read_kv(self.handle, slot, layer, first, count, keys.ctypes.data, values.ctypes.data)
        )
        return keys, values


