"""ctypes binding of libsynapse_kv, mirroring Synapse's managed loader.

The conventions follow ``NativeGpuLibrary`` (src/Synapse.Runtime/Features/GpuKernels/NativeGpuLibrary.cs):
the library is loaded from an explicit path, its ABI version is checked before any other call
(``NativeGpuLibrary.cs:49-75``), and failing status codes become exceptions with the library's
thread-local message (``ThrowIfFailed``): status 3 -> :class:`NotSupportedError`
(NotSupportedException), 5 -> :class:`InsufficientMemoryError` (InsufficientMemoryException), anything
else -> :class:`InvalidOperationError` (InvalidOperationException).

There is no fallback: a missing or mismatched library raises :class:`NotSupportedError`.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

ABI_VERSION = 4
LIBRARY_PATH = Path(__file__).resolve().parent / "_lib" / "libsynapse_kv.so"

STATUS_OK = 0
STATUS_NULL_POINTER = 1
STATUS_INVALID_ARGUMENT = 2
STATUS_UNAVAILABLE = 3
STATUS_DEVICE_ERROR = 4
STATUS_OUT_OF_MEMORY = 5
STATUS_PANIC = 6

KV_F32 = 0
KV_F16 = 1

OPTION_SPLIT_KEYS = 1
OPTION_PREFILL_RUNS = 2
OPTION_PREFILL_SPLIT_KEYS = 3
OPTION_DECODE_PREFETCH = 4
OPTION_PROFILE_EVERY = 5
OPTION_SHARED_PREFIX = 6
OPTION_FUSED_SUMS = 7
OPTION_SEGMENT_COST = 8
OPTION_ADAPTIVE_SPLIT = 9

SELECT_KEY_BOUND = 0
SELECT_RANDOM = 1


class SynapseKvError(RuntimeError):
    """A failing status from the library, with its status code and message."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class NotSupportedError(SynapseKvError):
    """Status 3: the library, device or requested shape is unavailable."""


class InsufficientMemoryError(SynapseKvError, MemoryError):
    """Status 5: a device allocation failed or the page pool is exhausted."""


class InvalidOperationError(SynapseKvError):
    """Any other failing status (null pointer, invalid argument, device error, caught exception)."""


class DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_uint8 * 128),
        ("recommended_working_set_bytes", ctypes.c_uint64),
        ("max_buffer_bytes", ctypes.c_uint64),
        ("unified_memory", ctypes.c_uint32),
        ("apple_family", ctypes.c_uint32),
    ]


class BatchToken(ctypes.Structure):
    """BatchToken (native/synapse-gpu/src/Features/GpuKernels/decoder.rs:133-141)."""

    _fields_ = [
        ("slot", ctypes.c_int32),
        ("token", ctypes.c_int32),
        ("position", ctypes.c_int32),
        ("logits_row", ctypes.c_int32),
    ]


class CacheDesc(ctypes.Structure):
    _fields_ = [
        ("rope_cosines", ctypes.POINTER(ctypes.c_float)),
        ("rope_sines", ctypes.POINTER(ctypes.c_float)),
        ("layer_count", ctypes.c_uint32),
        ("heads", ctypes.c_uint32),
        ("kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("max_positions", ctypes.c_uint32),
        ("kv_growth_positions", ctypes.c_uint32),
        ("page_tokens", ctypes.c_uint32),
        ("kv_precision", ctypes.c_uint32),
        ("session_slots", ctypes.c_uint32),
        ("step_tokens", ctypes.c_uint32),
        ("max_pages", ctypes.c_uint32),
        ("device", ctypes.c_int32),
    ]


class PageStats(ctypes.Structure):
    _fields_ = [
        ("max_pages", ctypes.c_uint32),
        ("free_pages", ctypes.c_uint32),
        ("used_pages", ctypes.c_uint32),
        ("shared_pages", ctypes.c_uint32),
        ("page_bytes", ctypes.c_uint64),
        ("kv_bytes", ctypes.c_uint64),
        ("device_status", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
    ]


KERNEL_KINDS = ("table", "pages", "append", "decode", "merge", "prefill", "gather", "page_select")

NO_BIAS = (1 << 64) - 1


class Matrix(ctypes.Structure):
    """SynapseKvMatrix: one GGML Q8_0 matrix of a host blob (matmul_segment's weight/bias/rows)."""

    _fields_ = [
        ("weight", ctypes.c_uint64),
        ("bias", ctypes.c_uint64),
        ("rows", ctypes.c_uint32),
        ("columns", ctypes.c_uint32),
    ]


class Projection(ctypes.Structure):
    """SynapseKvProjection: matmul_args (common.metal:61-71) with matrices named by index."""

    _fields_ = [
        ("matrix", ctypes.c_uint32 * 3),
        ("out_column", ctypes.c_uint32 * 3),
        ("segments", ctypes.c_uint32),
        ("tokens", ctypes.c_uint32),
        ("in_stride", ctypes.c_uint32),
        ("out_stride", ctypes.c_uint32),
        ("accumulate", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
    ]


class PageActivation(ctypes.Structure):
    """SynapseKvPageActivation: KvPageActivation (KvPageActivation.cs:10-37) plus an enable flag."""

    _fields_ = [
        ("enabled", ctypes.c_uint32),
        ("budget_pages", ctypes.c_uint32),
        ("window_tokens", ctypes.c_uint32),
        ("page_tokens", ctypes.c_uint32),
        ("selection", ctypes.c_uint32),
        ("seed", ctypes.c_int32),
    ]


NO_TENSOR = (1 << 64) - 1
ENCODING_Q8_0 = 8
ENCODING_Q4_K = 12
ENCODING_Q6_K = 14
ALL_Q8_0 = 0x08888888


class LayerOffsets(ctypes.Structure):
    """SynapseKvLayerOffsets: DecoderLayerOffsets (decoder.rs:60-81)."""

    _fields_ = [(name, ctypes.c_uint64) for name in (
        "attention_norm", "query", "key", "value", "query_bias", "key_bias", "value_bias", "query_norm", "key_norm",
        "attention_output", "feed_forward_norm", "gate", "up", "down", "encodings")]


class DecoderDesc(ctypes.Structure):
    """SynapseKvDecoderDesc: DecoderDesc (decoder.rs:85-116)."""

    _fields_ = [
        ("weights", ctypes.c_void_p),
        ("weights_length", ctypes.c_uint64),
        ("layers", ctypes.POINTER(LayerOffsets)),
        ("rope_cosines", ctypes.POINTER(ctypes.c_float)),
        ("rope_sines", ctypes.POINTER(ctypes.c_float)),
        ("token_embedding", ctypes.c_uint64),
        ("output_norm", ctypes.c_uint64),
        ("output", ctypes.c_uint64),
        ("layer_count", ctypes.c_uint32),
        ("hidden", ctypes.c_uint32),
        ("feed_forward", ctypes.c_uint32),
        ("heads", ctypes.c_uint32),
        ("kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("vocabulary", ctypes.c_uint32),
        ("context", ctypes.c_uint32),
        ("session_slots", ctypes.c_uint32),
        ("step_tokens", ctypes.c_uint32),
        ("logits_rows", ctypes.c_uint32),
        ("rms_epsilon", ctypes.c_float),
        ("embedding_encoding", ctypes.c_uint32),
        ("rope_layout", ctypes.c_uint32),
        ("activation", ctypes.c_uint32),
        ("kv_precision", ctypes.c_uint32),
        ("kv_growth_positions", ctypes.c_uint32),
        ("output_encoding", ctypes.c_uint32),
    ]


class Profile(ctypes.Structure):
    _fields_ = [("launches", ctypes.c_uint64 * 8), ("milliseconds", ctypes.c_double * 8)]


# Sizes pinned on both sides of the ABI (include/synapse_kv.h static assertions).
class PrefixKey(ctypes.Structure):
    """SynapseKvPrefixKey: what a persistent prefix payload is keyed by (ADR-018-prompt-prefix-reuse.md:42-44)."""

    _fields_ = [("model", ctypes.c_uint64), ("tokenizer", ctypes.c_uint64), ("rope", ctypes.c_uint64), ("prefix", ctypes.c_uint64)]


class PrefixHeader(ctypes.Structure):
    """SynapseKvPrefixHeader: the 128-byte header of a prefix payload."""

    _fields_ = [
        ("magic", ctypes.c_char * 8),
        ("version", ctypes.c_uint32),
        ("header_bytes", ctypes.c_uint32),
        ("key", PrefixKey),
        ("kv_precision", ctypes.c_uint32),
        ("layer_count", ctypes.c_uint32),
        ("kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("length", ctypes.c_uint32),
        ("reserved0", ctypes.c_uint32),
        ("payload_bytes", ctypes.c_uint64),
        ("checksum", ctypes.c_uint64),
        ("reserved", ctypes.c_uint8 * 40),
    ]


STRUCT_SIZES = {DeviceInfo: 152, BatchToken: 16, CacheDesc: 64, PageStats: 40, Profile: 128, Matrix: 24,
                Projection: 48, PageActivation: 24, LayerOffsets: 120, DecoderDesc: 136, PrefixKey: 32,
                PrefixHeader: 128}
for _struct, _size in STRUCT_SIZES.items():
    assert ctypes.sizeof(_struct) == _size, (_struct.__name__, ctypes.sizeof(_struct))

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_SIZE = ctypes.c_size_t

# name -> (restype, argtypes); the complete exported surface of include/synapse_kv.h.
EXPORTS = {
    "synapse_kv_abi_version": (_U32, []),
    "synapse_kv_prefix_hash": (_U64, [_P, _SIZE]),
    "synapse_kv_export_prefix": (_I32, [_P, _U32, _U32, ctypes.POINTER(PrefixKey), _P, _U64, ctypes.POINTER(_U64)]),
    "synapse_kv_import_prefix": (_I32, [_P, _U32, ctypes.POINTER(PrefixKey), _P, _U64, ctypes.POINTER(_U32)]),
    "synapse_kv_probe": (_I32, [ctypes.POINTER(DeviceInfo)]),
    "synapse_kv_last_error": (_SIZE, [ctypes.c_char_p, _SIZE]),
    "synapse_kv_cache_create": (_I32, [ctypes.POINTER(CacheDesc), ctypes.POINTER(_P)]),
    "synapse_kv_cache_destroy": (None, [_P]),
    "synapse_kv_set_stream": (_I32, [_P, _P]),
    "synapse_kv_set_option": (_I32, [_P, _U32, _U32]),
    "synapse_kv_bytes": (_U64, [_P]),
    "synapse_kv_reserve": (_I32, [_P, _U32, _U32]),
    "synapse_kv_release": (_I32, [_P, _U32]),
    "synapse_kv_truncate": (_I32, [_P, _U32, _U32]),
    "synapse_kv_fork": (_I32, [_P, _U32, _U32]),
    "synapse_kv_step": (_I32, [_P, ctypes.POINTER(BatchToken), _SIZE]),
    "synapse_kv_step_prompt": (_I32, [_P, ctypes.POINTER(BatchToken), _SIZE, _SIZE]),
    "synapse_kv_step_static": (_I32, [_P, ctypes.POINTER(BatchToken), _SIZE, _SIZE]),
    "synapse_kv_set_page_activation": (_I32, [_P, ctypes.POINTER(PageActivation)]),
    "synapse_kv_append_rope": (_I32, [_P, _U32, _P, _U32]),
    "synapse_kv_attention": (_I32, [_P, _U32, _P, _U32, _P, _U32]),
    "synapse_kv_append_attention": (_I32, [_P, _U32, _P, _U32, _P, _U32]),
    "synapse_kv_synchronize": (_I32, [_P]),
    "synapse_kv_profile_begin": (_I32, [_P]),
    "synapse_kv_profile_end": (_I32, [_P, ctypes.POINTER(Profile)]),
    "synapse_kv_slot_info": (
        _I32,
        [_P, _U32, ctypes.POINTER(_U32), ctypes.POINTER(_U32), ctypes.POINTER(_U32)],
    ),
    "synapse_kv_read_block_table": (_I32, [_P, _U32, _P, _SIZE, ctypes.POINTER(_SIZE)]),
    "synapse_kv_read_refcounts": (_I32, [_P, _P, _SIZE]),
    "synapse_kv_read_free_list": (_I32, [_P, _P, _SIZE, ctypes.POINTER(_SIZE)]),
    "synapse_kv_page_stats": (_I32, [_P, ctypes.POINTER(PageStats)]),
    "synapse_kv_read_kv": (_I32, [_P, _U32, _U32, _U32, _U32, _P, _P]),
    "synapse_kv_rope_table": (_I32, [_U32, ctypes.c_float, ctypes.c_float, _U32, _U32, _P, _P]),
    "synapse_kv_weights_create": (_I32, [_P, _U64, ctypes.POINTER(Matrix), _U32, ctypes.POINTER(_P)]),
    "synapse_kv_weights_create_encoded": (_I32, [_P, _U64, ctypes.POINTER(Matrix), ctypes.POINTER(_U32), _U32,
                                                 ctypes.POINTER(_P)]),
    "synapse_kv_weights_destroy": (None, [_P]),
    "synapse_kv_weights_bytes": (_U64, [_P]),
    "synapse_kv_weights_set_stream": (_I32, [_P, _P]),
    "synapse_kv_project": (_I32, [_P, ctypes.POINTER(Projection), _P, _P]),
    "synapse_kv_weights_read": (_I32, [_P, _U32, _P, _U64]),
    "synapse_kv_decoder_create": (_I32, [ctypes.POINTER(DecoderDesc), _I32, ctypes.POINTER(_P)]),
    "synapse_kv_decoder_forward": (_I32, [_P, ctypes.POINTER(BatchToken), _SIZE, _P, _SIZE]),
    "synapse_kv_decoder_forward_prompt": (_I32, [_P, ctypes.POINTER(BatchToken), _SIZE, _SIZE, _P, _SIZE]),
    "synapse_kv_decoder_destroy": (None, [_P]),
    "synapse_kv_decoder_kv_bytes": (_U64, [_P]),
    "synapse_kv_decoder_reserve": (_I32, [_P, _U32, _U32]),
    "synapse_kv_decoder_cache": (_I32, [_P, ctypes.POINTER(_P)]),
    "synapse_kv_decoder_set_stream": (_I32, [_P, _P]),
}

# libsynapse_gpu's ABI version 3 (include/synapse_gpu.h), exported by the same library for the HIP backend.
GPU_ABI_VERSION = 3
GPU_BACKEND_METAL = 1
GPU_BACKEND_CUDA = 2
GPU_BACKEND_HIP = 3
GPU_EXPORTS = {
    "synapse_gpu_abi_version": (_U32, []),
    "synapse_gpu_probe": (_I32, [_U32, ctypes.POINTER(DeviceInfo)]),
    "synapse_gpu_last_error": (_SIZE, [ctypes.c_char_p, _SIZE]),
    "synapse_gpu_decoder_create": (_I32, [_U32, ctypes.POINTER(DecoderDesc), ctypes.POINTER(_P)]),
    "synapse_gpu_decoder_forward": (_I32, [_P, ctypes.POINTER(BatchToken), _SIZE, _P, _SIZE]),
    "synapse_gpu_decoder_destroy": (None, [_P]),
    "synapse_gpu_decoder_kv_bytes": (_U64, [_P]),
    "synapse_gpu_decoder_reserve": (_I32, [_P, _U32, _U32]),
}


class NativeKvLibrary:
    """The loaded library with typed entry points and status checking."""

    _lock = threading.Lock()
    _loaded: "NativeKvLibrary | None" = None

    def __init__(self, path: Path):
        self.path = Path(path)
        if not self.path.exists():
            raise NotSupportedError(STATUS_UNAVAILABLE, f"{self.path}: the library file is missing; build it first")
        try:
            self.handle = ctypes.CDLL(str(self.path))
        except OSError as error:
            raise NotSupportedError(STATUS_UNAVAILABLE, f"{self.path}: the loader could not load it: {error}")
        version_function = self.handle.synapse_kv_abi_version
        version_function.restype = _U32
        version_function.argtypes = []
        version = version_function()
        if version != ABI_VERSION:
            raise NotSupportedError(
                STATUS_UNAVAILABLE, f"{self.path}: its ABI version {version} differs from the required {ABI_VERSION}"
            )
        for name, (restype, argtypes) in EXPORTS.items():
            function = getattr(self.handle, name)
            function.restype = restype
            function.argtypes = argtypes
            setattr(self, "c_" + name[len("synapse_kv_"):], function)
        for name, (restype, argtypes) in GPU_EXPORTS.items():
            function = getattr(self.handle, name)
            function.restype = restype
            function.argtypes = argtypes
            setattr(self, "g_" + name[len("synapse_gpu_"):], function)

    @classmethod
    def load(cls, path: Path | None = None) -> "NativeKvLibrary":
        with cls._lock:
            if path is not None:
                return cls(path)
            if cls._loaded is None:
                cls._loaded = cls(LIBRARY_PATH)
            return cls._loaded

    def last_error(self) -> str:
        """NativeGpuLibrary.LastError: query the length, then copy the message out."""
        length = self.c_last_error(None, 0)
        buffer = ctypes.create_string_buffer(max(1, length))
        self.c_last_error(buffer, length)
        return buffer.raw[:length].decode("utf-8", "replace")

    def check(self, status: int) -> None:
        """ThrowIfFailed: maps a failing status to the matching exception."""
        if status == STATUS_OK:
            return
        message = self.last_error()
        if status == STATUS_UNAVAILABLE:
            raise NotSupportedError(status, message)
        if status == STATUS_OUT_OF_MEMORY:
            raise InsufficientMemoryError(status, message)
        raise InvalidOperationError(status, message)

    def probe(self) -> dict:
        info = DeviceInfo()
        self.check(self.c_probe(ctypes.byref(info)))
        raw = bytes(info.name)
        return {
            "name": raw.split(b"\0", 1)[0].decode("utf-8", "replace"),
            "recommended_working_set_bytes": info.recommended_working_set_bytes,
            "max_buffer_bytes": info.max_buffer_bytes,
            "unified_memory": bool(info.unified_memory),
        }
