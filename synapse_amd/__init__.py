"""MI355X-native KV-cache and attention path for Synapse (libsynapse_kv behind a C ABI)."""

from .native import (
    ABI_VERSION,
    InsufficientMemoryError,
    InvalidOperationError,
    NativeKvLibrary,
    NotSupportedError,
    SynapseKvError,
)
from .kv_cache import PagedKvCache, batch_tokens, rope_table

__all__ = [
    "ABI_VERSION",
    "InsufficientMemoryError",
    "InvalidOperationError",
    "NativeKvLibrary",
    "NotSupportedError",
    "PagedKvCache",
    "SynapseKvError",
    "batch_tokens",
    "rope_table",
]
