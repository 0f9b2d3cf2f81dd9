"""The C ABI without a GPU: every declared symbol is exported, struct sizes are pinned, and the error paths follow
the reference's conventions (ffi.rs: status codes, thread-local last error, null-safe destroy and kv_bytes)."""

import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle_ffi import rope_table as oracle_rope_table

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "synapse_kv.h"
GPU_HEADER = ROOT / "include" / "synapse_gpu.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(synapse_kv_\w+)\s*\(", text, flags=re.MULTILINE)))


def test_every_declared_function_is_exported(native):
    names = declared_functions()
    assert len(names) >= 20
    exported = subprocess.run(["nm", "-D", "--defined-only", str(native.path)], capture_output=True, text=True,
                              check=True).stdout
    symbols = set(re.findall(r"\b(synapse_kv_\w+)\b", exported))
    assert set(names) == symbols, (set(names) ^ symbols)
    from synapse_amd.native import EXPORTS
    assert set(EXPORTS) == set(names)


@pytest.mark.parametrize("compiler,flag", [("gcc", "-std=c11"), ("g++", "-std=c++17")])
def test_header_compiles_with_pinned_sizes(compiler, flag, tmp_path):
    source = tmp_path / ("probe.c" if compiler == "gcc" else "probe.cpp")
    source.write_text('#include "synapse_kv.h"\nint main(void) { return (int)sizeof(SynapseKvDesc) - 64; }\n')
    subprocess.run([compiler, flag, "-fsyntax-only", "-I", str(HEADER.parent), str(source)], check=True)


def test_abi_version_and_struct_sizes(native):
    from synapse_amd.native import ABI_VERSION, STRUCT_SIZES

    assert native.c_abi_version() == ABI_VERSION == 4
    for struct, size in STRUCT_SIZES.items():
        assert ctypes.sizeof(struct) == size


def test_status_codes_match_the_reference():
    # error.rs:4-16.
    from synapse_amd import native as n

    assert [n.STATUS_OK, n.STATUS_NULL_POINTER, n.STATUS_INVALID_ARGUMENT, n.STATUS_UNAVAILABLE,
            n.STATUS_DEVICE_ERROR, n.STATUS_OUT_OF_MEMORY, n.STATUS_PANIC] == list(range(7))


def test_null_pointers_and_last_error_protocol(native):
    assert native.c_probe(None) == 1
    message = native.last_error()
    assert "null pointer" in message
    length = native.c_last_error(None, 0)
    assert length == len(message.encode())
    short = ctypes.create_string_buffer(4)
    assert native.c_last_error(short, 4) == length
    assert short.raw == message.encode()[:4]
    assert native.c_cache_create(None, None) == 1
    assert native.c_reserve(None, 0, 0) == 1
    assert native.c_step(None, None, 0) == 1
    assert native.c_attention(None, 0, None, 0, None, 0) == 1
    assert native.c_bytes(None) == 0
    native.c_cache_destroy(None)  # null is ignored
    assert native.c_weights_create(None, 0, None, 0, None) == 1
    assert native.c_project(None, None, None, None) == 1
    assert native.c_weights_set_stream(None, None) == 1
    assert native.c_weights_read(None, 0, None, 0) == 1
    assert native.c_weights_bytes(None) == 0
    native.c_weights_destroy(None)  # null is ignored


def test_status_maps_to_the_managed_exceptions(native):
    from synapse_amd.native import InsufficientMemoryError, InvalidOperationError, NotSupportedError

    with pytest.raises(InvalidOperationError):
        native.check(native.c_probe(None))
    for status, kind in [(3, NotSupportedError), (5, InsufficientMemoryError), (2, InvalidOperationError),
                         (4, InvalidOperationError), (6, InvalidOperationError)]:
        with pytest.raises(kind):
            native.check(status)


def cpu_desc(**overrides):
    from synapse_amd.native import CacheDesc

    cos = np.zeros((64, 32), dtype=np.float32)
    fields = dict(layer_count=2, heads=14, kv_heads=2, head_dim=64, max_positions=64, kv_growth_positions=64,
                  page_tokens=64, kv_precision=1, session_slots=1, step_tokens=8, max_pages=2, device=0)
    fields.update(overrides)
    pointer = cos.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    return CacheDesc(pointer, pointer, *fields.values()), cos


@pytest.mark.parametrize("overrides,status", [
    ({"head_dim": 96}, 3), ({"kv_precision": 2}, 2), ({"heads": 15}, 2), ({"kv_growth_positions": 32}, 2),
    ({"page_tokens": 100}, 2), ({"max_pages": 0}, 2), ({"heads": 18, "kv_heads": 2}, 2)])
def test_create_validates_the_shape_before_the_device(native, overrides, status):
    desc, _keep = cpu_desc(**overrides)
    handle = ctypes.c_void_p()
    assert native.c_cache_create(ctypes.byref(desc), ctypes.byref(handle)) == status
    assert not handle.value


def test_rope_table_entry_point_matches_the_restatement(native):
    from synapse_amd import rope_table

    for head_dim, factor, original in [(64, 0.0, 0), (128, 0.0, 0), (64, 4.0, 32768)]:
        cos, sin = rope_table(head_dim, 1e6, 3000, factor, original, library=native)
        ocos, osin = oracle_rope_table(head_dim, 1e6, 3000, factor, original)
        assert np.array_equal(cos.view(np.uint32), ocos.view(np.uint32))
        assert np.array_equal(sin.view(np.uint32), osin.view(np.uint32))
    out = np.zeros(4, dtype=np.float32)
    assert native.c_rope_table(63, 1e6, 0.0, 0, 1, out.ctypes.data, out.ctypes.data) == 2


@pytest.mark.parametrize("rows,columns,weight,bias,count", [
    (4, 48, 0, None, 1),        # columns not a multiple of 32
    (0, 64, 0, None, 1),        # no rows
    (4, 64, 40, None, 1),       # rows run past the blob (4 * 2 * 34 = 272 bytes from offset 40 of 300)
    (4, 64, 0, 298, 1),         # biases run past the blob
    (4, 64, 0, 2, 1),           # biases not 4-byte aligned
    (4, 64, 0, None, 0),        # no matrices
])
def test_weights_create_validates_before_the_device(native, rows, columns, weight, bias, count):
    from synapse_amd.native import NO_BIAS, Matrix

    blob = np.zeros(300, dtype=np.uint8)
    matrix = Matrix(weight, NO_BIAS if bias is None else bias, rows, columns)
    handle = ctypes.c_void_p()
    assert native.c_weights_create(blob.ctypes.data, blob.nbytes, ctypes.byref(matrix), count,
                                   ctypes.byref(handle)) == 2
    assert "invalid argument" in native.last_error()
    assert not handle.value


def decoder_desc(**overrides):
    """A valid SynapseKvDecoderDesc over a tiny synthetic model file, with fields overridden."""
    from synapse_amd.decoder import DecoderShape, synthetic_model
    from synapse_amd.native import DecoderDesc, LayerOffsets

    shape = DecoderShape(layers=1, hidden=128, feed_forward=256, heads=2, kv_heads=1, head_dim=64, vocabulary=64,
                         context=128, session_slots=2, step_tokens=8, logits_rows=4, growth=64)
    blob, layout = synthetic_model(shape, seed=1)
    layer_overrides = overrides.pop("layer", {})
    layers = (LayerOffsets * 1)()
    for name, _ in LayerOffsets._fields_:
        setattr(layers[0], name, int(layer_overrides.get(name, layout["layers"][0][name])))
    cos = np.zeros((128, 32), dtype=np.float32)
    desc = DecoderDesc()
    desc.weights = blob.ctypes.data
    desc.weights_length = blob.nbytes
    desc.layers = layers
    desc.rope_cosines = cos.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    desc.rope_sines = cos.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    fields = dict(token_embedding=layout["token_embedding"], output_norm=layout["output_norm"],
                  output=layout["output"], layer_count=1, hidden=128, feed_forward=256, heads=2, kv_heads=1,
                  head_dim=64, vocabulary=64, context=128, session_slots=2, step_tokens=8, logits_rows=4,
                  rms_epsilon=1e-6, embedding_encoding=8, rope_layout=0, activation=0, kv_precision=0,
                  kv_growth_positions=64, output_encoding=8)
    fields.update(overrides)
    for name, value in fields.items():
        setattr(desc, name, value)
    return desc, (blob, layers, cos)


@pytest.mark.parametrize("overrides,status,message", [
    ({"output_encoding": 12}, 3, "tensor output has 128 columns, not a multiple of its 256-value blocks"),
    ({"output_encoding": 14}, 3, "256-value blocks"),
    ({"embedding_encoding": 2}, 3, "not GGML type 2"),
    ({"rope_layout": 2}, 3, "NeoX RoPE"),
    ({"activation": 1}, 3, "SwiGLU"),
    ({"head_dim": 96, "hidden": 192}, 3, "head dimensions"),
    ({"heads": 18, "kv_heads": 2, "hidden": 18 * 64}, 3, "at most 8"),
    ({"rms_epsilon": 0.0}, 2, "epsilon"),
    ({"kv_growth_positions": 32}, 2, "multiple of 64"),
    ({"feed_forward": 0}, 2, "positive"),
    ({"output": 10**9}, 2, "tensor output"),
    ({"output_norm": 2}, 2, "tensor output_norm"),
    ({"layer": {"query_norm": 0}}, 3, "query/key normalization"),
    ({"layer": {"encodings": 0x08888C88}}, 3, "tensor attn_v has 128 columns"),
    ({"layer": {"encodings": 0x08888388}}, 3, "not GGML type 3"),
    ({"layer": {"key_bias": 10**9}}, 2, "layer 0: tensor attn_k.bias"),
    ({"layer": {"gate": 1}}, 2, "layer 0: tensor ffn_gate"),
])
def test_decoder_create_validates_the_description_first(native, overrides, status, message):
    # DecoderPlan::new (decoder.rs:246-294, checks.rs) runs before any device work.
    desc, _keep = decoder_desc(**overrides)
    handle = ctypes.c_void_p()
    assert native.c_decoder_create(ctypes.byref(desc), 0, ctypes.byref(handle)) == status
    assert message in native.last_error()
    assert not handle.value


def test_encoded_weights_validate_before_device_work(native):
    """synapse_kv_weights_create_encoded checks every matrix (encoding, whole blocks, range) before any HIP call."""
    from synapse_amd.native import Matrix

    blob = np.zeros(4096, dtype=np.uint8)
    matrices = (Matrix * 1)()
    matrices[0].weight = 0
    matrices[0].bias = (1 << 64) - 1
    handle = ctypes.c_void_p()
    for encoding, rows, columns, status, message in ((3, 4, 256, 3, "not GGML type 3"),
                                                     (12, 4, 128, 2, "multiple of 256"),
                                                     (14, 10, 512, 2, "extend past the blob"),
                                                     (12, 8, 1024, 2, "extend past the blob")):
        matrices[0].rows = rows
        matrices[0].columns = columns
        ids = (ctypes.c_uint32 * 1)(encoding)
        assert native.c_weights_create_encoded(blob.ctypes.data, blob.nbytes, matrices, ids, 1,
                                               ctypes.byref(handle)) == status
        assert message in native.last_error()
        assert not handle.value
    assert native.c_weights_create_encoded(None, 0, None, None, 0, None) == 1


def test_decoder_null_pointers(native):
    assert native.c_decoder_create(None, 0, None) == 1
    assert native.c_decoder_forward(None, None, 0, None, 0) == 1
    assert native.c_decoder_reserve(None, 0, 0) == 1
    assert native.c_decoder_kv_bytes(None) == 0
    assert native.c_decoder_cache(None, None) == 1
    native.c_decoder_destroy(None)


# ---- libsynapse_gpu's ABI version 3 (include/synapse_gpu.h) ----

def test_gpu_abi_is_declared_exported_and_versioned(native, tmp_path):
    """The eight functions NativeGpuLibrary binds (NativeGpuLibrary.cs:49-75) are exported with ABI version 3, and
    the header compiles in C and C++ with the reference's type names."""
    from synapse_amd.native import GPU_ABI_VERSION, GPU_EXPORTS

    declared = sorted(set(re.findall(r"^\w[\w\s\*]*?\b(synapse_gpu_\w+)\s*\(", GPU_HEADER.read_text(),
                                     flags=re.MULTILINE)))
    exported = subprocess.run(["nm", "-D", "--defined-only", str(native.path)], capture_output=True, text=True,
                              check=True).stdout
    assert set(declared) == set(re.findall(r"\b(synapse_gpu_\w+)\b", exported)) == set(GPU_EXPORTS)
    assert len(declared) == 8
    assert native.g_abi_version() == GPU_ABI_VERSION == 3
    for compiler, flag, suffix in (("gcc", "-std=c11", "c"), ("g++", "-std=c++17", "cpp")):
        source = tmp_path / f"gpu.{suffix}"
        source.write_text('#include "synapse_gpu.h"\n'
                          "int main(void) { return (int)(sizeof(DecoderDesc) + sizeof(DecoderLayerOffsets) +"
                          " sizeof(BatchToken) + sizeof(GpuDeviceInfo)) - (136 + 120 + 16 + 152); }\n")
        subprocess.run([compiler, flag, "-fsyntax-only", "-I", str(GPU_HEADER.parent), str(source)], check=True)


def test_gpu_abi_errors_follow_ffi_rs(native):
    """ffi.rs order: null checks, then DecoderPlan::new, then the backend (Metal and CUDA status 3 here, unknown
    ids status 2); the last error is the thread's, shared with synapse_kv_last_error; null-safe destroy/kv_bytes."""
    from synapse_amd.native import DeviceInfo

    info = DeviceInfo()
    assert native.g_probe(3, None) == 1
    assert native.g_probe(1, ctypes.byref(info)) == 3 and "macOS" in native.last_error()
    assert native.g_probe(2, ctypes.byref(info)) == 3 and "CUDA" in native.last_error()
    assert native.g_probe(9, ctypes.byref(info)) == 2 and "unknown GPU backend 9" in native.last_error()
    handle = ctypes.c_void_p()
    assert native.g_decoder_create(3, None, ctypes.byref(handle)) == 1
    desc, _keep = decoder_desc()
    for backend, status, message in ((1, 3, "macOS"), (2, 3, "CUDA"), (7, 2, "unknown GPU backend 7")):
        assert native.g_decoder_create(backend, ctypes.byref(desc), ctypes.byref(handle)) == status
        assert message in native.last_error()
        assert not handle.value
    bad, _keep_bad = decoder_desc(rope_layout=2)
    assert native.g_decoder_create(7, ctypes.byref(bad), ctypes.byref(handle)) == 3  # validation comes first
    assert "NeoX RoPE" in native.last_error()
    buffer = ctypes.create_string_buffer(256)
    length = native.g_last_error(buffer, 256)
    assert buffer.raw[:length].decode() == native.last_error()
    assert native.g_decoder_forward(None, None, 0, None, 0) == 1
    assert native.g_decoder_reserve(None, 0, 0) == 1
    assert native.g_decoder_kv_bytes(None) == 0
    native.g_decoder_destroy(None)


def test_prefix_hash_is_fnv1a_64(native):
    """Published FNV-1a 64 vectors (offset basis for the empty input; "a"; "foobar"), and token ids hash as their
    little-endian int32 bytes."""
    def digest(data: bytes) -> int:
        buffer = (ctypes.c_uint8 * max(1, len(data))).from_buffer_copy(data or b"\0")
        return int(native.c_prefix_hash(buffer, len(data)))

    assert digest(b"") == 0xcbf29ce484222325
    assert digest(b"a") == 0xaf63dc4c8601ec8c
    assert digest(b"foobar") == 0x85944171f73967e8
    assert int(native.c_prefix_hash(None, 0)) == 0xcbf29ce484222325
    tokens = np.array([7, 151643, 0, -1], dtype="<i4")
    assert digest(tokens.tobytes()) != digest(tokens[:3].tobytes())


def test_prefix_entry_points_check_pointers(native):
    from synapse_amd.native import PrefixKey

    key = PrefixKey(1, 2, 3, 4)
    size = ctypes.c_uint64()
    length = ctypes.c_uint32()
    assert native.c_export_prefix(None, 0, 0, ctypes.byref(key), None, 0, ctypes.byref(size)) == 1
    assert native.c_import_prefix(None, 0, ctypes.byref(key), None, 0, ctypes.byref(length)) == 1
    assert "null pointer" in native.last_error()
