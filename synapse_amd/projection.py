"""Q8_0 projections over libsynapse_kv: the QKV and o_proj matrices around the attention path.

``Q8Weights`` mirrors what the reference's GPU step does with a layer's matrices
(native/synapse-gpu/src/Features/GpuKernels/step/projection.rs:51-141 over matmul.cu / matmul.metal): the model
file's GGML Q8_0 rows are selected by byte offset (GpuLayoutMapping.cs:14-32), uploaded once, and each
``project`` call computes

    output[t][out_column[s] + row] = (accumulate ? output : 0) + sum_k (d * code)[row][k] * input[t][k] + bias[row]

for the rows of up to three matrices (``matmul_args``, common.metal:54-71), in FP32. Device buffers are torch
tensors (or raw device addresses). There is no CPU fallback.
"""

from __future__ import annotations

import ctypes

import numpy as np

from .native import NO_BIAS, Matrix, NativeKvLibrary, Projection

BLOCK_ELEMENTS = 32
BLOCK_BYTES = 34


def _address(buffer) -> int:
    if isinstance(buffer, int):
        return buffer
    if hasattr(buffer, "data_ptr"):
        return int(buffer.data_ptr())
    raise TypeError("expected a device tensor or a device address")


class Q8Weights:
    """Q8_0 matrices of one host blob, resident on the device in the projection kernel's layout."""

    def __init__(self, blob: np.ndarray, matrices: list[dict], library: NativeKvLibrary | None = None):
        """``blob``: uint8 bytes of the model file (or any buffer holding the matrices); ``matrices``: dicts with
        ``weight`` (byte offset), ``rows``, ``columns`` and optional ``bias`` (byte offset of FP32 biases)."""
        self.library = library or NativeKvLibrary.load()
        blob = np.ascontiguousarray(blob, dtype=np.uint8)
        described = (Matrix * len(matrices))()
        for index, matrix in enumerate(matrices):
            described[index].weight = int(matrix["weight"])
            bias = matrix.get("bias")
            described[index].bias = NO_BIAS if bias is None else int(bias)
            described[index].rows = int(matrix["rows"])
            described[index].columns = int(matrix["columns"])
        handle = ctypes.c_void_p()
        self.library.check(
            self.library.c_weights_create(blob.ctypes.data, blob.nbytes, described, len(matrices), ctypes.byref(handle))
        )
        self.handle = handle
        self.shapes = [(int(m["rows"]), int(m["columns"])) for m in matrices]

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.library.c_weights_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    @property
    def device_bytes(self) -> int:
        return int(self.library.c_weights_bytes(self.handle))

    def set_stream(self, stream) -> None:
        """Orders the projections on a torch stream (or a raw hipStream_t address)."""
        raw = stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream or 0)
        self.library.check(self.library.c_weights_set_stream(self.handle, ctypes.c_void_p(raw)))

    def project(self, segments, inputs, output, tokens: int | None = None, in_stride: int | None = None,
                out_stride: int | None = None, accumulate: bool = False) -> None:
        """``segments``: [(matrix index, first output column)] (1..3); ``inputs`` [tokens][>= columns] and
        ``output`` [tokens][out_stride] FP32 device buffers."""
        projection = Projection()
        for s, (matrix, column) in enumerate(segments):
            projection.matrix[s] = int(matrix)
            projection.out_column[s] = int(column)
        projection.segments = len(segments)
        projection.tokens = int(tokens if tokens is not None else inputs.shape[0])
        projection.in_stride = int(in_stride if in_stride is not None else inputs.shape[-1])
        projection.out_stride = int(out_stride if out_stride is not None else output.shape[-1])
        projection.accumulate = 1 if accumulate else 0
        self.library.check(
            self.library.c_project(self.handle, ctypes.byref(projection), _address(inputs), _address(output))
        )

    def read(self, index: int) -> np.ndarray:
        """Matrix ``index`` copied back as GGML Q8_0 blocks (uint8 [rows][columns / 32 * 34])."""
        rows, columns = self.shapes[index]
        out = np.empty((rows, columns // BLOCK_ELEMENTS * BLOCK_BYTES), dtype=np.uint8)
        self.library.check(self.library.c_weights_read(self.handle, index, out.ctypes.data, out.nbytes))
        return out


def quantize_q8_0(values: np.ndarray) -> np.ndarray:
    """GGML Q8_0 rows of a float matrix (ggml quantize_row_q8_0; the reference's test writer
    TinyQwen2Gguf.QuantizeQ8Zero): per 32 values d = max|x| / 127 stored as FP16 (round to nearest even), codes
    round_half_even(x / d) with the unrounded d. Returns uint8 [rows][columns / 32 * 34]."""
    values = np.asarray(values, dtype=np.float32)
    rows, columns = values.shape
    blocks = values.reshape(rows, columns // BLOCK_ELEMENTS, BLOCK_ELEMENTS)
    scale = np.abs(blocks).max(axis=2) / np.float32(127.0)
    inverse = np.where(scale == 0, np.float32(0.0), np.float32(1.0) / np.where(scale == 0, 1, scale)).astype(np.float32)
    codes = np.rint(blocks * inverse[:, :, None]).astype(np.int8)
    out = np.empty((rows, columns // BLOCK_ELEMENTS, BLOCK_BYTES), dtype=np.uint8)
    out[:, :, :2] = scale.astype(np.float16).view(np.uint8).reshape(rows, -1, 2)
    out[:, :, 2:] = codes.view(np.uint8)
    return out.reshape(rows, -1)


def dequantize_q8_0(blocks: np.ndarray, columns: int) -> np.ndarray:
    """FP32 elements d * code of GGML Q8_0 rows (exact)."""
    blocks = np.asarray(blocks, dtype=np.uint8).reshape(-1, columns // BLOCK_ELEMENTS, BLOCK_BYTES)
    scale = blocks[:, :, :2].copy().view(np.float16).astype(np.float32)
    codes = blocks[:, :, 2:].view(np.int8).astype(np.float32)
    return (codes * scale).reshape(-1, columns)
