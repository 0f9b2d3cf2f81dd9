"""Q8_0 and K-quant projections over libsynapse_kv: the QKV and o_proj matrices around the attention path.

``Q8Weights`` mirrors what the reference's GPU step does with a layer's matrices
(native/synapse-gpu/src/Features/GpuKernels/step/projection.rs:51-141 over matmul.cu / matmul.metal): the model
file's GGML Q8_0 rows are selected by byte offset (GpuLayoutMapping.cs:14-32), uploaded once, and each
``project`` call computes

    output[t][out_column[s] + row] = (accumulate ? output : 0) + sum_k (d * code)[row][k] * input[t][k] + bias[row]

for the rows of up to three matrices (``matmul_args``, common.metal:54-71), in FP32. Matrices may also be GGML
Q4_K or Q6_K (ADR-021; matmul_kquant.metal), named per matrix by ``encoding``. Device buffers are torch tensors (or
raw device addresses). There is no CPU fallback.

The numpy codecs below (GGML block layouts, written from ggml's published dequantize_row_q4_K / q6_K and the
reference's test encoder TinyKQuantEncoder.cs) make test and benchmark models; they are not used by the projections.
"""

from __future__ import annotations

import ctypes

import numpy as np

from .native import ENCODING_Q4_K, ENCODING_Q6_K, ENCODING_Q8_0, NO_BIAS, Matrix, NativeKvLibrary, Projection

BLOCK_ELEMENTS = 32
BLOCK_BYTES = 34
SUPER_BLOCK = 256
Q4_K_BYTES = 144
Q6_K_BYTES = 210


def matrix_bytes(encoding: int, rows: int, columns: int) -> int:
    """Bytes of a rows x columns GGML matrix (Encoding::matrix_bytes, decoder/encoding.rs:59-62)."""
    if encoding == ENCODING_Q8_0:
        return rows * (columns // BLOCK_ELEMENTS) * BLOCK_BYTES
    per = {ENCODING_Q4_K: Q4_K_BYTES, ENCODING_Q6_K: Q6_K_BYTES}[encoding]
    return rows * (columns // SUPER_BLOCK) * per


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
        ``weight`` (byte offset), ``rows``, ``columns``, optional ``bias`` (byte offset of FP32 biases) and optional
        ``encoding`` (GGML type id, Q8_0 when absent)."""
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
        encodings = [int(m.get("encoding", ENCODING_Q8_0)) for m in matrices]
        if all(e == ENCODING_Q8_0 for e in encodings):
            status = self.library.c_weights_create(blob.ctypes.data, blob.nbytes, described, len(matrices),
                                                   ctypes.byref(handle))
        else:
            ids = (ctypes.c_uint32 * len(matrices))(*encodings)
            status = self.library.c_weights_create_encoded(blob.ctypes.data, blob.nbytes, described, ids,
                                                           len(matrices), ctypes.byref(handle))
        self.library.check(status)
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


def _f16(raw: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(raw).view(np.float16).astype(np.float32)


def _q4_k_scales(packed: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """get_scale_min_k4 over [n][12] packed bytes: ([n][8] scales, [n][8] minima)."""
    packed = packed.astype(np.int32)
    scale = np.empty((packed.shape[0], 8), dtype=np.int32)
    minimum = np.empty_like(scale)
    scale[:, :4] = packed[:, 0:4] & 63
    minimum[:, :4] = packed[:, 4:8] & 63
    scale[:, 4:] = (packed[:, 8:12] & 0xF) | ((packed[:, 0:4] >> 6) << 4)
    minimum[:, 4:] = (packed[:, 8:12] >> 4) | ((packed[:, 4:8] >> 6) << 4)
    return scale, minimum


def dequantize_q4_k(blocks: np.ndarray, columns: int) -> np.ndarray:
    """FP32 values (d * sc) * q - (dmin * m) of GGML Q4_K rows (GgufKQuantBlocks.DecodeQ4K, :99-121), each product
    and the difference rounded to FP32 as the reference computes them."""
    b = np.asarray(blocks, dtype=np.uint8).reshape(-1, Q4_K_BYTES)
    d = _f16(b[:, 0:2])
    dmin = _f16(b[:, 2:4])
    scale, minimum = _q4_k_scales(b[:, 4:16])
    q = b[:, 16:].reshape(-1, 4, 32)
    codes = np.empty((b.shape[0], 8, 32), dtype=np.float32)
    codes[:, 0::2] = q & 0xF
    codes[:, 1::2] = q >> 4
    step = (d * scale.astype(np.float32)).astype(np.float32)
    offset = (dmin * minimum.astype(np.float32)).astype(np.float32)
    values = (step[:, :, None] * codes).astype(np.float32) - offset[:, :, None]
    return values.astype(np.float32).reshape(-1, columns)


def _q6_k_index() -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    i = np.arange(SUPER_BLOCK)
    half, rest = i // 128, i % 128
    quarter, lane = rest // 32, rest % 32
    low = half * 64 + np.where(quarter % 2 == 0, lane, lane + 32)
    high = 128 + half * 32 + lane
    return low, np.where(quarter < 2, 0, 4), high, 2 * quarter


def dequantize_q6_k(blocks: np.ndarray, columns: int) -> np.ndarray:
    """FP32 values (d * scale[i / 16]) * (q - 32) of GGML Q6_K rows (GgufKQuantBlocks.DecodeQ6K, :155-177)."""
    b = np.asarray(blocks, dtype=np.uint8).reshape(-1, Q6_K_BYTES)
    low, low_shift, high, high_shift = _q6_k_index()
    q = ((b[:, low] >> low_shift) & 0xF) | (((b[:, high] >> high_shift) & 3) << 4)
    d = _f16(b[:, 208:210])
    step = (d * b[:, 192:208].view(np.int8).astype(np.float32)).astype(np.float32)
    values = np.repeat(step, 16, axis=1) * (q.astype(np.float32) - 32.0)
    return values.astype(np.float32).reshape(-1, columns)


def dequantize(encoding: int, blocks: np.ndarray, columns: int) -> np.ndarray:
    """FP32 values of GGML rows in any of the three encodings."""
    if encoding == ENCODING_Q8_0:
        return dequantize_q8_0(blocks, columns)
    return {ENCODING_Q4_K: dequantize_q4_k, ENCODING_Q6_K: dequantize_q6_k}[encoding](blocks, columns)


def quantize_q4_k(values: np.ndarray) -> np.ndarray:
    """GGML Q4_K rows of a float matrix by the reference's simple test encoder (TinyKQuantEncoder.EncodeQ4KBlock):
    per 32-value sub-block a step (max - min(0, min)) / 15 and an offset -min(0, min); d and dmin the largest of each
    / 63 in FP16; 6-bit scale and minimum round(step / d), round(offset / dmin); codes round((x + dmin m) / (d sc))
    clamped to 0..15. Returns uint8 [rows][columns / 256 * 144]."""
    x = np.asarray(values, dtype=np.float32).reshape(-1, 8, 32)
    low = np.minimum(np.float32(0), x.min(axis=2))
    steps = ((x.max(axis=2) - low) / np.float32(15)).astype(np.float32)
    offsets = (-low).astype(np.float32)
    d = (steps.max(axis=1) / np.float32(63)).astype(np.float16).astype(np.float32)
    dmin = (offsets.max(axis=1) / np.float32(63)).astype(np.float16).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = np.where(d[:, None] == 0, 0, np.clip(np.rint(steps / d[:, None]), 0, 63)).astype(np.int32)
        minimum = np.where(dmin[:, None] == 0, 0, np.clip(np.rint(offsets / dmin[:, None]), 0, 63)).astype(np.int32)
        step = (d[:, None] * scale.astype(np.float32)).astype(np.float32)
        bias = (dmin[:, None] * minimum.astype(np.float32)).astype(np.float32)
        q = np.where(step[:, :, None] == 0, 0,
                     np.clip(np.rint((x + bias[:, :, None]) / step[:, :, None]), 0, 15)).astype(np.uint8)
    out = np.zeros((x.shape[0], Q4_K_BYTES), dtype=np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = dmin.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 4:8] = (scale[:, :4] & 63) | ((scale[:, 4:] >> 4) << 6)
    out[:, 8:12] = (minimum[:, :4] & 63) | ((minimum[:, 4:] >> 4) << 6)
    out[:, 12:16] = (scale[:, 4:] & 0xF) | ((minimum[:, 4:] & 0xF) << 4)
    out[:, 16:] = (q[:, 0::2] | (q[:, 1::2] << 4)).reshape(-1, 128)
    rows = np.asarray(values).shape[0]
    return out.reshape(rows, -1)


def quantize_q6_k(values: np.ndarray) -> np.ndarray:
    """GGML Q6_K rows by TinyKQuantEncoder.EncodeQ6KBlock: per 16 values a step max|x| / 31; d the largest step / 127
    in FP16; int8 scales round(step / d) clamped to 1..127 (1 when d is 0); codes round(x / (d sc)) clamped to
    -32..31, stored + 32. Returns uint8 [rows][columns / 256 * 210]."""
    x = np.asarray(values, dtype=np.float32).reshape(-1, SUPER_BLOCK)
    steps = (np.abs(x.reshape(-1, 16, 16)).max(axis=2) / np.float32(31)).astype(np.float32)
    d = (steps.max(axis=1) / np.float32(127)).astype(np.float16).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = np.where(d[:, None] == 0, 1, np.clip(np.rint(steps / d[:, None]), 1, 127)).astype(np.int32)
        step = (d[:, None] * scale.astype(np.float32)).astype(np.float32)
        full = np.repeat(step, 16, axis=1)
        q = (np.where(full == 0, 0, np.clip(np.rint(x / full), -32, 31)) + 32).astype(np.int32)
    out = np.zeros((x.shape[0], Q6_K_BYTES), dtype=np.uint8)
    low, low_shift, high, high_shift = _q6_k_index()
    for i in range(SUPER_BLOCK):
        out[:, low[i]] |= ((q[:, i] & 0xF) << low_shift[i]).astype(np.uint8)
        out[:, high[i]] |= (((q[:, i] >> 4) & 3) << high_shift[i]).astype(np.uint8)
    out[:, 192:208] = scale.astype(np.int8).view(np.uint8)
    out[:, 208:210] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    rows = np.asarray(values).shape[0]
    return out.reshape(rows, -1)


def quantize(encoding: int, values: np.ndarray) -> np.ndarray:
    if encoding == ENCODING_Q8_0:
        return quantize_q8_0(values)
    return {ENCODING_Q4_K: quantize_q4_k, ENCODING_Q6_K: quantize_q6_k}[encoding](values)
