"""K-quant matrices (ADR-021): the GGML Q4_K / Q6_K block decoders that test models and the oracle rely on.

The reference holds no golden K-quant vectors (its tests compare against ggml's own dequantize_row_* from a native
library, GgmlReferenceDecoderTests.cs, which is not here). These tests pin the decoders instead with:
  * known-answer blocks built byte by byte from ggml's published layout, whose expected values are written out as
    literals (worked by hand in the comments), covering the packed high bits of Q4_K's scales and minima
    (sub-blocks 4-7), both nibbles, all four Q6_K quarters, both 128-value halves and negative int8 scales;
  * an encode -> decode round trip through the reference's test encoder restated in numpy
    (TinyKQuantEncoder.cs), whose error stays within the quantization step;
  * the C restatement (orc_decoder_*) against the numpy decoder on a closed form: a model whose layer matrices are
    zero passes the embedding row through, so the logits are W_out(norm(embedding row)) with K-quant tables.
"""

import numpy as np
import pytest

from oracle_ffi import DecoderOracle
from synapse_amd.decoder import DecoderShape, q4_k_m, synthetic_model
from synapse_amd.projection import (
    dequantize,
    dequantize_q4_k,
    dequantize_q6_k,
    matrix_bytes,
    quantize_q4_k,
    quantize_q6_k,
)


def half_bytes(value):
    return list(np.array([value], dtype=np.float16).view(np.uint8))


def q4_k_block():
    """d = 0.5, dmin = 0.25; sub-block scales [1, 2, 3, 63, 17, 40, 33, 62] and minima [0, 5, 10, 63, 48, 1, 20, 35]
    packed as get_scale_min_k4 reads them (bytes 0-3: scale low 6 bits | scale[j+4] >> 4 in bits 6-7; bytes 4-7:
    the same for minima; bytes 8-11: scale[j+4] & 15 | (min[j+4] & 15) << 4), worked out by hand; code of value l of
    sub-block j is (5 j + l) % 16."""
    block = np.zeros(144, dtype=np.uint8)
    block[0:2] = half_bytes(0.5)
    block[2:4] = half_bytes(0.25)
    block[4:16] = [65, 130, 131, 255, 192, 5, 74, 191, 1, 24, 65, 62]
    for j in range(8):
        for lane in range(32):
            code = (5 * j + lane) % 16
            block[16 + (j // 2) * 32 + lane] |= code << (4 * (j % 2))
    return block


def q6_k_block():
    """d = 0.125; int8 scales [1, -1, 2, -2, 3, -3, 4, -4, 127, -128, 5, -5, 10, -10, 60, -60]; six-bit code of value i
    is 7 i % 64, its low nibble in ql[64 h + l (+ 32 for quarters 1, 3)] (high nibble for quarters 2, 3) and its two
    high bits in qh[32 h + l] at bit 2 * quarter, for i = 128 h + 32 quarter + l."""
    block = np.zeros(210, dtype=np.uint8)
    for i in range(256):
        q = 7 * i % 64
        h, rest = divmod(i, 128)
        quarter, lane = divmod(rest, 32)
        block[h * 64 + lane + (32 if quarter % 2 else 0)] |= (q & 0xF) << (0 if quarter < 2 else 4)
        block[128 + h * 32 + lane] |= (q >> 4) << (2 * quarter)
    block[192:208] = np.array([1, -1, 2, -2, 3, -3, 4, -4, 127, -128, 5, -5, 10, -10, 60, -60], dtype=np.int8).view(np.uint8)
    block[208:210] = half_bytes(0.125)
    return block


# (sub-block j, lane l) -> 0.5 * sc_j * code - 0.25 * m_j.
Q4_K_EXPECTED = {
    (0, 0): 0.0,      # code 0
    (3, 2): 15.75,    # code 1: 31.5 - 15.75
    (5, 7): -0.25,    # code 0: 0 - 0.25 * 1
    (7, 31): 53.25,   # code 2: 62 - 8.75
    (4, 10): 107.0,   # code 14: 119 - 12
    (6, 1): 242.5,    # code 15: 247.5 - 5
    (1, 9): 12.75,    # code 14: 14 - 1.25
}

# i -> 0.125 * scale[i / 16] * (7 i % 64 - 32).
Q6_K_EXPECTED = {
    0: -4.0,       # q 0, scale 1
    37: -7.25,     # q 3, scale 2
    100: 14.0,     # q 60, scale 4
    130: -285.75,  # q 14, scale 127
    150: 96.0,     # q 26, scale -128
    200: 30.0,     # q 56, scale 10
    255: -187.5,   # q 57, scale -60
    70: 3.75,      # q 42 (490 = 7 * 64 + 42), scale 3
}


def test_q4_k_known_answers():
    values = dequantize_q4_k(q4_k_block(), 256).reshape(8, 32)
    for (j, lane), expected in Q4_K_EXPECTED.items():
        assert values[j, lane] == np.float32(expected), (j, lane, values[j, lane], expected)


def test_q6_k_known_answers():
    values = dequantize_q6_k(q6_k_block(), 256).reshape(256)
    for i, expected in Q6_K_EXPECTED.items():
        assert values[i] == np.float32(expected), (i, values[i], expected)


def test_rows_of_several_blocks_decode_block_by_block():
    """Rows are super-blocks in order: a 2 x 512 matrix of four distinct blocks decodes each in its place."""
    blocks = [q4_k_block(), q4_k_block(), q4_k_block(), q4_k_block()]
    for index, block in enumerate(blocks):
        block[0:2] = half_bytes(0.5 * (index + 1))
    values = dequantize_q4_k(np.concatenate(blocks), 512).reshape(2, 2, 8, 32)
    single = dequantize_q4_k(q4_k_block(), 256).reshape(8, 32)
    offsets = np.array([0.0, 1.25, 2.5, 15.75, 12.0, 0.25, 5.0, 8.75], dtype=np.float32)[:, None]
    for index in range(4):
        scaled = (single + offsets) * (index + 1) - offsets  # d grows, dmin stays
        assert np.allclose(values[index // 2, index % 2], scaled, rtol=1e-6, atol=1e-5)


@pytest.mark.parametrize("encoding,quantize,budget", [(12, quantize_q4_k, 0.6), (14, quantize_q6_k, 0.55)])
def test_encode_decode_round_trip_stays_within_the_step(encoding, quantize, budget):
    """TinyKQuantEncoder restated: every value decodes within about half its block's step (round to nearest; a few
    values near the clamped ends within a step), and the whole matrix within a few percent RMS."""
    rng = np.random.default_rng(encoding)
    x = rng.standard_normal((6, 512)).astype(np.float32)
    x[0, :256] = 0.0  # an all-zero super-block: d = 0, every value 0
    blocks = quantize(x)
    assert blocks.nbytes == matrix_bytes(encoding, 6, 512)
    decoded = dequantize(encoding, blocks, 512)
    assert np.all(decoded[0, :256] == 0)
    group = 32 if encoding == 12 else 16
    span = x.reshape(-1, group)
    steps = (span.max(axis=1) - np.minimum(span.min(axis=1), 0)) / 15 if encoding == 12 else np.abs(span).max(axis=1) / 31
    error = np.abs(decoded - x).reshape(-1, group)
    assert np.all(error <= np.maximum(budget * 2 * steps[:, None], 1e-6))
    assert np.sqrt(np.mean((decoded - x) ** 2)) <= 0.05 * np.sqrt(np.mean(x ** 2)) * (4 if encoding == 12 else 1)


@pytest.mark.parametrize("embedding,output", [(12, 14), (14, 12), (12, 12)])
def test_oracle_decodes_k_quant_tables_as_numpy(embedding, output):
    """The C restatement's embedding lookup and logits projection on K-quant tables: with every layer matrix zero
    and no biases the residual stream is the embedding row, so logits = W_out (x / sqrt(mean(x^2) + eps) * w)."""
    shape = DecoderShape(layers=1, hidden=256, feed_forward=256, heads=4, kv_heads=1, head_dim=64, vocabulary=40,
                         context=64, session_slots=1, step_tokens=4, logits_rows=4, growth=64)
    choose = {"token_embd": embedding, "output": output}
    blob, layout = synthetic_model(shape, seed=2, biases=False, encodings=lambda name: choose.get(name, q4_k_m(name)))
    layer = layout["layers"][0]
    encodings = int(layer["encodings"])
    for index, (name, rows, columns) in enumerate((("query", 256, 256), ("key", 64, 256), ("value", 64, 256),
                                                    ("attention_output", 256, 256), ("gate", 256, 256),
                                                    ("up", 256, 256), ("down", 256, 256))):
        size = matrix_bytes((encodings >> (4 * index)) & 0xF, rows, columns)
        blob[layer[name]:layer[name] + size] = 0
    cos = np.ones((64, 32), dtype=np.float32)
    sin = np.zeros((64, 32), dtype=np.float32)
    logits = DecoderOracle(blob, layout, shape, cos, sin).forward([(0, 17, 0, 0), (0, 3, 1, 1)])
    table = dequantize(embedding, blob[layout["token_embedding"]:layout["token_embedding"] +
                                       matrix_bytes(embedding, 40, 256)], 256)
    weights = dequantize(output, blob[layout["output"]:layout["output"] + matrix_bytes(output, 40, 256)], 256)
    w = blob[layout["output_norm"]:layout["output_norm"] + 1024].view(np.float32).astype(np.float64)
    for row, token in enumerate((17, 3)):
        x = table[token].astype(np.float64)
        expected = weights.astype(np.float64) @ (x / np.sqrt(np.mean(x * x) + shape.rms_epsilon) * w)
        assert np.allclose(logits[row], expected, rtol=1e-5, atol=1e-5 * np.abs(expected).max())
