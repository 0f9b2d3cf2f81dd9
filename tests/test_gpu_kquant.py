"""K-quant (Q4_K / Q6_K) projections and decoder steps on the GPU through the C ABI.

Projections: against an FP64 product with the exactly decoded weights (projection.dequantize; the decoders are
pinned by tests/test_oracle_kquant.py). Bar: |gpu - fp64| <= 2^-18 * sum_k (|scale * q| + |offset|) * |x_k|
(+ |bias|, + |old output| when accumulating): the kernels multiply codes by a split of x on the matrix cores
(prompt runs: three bf16 parts, exact; decode: two FP16 parts of x scaled per token, x to 2^-22) and apply each block's FP32 factors to its sum, as the reference's factored form
scale * dot(q, x) - offset * sum(x) does (matmul_kquant.metal:115-119), in another FP32 order. A wrong nibble, a
swapped half-block scale or a dropped offset moves outputs by far more (about 1e-2 of that sum).

Decoder steps: the Q4_K_M mix (Q4_K, with Q6_K for V, down and output) against the CPU restatement, at the
reference's GPU bar (max |gpu - oracle| <= 0.002 x the oracle's logits range).
"""

import sys

import numpy as np
import pytest

from oracle_ffi import DecoderOracle
from synapse_amd.decoder import Decoder, DecoderShape
from synthetic_models import q4_k_m, synthetic_model
from synapse_amd.projection import Q8Weights
from ggml_blocks import dequantize, quantize

pytestmark = pytest.mark.gpu

TOLERANCE = 2.0 ** -18


def say(*parts):
    print(*parts, flush=True)
    sys.stdout.flush()


def factor_magnitude(encoding, blocks, columns):
    """|scale * q| + |offset| per weight: Q4_K's two terms decoded apart (dmin zeroed, then d zeroed); the other
    encodings are a single product."""
    if encoding != 12:
        return np.abs(dequantize(encoding, blocks, columns).astype(np.float64))
    b = blocks.reshape(-1, 144).copy()
    scaled = b.copy()
    scaled[:, 2:4] = 0
    offsets = b.copy()
    offsets[:, 0:2] = 0
    return (np.abs(dequantize(12, scaled, columns).astype(np.float64)) +
            np.abs(dequantize(12, offsets, columns).astype(np.float64)))


def build_blob(rng, specs):
    """specs: [(rows, columns, encoding, with_bias)] -> blob, matrices, (dense FP64 weights, per-weight magnitudes),
    biases."""
    parts, matrices, dense, biases = [], [], [], []
    offset = 0
    for rows, columns, encoding, with_bias in specs:
        values = rng.standard_normal((rows, columns)).astype(np.float32) * np.float32(0.03)
        values[:, :32] += np.float32(0.02)  # an off-centre block: Q4_K minima are non-zero
        q = quantize(encoding, values)
        dense.append((dequantize(encoding, q, columns).astype(np.float64), factor_magnitude(encoding, q, columns)))
        entry = {"weight": offset, "rows": rows, "columns": columns, "encoding": encoding}
        parts.append(q.reshape(-1))
        offset += q.nbytes
        pad = (-offset) % 4
        parts.append(np.zeros(pad, dtype=np.uint8))
        offset += pad
        bias = None
        if with_bias:
            bias = rng.standard_normal(rows).astype(np.float32) * np.float32(0.1)
            entry["bias"] = offset
            parts.append(bias.view(np.uint8))
            offset += bias.nbytes
        biases.append(bias)
        matrices.append(entry)
    return np.concatenate(parts), matrices, dense, biases


def check(torch, weights, dense, biases, segments, x, out_width, accumulate):
    tokens = x.shape[0]
    rng = np.random.default_rng(tokens)
    initial = rng.standard_normal((tokens, out_width)).astype(np.float32) if accumulate else \
        np.zeros((tokens, out_width), dtype=np.float32)
    device_x = torch.from_numpy(x).cuda()
    device_out = torch.from_numpy(initial.copy()).cuda()
    weights.project(segments, device_x, device_out, accumulate=accumulate)
    torch.cuda.synchronize()
    got = device_out.cpu().numpy().astype(np.float64)
    expected = initial.astype(np.float64).copy()
    magnitude = np.zeros_like(expected)
    x64 = x.astype(np.float64)
    for m, column in segments:
        w, size = dense[m]
        rows = w.shape[0]
        product = x64 @ w.T + (0 if biases[m] is None else biases[m].astype(np.float64))
        base = expected[:, column:column + rows] if accumulate else 0
        expected[:, column:column + rows] = base + product
        magnitude[:, column:column + rows] = (np.abs(x64) @ size.T + np.abs(expected[:, column:column + rows])
                                              + (0 if biases[m] is None else np.abs(biases[m])))
    error = np.abs(got - expected)
    bound = TOLERANCE * magnitude + 1e-30
    assert np.all(error <= bound), (float((error / np.maximum(magnitude, 1e-30)).max()), segments, tokens)
    written = np.zeros(out_width, dtype=bool)
    for m, column in segments:
        written[column:column + dense[m][0].shape[0]] = True
    assert np.array_equal(got[:, ~written], initial[:, ~written].astype(np.float64))


SPECS = {
    # name: ([(rows, columns, encoding, bias)], segments as (matrix, first column), output width)
    "q4_k qkv": ([(512, 1024, 12, True), (128, 1024, 12, True), (128, 1024, 12, True)],
                 [(0, 0), (1, 512), (2, 640)], 768),
    "q4_k_m qkv (mixed)": ([(512, 1024, 12, True), (128, 1024, 12, True), (128, 1024, 14, True)],
                           [(0, 0), (1, 512), (2, 640)], 768),
    "q6_k down": ([(256, 2816, 14, False)], [(0, 0)], 256),
    "q8 + q4_k + q6_k": ([(40, 512, 8, False), (37, 512, 12, True), (19, 512, 14, False)],
                         [(2, 0), (0, 19), (1, 59)], 100),
}


@pytest.mark.parametrize("name", list(SPECS))
@pytest.mark.parametrize("tokens", [1, 5, 16, 17, 100])
def test_kquant_projection_matches_fp64(torch_gpu, name, tokens):
    torch = torch_gpu
    say("kquant projection", name, tokens)
    specs, segments, width = SPECS[name]
    rng = np.random.default_rng(tokens + len(name))
    blob, matrices, dense, biases = build_blob(rng, specs)
    weights = Q8Weights(blob, matrices)
    x = rng.standard_normal((tokens, specs[0][1])).astype(np.float32)
    x[:, 100] = 0.0
    x[0, 200] = 3e-7  # small values split into exact bf16 parts
    check(torch, weights, dense, biases, segments, x, width, accumulate=False)
    check(torch, weights, dense, biases, segments, x, width, accumulate=True)
    weights.close()


@pytest.mark.parametrize("encoding", [12, 14])
def test_kquant_prompt_run_at_full_size_on_sampled_tokens(torch_gpu, encoding):
    """A 7B-wide K-quant matrix (4,608 x 3,584) over a 512-token prompt chunk: 36 x 16 GEMM workgroups; 40 sampled
    tokens against the FP64 product of the exactly decoded weights."""
    torch = torch_gpu
    say("kquant prompt run, full size", encoding)
    rng = np.random.default_rng(encoding * 7 + 512)
    blob, matrices, dense, biases = build_blob(rng, [(4608, 3584, encoding, True)])
    weights = Q8Weights(blob, matrices)
    tokens = 512
    x = rng.standard_normal((tokens, 3584)).astype(np.float32)
    device_x = torch.from_numpy(x).cuda()
    device_out = torch.zeros((tokens, 4608), device="cuda")
    weights.project([(0, 0)], device_x, device_out)
    torch.cuda.synchronize()
    got = device_out.cpu().numpy().astype(np.float64)
    assert np.all(np.isfinite(got))
    sample = sorted({0, 31, 32, 511} | set(int(t) for t in rng.choice(tokens, size=36, replace=False)))
    w, size = dense[0]
    x64 = x[sample].astype(np.float64)
    expected = x64 @ w.T + biases[0].astype(np.float64)
    magnitude = np.abs(x64) @ size.T + np.abs(biases[0])
    error = np.abs(got[sample] - expected)
    assert np.all(error <= TOLERANCE * magnitude + 1e-30), float((error / np.maximum(magnitude, 1e-30)).max())
    weights.close()


def test_kquant_weights_read_back_is_unavailable(torch_gpu):
    from synapse_amd.native import NotSupportedError

    say("kquant read-back")
    rng = np.random.default_rng(1)
    blob, matrices, _, _ = build_blob(rng, [(16, 256, 12, False), (16, 256, 8, False)])
    weights = Q8Weights(blob, matrices)
    with pytest.raises(NotSupportedError, match="K-quant"):
        weights.read(0)
    assert weights.read(1).shape == (16, 256 // 32 * 34)
    weights.close()


SHAPES = [
    ("q4_k_m f16", DecoderShape(layers=2, hidden=1024, feed_forward=2816, heads=8, kv_heads=2, head_dim=128,
                                vocabulary=1000, context=1024, session_slots=3, step_tokens=256, logits_rows=8,
                                growth=256, kv_precision="f16"), q4_k_m),
    ("all q6_k f32", DecoderShape(layers=2, hidden=512, feed_forward=1024, heads=8, kv_heads=2, head_dim=64,
                                  vocabulary=300, context=512, session_slots=3, step_tokens=128, logits_rows=8,
                                  growth=256), lambda name: 14),
]


@pytest.mark.parametrize("name,shape,encodings", SHAPES)
def test_kquant_decoder_matches_the_restatement(torch_gpu, name, shape, encodings):
    from synapse_amd.kv_cache import rope_table

    say("kquant decoder", name)
    rng = np.random.default_rng(len(name))
    blob, layout = synthetic_model(shape, seed=len(name), encodings=encodings)
    gpu = Decoder(blob, layout, shape)
    cos, sin = rope_table(shape.head_dim, shape.theta, shape.context)
    oracle = DecoderOracle(blob, layout, shape, cos, sin, page_tokens=256)
    vocab = shape.vocabulary
    prompt = [(0, int(rng.integers(vocab)), p, 0 if p == 39 else -1) for p in range(40)]
    batches = [prompt, [(1, int(rng.integers(vocab)), p, 0 if p == 20 else -1) for p in range(21)]]
    positions = {0: 40, 1: 21}
    for _ in range(3):
        batches.append([(slot, int(rng.integers(vocab)), positions[slot] + 0, row)
                        for row, slot in enumerate((0, 1))])
        positions = {slot: value + 1 for slot, value in positions.items()}
    for index, tokens in enumerate(batches):
        got = gpu.forward(tokens)
        expected = oracle.forward(tokens)
        bar = 0.002 * (expected.max() - expected.min())
        error = np.abs(got - expected).max()
        assert error <= bar, (name, index, float(error), float(bar))
    gpu.close()


@pytest.mark.parametrize("columns", [512, 1280, 1024])
def test_prompt_first_call_on_fresh_weights(torch_gpu, columns):
    """The first prompt run on newly created weights (cold memory: slow loads), for column counts whose last round
    of the GEMM's three-chunk ring holds two chunks (512, 1,280) or one (1,024): the call must equal the next one
    bit for bit and the FP64 product, on several fresh objects. Q4_K, Q4_K and Q6_K segments (two launches) over
    57 tokens (a padded last token tile)."""
    torch = torch_gpu
    say("kquant first call", columns)
    specs = [(512, columns, 12, True), (128, columns, 12, True), (128, columns, 14, True)]
    segments = [(0, 0), (1, 512), (2, 640)]
    tokens, width = 57, 768
    rng = np.random.default_rng(columns)
    blob, matrices, dense, biases = build_blob(rng, specs)
    x = rng.standard_normal((tokens, columns)).astype(np.float32)
    device_x = torch.from_numpy(x).cuda()
    for trial in range(6):
        weights = Q8Weights(blob, matrices)
        first = torch.zeros((tokens, width), device="cuda")
        second = torch.zeros((tokens, width), device="cuda")
        weights.project(segments, device_x, first)
        weights.project(segments, device_x, second)
        torch.cuda.synchronize()
        assert torch.equal(first.view(torch.int32), second.view(torch.int32)), trial
        weights.close()
    weights = Q8Weights(blob, matrices)
    check(torch, weights, dense, biases, segments, x, width, accumulate=False)
    weights.close()
