"""Q8_0 projections on the GPU through the C ABI, against the FP64 restatement on the same seeded inputs.

Bar: |gpu - fp64| <= 2^-18 * sum_k |d * code * x| (+ |bias|, + |old output| when accumulating) per element: FP32
summation in another order of products that are exact (prompt runs: three bf16 parts of x) or within 2^-22 of
exact (decode: two FP16 parts of x scaled per token); the reference's own FP32 matrix-vector order stays within
2^-20 of the anchor, tests/test_oracle_projection.py. A dropped or mis-scaled 32-column block moves an output by
about 1e-3 of that sum at these widths. Weights read back from the device are bit-exact with the uploaded blocks.
"""

import sys

import numpy as np
import pytest

from oracle_ffi import q8_project
from synapse_amd.projection import Q8Weights
from ggml_blocks import quantize_q8_0

pytestmark = pytest.mark.gpu

TOLERANCE = 2.0 ** -18


def say(*parts):
    print(*parts, flush=True)
    sys.stdout.flush()


def build_blob(rng, shapes, bias_flags, scale=0.03):
    """A blob holding Q8_0 matrices (and FP32 biases) at 4-byte aligned offsets, like a mapped model file."""
    parts, matrices, blocks, biases = [], [], [], []
    offset = 0
    for (rows, columns), with_bias in zip(shapes, bias_flags):
        q = quantize_q8_0(rng.standard_normal((rows, columns)).astype(np.float32) * np.float32(scale))
        blocks.append(q)
        entry = {"weight": offset, "rows": rows, "columns": columns}
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
    return np.concatenate(parts), matrices, blocks, biases


def check(torch, weights, blocks, biases, segments, x, out_width, accumulate, initial=None):
    tokens = x.shape[0]
    out = np.zeros((tokens, out_width), dtype=np.float32) if initial is None else initial.copy()
    device_x = torch.from_numpy(x).cuda()
    device_out = torch.from_numpy(out.copy()).cuda()
    weights.project(segments, device_x, device_out, accumulate=accumulate)
    torch.cuda.synchronize()
    got = device_out.cpu().numpy()
    expected = out.copy()
    magnitude = q8_project([(blocks[m], biases[m], column) for m, column in segments], x, expected,
                           accumulate=accumulate, exact=True)
    error = np.abs(got.astype(np.float64) - expected.astype(np.float64))
    bound = TOLERANCE * magnitude + 1e-30
    assert np.all(error <= bound), (float((error / np.maximum(magnitude, 1e-30)).max()), segments, tokens)
    # Columns no segment writes keep their values.
    written = np.zeros(out_width, dtype=bool)
    for m, column in segments:
        written[column:column + blocks[m].shape[0]] = True
    assert np.array_equal(got[:, ~written], out[:, ~written])
    return got


SHAPES = [
    # (name, [(rows, columns) per matrix], bias per matrix)
    ("0.5B qkv", [(896, 896), (128, 896), (128, 896)], [True, True, True]),
    ("7B qkv", [(3584, 3584), (512, 3584), (512, 3584)], [True, True, True]),
    ("odd", [(37, 96), (5, 96)], [False, True]),
]


@pytest.mark.parametrize("name,shapes,bias_flags", SHAPES)
@pytest.mark.parametrize("tokens", [1, 3, 16, 17, 100])
def test_projection_matches_the_restatement(torch_gpu, name, shapes, bias_flags, tokens):
    say("projection", name, tokens)
    rng = np.random.default_rng(len(name) * 100 + tokens)
    blob, matrices, blocks, biases = build_blob(rng, shapes, bias_flags)
    weights = Q8Weights(blob, matrices)
    weights.set_stream(torch_gpu.cuda.current_stream())
    columns = shapes[0][1]
    x = rng.standard_normal((tokens, columns)).astype(np.float32)
    rows = [shape[0] for shape in shapes]
    segments = [(m, sum(rows[:m])) for m in range(len(shapes))]
    check(torch_gpu, weights, blocks, biases, segments, x, sum(rows), accumulate=False)
    weights.close()


def test_o_proj_accumulates_into_the_residual_with_strides(torch_gpu):
    say("o_proj accumulate")
    torch = torch_gpu
    rng = np.random.default_rng(11)
    blob, matrices, blocks, biases = build_blob(rng, [(3584, 3584)], [False])
    weights = Q8Weights(blob, matrices)
    weights.set_stream(torch.cuda.current_stream())
    for tokens in (1, 16, 40):
        # Inputs with a wider row stride than the matrix, outputs into a wider residual row at column 8.
        wide = rng.standard_normal((tokens, 3584 + 64)).astype(np.float32)
        residual = rng.standard_normal((tokens, 3600)).astype(np.float32)
        device_x = torch.from_numpy(wide).cuda()
        device_out = torch.from_numpy(residual.copy()).cuda()
        weights.project([(0, 8)], device_x, device_out, in_stride=3584 + 64, out_stride=3600, accumulate=True)
        weights.project([(0, 8)], device_x, device_out, in_stride=3584 + 64, out_stride=3600, accumulate=True)
        torch.cuda.synchronize()
        got = device_out.cpu().numpy()
        expected = residual.copy()
        x = np.ascontiguousarray(wide[:, :3584])
        once = q8_project([(blocks[0], None, 8)], x, expected, accumulate=True, exact=True)
        twice = q8_project([(blocks[0], None, 8)], x, expected, accumulate=True, exact=True)
        error = np.abs(got.astype(np.float64) - expected)
        assert np.all(error <= TOLERANCE * (once + twice) + 1e-30), float(error.max())
        assert np.array_equal(got[:, :8], residual[:, :8]) and np.array_equal(got[:, 8 + 3584:], residual[:, 8 + 3584:])
    weights.close()


@pytest.mark.parametrize("tokens", [2048, 512])
def test_prompt_run_at_full_size_on_sampled_tokens(torch_gpu, tokens):
    """The 7B QKV (4,608 x 3,584, biases) over a prompt chunk of 2,048 tokens (128-row x 64-token workgroup
    tiles) and of 512 tokens (128 x 32: the larger tile would not give two workgroups per CU). Every token is
    computed on the GPU; 64 sampled tokens (the first, the last, both sides of workgroup edges, and random ones)
    are checked against the FP64 restatement, and the unsampled rows must be finite."""
    say("prompt run, full size", tokens)
    torch = torch_gpu
    rng = np.random.default_rng(tokens)
    shapes = [(3584, 3584), (512, 3584), (512, 3584)]
    blob, matrices, blocks, biases = build_blob(rng, shapes, [True, True, True])
    weights = Q8Weights(blob, matrices)
    weights.set_stream(torch.cuda.current_stream())
    x = rng.standard_normal((tokens, 3584)).astype(np.float32)
    device_x = torch.from_numpy(x).cuda()
    device_out = torch.zeros((tokens, 4608), device="cuda")
    segments = [(0, 0), (1, 3584), (2, 4096)]
    weights.project(segments, device_x, device_out)
    torch.cuda.synchronize()
    got = device_out.cpu().numpy()
    assert np.all(np.isfinite(got))
    sample = sorted({t for t in (0, 1, 31, 32, 33, 63, 64, 1023, 1024, 2015, 2016, 2047) if t < tokens} |
                    {tokens - 1} | set(int(t) for t in rng.choice(tokens, size=52, replace=False)))
    expected = np.zeros((len(sample), 4608), dtype=np.float32)
    magnitude = q8_project([(blocks[m], biases[m], column) for m, column in segments], x[sample], expected,
                           exact=True)
    error = np.abs(got[sample].astype(np.float64) - expected.astype(np.float64))
    assert np.all(error <= TOLERANCE * magnitude + 1e-30), float((error / np.maximum(magnitude, 1e-30)).max())
    weights.close()


def test_prompt_rows_do_not_depend_on_the_batch(torch_gpu):
    """The prompt kernel's workgroup tile depends on the launch (token count, matrix size), but every tile runs the
    same per-chunk multiplies in the same order: a token's outputs are bit-identical whether it is projected in a
    2,048-token batch (128 x 64 tiles), a 512-token batch (128 x 32) or a 40-token batch (64 x 32)."""
    say("prompt batch invariance")
    torch = torch_gpu
    rng = np.random.default_rng(4040)
    blob, matrices, blocks, biases = build_blob(rng, [(3584, 3584), (512, 3584), (512, 3584)], [True, True, True])
    weights = Q8Weights(blob, matrices)
    weights.set_stream(torch.cuda.current_stream())
    x = torch.from_numpy(rng.standard_normal((2048, 3584)).astype(np.float32)).cuda()
    segments = [(0, 0), (1, 3584), (2, 4096)]
    results = {}
    for tokens in (2048, 512, 40):
        out = torch.zeros((tokens, 4608), device="cuda")
        weights.project(segments, x[:tokens].contiguous(), out)
        torch.cuda.synchronize()
        results[tokens] = out.cpu().numpy()
    assert np.array_equal(results[2048][:512].view(np.uint32), results[512].view(np.uint32))
    assert np.array_equal(results[2048][:40].view(np.uint32), results[40].view(np.uint32))
    weights.close()


def test_weights_read_back_bit_exact_and_errors(torch_gpu):
    from synapse_amd import InvalidOperationError

    say("weights read back")
    torch = torch_gpu
    rng = np.random.default_rng(5)
    blob, matrices, blocks, _ = build_blob(rng, [(37, 96), (20, 64)], [True, False])
    weights = Q8Weights(blob, matrices)
    for index in range(2):
        assert np.array_equal(weights.read(index), blocks[index])
    x = torch.zeros((2, 96), device="cuda")
    out = torch.zeros((2, 64), device="cuda")
    with pytest.raises(InvalidOperationError, match="equal column counts"):
        weights.project([(0, 0), (1, 37)], x, out)
    with pytest.raises(InvalidOperationError, match="out_stride"):
        weights.project([(0, 40)], x, out)
    with pytest.raises(InvalidOperationError, match="device memory"):
        weights.project([(0, 0)], np.zeros((2, 96), dtype=np.float32).ctypes.data, out, tokens=2, in_stride=96)
    weights.close()


@pytest.mark.parametrize("columns", [192, 256, 320])
def test_prompt_first_call_on_fresh_weights(torch_gpu, columns):
    """The first prompt run on newly created Q8_0 weights (cold memory: slow loads), for column counts of 3, 4 and 5
    64-column chunks, so that the GEMM's three-chunk ring ends on a full round, one chunk or two: its first tail
    chunk waits only for the copies the last full step (or the prologue) issued. The first call must equal the next
    bit for bit, on several fresh objects, and the restatement's product."""
    torch = torch_gpu
    say("q8 first call", columns)
    shapes = [(512, columns), (128, columns), (128, columns)]
    tokens = 57
    rng = np.random.default_rng(columns)
    blob, matrices, blocks, biases = build_blob(rng, shapes, [True, False, True])
    segments = [(0, 0), (1, 512), (2, 640)]
    x = rng.standard_normal((tokens, columns)).astype(np.float32)
    device_x = torch.from_numpy(x).cuda()
    for trial in range(6):
        weights = Q8Weights(blob, matrices)
        first = torch.zeros((tokens, 768), device="cuda")
        second = torch.zeros((tokens, 768), device="cuda")
        weights.project(segments, device_x, first)
        weights.project(segments, device_x, second)
        torch.cuda.synchronize()
        assert torch.equal(first.view(torch.int32), second.view(torch.int32)), trial
        weights.close()
    weights = Q8Weights(blob, matrices)
    check(torch, weights, blocks, biases, segments, x, 768, accumulate=False)
    weights.close()
