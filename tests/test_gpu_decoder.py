"""The decoder step on the GPU through the C ABI, against the CPU restatement (orc_decoder_*) on the same model
file and tokens.

Bar (the reference's Metal-vs-reference bar, MetalBackendTests.cs:60): max |gpu - oracle| <= 0.002 x the range of
the oracle's logits, per step. The GPU sums in other orders (MFMA projections over an FP16 or bf16 split of the inputs,
split-K attention); the oracle follows the reference kernels' FP32 order. Both KV precisions; FP16 KV rounds K and V
to nearest even on both sides.
"""

import sys

import numpy as np
import pytest

from oracle_ffi import DecoderOracle
from synapse_amd.decoder import Decoder, DecoderShape
from synthetic_models import synthetic_model

pytestmark = pytest.mark.gpu


def say(*parts):
    print(*parts, flush=True)
    sys.stdout.flush()


SHAPES = [
    ("tiny f32", DecoderShape(layers=2, hidden=128, feed_forward=256, heads=2, kv_heads=1, head_dim=64, vocabulary=96,
                              context=512, session_slots=3, step_tokens=64, logits_rows=8, growth=256)),
    ("gqa7 f16", DecoderShape(layers=2, hidden=896, feed_forward=1024, heads=14, kv_heads=2, head_dim=64,
                              vocabulary=512, context=1024, session_slots=3, step_tokens=256, logits_rows=8,
                              growth=256, kv_precision="f16")),
    ("d128 f16", DecoderShape(layers=2, hidden=1024, feed_forward=2816, heads=8, kv_heads=2, head_dim=128,
                              vocabulary=1000, context=1024, session_slots=3, step_tokens=256, logits_rows=8,
                              growth=256, kv_precision="f16")),
    ("d128 f32 no-bias", DecoderShape(layers=3, hidden=512, feed_forward=1024, heads=4, kv_heads=4, head_dim=128,
                                      vocabulary=300, context=512, session_slots=3, step_tokens=128, logits_rows=8,
                                      growth=256)),
    # hidden 4,608: the norm kernels' 1,024 threads hold a second, partly filled float4 group of the row.
    ("wide f16", DecoderShape(layers=1, hidden=4608, feed_forward=1024, heads=36, kv_heads=6, head_dim=128,
                              vocabulary=256, context=512, session_slots=3, step_tokens=128, logits_rows=8,
                              growth=256, kv_precision="f16")),
]


def steps(rng, shape):
    """A prompt run per slot (logits on the last token), then ragged decode steps, one token without logits."""
    vocab = shape.vocabulary
    prompt = [(0, int(rng.integers(vocab)), p, -1) for p in range(40)] + \
             [(1, int(rng.integers(vocab)), p, -1) for p in range(17)]
    prompt[39] = prompt[39][:3] + (0,)
    prompt[56] = prompt[56][:3] + (1,)
    out = [prompt, [(2, int(rng.integers(vocab)), p, 0 if p == 8 else -1) for p in range(9)]]
    positions = {0: 40, 1: 17, 2: 9}
    for step in range(6):
        tokens = []
        for slot in ((0, 1, 2) if step % 2 == 0 else (2, 0)):
            tokens.append((slot, int(rng.integers(vocab)), positions[slot], len(tokens)))
            positions[slot] += 1
        if step == 3:
            tokens.append((1, int(rng.integers(vocab)), positions[1], -1))
            positions[1] += 1
        out.append(tokens)
    return out


@pytest.mark.parametrize("name,shape", SHAPES)
def test_decoder_matches_the_restatement(torch_gpu, name, shape):
    from synapse_amd.kv_cache import rope_table

    say("decoder", name)
    rng = np.random.default_rng(len(name))
    blob, layout = synthetic_model(shape, seed=len(name), biases="no-bias" not in name)
    gpu = Decoder(blob, layout, shape)
    cos, sin = rope_table(shape.head_dim, shape.theta, shape.context)
    oracle = DecoderOracle(blob, layout, shape, cos, sin, page_tokens=256)
    for index, tokens in enumerate(steps(rng, shape)):
        got = gpu.forward(tokens)
        expected = oracle.forward(tokens)
        assert got.shape == expected.shape
        bar = 0.002 * (expected.max() - expected.min())
        error = np.abs(got - expected).max()
        assert error <= bar, (name, index, float(error), float(bar))
    assert gpu.kv_bytes > 0
    gpu.close()


def test_decoder_errors_and_reserve(torch_gpu):
    from synapse_amd import InvalidOperationError

    say("decoder errors")
    shape = SHAPES[0][1]
    blob, layout = synthetic_model(shape, seed=3)
    gpu = Decoder(blob, layout, shape)
    with pytest.raises(InvalidOperationError, match="0..k-1"):
        gpu.forward([(0, 1, 0, 1)])
    with pytest.raises(InvalidOperationError, match="invalid batch token"):
        gpu.forward([(0, shape.vocabulary, 0, 0)])
    with pytest.raises(InvalidOperationError, match="invalid batch token"):
        gpu.forward([(shape.session_slots, 1, 0, 0)])
    with pytest.raises(InvalidOperationError, match="1..64"):
        gpu.forward([(0, 1, p, -1) for p in range(65)])
    before = gpu.kv_bytes
    gpu.reserve(1, 300)
    assert gpu.kv_bytes > before
    # A failed step leaves the model usable.
    logits = gpu.forward([(0, 1, 0, 0), (1, 2, 0, 1)])
    assert logits.shape == (2, shape.vocabulary) and np.isfinite(logits).all()
    gpu.close()


def test_decoder_with_page_activation_runs_and_differs(torch_gpu):
    """KV page activation on the model's cache: decode units attend their selected pages (parity of the selection
    itself is tests/test_gpu_pages.py); with a covering budget the logits equal dense ones (1e-5 of the range: the
    dense step may take the fused append + decode launch, the activated one does not)."""
    say("decoder page activation")
    shape = DecoderShape(layers=2, hidden=256, feed_forward=512, heads=4, kv_heads=2, head_dim=64, vocabulary=200,
                         context=2048, session_slots=2, step_tokens=512, logits_rows=4, growth=256,
                         kv_precision="f16")
    blob, layout = synthetic_model(shape, seed=5)
    rng = np.random.default_rng(5)
    prompt = [(0, int(rng.integers(200)), p, -1) for p in range(1500)]
    results = []
    for budget in (None, 64, 2):
        gpu = Decoder(blob, layout, shape)
        for first in range(0, 1500, 500):
            gpu.forward(prompt[first:first + 500])
        if budget is not None:
            gpu.set_page_activation(budget, 64)
        results.append(np.concatenate([gpu.forward([(0, 7 + i, 1500 + i, 0)]) for i in range(3)]))
        gpu.close()
    spread = results[0].max() - results[0].min()
    assert np.abs(results[0] - results[1]).max() <= 1e-5 * spread
    assert np.abs(results[0] - results[2]).max() > 1e-3 * spread


def test_decoder_through_the_libsynapse_gpu_abi(torch_gpu):
    """The reference loader's calls (synapse_gpu_probe / _decoder_create with backend 3 / _forward / _reserve /
    _kv_bytes / _destroy) drive the same model: logits bit-identical to synapse_kv_decoder_* on the same steps."""
    import ctypes

    from synapse_amd.native import DeviceInfo, NativeKvLibrary

    say("decoder via synapse_gpu ABI")
    library = NativeKvLibrary.load()
    info = DeviceInfo()
    library.check(library.g_probe(3, ctypes.byref(info)))
    shape = SHAPES[1][1]
    blob, layout = synthetic_model(shape, seed=11)
    native_abi = Decoder(blob, layout, shape)
    gpu_abi = Decoder(blob, layout, shape, abi="gpu")
    rng = np.random.default_rng(11)
    for tokens in steps(rng, shape)[:4]:
        assert np.array_equal(native_abi.forward(tokens), gpu_abi.forward(tokens))
    library.check(library.g_decoder_reserve(gpu_abi.handle, 2, 700))
    assert library.g_decoder_kv_bytes(gpu_abi.handle) == library.c_decoder_kv_bytes(gpu_abi.handle)
    assert library.g_decoder_kv_bytes(gpu_abi.handle) > native_abi.kv_bytes
    native_abi.close()
    gpu_abi.close()


@pytest.mark.parametrize("encodings,hidden,feed_forward", [(None, 512, 1024), ("q4_k_m", 512, 1024), (None, 4608, 1024),
                                                          (None, 512, 1056)])
def test_fused_slice_sums_are_bit_identical_to_separate_reduces(torch_gpu, encodings, hidden, feed_forward):
    """Decode steps add the o_proj and gate/up slice sums inside the feed-forward norm and SwiGLU kernels, and
    prompt steps (more than 16 tokens) have the norms and SwiGLU write the next projection's split input; with
    SYNAPSE_KV_OPTION_FUSED_SUMS = 0 they run as separate reduce launches and FP32 rows through split_kernel. The
    arithmetic is the same and in the same order, so the logits are bit-identical. A feed-forward width of 1,056
    (33 blocks of 32) leaves the down projection's split input a zero-padded last 64-column chunk."""
    from synthetic_models import q4_k_m
    from synapse_amd.native import OPTION_FUSED_SUMS

    say("decoder fused sums", encodings, hidden, feed_forward)
    shape = DecoderShape(layers=2, hidden=hidden, feed_forward=feed_forward, heads=hidden // 64,
                         kv_heads=2 if hidden == 512 else 9, head_dim=64, vocabulary=300, context=512,
                         session_slots=3, step_tokens=128, logits_rows=8, growth=256, kv_precision="f16")
    blob, layout = synthetic_model(shape, seed=13, encodings=q4_k_m if encodings else None)
    fused = Decoder(blob, layout, shape)
    separate = Decoder(blob, layout, shape)
    separate.set_option(OPTION_FUSED_SUMS, 0)
    rng = np.random.default_rng(13)
    for tokens in steps(rng, shape):
        assert np.array_equal(fused.forward(tokens).view(np.uint32), separate.forward(tokens).view(np.uint32))
    fused.close()
    separate.close()
