"""Attention with scaled values on the GPU (7B shape: 28 query heads, 4 KV heads, head_dim 128, FP16 pages)
against the restatement's FP32-accumulate attention (Qwen2CpuAttention order).

The output is a weighted mean of value rows. Weights perturbed by a relative e (a probability rounded to FP16:
e up to 2^-11) move it by about e * |v_i - mean|, so the error of an inexact probability grows with the spread of
V and is largest where few keys carry the weight: the first positions of a fresh prompt, and queries scaled up.
Each case scales V (and Q) by fixed factors; the cached K/V are written through the append path with the same
scale, so the pages hold the scaled values. Inputs are seeded; the scales are fixed.
"""

import numpy as np
import pytest

from test_gpu_peaked import ATOL, RTOL, expected_rows, say, seven_b

pytestmark = pytest.mark.gpu

SEED = 20261213
# (query scale, value scale)
CASES = ((1.0, 1.0), (1.0, 4.0), (1.0, 8.0), (4.0, 4.0), (8.0, 8.0))


def scaled_rows(cache, rng, count, q_scale, v_scale):
    heads_width = cache.heads * cache.head_dim
    kv_width = cache.kv_heads * cache.head_dim
    rows = rng.standard_normal((count, cache.qkv_width)).astype(np.float32)
    rows[:, :heads_width] *= np.float32(q_scale)
    rows[:, heads_width + kv_width:] *= np.float32(v_scale)
    return rows


def run(cache, torch, tokens, rows):
    cache.step(tokens)
    qkv = torch.from_numpy(rows).cuda()
    out = torch.empty((len(tokens), cache.heads * cache.head_dim), device="cuda")
    cache.append_attention(0, qkv, out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def measure(got, expected, label):
    error = np.abs(got - expected)
    ratio = float((error / (ATOL + RTOL * np.abs(expected))).max())
    say(f"{label}: max abs error {float(error.max()):.3e}, worst fraction of the bound {ratio:.3f}")
    return ratio


def test_fresh_prompt_with_scaled_values(torch_gpu):
    """A 256-token prompt from position 0 (MFMA prefill kernel, causal): position p attends p + 1 keys, so the
    first rows put their whole weight on a handful of keys. Every row of the first 64 positions is checked."""
    torch = torch_gpu
    rng = np.random.default_rng(SEED)
    cache = seven_b(torch, 1024, 1, 8)
    tokens = [(0, p) for p in range(256)]
    sample = list(range(64)) + list(range(64, 256, 5)) + [255]
    worst = []
    for q_scale, v_scale in CASES:
        cache.truncate(0, 0)
        rows = scaled_rows(cache, rng, len(tokens), q_scale, v_scale)
        got = run(cache, torch, tokens, rows)[sample]
        expected = expected_rows(cache, rows[sample], [tokens[j] for j in sample])
        worst.append(measure(got, expected, f"fresh prompt q x{q_scale:g} v x{v_scale:g}"))
    cache.close()
    assert max(worst) <= 1.0, worst


def test_decode_at_short_positions_with_scaled_values(torch_gpu):
    """Single-token decode at positions 1-40 of 8 sequences (decode kernel) with scaled Q and V."""
    torch = torch_gpu
    rng = np.random.default_rng(SEED + 1)
    cache = seven_b(torch, 1024, 8, 8 * 4)
    worst = []
    for q_scale, v_scale in CASES:
        lengths = [int(x) for x in rng.integers(1, 41, size=8)]
        for slot, length in enumerate(lengths):
            cache.truncate(slot, 0)
            prompt = [(slot, p) for p in range(length)]
            run(cache, torch, prompt, scaled_rows(cache, rng, length, q_scale, v_scale))
        tokens = [(slot, length) for slot, length in enumerate(lengths)]
        rows = scaled_rows(cache, rng, len(tokens), q_scale, v_scale)
        got = run(cache, torch, tokens, rows)
        worst.append(measure(got, expected_rows(cache, rows, tokens), f"decode q x{q_scale:g} v x{v_scale:g}"))
    cache.close()
    assert max(worst) <= 1.0, worst


def test_shared_prefix_decode_with_scaled_values(torch_gpu):
    """C4's form at a smaller size: a 2,000-token prefix forked into 6 sequences that share its pages; their
    decode tokens read the shared pages through listed prefill items (MFMA kernel) and their own keys through the
    decode kernel, then merge."""
    torch = torch_gpu
    rng = np.random.default_rng(SEED + 2)
    worst = []
    for q_scale, v_scale in CASES:
        cache = seven_b(torch, 4096, 7, 7 * 16)
        prefix = 2000
        for start in range(0, prefix, 500):
            tokens = [(0, p) for p in range(start, start + 500)]
            run(cache, torch, tokens, scaled_rows(cache, rng, len(tokens), q_scale, v_scale))
        for target in range(1, 7):
            cache.fork(0, target)
        for step in range(3):
            tokens = [(slot, prefix + step) for slot in range(1, 7)]
            rows = scaled_rows(cache, rng, len(tokens), q_scale, v_scale)
            got = run(cache, torch, tokens, rows)
        worst.append(measure(got, expected_rows(cache, rows, tokens), f"shared prefix q x{q_scale:g} v x{v_scale:g}"))
        cache.close()
    assert max(worst) <= 1.0, worst


def test_prefill_over_a_long_cache_with_scaled_values(torch_gpu):
    """A 256-token chunk over 4,096 cached tokens whose values are scaled too: past the first keys most 64-key
    steps hold a small share of each row's weight, so an error of the probabilities would average over many keys
    here, unlike the fresh prompt above; both must meet the bar."""
    torch = torch_gpu
    rng = np.random.default_rng(SEED + 3)
    cached, chunk = 4096, 256
    tokens = [(0, cached + j) for j in range(chunk)]
    sample = list(range(0, chunk, 3)) + [chunk - 1]
    worst = []
    for q_scale, v_scale in CASES:
        cache = seven_b(torch, 8192, 1, 32)
        for start in range(0, cached, 1024):
            fill_tokens = [(0, p) for p in range(start, start + 1024)]
            run(cache, torch, fill_tokens, scaled_rows(cache, rng, len(fill_tokens), q_scale, v_scale))
        rows = scaled_rows(cache, rng, chunk, q_scale, v_scale)
        got = run(cache, torch, tokens, rows)[sample]
        expected = expected_rows(cache, rows[sample], [tokens[j] for j in sample])
        worst.append(measure(got, expected, f"long prefill q x{q_scale:g} v x{v_scale:g}"))
        cache.close()
    assert max(worst) <= 1.0, worst
