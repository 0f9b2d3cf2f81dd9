"""Pins the oracle's RoPE and attention restatements against closed forms, the reference's own known coordinates
and independent FP64 computations (numpy), so that a dropped term, a wrong index or a transposed operand fails."""

import math

import numpy as np
import pytest

from oracle_ffi import ORACLE, attention, ptr, rope_apply, rope_table

THETA = 1_000_000.0


def fp64_reference(query, keys, values, heads, kv_heads, head_dim, position, valid=None):
    """numpy FP64 causal GQA attention, written independently of the oracle (vectorised)."""
    q = query.reshape(heads, head_dim).astype(np.float64)
    k = keys[: position + 1].astype(np.float64)
    v = values[: position + 1].astype(np.float64)
    scale = 1.0 / math.sqrt(head_dim)
    group = heads // kv_heads
    out = np.zeros((heads, head_dim))
    for head in range(heads):
        scores = k[:, head // group, :] @ q[head] * scale
        if valid is not None:
            scores = np.where(valid[: position + 1], scores, -np.inf)
        weights = np.exp(scores - scores.max())
        out[head] = weights @ v[:, head // group, :] / weights.sum()
    return out.reshape(-1)


def test_causal_mask_prevents_future_leak_known_coordinates():
    # ReferenceOperatorsTests.cs:61-93: one KV head, head dim 2, two query heads, query position 1, scale 1.
    query = np.array([1, 0, 0, 1], dtype=np.float32)
    keys = np.array([1, 0, 0, 1, 0.5, 0.5], dtype=np.float32)
    values = np.array([10, 20, 30, 40, 50, 60], dtype=np.float32)
    valid = np.ones(3, dtype=np.uint8)
    before = np.zeros(4, dtype=np.float32)
    assert ORACLE.orc_attention_fp64(ptr(query), ptr(keys), ptr(values), ptr(valid), 2, 1, 2, 1, 1.0, ptr(before)) == 0
    keys[4], keys[5], values[4], values[5] = np.nan, 1000.0, np.nan, -1e6
    after = np.zeros(4, dtype=np.float32)
    assert ORACLE.orc_attention_fp64(ptr(query), ptr(keys), ptr(values), ptr(valid), 2, 1, 2, 1, 1.0, ptr(after)) == 0
    assert np.array_equal(before, after)
    first = math.exp(1) / (math.exp(1) + 1)
    assert abs(before[0] - (first * 10 + (1 - first) * 30)) <= 1e-5 + 1e-4 * 30
    assert abs(before[2] - ((1 - first) * 10 + first * 30)) <= 1e-5 + 1e-4 * 30


def test_all_masked_row_is_an_error_and_leaves_output():
    # ReferenceOperatorsTests.cs:96-117.
    query = np.array([1, 0], dtype=np.float32)
    keys = np.array([1, 0, 0, 1], dtype=np.float32)
    values = np.array([10, 20, 30, 40], dtype=np.float32)
    valid = np.zeros(2, dtype=np.uint8)
    output = np.array([42, 43], dtype=np.float32)
    assert ORACLE.orc_attention_fp64(ptr(query), ptr(keys), ptr(values), ptr(valid), 1, 1, 2, 1, 1.0, ptr(output)) == 8
    assert output.tolist() == [42, 43]


def random_case(seed, positions, heads, kv_heads, head_dim):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(heads * head_dim).astype(np.float32)
    k = rng.standard_normal((positions, kv_heads, head_dim)).astype(np.float32)
    v = rng.standard_normal((positions, kv_heads, head_dim)).astype(np.float32)
    return q, k, v


@pytest.mark.parametrize("heads,kv_heads,head_dim,position", [(14, 2, 64, 0), (14, 2, 64, 300), (28, 4, 128, 1000),
                                                               (4, 4, 64, 37)])
@pytest.mark.parametrize("kind", ["scalar", "managed", "fp64"])
def test_restatements_match_independent_fp64(kind, heads, kv_heads, head_dim, position):
    q, k, v = random_case(position + head_dim, position + 1, heads, kv_heads, head_dim)
    expected = fp64_reference(q, k, v, heads, kv_heads, head_dim, position)
    got = attention(kind, q, k, v, heads, kv_heads, head_dim, position)
    tolerance = 1e-6 if kind == "fp64" else 2e-5
    assert np.max(np.abs(got - expected)) <= tolerance


def test_gqa_head_mapping_uses_head_over_group():
    # Changing KV head 1 must change only query heads 7..13 (kvh = head / group, Qwen2Attention.cs:12).
    q, k, v = random_case(3, 50, 14, 2, 64)
    base = attention("scalar", q, k, v, 14, 2, 64, 49)
    v2 = v.copy()
    v2[:, 1, :] += 1.0
    moved = attention("scalar", q, k, v2, 14, 2, 64, 49).reshape(14, 64)
    base = base.reshape(14, 64)
    assert np.array_equal(moved[:7], base[:7])
    assert np.allclose(moved[7:], base[7:] + 1.0, atol=1e-5)


def test_identical_keys_average_the_values():
    q, k, v = random_case(5, 64, 2, 1, 64)
    k[:] = k[0]
    expected = v[:, 0, :].astype(np.float64).mean(axis=0)
    got = attention("managed", q, k, v, 2, 1, 64, 63).reshape(2, 64)
    assert np.allclose(got[0], expected, atol=1e-5) and np.allclose(got[1], expected, atol=1e-5)


def test_dominant_key_selects_its_value():
    q, k, v = random_case(9, 20, 1, 1, 64)
    q[:] = 0
    q[0] = 100.0
    k[:] = 0
    k[13, 0, 0] = 100.0  # score 100 * 100 / 8 dominates every other key
    got = attention("scalar", q, k, v, 1, 1, 64, 19)
    assert np.allclose(got, v[13, 0], atol=1e-6)


def test_position_limits_the_keys():
    q, k, v = random_case(11, 10, 2, 1, 64)
    k2, v2 = k.copy(), v.copy()
    k2[6:], v2[6:] = 1e3, -1e3  # beyond position 5
    assert np.array_equal(attention("scalar", q, k, v, 2, 1, 64, 5), attention("scalar", q, k2, v2, 2, 1, 64, 5))


@pytest.mark.parametrize("split_keys", [1, 7, 64, 1000])
def test_split_merge_tracks_the_unsplit_result(split_keys):
    # One split = many splits within tolerance (MetalFp16KvSplitDecodeTracksPromptRun, MetalKvPrecisionTests.cs:35-46).
    q, k, v = random_case(13, 777, 14, 2, 64)
    expected = fp64_reference(q, k, v, 14, 2, 64, 776)
    got = attention("split", q, k, v, 14, 2, 64, 776, split_keys=split_keys)
    assert np.max(np.abs(got - expected)) <= 2e-5


def test_rope_table_closed_forms():
    cos, sin = rope_table(64, THETA, 8)
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    # Pair 0 rotates by exactly `position` radians.
    assert np.allclose(cos[1:, 0], np.cos(np.arange(1, 8)), atol=1e-7)
    positions = np.array([1, 17, 4095, 32767], dtype=np.float64)
    cos, sin = rope_table(64, THETA, 32768)
    index = np.arange(32)
    angle = positions[:, None] / THETA ** (2.0 * index / 64)
    # FP32 angle rounding grows with the angle: 8 |angle| 2^-23 + 2e-6 as RopeFrequenciesTests.cs:52-54.
    tolerance = 8 * np.abs(angle) * 2.0**-23 + 2e-6
    rows = positions.astype(int)
    assert np.all(np.abs(cos[rows] - np.cos(angle)) <= tolerance)
    assert np.all(np.abs(sin[rows] - np.sin(angle)) <= tolerance)


def test_yarn_table_matches_fp64_formula():
    # RopeFrequenciesTests.cs:37-76 (factor 4, original context 32,768, head dim 64, theta 1e6).
    factor, original = 4.0, 32768
    positions = [0, 1, 17, 4095, 32767, 65536, 131071]
    cos, sin = rope_table(64, THETA, 131072, factor, original)
    worst = 0.0
    for position in positions:
        for index in range(32):
            extrapolated = position / THETA ** (2.0 * index / 64)
            interpolated = extrapolated / factor

            def correction(rotations):
                return 64 * math.log(original / (rotations * 2 * math.pi)) / (2 * math.log(THETA))

            low = max(0.0, math.floor(correction(32)))
            high = min(63.0, math.ceil(correction(1)))
            ramp = 1 - min(max((index - low) / max(0.001, high - low), 0.0), 1.0)
            angle = interpolated * (1 - ramp) + extrapolated * ramp
            magnitude = 1 + 0.1 * math.log(factor)
            tolerance = 8 * abs(angle) * 2.0**-23 + 2e-6
            worst = max(worst, abs(cos[position, index] - math.cos(angle) * magnitude) / tolerance)
            worst = max(worst, abs(sin[position, index] - math.sin(angle) * magnitude) / tolerance)
    assert worst <= 1.0


def test_rope_rotation_special_cases_and_order():
    rng = np.random.default_rng(21)
    x = rng.standard_normal(3 * 64).astype(np.float32)
    ones, zeros = np.ones(32, np.float32), np.zeros(32, np.float32)
    assert np.array_equal(rope_apply(x, 3, 64, ones, zeros), x)  # angle 0: identity, bit for bit
    swapped = rope_apply(x, 3, 64, zeros, ones).reshape(3, 2, 32)
    original = x.reshape(3, 2, 32)
    assert np.array_equal(swapped[:, 0], -original[:, 1]) and np.array_equal(swapped[:, 1], original[:, 0])
    # Separate FP32 products and sums (no fused multiply-add): numpy float32 arithmetic gives the same bits.
    cos = rng.standard_normal(32).astype(np.float32)
    sin = rng.standard_normal(32).astype(np.float32)
    got = rope_apply(x, 3, 64, cos, sin).reshape(3, 2, 32)
    first, second = original[:, 0], original[:, 1]
    assert np.array_equal(got[:, 0], first * cos - second * sin)
    assert np.array_equal(got[:, 1], first * sin + second * cos)


def test_rope_preserves_norm_and_inverts():
    cos, sin = rope_table(128, THETA, 5000)
    rng = np.random.default_rng(4)
    x = rng.standard_normal(4 * 128).astype(np.float32)
    y = rope_apply(x, 4, 128, cos[4321], sin[4321])
    assert np.allclose(np.linalg.norm(y.reshape(4, 128), axis=1), np.linalg.norm(x.reshape(4, 128), axis=1), rtol=1e-5)
    back = rope_apply(y, 4, 128, cos[4321], -sin[4321])
    assert np.allclose(back, x, atol=1e-5)
