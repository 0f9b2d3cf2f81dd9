"""Pins the oracle's restatement of query-aware KV page activation (ADR-016): the seeded generator of the random
control, the key bound, the selection rule, the decode-unit rule and masked attention.

Anchors: known outputs of .NET's System.Random for seeds 0 and 42 (the generator lives in the .NET runtime, not in
the reference tree); the reference's own selector tests (KvPageActivationTests.cs:14-95) restated on inputs of the
same construction; closed forms (a one-channel bound is the exact maximum score; a page of equal keys bounds at
the exact dot product); the FP64 attention of test_oracle_attention under the same masks.
"""

import math

import numpy as np
import pytest

from oracle_ffi import PagedCache, dotnet_random, page_bound, page_select, rope_table


def test_dotnet_random_known_answers():
    # new Random(0).Next() x 10, new Random(42).Next() x 5, new Random(0).Next(100) x 5.
    assert dotnet_random(0, 10).tolist() == [1559595546, 1755192844, 1649316166, 1198642031, 442452829,
                                             1200195957, 1945678308, 949569752, 2099272109, 587775847]
    assert dotnet_random(42, 5).tolist() == [1434747710, 302596119, 269548474, 1122627734, 361709742]
    assert dotnet_random(0, 5, 0, 100).tolist() == [72, 81, 76, 55, 20]


def test_dotnet_random_ranges_and_negative_seeds():
    draws = dotnet_random(-7, 2000, 3, 10)
    assert draws.min() == 3 and draws.max() == 9
    # Random(seed) seeds with |seed|.
    assert np.array_equal(dotnet_random(-12345, 20), dotnet_random(12345, 20))
    assert not np.array_equal(dotnet_random(1, 20), dotnet_random(2, 20))


def values(rng, count, scale=1.0):
    return ((rng.random(count) * 2 - 1) * scale).astype(np.float32)


def test_key_bound_never_underestimates_a_page_score():
    # KeyBoundNeverUnderestimatesAPageScore (KvPageActivationTests.cs:14-36).
    rng = np.random.default_rng(5)
    dimension = 64
    keys = values(rng, 640 * dimension).reshape(640, dimension)
    queries = values(rng, 3 * dimension).reshape(3, dimension)
    for page in range(10):
        bound = page_bound(queries, 3, dimension, keys, page * 64, page * 64 + 63)
        exact = (queries.astype(np.float64) @ keys[page * 64:page * 64 + 64].T.astype(np.float64)).max()
        assert bound >= exact - 1e-4


def test_key_bound_closed_forms():
    rng = np.random.default_rng(6)
    # One channel: sum_c max(q*min, q*max) is max over the page's keys of q * k, exactly (both one rounding).
    keys = values(rng, 128).reshape(128, 1)
    for q in (np.float32(0.75), np.float32(-1.25), np.float32(0.0)):
        bound = page_bound(np.array([q]), 1, 1, keys, 64, 127)
        assert bound == float((q * keys[64:128, 0]).max())
    # A page of identical keys: the bound is the sequential dot product of each head, maximised over heads.
    dimension = 32
    key = values(rng, dimension)
    keys = np.tile(key, (64, 1))
    queries = values(rng, 2 * dimension).reshape(2, dimension)
    expected = []
    for head in range(2):
        total = np.float32(0)
        for channel in range(dimension):
            total = np.float32(total + np.float32(queries[head, channel] * key[channel]))
        expected.append(total)
    assert page_bound(queries, 2, dimension, keys, 0, 63) == float(max(expected))
    # The bound of a page is the maximum over heads: adding a head can only raise it.
    wider = np.concatenate([queries, values(rng, dimension)[None]], axis=0)
    assert page_bound(wider, 3, dimension, keys, 0, 63) >= page_bound(queries, 2, dimension, keys, 0, 63)


def pages_of(selected, size=64):
    return sorted({index // size for index in np.flatnonzero(selected)})


def test_selection_keeps_sink_window_and_the_best_page():
    # SelectionKeepsSinkWindowAndTheBestPage (KvPageActivationTests.cs:38-54).
    rng = np.random.default_rng(7)
    dimension = 64
    keys = values(rng, 640 * dimension, 0.01).reshape(640, dimension)
    query = values(rng, dimension)
    keys[5 * 64:6 * 64] = query
    selected = page_select(1, 64, query, 1, dimension, keys, 639)
    assert pages_of(selected) == [0, 5, 9]
    assert selected[0:64].all() and selected[320:384].all() and selected[576:640].all()


def test_smaller_pages_select_at_their_own_granularity():
    # SmallerPagesSelectAtTheirOwnGranularity (KvPageActivationTests.cs:56-76).
    rng = np.random.default_rng(8)
    dimension = 64
    keys = values(rng, 640 * dimension, 0.01).reshape(640, dimension)
    query = values(rng, dimension)
    keys[208:224] = query
    selected = page_select(1, 64, query, 1, dimension, keys, 639, page_tokens=16)
    expected = list(range(0, 16)) + list(range(208, 224)) + list(range(576, 640))
    assert np.flatnonzero(selected).tolist() == expected


def test_random_control_selects_the_budget_deterministically():
    # RandomControlSelectsTheBudgetDeterministically (KvPageActivationTests.cs:78-95).
    dimension = 64
    keys = values(np.random.default_rng(9), 1280 * dimension).reshape(1280, dimension)
    query = values(np.random.default_rng(10), dimension)
    first = page_select(3, 64, query, 1, dimension, keys, 1279, seed=42, random=True)
    again = page_select(3, 64, query, 1, dimension, keys, 1279, seed=42, random=True)
    assert np.array_equal(first, again)
    assert len(pages_of(first)) == 1 + 3 + 1
    assert 0 in pages_of(first) and 19 in pages_of(first)
    # The draw is the first three entries of a partial Fisher-Yates shuffle of pages 1..18 under Random(42).
    pages = list(range(1, 19))
    generator = iter(dotnet_random(42, 3, 0, 0))  # raw samples; Next(i, 18) = i + trunc(sample / (2^31-1) * (18-i))
    for index in range(3):
        sample = next(generator)
        swap = index + int(sample * (1.0 / 2147483647) * (18 - index))
        pages[index], pages[swap] = pages[swap], pages[index]
    assert pages_of(first) == sorted([0, 19] + pages[:3])


@pytest.mark.parametrize("budget,window,position", [(64, 64, 999), (13, 64, 999), (0, 1000, 999), (5, 0, 383),
                                                    (2, 128, 100)])
def test_covering_budget_selects_every_position(budget, window, position):
    """The exactness boundary (ADR-016): budget * 64 + window + 64 covering the prefix selects all of it."""
    rng = np.random.default_rng(budget + window)
    keys = values(rng, (position + 1) * 16).reshape(position + 1, 16)
    query = values(rng, 16)
    selected = page_select(budget, window, query, 1, 16, keys, position)
    count = position + 1
    window_page = max(0, count - window) // 64
    covering = max(0, window_page - 1) <= budget
    assert selected.all() == covering
    if not covering:
        assert len(pages_of(selected)) == 1 + budget + (position // 64 - window_page + 1)


def test_window_zero_can_rank_the_page_being_completed():
    """With no window a full last page is a candidate: position 383 (page 5 just filled) ranks pages 1..5."""
    rng = np.random.default_rng(12)
    keys = values(rng, 384 * 8, 0.01).reshape(384, 8)
    query = values(rng, 8)
    keys[320:384] = query
    selected = page_select(1, 0, query, 1, 8, keys, 383)
    assert pages_of(selected) == [0, 5]


def fp64_masked(query, keys, values_, heads, kv_heads, head_dim, position, masks):
    q = query.reshape(heads, head_dim).astype(np.float64)
    group = heads // kv_heads
    out = np.zeros((heads, head_dim))
    for head in range(heads):
        kv = head // group
        scores = keys[: position + 1, kv].astype(np.float64) @ q[head] / math.sqrt(head_dim)
        scores = np.where(masks[kv][: position + 1], scores, -np.inf)
        weights = np.exp(scores - scores.max())
        out[head] = weights @ values_[: position + 1, kv].astype(np.float64) / weights.sum()
    return out.reshape(-1)


@pytest.mark.parametrize("selection", [0, 1])
def test_paged_attention_masks_decode_units_only(selection):
    """Qwen2KvPageMasks.Prepare + Qwen2CpuAttention.Attend: decode units (before the prompt boundary, alone in their
    slot) get their selection; others stay dense. Masked outputs equal FP64 attention under the same masks."""
    heads, kv_heads, head_dim, maximum = 4, 2, 16, 1024
    cache = PagedCache(1, heads, kv_heads, head_dim, maximum, 256, 64, 0, 4, 64, 512)
    cos, sin = rope_table(head_dim, 1e6, maximum)
    rng = np.random.default_rng(20 + selection)
    width = (heads + 2 * kv_heads) * head_dim
    # Prefill 700 positions of slots 0 and 1, 300 of slot 2.
    for slot, length in ((0, 700), (1, 700), (2, 300)):
        for first in range(0, length, 256):
            tokens = [(slot, p) for p in range(first, min(length, first + 256))]
            assert cache.step(tokens) == 0
            assert cache.append_rope(0, rng.standard_normal((len(tokens), width)).astype(np.float32), cos, sin) == 0
    # Slot 0: a lone decode token; slot 1: two tokens (not units); slot 2: lone but past the prompt boundary.
    tokens = [(0, 700), (1, 700), (1, 701), (2, 300)]
    assert cache.step(tokens) == 0
    rows = rng.standard_normal((4, width)).astype(np.float32)
    assert cache.append_rope(0, rows, cos, sin) == 0
    out = np.zeros((4, heads * head_dim), dtype=np.float32)
    activation = (2, 64, 64, selection, 3)
    masks = cache.attention(0, rows, out, activation=activation, prompt_start=3, maximum=maximum)
    assert masks[1:].sum() == 0
    for kv in range(kv_heads):
        assert len(pages_of(masks[0, kv, :701])) == 1 + 2 + 2  # 701 - 64 = 637 -> window pages 9, 10
    keys, values_ = cache.gather(0, 0, 0, 701)
    expected = fp64_masked(rows[0, :heads * head_dim], keys, values_, heads, kv_heads, head_dim, 700, masks[0])
    assert np.allclose(out[0], expected, atol=1e-5, rtol=1e-4)
    dense = np.zeros_like(out)
    cache.attention(0, rows, dense)
    assert np.array_equal(out[1:], dense[1:])
    assert not np.allclose(out[0], dense[0], atol=1e-3)
