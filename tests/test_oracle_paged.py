"""The paged KV-cache restatement: hand-derived block tables, allocator invariants, and equivalence with the
dense Qwen2KvCache restatement (capacity policy and stored contents) under growth, contraction and release."""

import numpy as np
import pytest

from oracle_ffi import DenseCache, PagedCache, rope_table
from paged_checks import check_allocator_invariants


def small(precision=1, slots=3, max_pages=12, layers=1, maximum=512, growth=128, page=64, heads=2, kv_heads=1,
          head_dim=64, step_tokens=64):
    return PagedCache(layers, heads, kv_heads, head_dim, maximum, growth, page, precision, slots, max_pages,
                      step_tokens)


def tables(cache, slots):
    return [cache.table(slot) for slot in range(slots)]


def mapped(cache, slot):
    table = cache.table(slot)
    return table[table >= 0].tolist()


def test_hand_derived_block_tables():
    # Page 64, growth 128 (two pages), context 512, 12 pages; the free stack pops page 0 first.
    cache = small()
    assert cache.free_list().tolist() == list(range(11, -1, -1))
    assert cache.reserve(0, 100) == 0 and mapped(cache, 0) == [0, 1]
    assert cache.reserve(1, 1) == 0 and mapped(cache, 1) == [2, 3]
    assert cache.step([(0, 130)]) == 0  # NextCapacity(131, 128) = 256: pages 4 and 5
    assert mapped(cache, 0) == [0, 1, 4, 5] and cache.slot(0)["capacity"] == 256
    assert cache.reserve(0, 512) == 0 and mapped(cache, 0) == [0, 1, 4, 5, 6, 7, 8, 9]
    assert cache.free_list().tolist() == [11, 10]
    assert cache.reserve(0, 100) == 0  # rounded 128 <= 512 / 4: contract, pushing pages 9..4
    assert mapped(cache, 0) == [0, 1]
    assert cache.free_list().tolist() == [11, 10, 9, 8, 7, 6, 5, 4]
    assert cache.slot(0) == {"capacity": 128, "length": 128, "pages": 2}
    assert cache.fork(0, 2) == 0 and mapped(cache, 2) == [0, 1]
    assert cache.refcounts()[:2].tolist() == [2, 2]
    assert cache.step([(2, 128)]) == 0  # growth of slot 2 only: pages 4, 5
    assert mapped(cache, 2) == [0, 1, 4, 5]
    assert cache.step([(2, 127)]) == 0  # write into shared page 1: copy to page 6
    assert mapped(cache, 2) == [0, 6, 4, 5]
    assert cache.release(0) == 0  # page 1 drops to zero and is freed; page 0 stays with slot 2
    assert cache.free_list().tolist() == [11, 10, 9, 8, 7, 1]
    refs = cache.refcounts()
    assert refs.tolist() == [1, 0, 1, 1, 1, 1, 1, 0, 0, 0, 0, 0]
    check_allocator_invariants(tables(cache, 3), refs, cache.free_list(), 12)


def test_out_of_pages_leaves_everything_unchanged():
    cache = small(max_pages=4)
    assert cache.reserve(0, 128) == 0
    before = (tables(cache, 3), cache.refcounts().copy(), cache.free_list().copy())
    assert cache.reserve(1, 300) == 5  # needs 6 pages, 2 are free
    assert cache.step([(1, 0), (2, 200)]) == 5
    after = (tables(cache, 3), cache.refcounts(), cache.free_list())
    assert all(np.array_equal(a, b) for a, b in zip(before[0], after[0]))
    assert np.array_equal(before[1], after[1]) and np.array_equal(before[2], after[2])


def test_step_rejects_bad_tokens_before_any_change():
    cache = small()
    assert cache.step([(0, 512)]) == 2
    assert cache.step([(3, 0)]) == 2
    assert cache.step([(0, -1)]) == 2
    assert cache.free_list().size == 12


def test_cow_last_writer_keeps_the_page():
    cache = small(slots=4, max_pages=16)
    assert cache.step([(0, p) for p in range(60)]) == 0
    assert cache.fork(0, 1) == 0 and cache.fork(0, 2) == 0
    cache.release(0)
    shared = cache.table(1)[0]
    assert cache.refcounts()[shared] == 2
    # Slot 1 then slot 2 write into the shared page in one step: slot 1 copies, slot 2 keeps the original.
    assert cache.step([(1, 60), (2, 60)]) == 0
    assert cache.table(2)[0] == shared and cache.table(1)[0] != shared
    assert cache.refcounts()[shared] == 1


def test_fork_shares_only_written_pages_and_rejects_busy_targets():
    cache = small(slots=3)
    cache.reserve(0, 512)
    assert cache.step([(0, p) for p in range(0, 64)]) == 0
    assert cache.step([(0, 64)]) == 0
    assert cache.fork(0, 1) == 0
    assert mapped(cache, 1) == mapped(cache, 0)[:2]
    assert cache.slot(1) == {"capacity": 128, "length": 65, "pages": 2}
    assert cache.fork(0, 1) == 2 and cache.fork(0, 0) == 2
    assert cache.truncate(1, 66) == 2 and cache.truncate(1, 10) == 0


def random_rows(rng, count, heads, kv_heads, head_dim):
    return rng.standard_normal((count, (heads + 2 * kv_heads) * head_dim)).astype(np.float32)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_fp32_paged_cache_equals_dense_cache(seed):
    # The paged restatement stores exactly what Qwen2KvCache stores, with the same capacity policy.
    layers, heads, kv_heads, head_dim, maximum, growth, page = 2, 4, 2, 64, 1024, 128, 64
    rng = np.random.default_rng(seed)
    cos, sin = rope_table(head_dim, 1e6, maximum)
    paged = PagedCache(layers, heads, kv_heads, head_dim, maximum, growth, page, 0, 1, 64, 4)
    dense = DenseCache(layers, maximum, kv_heads * head_dim, growth)
    length = 0
    for _ in range(120):
        action = rng.random()
        if action < 0.75:
            position = int(min(maximum - 1, max(0, length + rng.integers(-3, 40))))
            assert paged.step([(0, position)]) == 0
            for layer in range(layers):
                rows = random_rows(rng, 1, heads, kv_heads, head_dim)
                assert paged.append_rope(layer, rows, cos, sin) == 0
                key = rows[0, heads * head_dim:(heads + kv_heads) * head_dim]
                value = rows[0, (heads + kv_heads) * head_dim:]
                assert dense.store(layer, position, key, value) == 0
            length = max(length, position + 1)
        elif action < 0.95:
            positions = int(rng.integers(0, maximum + 1))
            assert paged.reserve(0, positions) == 0 and dense.reserve(positions) == 0
            length = min(length, paged.slot(0)["capacity"])
        else:
            assert paged.release(0) == 0
            dense.release()
            length = 0
        assert paged.slot(0)["capacity"] == dense.allocated
        check_allocator_invariants([paged.table(0)], paged.refcounts(), paged.free_list(), 64)
    capacity = paged.slot(0)["capacity"]
    for layer in range(layers):
        keys, values = paged.gather(0, layer, 0, capacity)
        for position in range(capacity):
            for kv_head in range(kv_heads):
                status, key = dense.get(layer, position, kv_head, head_dim)
                assert status == 0
                assert np.array_equal(keys[position, kv_head].view(np.uint32), key.view(np.uint32))
                _, value = dense.get(layer, position, kv_head, head_dim, value=True)
                assert np.array_equal(values[position, kv_head].view(np.uint32), value.view(np.uint32))


def test_fp16_append_stores_rne_of_the_rotated_rows():
    from oracle_ffi import f32_to_f16, rope_apply

    heads, kv_heads, head_dim = 14, 2, 64
    cos, sin = rope_table(head_dim, 1e6, 600)
    cache = PagedCache(1, heads, kv_heads, head_dim, 600, 256, 256, 1, 1, 4, 8)
    rng = np.random.default_rng(8)
    rows = random_rows(rng, 3, heads, kv_heads, head_dim)
    original = rows.copy()
    positions = [0, 255, 256]
    for position, row in zip(positions, rows):
        assert cache.step([(0, position)]) == 0
        assert cache.append_rope(0, row[None, :].copy(), cos, sin) == 0
    for index, position in enumerate(positions):
        keys, values = cache.gather(0, 0, position, 1, raw=True)
        rotated = rope_apply(original[index, heads * head_dim:(heads + kv_heads) * head_dim], kv_heads, head_dim,
                             cos[position], sin[position])
        assert np.array_equal(keys.reshape(-1), f32_to_f16(rotated))
        assert np.array_equal(values.reshape(-1), f32_to_f16(original[index, (heads + kv_heads) * head_dim:]))


def test_long_then_short_contracts_to_the_reserved_pages():
    # Config 2 in miniature: fill 8 pages, decode past them, then Reserve(1,024 / 8) contracts to its rounded need.
    cache = small(precision=1, slots=1, max_pages=32, maximum=2048, growth=128, page=64)
    for chunk in range(8):
        assert cache.step([(0, p) for p in range(chunk * 64, chunk * 64 + 64)]) == 0
    assert cache.slot(0)["capacity"] == 512
    assert cache.step([(0, 512)]) == 0
    assert cache.slot(0)["capacity"] == 1024
    assert cache.reserve(0, 128) == 0
    assert cache.slot(0) == {"capacity": 128, "length": 128, "pages": 2}
    assert cache.free_list().size == 30
    assert cache.kv_bytes == 2 * 64 * 2 * 64 * 2
