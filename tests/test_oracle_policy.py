"""Known-answer tests the reference holds for the KV capacity policy, the dense cache, the attention schedule and
prompt prefix reuse, transcribed against the oracle restatement."""

import numpy as np
import pytest

from oracle_ffi import DenseCache, Prefix, plan_attention, ORACLE


def next_capacity(needed, current, growth=1024, maximum=4096):
    return ORACLE.orc_next_capacity(needed, current, growth, maximum)


def test_kv_capacity_grows_by_unit_and_doubling_up_to_the_context():
    # decoder_tests.rs:235-250 (context 4096, growth 1024).
    assert next_capacity(1, 0) == 1024
    assert next_capacity(1025, 1024) == 2048
    assert next_capacity(3001, 1024) == 3072
    assert next_capacity(3500, 3072) == 4096


def test_kv_bytes_per_position_closed_forms():
    # DynamicKvCapacityTests.cs:57-58: 0.5B FP32 = 24 layers * 2 KV heads * 64 dims * 2 (K, V) * 4 bytes.
    assert 2 * 24 * 2 * 64 * 4 == 24_576
    # decoder_tests.rs:212-233 / 235-250: one layer, one KV head, head dim 64 FP32 -> 2 * 64 * 4; FP16 halves it.
    assert 2 * 1 * 1 * 64 * 4 == 512


def test_kv_cache_keeps_heads_separate_and_rejects_out_of_range_positions():
    # KvCacheParityTests.cs:72-85.
    cache = DenseCache(layers=2, maximum=3, kv_width=8, growth=1024)
    key = np.arange(8, dtype=np.float32)
    value = np.arange(10, 18, dtype=np.float32)
    assert cache.store(1, 2, key, value) == 0
    assert cache.get(1, 2, 1, 4)[1].tolist() == [4, 5, 6, 7]
    assert cache.get(1, 2, 0, 4, value=True)[1].tolist() == [10, 11, 12, 13]
    assert np.all(cache.get(0, 2, 0, 4)[1] == 0)
    assert cache.store(1, 3, key, value) != 0
    assert cache.store(0, 0, key[:4], value) != 0


def test_cpu_kv_cache_grows_and_keeps_contents():
    # DynamicKvCapacityTests.cs:16-34.
    cache = DenseCache(layers=2, maximum=8192, kv_width=4, growth=1024)
    key = np.array([1, 2, 3, 4], dtype=np.float32)
    value = np.array([5, 6, 7, 8], dtype=np.float32)
    cache.store(1, 5, key, value)
    first = cache.allocated
    for position in range(1500):
        cache.store(0, position, [position, 0, 0, 0], [0, 0, 0, position])
    assert first == 1024
    assert cache.allocated == 2048
    assert cache.get(1, 5, 0, 4)[1].tolist() == key.tolist()
    assert cache.get(1, 5, 0, 4, value=True)[1].tolist() == value.tolist()
    assert cache.get(0, 1499, 0, 4)[1][0] == 1499
    assert cache.store(0, 8192, key, value) != 0


def bits(values):
    return np.asarray(values, dtype=np.float32).view(np.uint32).tolist()


def test_cpu_reservation_contracts_at_fourfold_boundary_and_keeps_prefix_bits():
    # DynamicKvContractionTests.cs:16-36.
    cache = DenseCache(layers=2, maximum=512, kv_width=4, growth=64)
    key = np.array([1.25, -2.5, np.float32(1.4e-45), -0.0], dtype=np.float32)
    value = np.array([3.75, -4.5, -np.float32(1.4e-45), 0.0], dtype=np.float32)
    cache.reserve(512)
    cache.store(1, 127, key, value)
    cache.reserve(129)
    assert cache.allocated == 512
    cache.reserve(128)
    assert cache.allocated == 128
    assert bits(cache.get(1, 127, 0, 4)[1]) == bits(key)
    assert bits(cache.get(1, 127, 0, 4, value=True)[1]) == bits(value)
    cache.reserve(65)
    assert cache.allocated == 128


@pytest.mark.parametrize("positions", [-1, 513])
def test_reservation_rejects_bounds_outside_instance_context(positions):
    # DynamicKvContractionTests.cs:38-48.
    cache = DenseCache(layers=1, maximum=512, kv_width=4, growth=64)
    assert cache.reserve(positions) != 0


def test_kv_bytes_follow_the_context_in_use():
    # DynamicKvCapacityTests.cs:60-79 as an allocator scenario: 100 sequential positions -> 1,024; 1,500 -> 2,048.
    cache = DenseCache(layers=24, maximum=32768, kv_width=2 * 64, growth=1024)
    row = np.zeros(128, dtype=np.float32)
    for position in range(100):
        for layer in range(24):
            cache.store(layer, position, row, row)
    assert cache.allocated_bytes == 1024 * 24_576
    cache.release()
    for position in range(1500):
        cache.store(0, position, row, row)
    assert cache.allocated_bytes == 2048 * 24_576


def test_generate_reserves_prompt_and_output_once():
    # DynamicKvCapacityTests.cs:81-99: Reserve(1,500 + 600) allocates 3,072 positions once.
    cache = DenseCache(layers=24, maximum=8192, kv_width=128, growth=1024)
    cache.reserve(2100)
    assert cache.allocated_bytes == 3072 * 24_576


def token_rows(pairs):
    return np.array([[slot, 1, position, -1] for slot, position in pairs], dtype=np.int32)


def test_prompt_runs_split_into_eight_token_blocks_per_kv_head():
    # schedule_tests.rs:14-42.
    blocks, summary = plan_attention(token_rows([(0, p) for p in range(20)]), 2, 8)
    assert summary["run_blocks"] == 6 and summary["single_blocks"] == 0 and summary["splits"] == 1
    assert [tuple(b[:3]) for b in blocks] == [(0, 8, 0), (0, 8, 1), (8, 8, 0), (8, 8, 1), (16, 4, 0), (16, 4, 1)]
    assert all(b[3] == 0 for b in blocks)
    assert blocks[5][5] == 20


def test_decode_tokens_become_single_blocks_after_prompt_runs():
    # schedule_tests.rs:44-67.
    blocks, summary = plan_attention(token_rows([(1, 40), (2, 7), (3, 0), (3, 1), (3, 2)]), 2, 8)
    assert summary["run_blocks"] == 2 and summary["single_blocks"] == 4
    assert blocks[0][0] == 2 and blocks[0][5] == 3
    assert [(b[0], b[4], b[5], b[3]) for b in blocks[2:]] == [(0, 1, 41, 1), (0, 1, 41, 1), (1, 2, 8, 1), (1, 2, 8, 1)]


def test_non_consecutive_positions_break_a_run():
    # schedule_tests.rs:69-77.
    blocks, summary = plan_attention(token_rows([(0, 0), (0, 1), (0, 5), (0, 6)]), 1, 8)
    assert summary["run_blocks"] == 2
    assert blocks[1][0] == 2 and blocks[1][5] == 7


def test_long_decode_contexts_split_within_the_partial_buffer():
    # schedule_tests.rs:79-95.
    _, one = plan_attention(token_rows([(0, 32767)]), 2, 8)
    _, crowded = plan_attention(token_rows([(slot, 131071) for slot in range(64)]), 2, 8)
    _, short = plan_attention(token_rows([(0, 3)]), 2, 8)
    assert one["splits"] > 1
    assert one["split_keys"] % 32 == 0
    assert one["split_keys"] * one["splits"] >= 32768
    assert one["single_blocks"] * one["splits"] <= 512
    assert crowded["single_blocks"] * crowded["splits"] <= 512
    assert crowded["split_keys"] * crowded["splits"] >= 131072
    assert short["splits"] == 1 and short["split_keys"] >= 4


def test_run_block_size_is_a_parameter():
    # schedule_tests.rs:97-110.
    blocks, _ = plan_attention(token_rows([(0, p) for p in range(40)]), 2, 16)
    assert [(b[0], b[1], b[5]) for b in blocks if b[2] == 0] == [(0, 16, 16), (16, 16, 32), (32, 8, 40)]


DOCUMENT = [(index * 7919 % 150_000) + 100 for index in range(700)]
QUESTION = [785, 6722, 315, 9625, 374]


def test_reused_prefix_counts():
    # PromptPrefixReuseTests.cs:17-30 and :48-60 (claim counts; generation is out of scope here).
    prefix = Prefix(enabled=True)
    assert prefix.claim(DOCUMENT) == 0
    prefix.remember(DOCUMENT, [11, 12, 13, 14])
    assert prefix.claim(DOCUMENT + QUESTION) == len(DOCUMENT)
    cold = Prefix(enabled=False)
    cold.remember(DOCUMENT, [1, 2])
    assert cold.claim(DOCUMENT + QUESTION) == 0


def test_identical_prompt_reevaluates_only_its_last_token_and_other_work_invalidates():
    # PromptPrefixReuseTests.cs:48-60.
    prefix = Prefix(enabled=True)
    prefix.claim(DOCUMENT)
    prefix.remember(DOCUMENT, [5, 6])
    assert prefix.claim(DOCUMENT) == len(DOCUMENT) - 1
    prefix.clear()  # any other direct use of the slot
    assert prefix.claim(DOCUMENT) == 0


def test_failed_request_keeps_only_the_prefix_it_did_not_overwrite():
    # PromptPrefixReuseTests.cs:62-76: the claim forgets everything after the shared 300 before writing.
    prefix = Prefix(enabled=True)
    prefix.remember(DOCUMENT, [1, 2])
    diverging = DOCUMENT[:300] + QUESTION + QUESTION
    assert prefix.claim(diverging) == 300
    # The request fails before Remember: the next claim finds only the 300 untouched tokens.
    assert prefix.claim(DOCUMENT) == 300
