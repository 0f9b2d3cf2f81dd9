"""The BASELINE.json configurations at their full sizes on the GPU, checked through size-independent properties
and against the restatement on read-back data.

At these sizes the oracle does not replay every append; instead: appended K/V bits are checked for sampled tokens
against the restatement's rotation + RNE of the same rows, attention is checked against the restatement's
FP32-accumulate attention (Qwen2CpuAttention order) run on the K/V read back from the pages, and page tables,
counts and contraction outcomes are checked exactly.
"""

import sys

import numpy as np
import pytest

from oracle_ffi import PagedCache, attention, f16_to_f32, f32_to_f16, rope_apply

pytestmark = pytest.mark.gpu

ATOL = 2e-3
RTOL = 1e-3
SEED = 20261201


def say(*parts):
    print(*parts, flush=True)
    sys.stdout.flush()


def widen(bits):
    return f16_to_f32(bits) if bits.dtype == np.uint16 else bits


_READ = {}


def read_back(cache, slot, layer, count):
    """K/V positions [0, count) of (slot, layer), widened; one read per (cache, slot, layer) and length."""
    key = (id(cache), slot, layer)
    held = _READ.get(key)
    if held is None or held[0].shape[0] < count:
        keys, values = cache.read_kv(slot, layer, 0, count)
        held = (widen(keys), widen(values))
        _READ.clear()
        _READ[key] = held
    return held[0][:count], held[1][:count]


def check_token(cache, qkv_row, slot, position, layer, got, rotated_q=True, upto=None):
    """Restatement attention for one token over its slot's read-back K/V."""
    heads, kv_heads, d = cache.heads, cache.kv_heads, cache.head_dim
    keys, values = read_back(cache, slot, layer, max(position + 1, upto or 0))
    keys, values = keys[: position + 1], values[: position + 1]
    q = np.ascontiguousarray(qkv_row[: heads * d], dtype=np.float32)
    if not rotated_q:
        q = rope_apply(q, heads, d, cache.rope_cosines[position], cache.rope_sines[position])
    expected = attention("managed", np.ascontiguousarray(q), np.ascontiguousarray(keys), np.ascontiguousarray(values),
                         heads, kv_heads, d, position)
    error = np.abs(got - expected)
    assert np.all(error <= ATOL + RTOL * np.abs(expected)), (slot, position, layer, float(error.max()))
    return float(error.max())


def check_appended(cache, qkv_row, slot, position, layer):
    """The stored K/V of `position` are RNE (FP16) or copies (FP32) of the rotated K and the V of the row."""
    heads, kv_heads, d = cache.heads, cache.kv_heads, cache.head_dim
    keys, values = cache.read_kv(slot, layer, position, 1)
    k = rope_apply(qkv_row[heads * d:(heads + kv_heads) * d], kv_heads, d, cache.rope_cosines[position],
                   cache.rope_sines[position])
    v = np.ascontiguousarray(qkv_row[(heads + kv_heads) * d:], dtype=np.float32)
    if keys.dtype == np.uint16:
        assert np.array_equal(keys.reshape(-1), f32_to_f16(k)) and np.array_equal(values.reshape(-1), f32_to_f16(v))
    else:
        assert np.array_equal(keys.reshape(-1).view(np.uint32), k.view(np.uint32))
        assert np.array_equal(values.reshape(-1).view(np.uint32), v.view(np.uint32))


def fill(cache, torch, slot, first, count, chunk, generator, layers):
    """Appends positions [first, first + count) of `slot` in prompt chunks of fresh N(0,1) rows."""
    buffer = torch.empty((chunk, cache.qkv_width), device="cuda")
    for start in range(first, first + count, chunk):
        size = min(chunk, first + count - start)
        cache.step([(slot, p) for p in range(start, start + size)])
        for layer in range(layers):
            rows = buffer[:size]
            rows.normal_(generator=generator)
            cache.append_rope(layer, rows)
    torch.cuda.synchronize()


def test_c1_fp32_decode_over_4096_cached_tokens(torch_gpu):
    # Config 1: 0.5B shape, FP32 KV, 4,096 cached tokens + 1 appended per layer (24 layers).
    from synapse_amd import PagedKvCache

    torch = torch_gpu
    say("C1")
    layers, heads, kv_heads, d = 24, 14, 2, 64
    cache = PagedKvCache(layers=layers, heads=heads, kv_heads=kv_heads, head_dim=d, max_positions=8192,
                         growth_positions=1024, page_tokens=256, precision="f32", session_slots=1,
                         step_tokens=512, max_pages=32)
    generator = torch.Generator(device="cuda")
    generator.manual_seed(SEED + 1)
    fill(cache, torch, 0, 0, 4096, 512, generator, layers)
    assert cache.slot_info(0) == {"capacity": 4096, "length": 4096, "pages": 16}
    assert cache.allocated_bytes == 4096 * 24 * 2 * 2 * 64 * 4  # 24,576 B per position (DynamicKvCapacityTests)
    qkv = torch.empty((layers, 1, cache.qkv_width), device="cuda").normal_(generator=generator)
    out = torch.empty((layers, 1, heads * d), device="cuda")
    cache.step([(0, 4096)])
    host_rows = qkv.cpu().numpy()
    for layer in range(layers):
        cache.append_attention(layer, qkv[layer], out[layer])
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    worst = 0.0
    for layer in range(layers):
        check_appended(cache, host_rows[layer, 0], 0, 4096, layer)
        worst = max(worst, check_token(cache, host_rows[layer, 0], 0, 4096, layer, got[layer, 0], rotated_q=False))
    assert cache.slot_info(0)["capacity"] == 8192  # NextCapacity(4097, 4096) doubles
    say("C1 worst abs error", worst)
    cache.close()


def test_c2_fp16_fill_decode_and_contract(torch_gpu):
    # Config 2: 0.5B FP16, 256-token pages, fill to 32,768 in 512-token chunks, 256 decode steps, then a
    # 1,024-token request contracts the slot to exactly 4 pages.
    from synapse_amd import PagedKvCache

    torch = torch_gpu
    say("C2")
    layers, heads, kv_heads, d = 24, 14, 2, 64
    cache = PagedKvCache(layers=layers, heads=heads, kv_heads=kv_heads, head_dim=d, max_positions=65536,
                         growth_positions=1024, page_tokens=256, precision="f16", session_slots=1,
                         step_tokens=512, max_pages=256)
    generator = torch.Generator(device="cuda")
    generator.manual_seed(SEED + 2)
    fill(cache, torch, 0, 0, 32768, 512, generator, layers)
    assert cache.slot_info(0) == {"capacity": 32768, "length": 32768, "pages": 128}
    assert cache.allocated_bytes == 128 * 256 * 12_288  # 12,288 B per position for 0.5B FP16
    qkv = torch.empty((layers, 1, cache.qkv_width), device="cuda")
    out = torch.empty((layers, 1, heads * d), device="cuda")
    checked = {0: None, 255: None}
    for step in range(256):
        qkv.normal_(generator=generator)
        cache.step([(0, 32768 + step)])
        for layer in range(layers):
            cache.append_attention(layer, qkv[layer], out[layer])
        if step in checked:
            torch.cuda.synchronize()
            checked[step] = (qkv.cpu().numpy(), out.cpu().numpy())
    torch.cuda.synchronize()
    assert cache.slot_info(0)["capacity"] == 65536  # NextCapacity(32769, 32768) doubles
    for step, (rows, got) in checked.items():
        for layer in (0, 23):
            check_appended(cache, rows[layer, 0], 0, 32768 + step, layer)
            check_token(cache, rows[layer, 0], 0, 32768 + step, layer, got[layer, 0], rotated_q=False)
    keys_before, values_before = cache.read_kv(0, 7, 0, 1024)
    cache.reserve(0, 1024)  # rounded 1,024 <= 65,536 / 4: contract, keeping the prefix
    stats = cache.page_stats()
    assert cache.slot_info(0) == {"capacity": 1024, "length": 1024, "pages": 4}
    assert stats["used_pages"] == 4 and stats["free_pages"] == 252 and stats["device_status"] == 0
    assert cache.allocated_bytes == 1024 * 12_288
    keys_after, values_after = cache.read_kv(0, 7, 0, 1024)
    assert np.array_equal(keys_before, keys_after) and np.array_equal(values_before, values_after)
    assert cache.free_list().size == 252
    cache.close()


def test_c3_batched_decode_ragged_lengths(torch_gpu):
    # Config 3 (the north-star shape): 7B, 16 sequences with lengths U[1,024, 32,768], one decode step checked on
    # two layers for every sequence.
    from synapse_amd import PagedKvCache

    torch = torch_gpu
    say("C3")
    layers, heads, kv_heads, d = 28, 28, 4, 128
    lengths = np.random.default_rng(SEED + 3).integers(1024, 32769, size=16)
    pages = int(sum(-(-(-(-(int(n) + 1) // 1024) * 1024) // 256) for n in lengths))
    cache = PagedKvCache(layers=layers, heads=heads, kv_heads=kv_heads, head_dim=d, max_positions=33792,
                         growth_positions=1024, page_tokens=256, precision="f16", session_slots=16,
                         step_tokens=4096, max_pages=pages)
    generator = torch.Generator(device="cuda")
    generator.manual_seed(SEED + 3)
    for slot, length in enumerate(lengths.tolist()):
        cache.reserve(slot, length + 1)
        fill(cache, torch, slot, 0, length, 4096, generator, layers)
    qkv = torch.empty((layers, 16, cache.qkv_width), device="cuda").normal_(generator=generator)
    out = torch.empty((layers, 16, heads * d), device="cuda")
    cache.step([(slot, int(length)) for slot, length in enumerate(lengths)])
    for layer in range(layers):
        cache.append_attention(layer, qkv[layer], out[layer])
    torch.cuda.synchronize()
    rows, got = qkv.cpu().numpy(), out.cpu().numpy()
    for layer in (0, 27):
        for slot, length in enumerate(lengths.tolist()):
            check_appended(cache, rows[layer, slot], slot, length, layer)
            check_token(cache, rows[layer, slot], slot, length, layer, got[layer, slot], rotated_q=False)
    stats = cache.page_stats()
    assert stats["used_pages"] == pages and stats["device_status"] == 0
    cache.close()


def test_c4_prefix_reuse_copy_on_write(torch_gpu):
    # Config 4: a 30,000-token FP16 prefix forked into 8 sequences that share its pages copy-on-write; each
    # appends a distinct 64-token suffix and decodes 128 tokens. Tables, reference counts and free stacks are
    # bit-exact with the restatement driven by the same calls.
    from synapse_amd import PagedKvCache

    torch = torch_gpu
    say("C4")
    layers, heads, kv_heads, d = 28, 28, 4, 128
    max_pages = 160
    cache = PagedKvCache(layers=layers, heads=heads, kv_heads=kv_heads, head_dim=d, max_positions=32768,
                         growth_positions=1024, page_tokens=256, precision="f16", session_slots=9,
                         step_tokens=4096, max_pages=max_pages)
    # The restatement tracks tables only here (one layer of page payload keeps its memory small).
    oracle = PagedCache(1, heads, kv_heads, d, 32768, 1024, 256, 1, 9, max_pages, 4096)
    generator = torch.Generator(device="cuda")
    generator.manual_seed(SEED + 4)
    cache.reserve(0, 30000)
    assert oracle.reserve(0, 30000) == 0
    for start in range(0, 30000, 4096):
        size = min(4096, 30000 - start)
        assert oracle.step([(0, p) for p in range(start, start + size)]) == 0
    fill(cache, torch, 0, 0, 30000, 4096, generator, layers)
    for target in range(1, 9):
        cache.fork(0, target)
        assert oracle.fork(0, target) == 0
    shared = cache.block_table(0)[:118]
    assert cache.refcounts()[shared].tolist() == [9] * 118  # 117 full pages + the partial page (48 tokens)
    suffix = torch.empty((64 * 8, cache.qkv_width), device="cuda")
    out = torch.empty((64 * 8, heads * d), device="cuda")
    tokens = [(slot, 30000 + j) for slot in range(1, 9) for j in range(64)]
    cache.step(tokens)
    assert oracle.step(tokens) == 0
    for layer in range(layers):
        suffix.normal_(generator=generator)
        cache.append_attention(layer, suffix, out)
        if layer == 3:
            torch.cuda.synchronize()
            suffix_rows, suffix_out = suffix.cpu().numpy(), out.cpu().numpy()
    torch.cuda.synchronize()
    for slot in range(9):
        assert np.array_equal(cache.block_table(slot), oracle.table(slot)), slot
    assert np.array_equal(cache.refcounts(), oracle.refcounts())
    assert np.array_equal(cache.free_list(), oracle.free_list())
    # Each fork copied the partial page once; the original keeps slot 0's bits.
    assert cache.refcounts()[shared[117]] == 1 and cache.refcounts()[shared[0]] == 9
    for index in (0, 63, 64 * 7 + 5):
        slot, position = tokens[index]
        check_appended(cache, suffix_rows[index], slot, position, 3)
        check_token(cache, suffix_rows[index], slot, position, 3, suffix_out[index], rotated_q=False)
    qkv = torch.empty((8, cache.qkv_width), device="cuda")
    decode_out = torch.empty((8, heads * d), device="cuda")
    for step in range(128):
        tokens = [(slot, 30064 + step) for slot in range(1, 9)]
        cache.step(tokens)
        assert oracle.step(tokens) == 0
        for layer in range(layers):
            qkv.normal_(generator=generator)
            cache.append_attention(layer, qkv, decode_out)
    torch.cuda.synchronize()
    rows, got = qkv.cpu().numpy(), decode_out.cpu().numpy()
    for slot in (1, 8):
        check_token(cache, rows[slot - 1], slot, 30064 + 127, 27, got[slot - 1], rotated_q=False)
    for slot in range(9):
        assert np.array_equal(cache.block_table(slot), oracle.table(slot)), slot
    assert np.array_equal(cache.refcounts(), oracle.refcounts())
    assert np.array_equal(cache.free_list(), oracle.free_list())
    assert cache.page_stats()["device_status"] == 0
    # Releasing the forks frees their copied pages; the shared prefix stays with slot 0.
    for slot in range(1, 9):
        cache.release(slot)
        assert oracle.release(slot) == 0
    assert np.array_equal(cache.free_list(), oracle.free_list())
    assert cache.refcounts()[shared].tolist() == [1] * 118
    cache.close()


def test_c5_chunked_prefill_over_63488_cached_tokens(torch_gpu):
    # Config 5: a 2,048-token chunk attends causally over a 63,488-token FP16 cache plus itself (65,536), all 28
    # layers, QK^T and PV on FP16 MFMA. Rows of the first, middle and last tokens are checked on two layers.
    from synapse_amd import PagedKvCache

    torch = torch_gpu
    say("C5")
    layers, heads, kv_heads, d = 28, 28, 4, 128
    cache = PagedKvCache(layers=layers, heads=heads, kv_heads=kv_heads, head_dim=d, max_positions=65536,
                         growth_positions=1024, page_tokens=256, precision="f16", session_slots=1,
                         step_tokens=4096, max_pages=256)
    generator = torch.Generator(device="cuda")
    generator.manual_seed(SEED + 5)
    cache.reserve(0, 65536)
    fill(cache, torch, 0, 0, 63488, 4096, generator, layers)
    qkv = torch.empty((2048, cache.qkv_width), device="cuda")
    out = torch.empty((2048, heads * d), device="cuda")
    cache.step([(0, 63488 + j) for j in range(2048)])
    kept = {}
    for layer in range(layers):
        qkv.normal_(generator=generator)
        cache.append_attention(layer, qkv, out)
        if layer in (0, 27):
            torch.cuda.synchronize()
            kept[layer] = (qkv.cpu().numpy(), out.cpu().numpy())
    torch.cuda.synchronize()
    for layer, (rows, got) in kept.items():
        for j in (0, 1, 1023, 2047):
            check_appended(cache, rows[j], 0, 63488 + j, layer)
            check_token(cache, rows[j], 0, 63488 + j, layer, got[j], rotated_q=False, upto=65536)
        say("C5 layer", layer, "checked")
    cache.close()
