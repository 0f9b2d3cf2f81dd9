"""Persistent prefix payloads (ADR-018's next step) on the GPU through the C ABI.

Bar: bit-exact. An exported prefix imported into an empty slot holds the same K/V bytes in every layer
(synapse_kv_read_kv), and a decode step attends over it to the same output bits as over the original slot.
Payloads are deterministic (the same prefix exports the same bytes), truncated exports equal the leading part of
the full one's rows, and every mismatch (key, KV type or shape, size, checksum, occupied slot) is status 2 with the
slot left empty.
"""

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

KEY = (0x1111, 0x2222, 0x3333, 0x4444)


def say(*parts):
    print(*parts, flush=True)
    sys.stdout.flush()


def make_cache(precision, layers=3, head_dim=64, kv_heads=2, heads=14, page_tokens=64, growth=256, slots=3):
    from synapse_amd import PagedKvCache

    return PagedKvCache(layers=layers, heads=heads, kv_heads=kv_heads, head_dim=head_dim, max_positions=2048,
                        growth_positions=growth, page_tokens=page_tokens, precision=precision, session_slots=slots,
                        step_tokens=512, max_pages=96)


def fill(torch, cache, slot, length, rng):
    width = (cache.heads + 2 * cache.kv_heads) * cache.head_dim
    for first in range(0, length, 400):
        count = min(400, length - first)
        cache.step([(slot, p) for p in range(first, first + count)])
        for layer in range(cache.layers):
            rows = rng.standard_normal((count, width)).astype(np.float32)
            cache.append_rope(layer, torch.from_numpy(rows).cuda())


def decode(torch, cache, slot, position, rows, prompt_start=None):
    cache.step([(slot, position)], prompt_start)
    outputs = []
    for layer in range(cache.layers):
        qkv = torch.from_numpy(rows[layer].copy()).cuda()
        out = torch.zeros((1, cache.heads * cache.head_dim), device="cuda")
        cache.append_attention(layer, qkv, out)
        outputs.append(out.cpu().numpy())
    return np.concatenate(outputs)


@pytest.mark.parametrize("precision,page_tokens,length", [("f16", 64, 777), ("f32", 256, 300), ("f16", 256, 64)])
def test_export_import_round_trip_is_bit_exact(torch_gpu, precision, page_tokens, length):
    torch = torch_gpu
    say("prefix round trip", precision, page_tokens, length)
    rng = np.random.default_rng(length)
    cache = make_cache(precision, page_tokens=page_tokens)
    fill(torch, cache, 0, length, rng)
    payload = cache.export_prefix(0, length, KEY)
    assert payload == cache.export_prefix(0, length, KEY)  # deterministic
    assert cache.import_prefix(1, KEY, payload) == length
    for layer in range(cache.layers):
        k0, v0 = cache.read_kv(0, layer, 0, length)
        k1, v1 = cache.read_kv(1, layer, 0, length)
        assert k0.tobytes() == k1.tobytes() and v0.tobytes() == v1.tobytes(), layer
    # A shorter export is the leading part of the full one, layer by layer.
    short = cache.export_prefix(0, length // 2, KEY)
    element = 2 if precision == "f16" else 4
    full_rows = np.frombuffer(payload[128:], dtype=np.uint8).reshape(cache.layers, 2, length, -1)
    short_rows = np.frombuffer(short[128:], dtype=np.uint8).reshape(cache.layers, 2, length // 2, -1)
    assert full_rows.shape[-1] == cache.kv_heads * cache.head_dim * element
    assert np.array_equal(full_rows[:, :, :length // 2], short_rows)
    # Decoding the same token over both slots gives the same bits.
    width = (cache.heads + 2 * cache.kv_heads) * cache.head_dim
    rows = rng.standard_normal((cache.layers, 1, width)).astype(np.float32)
    a = decode(torch, cache, 0, length, rows)
    b = decode(torch, cache, 1, length, rows)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    cache.close()


def test_import_rejects_mismatches_and_leaves_the_slot_empty(torch_gpu):
    from synapse_amd import InvalidOperationError

    torch = torch_gpu
    say("prefix import errors")
    rng = np.random.default_rng(2)
    cache = make_cache("f16")
    fill(torch, cache, 0, 300, rng)
    payload = bytearray(cache.export_prefix(0, 300, KEY))
    with pytest.raises(InvalidOperationError, match="prefix key differs"):
        cache.import_prefix(1, (0x1111, 0x2222, 0x3333, 0x4445), bytes(payload))
    corrupt = bytearray(payload)
    corrupt[128 + 1000] ^= 1
    with pytest.raises(InvalidOperationError, match="checksum"):
        cache.import_prefix(1, KEY, bytes(corrupt))
    with pytest.raises(InvalidOperationError, match="size does not match"):
        cache.import_prefix(1, KEY, bytes(payload[:-2]))
    with pytest.raises(InvalidOperationError, match="version 1 prefix payload"):
        cache.import_prefix(1, KEY, b"X" * 200)
    with pytest.raises(InvalidOperationError, match="empty slot"):
        cache.import_prefix(0, KEY, bytes(payload))
    other = make_cache("f32")
    with pytest.raises(InvalidOperationError, match="KV type or shape"):
        other.import_prefix(0, KEY, bytes(payload))
    other.close()
    assert cache.import_prefix(1, KEY, bytes(payload)) == 300  # the failed attempts left slot 1 empty
    cache.close()


def test_import_under_page_activation_rebuilds_summaries(torch_gpu):
    """With KV page activation on, the imported blocks get key summaries: a sparse decode over the imported slot
    selects and attends exactly as over the original."""
    torch = torch_gpu
    say("prefix import with page activation")
    rng = np.random.default_rng(4)
    cache = make_cache("f16", layers=2)
    fill(torch, cache, 0, 1000, rng)
    cache.set_page_activation(2, 64)
    payload = cache.export_prefix(0, 1000, KEY)
    cache.import_prefix(1, KEY, payload)
    width = (cache.heads + 2 * cache.kv_heads) * cache.head_dim
    rows = rng.standard_normal((cache.layers, 1, width)).astype(np.float32)
    # prompt_start 1: the step's token comes before the prompt boundary, a decode unit that attends its selected
    # pages only (ADR-016).
    a = decode(torch, cache, 0, 1000, rows, prompt_start=1)
    b = decode(torch, cache, 1, 1000, rows, prompt_start=1)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    cache.set_page_activation(None)
    cache.import_prefix(2, KEY, payload)
    dense = decode(torch, cache, 2, 1000, rows, prompt_start=1)
    assert not np.allclose(a, dense, atol=1e-3)  # the sparse plan was taken
    cache.close()
