"""GPU parity through the C ABI: the HIP path against the CPU restatement on the same seeded inputs.

Bar: block tables, reference counts, free stacks, rotated Q/K and stored K/V bits are bit-exact; attention is
within |gpu - ref| <= 2e-3 + 1e-3 * |ref| of the FP32-accumulate restatement (Qwen2CpuAttention order).
"""

import sys

import numpy as np
import pytest

from oracle_ffi import PagedCache
from paged_checks import check_allocator_invariants

pytestmark = pytest.mark.gpu

ATOL = 2e-3
RTOL = 1e-3


def say(*parts):
    print(*parts, flush=True)
    sys.stdout.flush()


class Pair:
    """A GPU cache and its CPU restatement driven with identical calls."""

    def __init__(self, torch, *, layers=2, heads=14, kv_heads=2, head_dim=64, max_positions=4096, growth=256,
                 page=256, precision="f16", slots=4, max_pages=64, step_tokens=256):
        from synapse_amd import PagedKvCache

        self.torch = torch
        self.gpu = PagedKvCache(layers=layers, heads=heads, kv_heads=kv_heads, head_dim=head_dim,
                                max_positions=max_positions, growth_positions=growth, page_tokens=page,
                                precision=precision, session_slots=slots, step_tokens=step_tokens,
                                max_pages=max_pages)
        code = 1 if precision == "f16" else 0
        self.cpu = PagedCache(layers, heads, kv_heads, head_dim, max_positions, growth, page, code, slots,
                              max_pages, step_tokens)
        self.layers, self.heads, self.kv_heads, self.head_dim = layers, heads, kv_heads, head_dim
        self.slots, self.max_pages = slots, max_pages
        self.width = (heads + 2 * kv_heads) * head_dim
        self.cos, self.sin = self.gpu.rope_cosines, self.gpu.rope_sines

    def call(self, name, *args):
        """Runs one table operation on both sides; both must succeed or fail alike."""
        from synapse_amd import SynapseKvError

        expected = getattr(self.cpu, name)(*args)
        try:
            getattr(self.gpu, name)(*args)
            status = 0
        except SynapseKvError as error:
            status = error.status
        assert status == expected, (name, args, status, expected)
        return status

    def step(self, tokens, rng, attend=True, fused=False, key_scale=None):
        """One step: prepare, then per layer append (+ attention); checks every output. `fused` drives the layer
        through append_attention (qkv stays unrotated) instead of append_rope + attention. `key_scale(position)`
        multiplies each token's K row (rising scales move the running maximum often)."""
        torch = self.torch
        status = self.call("step", tokens)
        if status:
            return status
        count = len(tokens)
        for layer in range(self.layers):
            rows = rng.standard_normal((count, self.width)).astype(np.float32)
            if key_scale is not None:
                k0, k1 = self.heads * self.head_dim, (self.heads + self.kv_heads) * self.head_dim
                scales = np.array([key_scale(position) for _, position in tokens], dtype=np.float32)
                rows[:, k0:k1] *= scales[:, None]
            qkv = torch.from_numpy(rows.copy()).cuda()
            original = rows.copy()
            out = torch.full((count, self.heads * self.head_dim), float("nan"), device="cuda")
            if fused:
                self.gpu.append_attention(layer, qkv, out)
            else:
                self.gpu.append_rope(layer, qkv)
            assert self.cpu.append_rope(layer, rows, self.cos, self.sin) == 0
            if fused:
                assert np.array_equal(qkv.cpu().numpy().view(np.uint32), original.view(np.uint32)), "qkv changed"
            else:
                rotated = qkv.cpu().numpy()
                assert np.array_equal(rotated.view(np.uint32), rows.view(np.uint32)), "rotated Q/K differ"
            if attend or fused:
                if not fused:
                    self.gpu.attention(layer, qkv, out)
                expected = np.zeros((count, self.heads * self.head_dim), dtype=np.float32)
                self.cpu.attention(layer, rows, expected)
                got = out.cpu().numpy()
                error = np.abs(got - expected)
                bound = ATOL + RTOL * np.abs(expected)
                assert np.all(error <= bound), (layer, float(error.max()), tokens[:4])
        return 0

    def check_tables(self):
        tables = []
        for slot in range(self.slots):
            gpu_table = self.gpu.block_table(slot)
            assert np.array_equal(gpu_table, self.cpu.table(slot)), slot
            assert self.gpu.slot_info(slot) == self.cpu.slot(slot)
            tables.append(gpu_table)
        refcounts = self.gpu.refcounts()
        assert np.array_equal(refcounts, self.cpu.refcounts())
        free = self.gpu.free_list()
        assert np.array_equal(free, self.cpu.free_list())
        check_allocator_invariants(tables, refcounts, free, self.max_pages)
        stats = self.gpu.page_stats()
        assert stats["device_status"] == 0
        assert self.gpu.allocated_bytes == self.cpu.kv_bytes

    def check_contents(self, slot):
        capacity = self.cpu.slot(slot)["capacity"]
        if capacity == 0:
            return
        for layer in range(self.layers):
            keys, values = self.gpu.read_kv(slot, layer, 0, capacity)
            ckeys, cvalues = self.cpu.gather(slot, layer, 0, capacity, raw=True)
            assert np.array_equal(keys.view(np.uint8), ckeys.view(np.uint8)), (slot, layer)
            assert np.array_equal(values.view(np.uint8), cvalues.view(np.uint8)), (slot, layer)


SHAPES = [
    # (heads, kv_heads, head_dim, precision, page)
    (14, 2, 64, "f16", 256),
    (28, 4, 128, "f16", 256),
    (14, 2, 64, "f32", 64),
    (28, 4, 128, "f32", 128),
    (8, 8, 128, "f16", 64),
]


@pytest.mark.parametrize("heads,kv_heads,head_dim,precision,page", SHAPES)
def test_decode_steps_match_the_restatement(torch_gpu, heads, kv_heads, head_dim, precision, page):
    say("decode parity", heads, kv_heads, head_dim, precision, page)
    pair = Pair(torch_gpu, heads=heads, kv_heads=kv_heads, head_dim=head_dim, precision=precision, page=page,
                growth=max(page, 256), max_pages=96 if page == 64 else 48)
    rng = np.random.default_rng(heads * 1000 + head_dim)
    # Prefill three slots with ragged lengths through decode-only steps of many tokens (no prompt runs).
    pair.gpu.set_prefill_runs(False)
    lengths = [1, 300, 777]
    for slot, length in enumerate(lengths):
        for first in range(0, length, 200):
            positions = range(first, min(length, first + 200))
            assert pair.step([(slot, p) for p in positions], rng, attend=False) == 0
    pair.check_tables()
    for slot in range(3):
        pair.check_contents(slot)
    # Decode: one token per slot per step, unsplit and with many small splits.
    for split in (512, 64, 128):
        pair.gpu.set_split_keys(split)
        tokens = [(slot, lengths[slot]) for slot in range(3)]
        assert pair.step(tokens, rng) == 0
        lengths = [length + 1 for length in lengths]
    pair.check_tables()


@pytest.mark.parametrize("prefetch", [0, 1])
@pytest.mark.parametrize("heads,kv_heads,head_dim,precision,page", SHAPES[:4])
def test_append_attention_matches_the_restatement(torch_gpu, heads, kv_heads, head_dim, precision, page, prefetch):
    from synapse_amd.native import OPTION_DECODE_PREFETCH

    say("append_attention parity", heads, kv_heads, head_dim, precision, page, prefetch)
    pair = Pair(torch_gpu, heads=heads, kv_heads=kv_heads, head_dim=head_dim, precision=precision, page=page,
                growth=max(page, 256), max_pages=96 if page == 64 else 48)
    pair.gpu.set_option(OPTION_DECODE_PREFETCH, prefetch)
    rng = np.random.default_rng(head_dim + 7)
    lengths = [0, 257, 600]
    for slot, length in enumerate(lengths):
        for first in range(0, length, 200):
            assert pair.step([(slot, p) for p in range(first, min(length, first + 200))], rng, attend=False) == 0
    # Decode steps with one token per slot: one fused launch per layer, split and unsplit rows.
    for split in (256, 64):
        pair.gpu.set_split_keys(split)
        pair.gpu.profile_begin()
        assert pair.step([(slot, lengths[slot]) for slot in range(3)], rng, fused=True) == 0
        kernels = pair.gpu.profile_end()
        assert kernels["decode"][0] == pair.layers and "append" not in kernels
        assert all(milliseconds > 0 for _, milliseconds in kernels.values())
        lengths = [length + 1 for length in lengths]
    # Two tokens of one slot (an overwrite and an append) and a prompt run: the append runs first, then attention,
    # qkv still untouched.
    assert pair.step([(0, lengths[0] - 2), (0, lengths[0]), (1, lengths[1])], rng, fused=True) == 0
    lengths[0] += 1
    lengths[1] += 1
    assert pair.step([(2, p) for p in range(lengths[2], lengths[2] + 40)] + [(1, lengths[1])], rng, fused=True) == 0
    pair.check_tables()
    for slot in range(3):
        pair.check_contents(slot)


def test_rows_cut_into_many_pieces(torch_gpu):
    """A 79-step decode row cut as finely as the planner allows (79 pieces: one merge wave, two rounds of split
    loads), then the row grown to 146 steps: decode cut into up to 146 pieces and a prompt chunk with 64-key
    prefill pieces, 146 partial rows per token (the wide merge: a workgroup per row). Three layers reuse each
    plan."""
    say("many pieces")
    pair = Pair(torch_gpu, heads=28, kv_heads=4, head_dim=128, max_positions=16384, growth=1024, max_pages=72,
                layers=3, slots=2)
    rng = np.random.default_rng(77)
    for first in range(0, 5000, 256):
        assert pair.step([(0, p) for p in range(first, min(5000, first + 256))], rng, attend=False) == 0
    assert pair.step([(1, p) for p in range(100)], rng, attend=False) == 0
    lengths = [5000, 100]
    for split, fused in ((64, True), (64, False), (128, True), (256, False)):
        pair.gpu.set_split_keys(split)
        assert pair.step([(slot, lengths[slot]) for slot in range(2)], rng, fused=fused) == 0
        lengths = [length + 1 for length in lengths]
    for first in range(lengths[0], 9300, 256):
        assert pair.step([(0, p) for p in range(first, min(9300, first + 256))], rng, attend=False) == 0
    lengths[0] = 9300
    for split, fused in ((64, True), (64, False)):
        pair.gpu.set_split_keys(split)
        assert pair.step([(slot, lengths[slot]) for slot in range(2)], rng, fused=fused) == 0
        lengths = [length + 1 for length in lengths]
    pair.gpu.set_prefill_split_keys(64)
    assert pair.step([(0, p) for p in range(lengths[0], lengths[0] + 20)], rng) == 0
    pair.check_contents(0)


def test_rows_past_the_wide_merge(torch_gpu):
    """A 66,000-key cache (small heads): single-token decode with 64-key workers (about 516 pieces per row, the
    wide merge) and a prompt chunk with 64-key prefill pieces, 1,032 partial rows per token: more than one wide
    merge holds, so blocks of 64 partial rows are merged first, then the blocks."""
    say("two-level merge")
    length = 66000
    pair = Pair(torch_gpu, heads=2, kv_heads=1, head_dim=64, max_positions=131072, growth=1024, max_pages=600,
                layers=1, slots=1, step_tokens=4096)
    rng = np.random.default_rng(78)
    for first in range(0, length, 4096):
        assert pair.step([(0, p) for p in range(first, min(length, first + 4096))], rng, attend=False) == 0
    for fused in (True, False):
        pair.gpu.set_split_keys(64)
        assert pair.step([(0, length)], rng, fused=fused) == 0
        length += 1
    pair.gpu.set_prefill_split_keys(64)
    assert pair.step([(0, p) for p in range(length, length + 20)], rng) == 0
    pair.check_contents(0)


@pytest.mark.parametrize("cost", [0, 64])
def test_split_cost_extremes(torch_gpu, cost):
    """The decode split with no row-start cost and with the largest (16 steps per row start, which leaves some
    workers with empty ranges): three rows of very different lengths, fused and separate launches, against the
    restatement; out-of-range costs are rejected."""
    from synapse_amd import InvalidOperationError
    from synapse_amd.native import OPTION_SEGMENT_COST

    say("split cost", cost)
    pair = Pair(torch_gpu, heads=28, kv_heads=4, head_dim=128, max_positions=8192, growth=1024, max_pages=40,
                layers=2, slots=3)
    pair.gpu.set_option(OPTION_SEGMENT_COST, cost)
    with pytest.raises(InvalidOperationError, match="segment cost"):
        pair.gpu.set_option(OPTION_SEGMENT_COST, 65)
    rng = np.random.default_rng(101 + cost)
    lengths = [3000, 700, 64]
    for slot, length in enumerate(lengths):
        for first in range(0, length, 256):
            assert pair.step([(slot, p) for p in range(first, min(length, first + 256))], rng, attend=False) == 0
    for split, fused in ((64, True), (64, False), (256, True)):
        pair.gpu.set_split_keys(split)
        assert pair.step([(slot, lengths[slot]) for slot in range(3)], rng, fused=fused) == 0
        lengths = [length + 1 for length in lengths]
    for slot in range(3):
        pair.check_contents(slot)


@pytest.mark.parametrize("precision", ["f16", "f32"])
def test_adaptive_split(torch_gpu, precision):
    """SYNAPSE_KV_OPTION_ADAPTIVE_SPLIT: worker shares weighted by the XCD speeds measured on earlier steps' first
    four decode launches. Consecutive decode steps over rows of very different lengths, fused and separate launches,
    stay within the attention bar of the restatement while the weights move; the stored K/V stay bit-exact; turning
    the option off restores equal shares."""
    from synapse_amd.native import OPTION_ADAPTIVE_SPLIT

    say("adaptive split", precision)
    pair = Pair(torch_gpu, heads=28, kv_heads=4, head_dim=128, max_positions=8192, growth=1024, max_pages=40,
                layers=5, slots=3, precision=precision)
    rng = np.random.default_rng(303)
    lengths = [3000, 700, 64]
    for slot, length in enumerate(lengths):
        for first in range(0, length, 256):
            assert pair.step([(slot, p) for p in range(first, min(length, first + 256))], rng, attend=False) == 0
    pair.gpu.set_option(OPTION_ADAPTIVE_SPLIT, 1)
    for index in range(10):
        assert pair.step([(slot, lengths[slot]) for slot in range(3)], rng, fused=index % 3 != 2) == 0
        lengths = [length + 1 for length in lengths]
    pair.gpu.set_option(OPTION_ADAPTIVE_SPLIT, 0)
    assert pair.step([(slot, lengths[slot]) for slot in range(3)], rng, fused=True) == 0
    for slot in range(3):
        pair.check_contents(slot)


def test_single_position_and_page_boundaries(torch_gpu):
    say("page boundaries")
    pair = Pair(torch_gpu, page=64, growth=64, max_pages=64, heads=28, kv_heads=4, head_dim=128)
    rng = np.random.default_rng(5)
    filled = 0
    for position in [0, 1, 63, 64, 65, 127, 128, 191, 255, 256]:
        if position > filled:  # appends stay contiguous: the positions in between first
            assert pair.step([(0, p) for p in range(filled, position)], rng, attend=False) == 0
        assert pair.step([(0, position)], rng) == 0
        filled = position + 1
    pair.gpu.set_split_keys(64)
    assert pair.step([(0, 257)], rng) == 0
    pair.check_tables()
    pair.check_contents(0)


@pytest.mark.parametrize("head_dim", [64, 128])
def test_prompt_runs_match_the_restatement(torch_gpu, head_dim):
    say("prefill parity", head_dim)
    heads, kv_heads = (14, 2) if head_dim == 64 else (28, 4)
    pair = Pair(torch_gpu, heads=heads, kv_heads=kv_heads, head_dim=head_dim, max_pages=64)
    rng = np.random.default_rng(head_dim)
    # A first chunk, a second chunk that attends over the cache, and runs of two slots in one step.
    assert pair.step([(0, p) for p in range(0, 100)], rng) == 0
    assert pair.step([(0, p) for p in range(100, 233)], rng) == 0
    pair.gpu.set_prefill_split_keys(64)
    assert pair.step([(0, p) for p in range(233, 300)] + [(1, p) for p in range(0, 45)], rng) == 0
    pair.gpu.set_prefill_split_keys(16384)
    assert pair.step([(1, 45), (0, 300)] + [(2, p) for p in range(0, 31)], rng) == 0
    pair.gpu.set_prefill_split_keys(0)  # automatic: split to fill the device
    assert pair.step([(2, p) for p in range(31, 97)] + [(3, p) for p in range(0, 64)], rng) == 0
    pair.check_tables()
    for slot in range(4):
        pair.check_contents(slot)


@pytest.mark.parametrize("split", [0, 64, 256])
def test_prefill_running_maximum_moves_often(torch_gpu, split):
    """Keys whose scale rises with position push every column's maximum up many times, through the lazy offset
    update (threshold crossings, the first key of a column, split partial rows merged afterwards)."""
    say("prefill rising scores", split)
    pair = Pair(torch_gpu, heads=28, kv_heads=4, head_dim=128, max_pages=64, layers=1)
    rng = np.random.default_rng(40 + split)
    pair.gpu.set_prefill_split_keys(split)
    rising = lambda position: 0.5 + position / 160.0  # noqa: E731
    assert pair.step([(0, p) for p in range(0, 200)], rng, key_scale=rising) == 0
    assert pair.step([(0, p) for p in range(200, 420)], rng, key_scale=rising) == 0
    assert pair.step([(0, p) for p in range(420, 452)], rng, key_scale=rising, fused=True) == 0
    pair.check_contents(0)


def test_table_operations_match_the_restatement(torch_gpu):
    say("table operations")
    pair = Pair(torch_gpu, page=64, growth=128, max_positions=1024, slots=5, max_pages=40, layers=1)
    rng = np.random.default_rng(17)
    lengths = [0] * 5
    for round_index in range(60):
        action = rng.random()
        slot = int(rng.integers(0, 5))
        if action < 0.45:
            # An append at the length, an overwrite below it (rollback), or a gap past it, which both sides reject
            # (status 2) and which leaves every table unchanged.
            kind = rng.random()
            if kind < 0.6:
                position = lengths[slot]
            elif kind < 0.85:
                position = int(rng.integers(max(0, lengths[slot] - 80), lengths[slot] + 1))
            else:
                position = lengths[slot] + int(rng.integers(1, 100))
            position = min(1023, position)
            status = pair.step([(slot, position)], rng, attend=False)
            assert (status == 2) == (position > lengths[slot]), (position, lengths[slot], status)
            if status == 0:
                lengths[slot] = max(lengths[slot], position + 1)
        elif action < 0.65:
            pair.call("reserve", slot, int(rng.integers(0, 1025)))
            lengths[slot] = min(lengths[slot], pair.cpu.slot(slot)["capacity"])
        elif action < 0.8:
            target = int(rng.integers(0, 5))
            pair.call("fork", slot, target)
            lengths[target] = pair.cpu.slot(target)["length"]
        elif action < 0.9:
            pair.call("release", slot)
            lengths[slot] = 0
        else:
            pair.call("truncate", slot, int(rng.integers(0, lengths[slot] + 2)))
            lengths[slot] = pair.cpu.slot(slot)["length"]
        pair.check_tables()
    for slot in range(5):
        pair.check_contents(slot)


def test_copy_on_write_keeps_both_histories(torch_gpu):
    say("copy on write")
    pair = Pair(torch_gpu, page=64, growth=64, max_positions=1024, slots=4, max_pages=48, heads=28, kv_heads=4,
                head_dim=128)
    rng = np.random.default_rng(23)
    assert pair.step([(0, p) for p in range(150)], rng, attend=False) == 0
    for target in (1, 2, 3):
        pair.call("fork", 0, target)
    # Every fork writes its own suffix into the shared partial page, then all decode together.
    assert pair.step([(1, 150), (2, 150), (3, 150)], rng) == 0
    assert pair.step([(0, 150), (1, 151), (2, 151), (3, 151)], rng) == 0
    pair.check_tables()
    for slot in range(4):
        pair.check_contents(slot)


@pytest.mark.parametrize("heads,kv_heads,head_dim", [(28, 4, 128), (14, 2, 64), (8, 8, 128)])
def test_forks_read_shared_pages_once(torch_gpu, heads, kv_heads, head_dim):
    """A 700-token prefix forked into 10 slots: the 11 decode tokens share pages 0..9 copy-on-write, so the shared
    kernel attends those 640 keys once per set of members (8 + 3 under GQA 7:1, one set of 11 otherwise) and the
    merge joins each member's own keys; outputs are checked against the restatement with the shared path on and
    off, split and unsplit, through append_rope + attention and through append_attention."""
    from synapse_amd.native import OPTION_SHARED_PREFIX

    say("shared prefix decode", heads, kv_heads, head_dim)
    pair = Pair(torch_gpu, heads=heads, kv_heads=kv_heads, head_dim=head_dim, page=64, growth=64,
                max_positions=2048, slots=12, max_pages=160)
    rng = np.random.default_rng(head_dim + heads)
    for first in range(0, 700, 256):
        assert pair.step([(0, p) for p in range(first, min(700, first + 256))], rng, attend=False) == 0
    for target in range(1, 11):
        pair.call("fork", 0, target)
    position = 700
    for shared, split, fused in ((1, 256, False), (1, 64, True), (0, 256, True), (1, 512, True), (1, 128, False)):
        pair.gpu.set_option(OPTION_SHARED_PREFIX, shared)
        pair.gpu.set_split_keys(split)
        assert pair.step([(slot, position) for slot in range(11)], rng, fused=fused) == 0
        position += 1
    # Ragged: only some forks advance, and one slot holds two lone tokens of the step (an overwrite below its
    # length and an append).
    assert pair.step([(3, position), (5, position - 3), (5, position), (9, position)], rng) == 0
    pair.check_tables()
    for slot in range(11):
        pair.check_contents(slot)


def test_errors_follow_the_reference_mapping(torch_gpu):
    from synapse_amd import InsufficientMemoryError, InvalidOperationError

    say("error mapping")
    pair = Pair(torch_gpu, page=64, growth=64, max_positions=512, slots=2, max_pages=4, layers=1)
    with pytest.raises(InvalidOperationError):
        pair.gpu.attention(0, torch_gpu.zeros(1, pair.width, device="cuda"),
                           torch_gpu.zeros(1, pair.heads * pair.head_dim, device="cuda"))
    with pytest.raises(InsufficientMemoryError):
        pair.gpu.reserve(0, 512)
    with pytest.raises(InvalidOperationError):
        pair.gpu.reserve(0, 513)
    with pytest.raises(InvalidOperationError):
        pair.gpu.step([(2, 0)])
    pair.gpu.step([(0, 0)])
    host = np.zeros((1, pair.width), dtype=np.float32)
    with pytest.raises(InvalidOperationError):
        pair.gpu.append_rope(0, host.ctypes.data)  # host memory is rejected
    with pytest.raises(InvalidOperationError):
        pair.gpu.append_rope(1, torch_gpu.zeros(1, pair.width, device="cuda"))
    assert pair.gpu.allocated_bytes == pair.gpu.page_stats()["page_bytes"]
