"""Query-aware KV page activation (ADR-016) on the GPU through the C ABI, against the restatement
(KvPageSelector + Qwen2KvPageMasks + Qwen2CpuAttention.Attend) on the same seeded inputs.

Bar: the selection is bit-exact (the device bounds use the reference's channel order and rounding, on keys and
rotated queries that are bit-exact with the restatement's), so the outputs meet the attention bar of the dense
path, |gpu - ref| <= 2e-3 + 1e-3 * |ref|. A budget that covers the prefix gives bit-identical outputs to dense
attention. Every sparse case is also checked to differ from dense attention, so the test cannot pass on a dense
plan.
"""

import sys

import numpy as np
import pytest

from test_gpu_parity import ATOL, RTOL, Pair

pytestmark = pytest.mark.gpu


def say(*parts):
    print(*parts, flush=True)
    sys.stdout.flush()


class PagePair(Pair):
    """Pair with page activation on both sides and a prompt boundary per step."""

    def __init__(self, torch, **kwargs):
        super().__init__(torch, **kwargs)
        self.maximum = kwargs.get("max_positions", 4096)
        self.activation = None

    def activate(self, budget, window, selection="key_bound", seed=0, page_tokens=64):
        self.gpu.set_page_activation(budget, window, page_tokens=page_tokens, selection=selection, seed=seed)
        self.activation = (budget, window, page_tokens, 0 if selection == "key_bound" else 1, seed)

    def deactivate(self):
        self.gpu.set_page_activation(None)
        self.activation = None

    def run(self, tokens, rng, prompt_start=None, fused=False, expect_sparse=None):
        """One step through every layer; returns the number of (token, KV head) rows that attended sparsely."""
        torch = self.torch
        assert self.cpu.step(tokens) == 0
        self.gpu.step(tokens, prompt_start)
        count = len(tokens)
        sparse_rows = 0
        for layer in range(self.layers):
            rows = rng.standard_normal((count, self.width)).astype(np.float32)
            qkv = torch.from_numpy(rows.copy()).cuda()
            out = torch.full((count, self.heads * self.head_dim), float("nan"), device="cuda")
            if fused:
                self.gpu.append_attention(layer, qkv, out)
            else:
                self.gpu.append_rope(layer, qkv)
            assert self.cpu.append_rope(layer, rows, self.cos, self.sin) == 0
            if not fused:
                assert np.array_equal(qkv.cpu().numpy().view(np.uint32), rows.view(np.uint32)), "rotated Q/K differ"
                self.gpu.attention(layer, qkv, out)
            expected = np.zeros((count, self.heads * self.head_dim), dtype=np.float32)
            if self.activation is None:
                self.cpu.attention(layer, rows, expected)
                masks = np.zeros((count, self.kv_heads, 1), dtype=bool)
            else:
                masks = self.cpu.attention(layer, rows, expected, activation=self.activation,
                                           prompt_start=prompt_start, maximum=self.maximum)
            got = out.cpu().numpy()
            error = np.abs(got - expected)
            assert np.all(error <= ATOL + RTOL * np.abs(expected)), (layer, float(error.max()), tokens[:4])
            partial = [(t, kv) for t in range(count) for kv in range(self.kv_heads)
                       if masks[t, kv].any() and not masks[t, kv, :tokens[t][1] + 1].all()]
            sparse_rows += len(partial)
            if partial and layer == 0:
                dense = np.zeros_like(expected)
                self.cpu.attention(layer, rows, dense)
                token = partial[0][0]
                assert not np.allclose(got[token], dense[token], atol=1e-3), "sparse row equals dense attention"
        if expect_sparse is not None:
            assert (sparse_rows > 0) == expect_sparse, sparse_rows
        return sparse_rows


def prefill(pair, rng, lengths):
    for slot, length in lengths:
        for first in range(0, length, 256):
            tokens = [(slot, p) for p in range(first, min(length, first + 256))]
            assert pair.cpu.step(tokens) == 0
            pair.gpu.step(tokens)
            for layer in range(pair.layers):
                rows = rng.standard_normal((len(tokens), pair.width)).astype(np.float32)
                qkv = pair.torch.from_numpy(rows.copy()).cuda()
                pair.gpu.append_rope(layer, qkv)
                assert pair.cpu.append_rope(layer, rows, pair.cos, pair.sin) == 0


SHAPES = [
    # (heads, kv_heads, head_dim, precision, page)
    (14, 2, 64, "f16", 256),
    (28, 4, 128, "f16", 64),
    (14, 2, 64, "f32", 64),
    (8, 8, 128, "f16", 128),
    (28, 4, 128, "f32", 256),
]


@pytest.mark.parametrize("heads,kv_heads,head_dim,precision,page", SHAPES)
@pytest.mark.parametrize("selection", ["key_bound", "random"])
def test_decode_units_attend_their_selected_pages(torch_gpu, heads, kv_heads, head_dim, precision, page, selection):
    """Summaries built when activation is switched on over a cached prefix, then kept by appends; ragged decode
    steps (units, a slot with two tokens, a token past the prompt boundary) over several budgets and windows."""
    say("page activation", heads, kv_heads, head_dim, precision, page, selection)
    pair = PagePair(torch_gpu, heads=heads, kv_heads=kv_heads, head_dim=head_dim, precision=precision, page=page,
                    growth=256, max_positions=2048, slots=4, max_pages=2048 // page * 4 + 8)
    rng = np.random.default_rng(head_dim + heads + len(selection))
    prefill(pair, rng, [(0, 1200), (1, 900), (2, 300)])
    pair.activate(2, 128, selection=selection, seed=11)
    pair.run([(0, 1200), (1, 900), (2, 300)], rng, expect_sparse=True)
    pair.run([(0, 1201), (1, 901), (1, 902), (2, 301)], rng, prompt_start=3, expect_sparse=True)
    pair.activate(5, 0, selection=selection, seed=-3)
    pair.run([(0, 1202), (1, 903)], rng, expect_sparse=True)
    pair.run([(0, 1203), (1, 904), (2, 302)], rng, fused=True, expect_sparse=True)
    pair.activate(1, 64, selection=selection)
    for position in range(1204, 1220):
        pair.run([(0, position), (1, position - 300)], rng, expect_sparse=True)
    pair.check_contents(0)


def test_window_zero_ranks_the_page_completed_in_the_same_step(torch_gpu):
    """Position 64k + 63 with no window: the block the step completes is a candidate, so its summary must be
    recomputed by the append before the selection reads it."""
    say("page activation window 0")
    pair = PagePair(torch_gpu, page=256, max_positions=2048, max_pages=40)
    rng = np.random.default_rng(3)
    prefill(pair, rng, [(0, 447)])
    pair.activate(1, 0)
    for position in range(447, 452):
        pair.run([(0, position)], rng, expect_sparse=True)


def test_copy_on_write_keeps_summaries(torch_gpu):
    """Forks share pages; a decode token copies its page on write, and the blocks of that page it does not write
    keep their summaries (window 0 makes them candidates)."""
    say("page activation fork")
    pair = PagePair(torch_gpu, page=256, max_positions=2048, slots=4, max_pages=40)
    rng = np.random.default_rng(4)
    prefill(pair, rng, [(0, 700)])
    pair.activate(2, 0)
    for target in (1, 2):
        pair.call("fork", 0, target)
    pair.run([(0, 700), (1, 700), (2, 700)], rng, expect_sparse=True)
    pair.run([(1, 701), (2, 701)], rng, fused=True, expect_sparse=True)
    pair.check_tables()


def test_covering_budget_is_bit_identical_to_dense(torch_gpu):
    """KvPagesCoveringThePrefixEqualDense (KvPageActivationTests.cs:97-112): the same inputs through a cache with a
    covering budget and one without activation give bit-identical outputs; a sparse budget does not. (Both run
    append_rope + attention: without activation append_attention would take the fused launch, whose rounding
    differs within the tolerance.)"""
    say("page activation covering")
    outputs = []
    for budget in (None, 64, 2):
        from synapse_amd import PagedKvCache

        cache = PagedKvCache(layers=1, heads=14, kv_heads=2, head_dim=64, max_positions=2048, growth_positions=256,
                             page_tokens=64, precision="f16", session_slots=2, step_tokens=256, max_pages=64)
        rng = np.random.default_rng(9)
        width = (14 + 4) * 64
        for first in range(0, 1000, 250):
            cache.step([(0, p) for p in range(first, first + 250)])
            cache.append_rope(0, torch_gpu.from_numpy(rng.standard_normal((250, width)).astype(np.float32)).cuda())
        if budget is not None:
            cache.set_page_activation(budget, 64)
        step_out = []
        for position in range(1000, 1004):
            cache.step([(0, position)])
            qkv = torch_gpu.from_numpy(rng.standard_normal((1, width)).astype(np.float32)).cuda()
            out = torch_gpu.zeros((1, 14 * 64), device="cuda")
            cache.append_rope(0, qkv)
            cache.attention(0, qkv, out)
            step_out.append(out.cpu().numpy())
        outputs.append(np.concatenate(step_out))
        cache.close()
    assert np.array_equal(outputs[0].view(np.uint32), outputs[1].view(np.uint32))
    assert not np.allclose(outputs[0], outputs[2], atol=1e-3)


def test_prompt_tokens_stay_dense(torch_gpu):
    """PromptTokensStayDenseEvenAloneInAStep (KvPageActivationTests.cs:114-133): a lone token past the prompt
    boundary attends densely; the same token before the boundary does not."""
    say("page activation prompt boundary")
    pair = PagePair(torch_gpu, page=64, max_positions=2048, max_pages=80)
    rng = np.random.default_rng(5)
    prefill(pair, rng, [(0, 640)])
    pair.activate(1, 64)
    assert pair.run([(0, 640)], rng, prompt_start=0) == 0
    assert pair.run([(0, 641)], rng, prompt_start=1) > 0


def test_page_activation_arguments(torch_gpu):
    from synapse_amd import InvalidOperationError, PagedKvCache
    from synapse_amd.native import PageActivation

    say("page activation arguments")
    cache = PagedKvCache(layers=1, heads=14, kv_heads=2, head_dim=64, max_positions=512, growth_positions=256,
                         page_tokens=64, precision="f16", session_slots=1, step_tokens=8, max_pages=8)
    with pytest.raises(InvalidOperationError, match="16, 32, or 64"):
        cache.set_page_activation(1, 64, page_tokens=24)
    with pytest.raises(ValueError):
        cache.set_page_activation(-1, 64)
    bad = PageActivation(1, 1, 64, 64, 7, 0)
    status = cache.library.c_set_page_activation(cache.handle, bad)
    assert status == 2 and "selection" in cache.library.last_error()
    assert cache.library.c_set_page_activation(None, bad) == 1
    with pytest.raises(InvalidOperationError, match="prompt_start"):
        cache.step([(0, 0)], prompt_start=2)
    cache.close()


def test_long_lists_take_the_even_split(torch_gpu):
    """A budget of 270 pages over an 18,000-position slot gives rows of 273 listed blocks, cut over many decode
    waves and merged (partial rows of one row in several merge levels), next to a slot with a short list."""
    say("page activation long lists")
    pair = PagePair(torch_gpu, page=256, growth=1024, max_positions=20480, slots=2, max_pages=2 * 80 + 8,
                    step_tokens=1024)
    rng = np.random.default_rng(6)
    for slot, length in ((0, 18000), (1, 3000)):
        for first in range(0, length, 1024):
            tokens = [(slot, p) for p in range(first, min(length, first + 1024))]
            assert pair.cpu.step(tokens) == 0
            pair.gpu.step(tokens)
            for layer in range(pair.layers):
                rows = rng.standard_normal((len(tokens), pair.width)).astype(np.float32)
                pair.gpu.append_rope(layer, torch_gpu.from_numpy(rows.copy()).cuda())
                assert pair.cpu.append_rope(layer, rows, pair.cos, pair.sin) == 0
    pair.activate(270, 64)
    pair.run([(0, 18000), (1, 3000)], rng, expect_sparse=True)
    pair.run([(0, 18001), (1, 3001)], rng, fused=True, expect_sparse=True)


def test_folded_summaries_through_block_ends_and_truncation(torch_gpu):
    """One token per step from position 300: the first step after activation recomputes its block from the keys
    below the new length, later steps fold each key into the summary; with no window every completed block is a
    candidate at once (positions 383 and 447 rank the block they complete). After a truncation the next append
    recomputes (the summary covered keys past the new length), then folding resumes; a two-token step and a step
    that overwrites an earlier position recompute too."""
    say("page activation folds")
    pair = PagePair(torch_gpu, page=128, max_positions=1024, slots=2, max_pages=24)
    rng = np.random.default_rng(8)
    prefill(pair, rng, [(0, 300)])
    pair.activate(2, 0)
    for position in range(300, 460):
        pair.run([(0, position)], rng, expect_sparse=True)
    pair.call("truncate", 0, 430)
    for position in range(430, 470):
        pair.run([(0, position)], rng, expect_sparse=True)
    pair.run([(0, 470), (0, 471)], rng, prompt_start=0)
    for position in range(472, 480):
        pair.run([(0, position)], rng, expect_sparse=True)
    pair.check_contents(0)


SMALL_PAGE_SHAPES = [
    # (heads, kv_heads, head_dim, precision, page)
    (28, 4, 128, "f16", 256),
    (14, 2, 64, "f32", 64),
    (8, 8, 128, "f16", 128),
]


@pytest.mark.parametrize("heads,kv_heads,head_dim,precision,page", SMALL_PAGE_SHAPES)
@pytest.mark.parametrize("activation_page", [16, 32])
@pytest.mark.parametrize("selection", ["key_bound", "random"])
def test_small_activation_pages(torch_gpu, heads, kv_heads, head_dim, precision, page, activation_page, selection):
    """KvPageActivation.PageTokens 16 and 32 (KvPageActivation.cs:12-13, 33-36): summaries per 16- or 32-position
    page, selection over those pages, and decode steps that read a listed page's 64-key block with the keys outside
    the page masked. Windows that end inside a 64-key block, a budget past one tile of 64 candidates, a slot with
    two tokens and a token past the prompt boundary; then the page size changes while activation stays on (the
    summaries are rebuilt) and back."""
    say("small activation pages", heads, kv_heads, head_dim, precision, page, activation_page, selection)
    pair = PagePair(torch_gpu, heads=heads, kv_heads=kv_heads, head_dim=head_dim, precision=precision, page=page,
                    growth=256, max_positions=4096, slots=4, max_pages=4096 // page * 4 + 8)
    rng = np.random.default_rng(head_dim + heads + activation_page + len(selection))
    prefill(pair, rng, [(0, 2500), (1, 900), (2, 300)])
    pair.activate(3, 40, selection=selection, seed=5, page_tokens=activation_page)
    pair.run([(0, 2500), (1, 900), (2, 300)], rng, expect_sparse=True)
    pair.run([(0, 2501), (1, 901), (1, 902), (2, 301)], rng, prompt_start=3, expect_sparse=True)
    pair.activate(70, 100, selection=selection, seed=-7, page_tokens=activation_page)
    pair.run([(0, 2502), (1, 903)], rng, expect_sparse=True)
    pair.run([(0, 2503), (1, 904), (2, 302)], rng, fused=True, expect_sparse=True)
    other = 48 - activation_page  # 16 <-> 32
    pair.activate(4, 0, selection=selection, page_tokens=other)
    pair.run([(0, 2504), (1, 905)], rng, expect_sparse=True)
    pair.activate(2, 17, selection=selection, page_tokens=activation_page)
    for position in range(2505, 2525):
        pair.run([(0, position), (1, position - 1600)], rng, expect_sparse=True)
    pair.check_contents(0)


@pytest.mark.parametrize("activation_page", [16, 32])
def test_small_page_folds_through_page_ends_and_truncation(torch_gpu, activation_page):
    """One token per step with no window: each completed 16- or 32-position page is a candidate at once, its
    summary folded key by key from the page's first position; a truncation inside a page and a two-token step make
    the next append recompute, then folding resumes."""
    say("small page folds", activation_page)
    pair = PagePair(torch_gpu, page=128, max_positions=1024, slots=2, max_pages=24)
    rng = np.random.default_rng(80 + activation_page)
    prefill(pair, rng, [(0, 300)])
    pair.activate(2, 0, page_tokens=activation_page)
    for position in range(300, 380):
        pair.run([(0, position)], rng, expect_sparse=True)
    pair.call("truncate", 0, 357)
    for position in range(357, 380):
        pair.run([(0, position)], rng, expect_sparse=True)
    pair.run([(0, 380), (0, 381)], rng, prompt_start=0)
    for position in range(382, 400):
        pair.run([(0, position)], rng, expect_sparse=True)
    pair.check_contents(0)


@pytest.mark.parametrize("activation_page,budget", [(16, 70), (16, 5), (32, 300)])
def test_many_candidates_take_the_sort(torch_gpu, activation_page, budget):
    """Rows of more than 1,024 candidate pages (16-position pages over an 18,000-position slot: 1,108 candidates;
    32-position pages over 40,000: 1,235), whose per-job merge sorts the kept keys instead of ranking each by binary
    searches, next to a short row that takes the search (both merges run in one step: the step's largest job picks
    the kernel)."""
    say("page activation many candidates", activation_page, budget)
    length = 18000 if activation_page == 16 else 40000
    pair = PagePair(torch_gpu, page=256, growth=1024, max_positions=length + 2048, slots=2,
                    max_pages=2 * ((length + 2048) // 256) + 8, step_tokens=1024)
    rng = np.random.default_rng(60 + activation_page + budget)
    for slot, count in ((0, length), (1, 3000)):
        for first in range(0, count, 1024):
            tokens = [(slot, p) for p in range(first, min(count, first + 1024))]
            assert pair.cpu.step(tokens) == 0
            pair.gpu.step(tokens)
            for layer in range(pair.layers):
                rows = rng.standard_normal((len(tokens), pair.width)).astype(np.float32)
                pair.gpu.append_rope(layer, torch_gpu.from_numpy(rows.copy()).cuda())
                assert pair.cpu.append_rope(layer, rows, pair.cos, pair.sin) == 0
    pair.activate(budget, 64, page_tokens=activation_page)
    pair.run([(0, length), (1, 3000)], rng, expect_sparse=True)
    pair.run([(0, length + 1), (1, 3001)], rng, fused=True, expect_sparse=True)


def test_page_activation_under_the_adaptive_split(torch_gpu):
    """Listed rows (KV page activation) split by measured XCD speeds (SYNAPSE_KV_OPTION_ADAPTIVE_SPLIT): several
    steps, so the weights move, each against the restatement's sparse attention."""
    from synapse_amd.native import OPTION_ADAPTIVE_SPLIT

    say("page activation, adaptive split")
    pair = PagePair(torch_gpu, heads=28, kv_heads=4, head_dim=128, precision="f16", page=64, growth=256,
                    max_positions=2048, slots=4, max_pages=2048 // 64 * 4 + 8)
    rng = np.random.default_rng(505)
    prefill(pair, rng, [(0, 1500), (1, 700), (2, 1100)])
    pair.gpu.set_option(OPTION_ADAPTIVE_SPLIT, 1)
    pair.activate(6, 128, selection="key_bound")
    for step in range(8):
        pair.run([(0, 1500 + step), (1, 700 + step), (2, 1100 + step)], rng, fused=step % 2 == 0, expect_sparse=True)
    pair.check_contents(0)
