"""Benchmark of the north-star workload: Qwen2.5-7B-shaped batched decode (config C3).

One step = one decode token for each of 16 sequences: for each of the 28 layers, the fused RoPE + FP16 KV append
and the GQA split-K flash-decode attention over the paged cache (the per-layer pairs run back to back; the
projections around them are outside this path). Lengths are drawn uniform in [1,024, 32,768] from the seed;
the KV cache is pre-filled through the same append path with N(0,1) fp32 K/V. Inputs are resident in HBM when
the timed region starts.

Prints one JSON line: the whole-job tokens/s, the step's algorithmic HBM GB/s (mean, median and p95 step time),
the dominant kernel's roofline (decode attention, timed with HIP events on the cache's stream over the timed
region, against the published 8 TB/s and the streaming-read ceiling measured in the same run) and the CPU baseline
(the restatement of Qwen2CpuAttention + the append, timed on host threads over one layer of the same workload and
the same rows).

Inputs come from bench_support/inputs.py: splitmix64 counters -> Box-Muller in double -> fp32 N(0,1), stream seed
20261201 + the config's offset (fill rows) or + 100 + offset (the decode rows); C3's lengths are
1024 + splitmix64 output mod 31,745 of stream 20261201 + 3. The seeds are recorded in the JSON line.
"""

from __future__ import annotations

import argparse
import gc
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from bench_support.inputs import BASE_SEED, TorchNormals, row_base  # noqa: E402
from bench_support.inputs import lengths as draw_lengths  # noqa: E402

METRIC = "decode attn+KV-append tokens/s, HBM GB/s (% of peak), 7B shape @32k ctx"
PEAK_HBM_GBPS = 8000.0
SEED = BASE_SEED
CONFIG_OFFSET = 3  # config C3
ROWS_OFFSET = 100  # decode / query rows: stream SEED + ROWS_OFFSET + config offset
LAYERS, HEADS, KV_HEADS, HEAD_DIM = 28, 28, 4, 128
SEQUENCES = 16
PAGE_TOKENS = 256
GROWTH = 1024
KV_BYTES_PER_TOKEN_LAYER = 2 * KV_HEADS * HEAD_DIM * 2  # K + V, FP16
PROFILES = ROOT / "profiles"


def log(message: str) -> None:
    print(message, file=sys.stderr, flush=True)


def lengths_for(seed: int) -> np.ndarray:
    return np.array(draw_lengths(seed, SEQUENCES, 1024, 32768), dtype=np.int64)


def cpu_info() -> dict:
    """The host the CPU baseline runs on: model string, nproc, and the CPUs this process may use."""
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return {"model": model, "nproc": os.cpu_count(), "usable": usable}


def cpu_threads(args) -> int:
    """Threads for the CPU baseline: --cpu-threads, else the usable CPUs capped at 16, the CPU share a one-GPU box
    grants a job whatever nproc shows."""
    return args.cpu_threads or min(16, cpu_info()["usable"])


class Rows:
    """Seeded rows of one config on the device: the fill stream (K/V columns of [slot][layer][position] rows) and
    the decode-row stream."""

    def __init__(self, torch, offset: int, heads: int, head_dim: int, width: int):
        self.torch = torch
        self.generator = TorchNormals(torch)
        self.fill_seed = SEED + offset
        self.rows_seed = SEED + ROWS_OFFSET + offset
        self.width = width
        self.kv_columns = slice(heads * head_dim, width)

    def fill(self, out, slot: int, layer: int, first: int) -> None:
        """out[r] = the K/V columns of row `first + r` of (slot, layer) (Q columns zero: append reads K and V)."""
        self.generator.fill_rows(out, self.fill_seed, row_base(slot, layer, first, self.width), self.kv_columns)

    def decode(self, layers: int, tokens: int):
        """[layers][tokens][width] decode rows: row t of layer l is row t of block (0, l) of the decode stream."""
        out = self.torch.empty((layers, tokens, self.width), device="cuda")
        for layer in range(layers):
            self.generator.fill_rows(out[layer], self.rows_seed, row_base(0, layer, 0, self.width))
        return out

    def seeds(self) -> dict:
        return {"fill": self.fill_seed, "rows": self.rows_seed, "generator": "bench_support/inputs.py splitmix64 "
                "counters -> Box-Muller (double) -> fp32"}


def step_times(torch, stream, run, repetitions: int):
    """Runs run(index) `repetitions` times with an event after each; returns (wall seconds, per-step seconds).
    Python's garbage collector is paused over the timed region (a collection there can hold the host back long
    enough for the device to run dry)."""
    events = [torch.cuda.Event(enable_timing=True) for _ in range(repetitions + 1)]
    torch.cuda.synchronize()
    collecting = gc.isenabled()
    gc.collect()
    gc.disable()
    try:
        begin = time.perf_counter()
        events[0].record(stream)
        for index in range(repetitions):
            run(index)
            events[index + 1].record(stream)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - begin
    finally:
        if collecting:
            gc.enable()
    steps = [events[i].elapsed_time(events[i + 1]) * 1e-3 for i in range(repetitions)]
    return elapsed, steps


def step_statistics(steps) -> dict:
    ordered = sorted(steps)
    p95 = ordered[min(len(ordered) - 1, int(math.ceil(0.95 * len(ordered))) - 1)]
    return {"ms_per_step_median": round(statistics.median(ordered) * 1e3, 4), "ms_per_step_p95": round(p95 * 1e3, 4),
            "ms_per_step_min": round(ordered[0] * 1e3, 4)}


def measured_peaks(mfma: bool = False, read_bytes: int | None = None) -> dict:
    """The device's measured ceilings in this run (bench_support/calibrate.py).

    With `read_bytes`, also the plain streaming read rate over that many bytes (the launch's own transfer size).
    """
    from bench_support.calibrate import measure

    result = measure(gib=2.0, repeats=5, mfma=mfma, read_sizes=(read_bytes,) if read_bytes else (),
                     pattern_sizes=(read_bytes,) if read_bytes else ())
    out = {"read_gbps": result["read_gbps"], "copy_gbps": result["copy_gbps"],
           "source": "bench_support/calibrate.py: 2 GiB streaming read with 16-byte non-temporal loads (best of "
                     "8/16/32 waves per CU) and copy, measured in this run"}
    if mfma:
        out["mfma_f16_tflops"] = result["mfma_f16_tflops"]
        out["mfma_f16_16x16x32_tflops"] = max(v for k, v in result.items() if k.startswith("mfma_f16_16x16x32"))
        out["source"] += "; FP16 MFMA chains (v_mfma_f32_32x32x16_f16 and _16x16x32_f16, 8 or 16 waves per CU)"
    if read_bytes:
        (size, gbps), = result["read_gbps_at_bytes"].items()
        out["read_gbps_same_size"] = gbps
        out["same_size_bytes"] = size
        if result.get("pattern_gbps_at_bytes"):
            (size, gbps), = result["pattern_gbps_at_bytes"].items()
            out["pattern_gbps_same_size"] = gbps
            out["pattern_source"] = ("bench_support/calibrate.py pattern_kernel: the decode kernel's loads without its "
                                     "arithmetic (one wave per SIMD, 32 KiB steps through two register sets), "
                                     f"{size} bytes")
    return out


def measured_traffic() -> dict | None:
    """HBM bytes per decode launch from the committed rocprofv3 PMC summary, when it exists."""
    path = PROFILES / "decode_attention_c3_traffic.json"
    if not path.exists():
        return None
    return json.loads(path.read_text())


def prefill(cache, torch, lengths, rows: Rows, chunk=4096):
    """Fills every sequence through step + append_rope in prompt chunks of the fill stream's rows."""
    buffer = torch.empty((chunk, rows.width), device="cuda")
    for slot, length in enumerate(lengths.tolist()):
        for first in range(0, length, chunk):
            count = min(chunk, length - first)
            cache.step([(slot, p) for p in range(first, first + count)])
            for layer in range(LAYERS):
                rows.fill(buffer[:count], slot, layer, first)
                cache.append_rope(layer, buffer[:count])
    torch.cuda.synchronize()


def parse_kv_pages(text: str | None) -> dict | None:
    """--kv-pages <budget>:<window>[:p16|p32|p64][:random[:seed]] (the reference CLI's option, ADR-016;
    GenerationOptions.cs:31)."""
    if text is None:
        return None
    usage = "--kv-pages takes <budget>:<window>[:p16|p32|p64][:random[:seed]]"
    parts = text.split(":")
    if len(parts) < 2:
        sys.exit(usage)
    budget, window = int(parts[0]), int(parts[1])
    rest = parts[2:]
    page = 64
    if rest and rest[0] in ("p16", "p32", "p64"):
        page = int(rest[0][1:])
        rest = rest[1:]
    if len(rest) > 2 or (rest and rest[0] != "random"):
        sys.exit(usage)
    random = bool(rest)
    seed = int(rest[1]) if len(rest) > 1 else 0
    name = f"kvpages{budget}w{window}" + ("" if page == 64 else f"p{page}") + ("r" if random else "")
    return {"budget": budget, "window": window, "page": page, "selection": "random" if random else "key_bound",
            "seed": seed, "name": name}


def attended_keys(position: int, activation: dict) -> int:
    """Positions a decode token at `position` attends (KvPageSelector.Select)."""
    size = activation["page"]
    count = position + 1
    window_page = max(0, count - activation["window"]) // size
    if max(0, window_page - 1) <= activation["budget"]:
        return count
    return size + activation["budget"] * size + (count - window_page * size)


def read_keys(position: int, activation: dict) -> int:
    """Keys the decode kernel reads for that token: one 64-key block per listed page (its keys outside the page
    masked), or the dense row."""
    size = activation["page"]
    count = position + 1
    window_page = max(0, count - activation["window"]) // size
    if max(0, window_page - 1) <= activation["budget"]:
        return count
    return 64 * (1 + activation["budget"] + position // size - window_page + 1)


def cpu_baseline(torch, lengths, rows: Rows, decode_rows, threads: int) -> dict:
    """The reference CPU path restated in C++ (oracle/: Qwen2CpuAttention with the fused RoPE + FP16 append), timed
    on host threads over one layer of one decode step: the same lengths and the same rows as the GPU run (layer 0's
    fill rows and decode rows, generated on the device and copied), extrapolated to 28 layers."""
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_ffi import PagedCache, rope_table

    max_positions = int(lengths.max()) + 1024
    pages = int(sum(-(-(int(n) + 1) // PAGE_TOKENS) for n in lengths)) + SEQUENCES
    cache = PagedCache(1, HEADS, KV_HEADS, HEAD_DIM, max_positions, PAGE_TOKENS, PAGE_TOKENS, 1, SEQUENCES, pages,
                       4096)
    cos, sin = rope_table(HEAD_DIM, 1e6, max_positions)
    buffer = torch.empty((4096, rows.width), device="cuda")
    start = time.perf_counter()
    for slot, length in enumerate(lengths.tolist()):
        assert cache.reserve(slot, length + 1) == 0
        for first in range(0, length, 4096):
            count = min(4096, length - first)
            rows.fill(buffer[:count], slot, 0, first)
            block = buffer[:count].cpu().numpy()
            assert cache.step([(slot, p) for p in range(first, first + count)]) == 0
            assert cache.append_rope(0, block, cos, sin) == 0
    fill_seconds = time.perf_counter() - start
    tokens = [(slot, int(length)) for slot, length in enumerate(lengths)]
    assert cache.step(tokens) == 0
    layer_rows = decode_rows[0].cpu().numpy()
    out = np.zeros((SEQUENCES, HEADS * HEAD_DIM), dtype=np.float32)

    def layer() -> float:
        # The append's wall time plus the attention's own time as the restatement reports it: the restatement
        # first widens the paged FP16 rows into a dense FP32 view, a step of its own layout that the reference's
        # CPU path (dense FP32 arrays) does not have, so that part is not counted.
        qkv = layer_rows.copy()
        begin = time.perf_counter()
        assert cache.append_rope(0, qkv, cos, sin) == 0
        append = time.perf_counter() - begin
        return append + cache.attention(0, qkv, out, threads)

    layer()  # warm-up
    times = [layer() for _ in range(3)]
    layer_seconds = statistics.median(times)
    step_seconds = layer_seconds * LAYERS
    return {
        "value": round(SEQUENCES / step_seconds, 3),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (
            f"one layer of one decode step for the 16 drawn lengths (sum {int(lengths.sum())} keys): the fused RoPE + "
            f"FP16 append and Qwen2CpuAttention (4-lane dot, 3-pass softmax) over FP16 pages widened per "
            f"Fp16.ToSingle (the widening into the restatement's dense view not timed), C++ restatement, "
            f"{threads} std::threads; median of 3 after 1 warm-up = "
            f"{layer_seconds * 1e3:.1f} ms, x28 layers; the GPU run's layer-0 rows; fill {fill_seconds:.1f} s"
        ),
        "cpu": cpu_info(),
        "ms_per_layer": round(layer_seconds * 1e3, 3),
    }


def prefill_config(args, torch) -> dict:
    """Config C5: a 2,048-token chunk attends causally over a 63,488-token FP16 cache plus itself (65,536 keys) in
    all 28 layers; one timed repetition = the chunk's 28 append_attention calls (append + MFMA prefill + merge)."""
    from synapse_amd import PagedKvCache

    cached, chunk = 63488, 2048
    cache = PagedKvCache(layers=LAYERS, heads=HEADS, kv_heads=KV_HEADS, head_dim=HEAD_DIM, max_positions=65536,
                         growth_positions=GROWTH, page_tokens=PAGE_TOKENS, precision="f16", session_slots=1,
                         step_tokens=4096, max_pages=256)
    stream = torch.cuda.current_stream()
    cache.set_stream(stream)
    if args.prefill_split_keys:
        cache.set_prefill_split_keys(args.prefill_split_keys)
    cache.reserve(0, cached + chunk)
    width = (HEADS + 2 * KV_HEADS) * HEAD_DIM
    rows = Rows(torch, 5, HEADS, HEAD_DIM, width)
    fill_slot(cache, torch, 0, 0, cached, 4096, LAYERS, rows)
    qkv = rows.decode(LAYERS, chunk)
    out = torch.empty((LAYERS, chunk, HEADS * HEAD_DIM), device="cuda")
    cache.step([(0, cached + j) for j in range(chunk)])

    def run(_index) -> None:
        for layer in range(LAYERS):
            cache.append_attention(layer, qkv[layer], out[layer])

    for index in range(args.warmup):
        run(index)
    torch.cuda.synchronize()
    cache.profile_begin()
    elapsed, per_step = step_times(torch, stream, run, args.steps)
    kernels = cache.profile_end()
    cache.close()
    # Key visits per query head: each chunk token sees the whole cache plus the chunk up to itself.
    visits = chunk * cached + chunk * (chunk + 1) // 2
    flops_per_layer = HEADS * visits * 4 * HEAD_DIM
    seconds = elapsed / args.steps
    tflops = LAYERS * flops_per_layer / seconds / 1e12
    prefill_launches, prefill_ms = kernels["prefill"]
    kernel_tflops = flops_per_layer / (prefill_ms * 1e-3 / prefill_launches) / 1e12
    peaks = measured_peaks(mfma=True)
    line = {
        "metric": "chunked-prefill attention TFLOP/s (MFMA FP16), 7B shape, 2,048-token chunk over 63,488 cached",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(seconds * 1e3, 3), **step_statistics(per_step), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic N(0,1) fp32 rows (splitmix64/Box-Muller)", "seeds": rows.seeds(),
        "config": {"workload": "C5: 28 layers x (append + causal prefill, split-K merge when planned), 65,536 keys",
                   "flops_per_layer": flops_per_layer},
        "roofline": {"bound": "mfma", "kernel": "prefill_f16_kernel<128>", "achieved": round(kernel_tflops, 2),
                     "peak": 2500.0, "unit": "TFLOP/s", "frac": round(kernel_tflops / 2500.0, 4), "traffic": None,
                     "measured_peak": peaks,
                     "frac_of_measured_mfma": round(kernel_tflops / peaks["mfma_f16_tflops"], 4),
                     "avg_launch_us": round(prefill_ms * 1e3 / prefill_launches, 2),
                     "kernels_ms": {kind: round(ms, 3) for kind, (count, ms) in kernels.items()}},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_c5(torch, rows, qkv, cached, chunk, cpu_threads(args))
    return line


def cpu_baseline_c5(torch, rows: Rows, qkv, cached: int, chunk: int, threads: int) -> dict:
    """C5's CPU baseline: the C++ restatement of the reference's prompt attention (Qwen2CpuAttention over every
    query token, causal) on one layer with the GPU run's layer-0 rows. The sample is the chunk's last 128 tokens
    (each attends about 65,400 keys) after the other 1,920 were appended; reported as TFLOP/s of that sample, the
    GPU figure's unit (the whole layer would take minutes of CPU time)."""
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_ffi import PagedCache, rope_table

    sample = 128
    total = cached + chunk
    cache = PagedCache(1, HEADS, KV_HEADS, HEAD_DIM, total, GROWTH, PAGE_TOKENS, 1, 1, total // PAGE_TOKENS, 4096)
    cos, sin = rope_table(HEAD_DIM, 1e6, total)
    assert cache.reserve(0, total) == 0
    buffer = torch.empty((4096, rows.width), device="cuda")
    for first in range(0, cached, 4096):
        rows.fill(buffer, 0, 0, first)
        assert cache.step([(0, p) for p in range(first, first + 4096)]) == 0
        assert cache.append_rope(0, buffer.cpu().numpy(), cos, sin) == 0
    layer_rows = qkv[0].cpu().numpy()
    head = chunk - sample
    assert cache.step([(0, cached + j) for j in range(head)]) == 0
    assert cache.append_rope(0, layer_rows[:head].copy(), cos, sin) == 0
    assert cache.step([(0, cached + j) for j in range(head, chunk)]) == 0
    block = layer_rows[head:].copy()
    out = np.zeros((sample, HEADS * HEAD_DIM), dtype=np.float32)
    begin = time.perf_counter()
    assert cache.append_rope(0, block, cos, sin) == 0
    seconds = time.perf_counter() - begin
    seconds += cache.attention(0, block, out, threads)  # without the restatement's dense-view copy
    visits = sum(cached + j + 1 for j in range(head, chunk))
    flops = HEADS * visits * 4 * HEAD_DIM
    return {
        "value": round(flops / seconds / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
        "sample": f"the chunk's last {sample} query tokens of one layer ({flops / 1e9:.0f} GFLOP, {seconds:.2f} s): "
                  f"RoPE + FP16 append + Qwen2CpuAttention, C++ restatement on {threads} std::threads, the GPU run's "
                  f"layer-0 rows; x28 layers and the whole chunk scale linearly in FLOPs",
        "cpu": cpu_info(),
    }


def fill_slot(cache, torch, slot, first, count, chunk, layers, rows: Rows):
    """Appends positions [first, first + count) of `slot` through step + append_rope in prompt chunks."""
    buffer = torch.empty((chunk, cache.qkv_width), device="cuda")
    for start in range(first, first + count, chunk):
        size = min(chunk, first + count - start)
        cache.step([(slot, p) for p in range(start, start + size)])
        for layer in range(layers):
            rows.fill(buffer[:size], slot, layer, start)
            cache.append_rope(layer, buffer[:size])
    torch.cuda.synchronize()


def apply_options(args, cache) -> None:
    if args.split_keys:
        cache.set_split_keys(args.split_keys)
    if args.prefetch is not None:
        from synapse_amd.native import OPTION_DECODE_PREFETCH

        cache.set_option(OPTION_DECODE_PREFETCH, args.prefetch)
    if args.segment_cost is not None:
        from synapse_amd.native import OPTION_SEGMENT_COST

        cache.set_option(OPTION_SEGMENT_COST, args.segment_cost)
    if args.adaptive_split is not None:
        from synapse_amd.native import OPTION_ADAPTIVE_SPLIT

        cache.set_option(OPTION_ADAPTIVE_SPLIT, args.adaptive_split)


def timed(torch, cache, run, repetitions, profile_every=1):
    """Wall seconds per repetition of `run` (between synchronizations), the cache's kernel profile, and each
    repetition's seconds (HIP events on the stream)."""
    from synapse_amd.native import OPTION_PROFILE_EVERY

    cache.set_option(OPTION_PROFILE_EVERY, profile_every)
    cache.profile_begin()
    elapsed, per_step = step_times(torch, torch.cuda.current_stream(), run, repetitions)
    return elapsed / repetitions, cache.profile_end(), per_step


def kernel_us(kernels, kind):
    launches, ms = kernels.get(kind, (0, 0.0))
    return ms * 1e3 / launches if launches else None


def decode_line(args, *, metric, workload, tokens_per_step, seconds, bytes_per_step, layers, decode_bytes_per_launch,
                kernels, data, extra=None):
    decode_us = kernel_us(kernels, "decode")
    decode_gbps = decode_bytes_per_launch / (decode_us * 1e-6) / 1e9 if decode_us else None
    line = {
        "metric": metric, "value": round(tokens_per_step / seconds, 2), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(seconds * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16" if "FP16" in workload else "f32", "data": data,
        "config": {"workload": workload, "layers": layers},
        "hbm_gbps": round(bytes_per_step / seconds / 1e9, 1),
        "hbm_frac_of_peak": round(bytes_per_step / seconds / 1e9 / PEAK_HBM_GBPS, 4),
        "roofline": {"bound": "hbm", "kernel": "decode_kernel (fused append + split-K decode)",
                     "achieved": round(decode_gbps, 1) if decode_gbps else None, "peak": PEAK_HBM_GBPS,
                     "unit": "GB/s", "frac": round(decode_gbps / PEAK_HBM_GBPS, 4) if decode_gbps else None,
                     "traffic": None, "algorithmic_bytes_per_launch": int(decode_bytes_per_launch),
                     "avg_launch_us": round(decode_us, 2) if decode_us else None,
                     "kernels_ms": {kind: round(ms, 3) for kind, (count, ms) in kernels.items()}},
    }
    if extra:
        line.update(extra)
    return line


def config_c1(args, torch) -> dict:
    """Config C1: 0.5B shape (24 layers, 14 q / 2 KV heads, head_dim 64), FP32 KV, one sequence decoding over
    4,096 cached tokens. One step = 24 x append_attention for the next position."""
    from synapse_amd import PagedKvCache

    layers, heads, kv_heads, d, cached = 24, 14, 2, 64, 4096
    total = args.warmup + args.steps
    cache = PagedKvCache(layers=layers, heads=heads, kv_heads=kv_heads, head_dim=d, max_positions=8192,
                         growth_positions=1024, page_tokens=256, precision="f32", session_slots=1,
                         step_tokens=512, max_pages=32)
    cache.set_stream(torch.cuda.current_stream())
    apply_options(args, cache)
    cache.reserve(0, cached + total + 1)
    rows = Rows(torch, 1, heads, d, cache.qkv_width)
    fill_slot(cache, torch, 0, 0, cached, 512, layers, rows)
    qkv = rows.decode(layers, 1)
    out = torch.empty((layers, 1, heads * d), device="cuda")

    def run(index):
        cache.step([(0, cached + index)])
        for layer in range(layers):
            cache.append_attention(layer, qkv[layer], out[layer])

    for index in range(args.warmup):
        run(index)
    seconds, kernels, per_step = timed(torch, cache, lambda i: run(args.warmup + i), args.steps,
                                       profile_every=layers // 2)
    row = 2 * kv_heads * d * 4  # K + V bytes per position per layer (FP32)
    keys = cached + args.warmup + (args.steps + 1) / 2
    launch_bytes = keys * row + row + heads * d * 4 + 2 * kv_heads * d * 4
    cache.close()
    line = decode_line(args, metric="C1 decode attn+KV-append tokens/s, 0.5B FP32 KV @4k ctx",
                       workload="C1: Qwen2.5-0.5B-shaped single-sequence decode, FP32 KV, 4,096 cached tokens, "
                                "24 layers", tokens_per_step=1, seconds=seconds,
                       bytes_per_step=layers * (launch_bytes + heads * d * 4), layers=layers,
                       decode_bytes_per_launch=launch_bytes, kernels=kernels,
                       data="synthetic N(0,1) fp32 rows (splitmix64/Box-Muller)",
                       extra={"seeds": rows.seeds(), **step_statistics(per_step)})
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_c1(torch, rows, cached, args.warmup + args.steps, cpu_threads(args))
    return line


def cpu_baseline_c1(torch, rows: Rows, cached: int, decoded: int, threads: int) -> dict:
    """C1 is the reference CPU configuration itself (Qwen2CpuAttention over an FP32 Qwen2KvCache): the C++
    restatement runs whole decode steps of all 24 layers (RoPE + append + attention per layer) over the same rows
    the GPU run used (fill rows of every layer, the decode rows), after the same 4,096-token fill."""
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_ffi import PagedCache, rope_table

    layers, heads, kv_heads, d = 24, 14, 2, 64
    steps = 200
    cache = PagedCache(layers, heads, kv_heads, d, 8192, 1024, 256, 0, 1, 32, 512)
    cos, sin = rope_table(d, 1e6, 8192)
    assert cache.reserve(0, cached + steps + 1) == 0
    buffer = torch.empty((512, rows.width), device="cuda")
    for first in range(0, cached, 512):
        assert cache.step([(0, p) for p in range(first, first + 512)]) == 0
        for layer in range(layers):
            rows.fill(buffer, 0, layer, first)
            assert cache.append_rope(layer, buffer.cpu().numpy(), cos, sin) == 0
    decode_rows = rows.decode(layers, 1).cpu().numpy()
    out = np.zeros((1, heads * d), dtype=np.float32)
    total = 0.0
    for step in range(steps):
        rotated = decode_rows.copy()
        begin = time.perf_counter()
        assert cache.step([(0, cached + step)]) == 0
        for layer in range(layers):
            assert cache.append_rope(layer, rotated[layer], cos, sin) == 0
        total += time.perf_counter() - begin
        for layer in range(layers):
            # The attention's own time as the restatement reports it (its copy of the paged rows into a dense
            # view is a step of its layout, not of the reference's dense FP32 cache).
            total += cache.attention(layer, rotated[layer], out, threads)
    seconds = total / steps
    return {
        "value": round(1.0 / seconds, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
        "sample": f"{steps} whole decode steps (24 layers each: RoPE + FP32 append + Qwen2CpuAttention) after the "
                  f"4,096-token fill, C++ restatement on {threads} std::threads, the GPU run's rows (attention timed "
                  f"as the restatement reports it, without its dense-view copy); "
                  f"{seconds * 1e3:.3f} ms per step",
        "cpu": cpu_info(),
    }


def config_c2(args, torch) -> dict:
    """Config C2: 0.5B FP16 paged cache filled to 32,768 positions in 64 x 512-token appends, then single-sequence
    decode steps over it, then a 1,024-position reserve that contracts the slot to 4 pages."""
    from synapse_amd import PagedKvCache

    layers, heads, kv_heads, d = 24, 14, 2, 64
    filled = 32768
    cache = PagedKvCache(layers=layers, heads=heads, kv_heads=kv_heads, head_dim=d, max_positions=65536,
                         growth_positions=1024, page_tokens=256, precision="f16", session_slots=1,
                         step_tokens=512, max_pages=256)
    cache.set_stream(torch.cuda.current_stream())
    apply_options(args, cache)
    source = Rows(torch, 2, heads, d, cache.qkv_width)
    rows = torch.empty((64, 512, cache.qkv_width), device="cuda")
    for chunk in range(64):
        source.fill(rows[chunk], 0, 0, chunk * 512)  # one set of rows serves every layer of a chunk
    torch.cuda.synchronize()

    # Fill: 64 chunks x 24 layers of append_rope (RoPE + FP16 RNE store), growth through the capacity policy.
    def fill_chunk(chunk):
        cache.step([(0, p) for p in range(chunk * 512, chunk * 512 + 512)])
        for layer in range(layers):
            cache.append_rope(layer, rows[chunk])

    fill_seconds, fill_kernels, _ = timed(torch, cache, fill_chunk, 64)
    width = cache.qkv_width * 4
    fill_bytes = 512 * layers * (width + (heads + kv_heads) * d * 4 + 2 * kv_heads * d * 2)
    qkv = source.decode(layers, 1)
    out = torch.empty((layers, 1, heads * d), device="cuda")

    def run(index):
        cache.step([(0, filled + index)])
        for layer in range(layers):
            cache.append_attention(layer, qkv[layer], out[layer])

    for index in range(args.warmup):
        run(index)
    seconds, kernels, per_step = timed(torch, cache, lambda i: run(args.warmup + i), args.steps,
                                       profile_every=layers // 2)
    row = 2 * kv_heads * d * 2
    keys = filled + args.warmup + (args.steps + 1) / 2
    launch_bytes = keys * row + row + heads * d * 4 + 2 * kv_heads * d * 4
    torch.cuda.synchronize()
    begin = time.perf_counter()
    cache.reserve(0, 1024)
    cache.synchronize()
    contract_ms = (time.perf_counter() - begin) * 1e3
    info = cache.slot_info(0)
    stats = cache.page_stats()
    cache.close()
    append_us = kernel_us(fill_kernels, "append")
    return decode_line(
        args, metric="C2 decode attn+KV-append tokens/s, 0.5B FP16 paged KV @32k ctx",
        workload="C2: Qwen2.5-0.5B-shaped single sequence, FP16 paged KV (256-token pages): fill to 32,768 in "
                 "64 x 512-token appends, decode, contract to 1,024", tokens_per_step=1, seconds=seconds,
        bytes_per_step=layers * (launch_bytes + heads * d * 4), layers=layers, decode_bytes_per_launch=launch_bytes,
        kernels=kernels, data="synthetic N(0,1) fp32 rows (splitmix64/Box-Muller)",
        extra={"seeds": source.seeds(), **step_statistics(per_step), "fill": {"ms": round(fill_seconds * 64 * 1e3, 3), "tokens_per_s": round(512 / fill_seconds, 1),
                        "append_avg_launch_us": round(append_us, 2) if append_us else None,
                        "append_gbps": round(fill_bytes / layers / (append_us * 1e-6) / 1e9, 1) if append_us else None,
                        "kernels_ms": {kind: round(ms, 3) for kind, (count, ms) in fill_kernels.items()}},
               "contract": {"ms": round(contract_ms, 3), "slot": info, "used_pages": stats["used_pages"],
                            "free_pages": stats["free_pages"]}})


def config_c4(args, torch) -> dict:
    """Config C4: a 30,000-token FP16 prefix forked copy-on-write into 8 sequences; each appends a distinct 64-token
    suffix (one step, prompt path, copying the shared partial page), then decodes. Unique bytes count the shared
    prefix once per layer."""
    from synapse_amd import PagedKvCache

    layers, heads, kv_heads, d = LAYERS, HEADS, KV_HEADS, HEAD_DIM
    prefix, forks = 30000, 8
    cache = PagedKvCache(layers=layers, heads=heads, kv_heads=kv_heads, head_dim=d, max_positions=32768,
                         growth_positions=1024, page_tokens=256, precision="f16", session_slots=forks + 1,
                         step_tokens=4096, max_pages=160)
    cache.set_stream(torch.cuda.current_stream())
    apply_options(args, cache)
    rows = Rows(torch, 4, heads, d, cache.qkv_width)
    cache.reserve(0, prefix)
    fill_slot(cache, torch, 0, 0, prefix, 4096, layers, rows)
    for target in range(1, forks + 1):
        cache.fork(0, target)
    suffix = torch.empty((64 * forks, cache.qkv_width), device="cuda")
    for fork in range(forks):
        rows.fill(suffix[64 * fork:64 * fork + 64], fork + 1, 0, prefix)
    suffix_out = torch.empty((64 * forks, heads * d), device="cuda")

    def suffix_step(_):
        cache.step([(slot, prefix + j) for slot in range(1, forks + 1) for j in range(64)])
        for layer in range(layers):
            cache.append_attention(layer, suffix, suffix_out)

    suffix_seconds, suffix_kernels, _ = timed(torch, cache, suffix_step, 1)
    qkv = rows.decode(layers, forks)
    out = torch.empty((layers, forks, heads * d), device="cuda")

    def run(index):
        cache.step([(slot, prefix + 64 + index) for slot in range(1, forks + 1)])
        for layer in range(layers):
            cache.append_attention(layer, qkv[layer], out[layer])

    for index in range(args.warmup):
        run(index)
    seconds, kernels, per_step = timed(torch, cache, lambda i: run(args.warmup + i), args.steps,
                                       profile_every=layers // 2)
    row = 2 * kv_heads * d * 2
    own = 64 + args.warmup + (args.steps + 1) / 2  # each fork's own positions (suffix + decoded), average
    unique = prefix * row + forks * own * row
    logical = forks * (prefix + own) * row
    q_rows = forks * (heads * d * 4 + 2 * kv_heads * d * 4)
    launch_unique = unique + forks * row + q_rows
    launch_logical = logical + forks * row + q_rows
    cache.close()
    line = decode_line(
        args, metric="C4 decode attn+KV-append tokens/s, 7B FP16, 8 COW forks of a 30,000-token prefix",
        workload="C4: Qwen2.5-7B-shaped prefix reuse: 30,000-token FP16 prefix forked copy-on-write into 8 "
                 "sequences, 64-token suffix each, then batched decode, 28 layers", tokens_per_step=forks,
        seconds=seconds, bytes_per_step=layers * (launch_unique + forks * heads * d * 4), layers=layers,
        decode_bytes_per_launch=launch_unique, kernels=kernels,
        data="synthetic N(0,1) fp32 rows (splitmix64/Box-Muller)",
        extra={"seeds": rows.seeds(), **step_statistics(per_step), "suffix_step_ms": round(suffix_seconds * 1e3, 3),
               "suffix_kernels_ms": {kind: round(ms, 3) for kind, (count, ms) in suffix_kernels.items()}})
    decode_us = kernel_us(kernels, "decode")
    if decode_us:
        line["roofline"]["logical_gbps"] = round(launch_logical / (decode_us * 1e-6) / 1e9, 1)
        line["roofline"]["logical_bytes_per_launch"] = int(launch_logical)
    return line


def projection_blob(rng, shapes, bias_flags):
    """One layer's Q8_0 matrices as GGML blocks (random codes, FP16 scales around 1/64) with FP32 biases."""
    parts, matrices, offset = [], [], 0
    for (rows, columns), with_bias in zip(shapes, bias_flags):
        blocks = np.empty((rows, columns // 32, 34), dtype=np.uint8)
        blocks[:, :, 2:] = rng.integers(-127, 128, size=(rows, columns // 32, 32), dtype=np.int8).view(np.uint8)
        scales = (rng.random((rows, columns // 32), dtype=np.float32) * np.float32(1 / 32)).astype(np.float16)
        blocks[:, :, :2] = scales.view(np.uint8).reshape(rows, columns // 32, 2)
        entry = {"weight": offset, "rows": rows, "columns": columns}
        parts.append(blocks.reshape(-1))
        offset += blocks.nbytes
        if with_bias:
            bias = rng.standard_normal(rows).astype(np.float32)
            entry["bias"] = offset
            parts.append(bias.view(np.uint8))
            offset += bias.nbytes
        matrices.append(entry)
    return np.concatenate(parts), matrices


def config_projection(args, torch) -> dict:
    """Q8_0 projections around the attention path on the 7B shape (hidden 3,584; QKV 4,608 rows with biases; o_proj
    3,584 rows accumulating into the residual), 28 layers of distinct weights. The headline is the decode step of
    C3 (16 tokens): weight bytes streamed per second against HBM. The prompt projection of C5 (2,048 tokens) is
    reported beside it in TFLOP/s against the FP32 MFMA peak (the reference's FP32 numeric contract)."""
    from synapse_amd.projection import Q8Weights

    hidden, kv = HEADS * HEAD_DIM, KV_HEADS * HEAD_DIM
    shapes = [(hidden, hidden), (kv, hidden), (kv, hidden), (hidden, hidden)]
    rng = np.random.default_rng(SEED + 7)
    layer_blob, layer_matrices = projection_blob(rng, shapes, [True, True, True, False])
    blob = np.tile(layer_blob, LAYERS)
    matrices = [dict(m, weight=m["weight"] + layer * layer_blob.nbytes,
                     **({"bias": m["bias"] + layer * layer_blob.nbytes} if "bias" in m else {}))
                for layer in range(LAYERS) for m in layer_matrices]
    weights = Q8Weights(blob, matrices)
    stream = torch.cuda.current_stream()
    weights.set_stream(stream)
    log(f"projection weights {weights.device_bytes / 2**20:.1f} MiB on the device")
    qkv_rows = hidden + 2 * kv
    element_bytes = 34 / 32  # codes plus FP16 scales per weight element, as in the GGML blocks

    def measure(tokens: int, repetitions: int):
        x = torch.randn((tokens, hidden), device="cuda")
        qkv = torch.empty((tokens, qkv_rows), device="cuda")
        attention = torch.randn((tokens, hidden), device="cuda")
        residual = torch.randn((tokens, hidden), device="cuda")

        def layer_pair(layer):
            base = 4 * layer
            weights.project([(base, 0), (base + 1, hidden), (base + 2, hidden + kv)], x, qkv)
            weights.project([(base + 3, 0)], attention, residual, accumulate=True)

        def qkv_only(layer):
            base = 4 * layer
            weights.project([(base, 0), (base + 1, hidden), (base + 2, hidden + kv)], x, qkv)

        def o_only(layer):
            weights.project([(4 * layer + 3, 0)], attention, residual, accumulate=True)

        results = {}
        for name, body in (("step", layer_pair), ("qkv", qkv_only), ("o_proj", o_only)):
            for _ in range(args.warmup):
                for layer in range(LAYERS):
                    body(layer)
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            start.record(stream)
            for _ in range(repetitions):
                for layer in range(LAYERS):
                    body(layer)
            stop.record(stream)
            torch.cuda.synchronize()
            results[name] = start.elapsed_time(stop) * 1e-3 / repetitions  # seconds per 28 layers
        return results

    decode_tokens, prompt_tokens = SEQUENCES, 2048
    decode = measure(decode_tokens, args.steps)
    prompt = measure(prompt_tokens, max(1, args.steps // 10))
    qkv_weight = qkv_rows * hidden * element_bytes
    o_weight = hidden * hidden * element_bytes
    qkv_bytes = qkv_weight + decode_tokens * (hidden + qkv_rows) * 4
    o_bytes = o_weight + decode_tokens * hidden * 4 * 3  # input, residual read and write
    step_bytes = LAYERS * (qkv_bytes + o_bytes)
    qkv_us = decode["qkv"] / LAYERS * 1e6
    qkv_gbps = qkv_bytes / (qkv_us * 1e-6) / 1e9
    flops = 2 * prompt_tokens * (qkv_rows + hidden) * hidden
    prompt_tflops = LAYERS * flops / prompt["step"] / 1e12
    qkv_flops = 2 * prompt_tokens * qkv_rows * hidden
    prompt_qkv_tflops = LAYERS * qkv_flops / prompt["qkv"] / 1e12
    line = {
        "metric": "Q8_0 projection (QKV + o_proj) weight-stream GB/s, 7B shape, 16 decode tokens",
        "value": round(step_bytes / decode["step"] / 1e9, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(decode["step"] * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "q8_0 x f32 (f32 accumulate)",
        "data": f"synthetic Q8_0 weights (numpy seed {SEED + 7}), 28 distinct layers; torch N(0,1) activations",
        "config": {"workload": "7B projections: QKV 4,608 x 3,584 with biases + o_proj 3,584 x 3,584 accumulating, "
                               "28 layers, 16 tokens", "decode_tokens": decode_tokens, "prompt_tokens": prompt_tokens},
        "roofline": {"bound": "hbm", "kernel": "project_decode_kernel + reduce_kernel (QKV, 3 segments)",
                     "achieved": round(qkv_gbps, 1),
                     "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": round(qkv_gbps / PEAK_HBM_GBPS, 4),
                     "traffic": None, "algorithmic_bytes_per_launch": int(qkv_bytes),
                     "avg_launch_us": round(qkv_us, 2),
                     "o_proj_avg_launch_us": round(decode["o_proj"] / LAYERS * 1e6, 2)},
        "prompt": {"tokens": prompt_tokens, "ms_per_28_layers": round(prompt["step"] * 1e3, 3),
                   "tflops": round(prompt_tflops, 1), "qkv_tflops": round(prompt_qkv_tflops, 1),
                   "peak_fp32_mfma_tflops": 157.3, "frac": round(prompt_tflops / 157.3, 4)},
    }
    weights.close()
    if not args.no_cpu_baseline:
        sys.path.insert(0, str(ROOT / "tests"))
        from oracle_ffi import q8_project

        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        layer = layer_blob
        segments = []
        for index, m in enumerate(layer_matrices[:3]):
            rows, columns = m["rows"], m["columns"]
            blocks = layer[m["weight"]:m["weight"] + rows * columns // 32 * 34].reshape(rows, -1)
            bias = layer[m["bias"]:m["bias"] + rows * 4].view(np.float32) if "bias" in m else None
            segments.append((blocks, bias, [0, hidden, hidden + kv][index]))
        o = layer_matrices[3]
        o_blocks = layer[o["weight"]:o["weight"] + hidden * hidden // 32 * 34].reshape(hidden, -1)
        x = rng.standard_normal((decode_tokens, hidden), dtype=np.float32)
        out = np.zeros((decode_tokens, qkv_rows), dtype=np.float32)
        residual = np.zeros((decode_tokens, hidden), dtype=np.float32)
        seconds = q8_project(segments, x, out, threads=threads)
        seconds += q8_project([(o_blocks, None, 0)], x, residual, accumulate=True, threads=threads)
        line["cpu_baseline"] = {
            "value": round(LAYERS * (qkv_bytes + o_bytes) / 1e9 / (LAYERS * seconds), 2), "unit": "GB/s",
            "cores": threads, "kind": "port",
            "sample": f"one layer's QKV + o_proj for 16 tokens ({seconds * 1e3:.0f} ms) in the reference's FP32 "
                      f"matrix-vector order (matmul.cu q8_matvec restated in C++), {threads} std::threads, x28 layers",
        }
    return line


def config_ttft(args, torch) -> dict:
    """Time to first token through the whole decoder (synapse_kv_decoder_forward) on a Qwen2.5-0.5B-shaped synthetic
    Q8_0 model with FP16 KV: a 30,000-token document as 512-token prompt chunks (the reference's chunked prefill,
    ADR-007) with logits for its last token only (cold), then a 32-token question over the cached document (warm;
    the question's positions are rewritten on every repetition). The reference's README reports, for this scenario
    on an Apple M2 Pro with the real 0.5B model, 23.8 s cold and 0.13 s for a second question over the cached
    document (context only: other hardware, other weights)."""
    sys.path.insert(0, str(ROOT / "tests"))
    from synapse_amd.decoder import Decoder, DecoderShape
    from synthetic_models import synthetic_model

    document, question, chunk = 30000, 32, 512
    shape = DecoderShape(layers=24, hidden=896, feed_forward=4864, heads=14, kv_heads=2, head_dim=64,
                         vocabulary=151936, context=32768, session_slots=1, step_tokens=chunk, logits_rows=1,
                         kv_precision="f16", growth=1024)
    started = time.perf_counter()
    blob, layout = synthetic_model(shape, seed=SEED + 9)
    model = Decoder(blob, layout, shape)
    log(f"model {blob.nbytes / 2**20:.0f} MiB built and uploaded in {time.perf_counter() - started:.1f} s")
    del blob
    rng = np.random.default_rng(SEED + 9)
    tokens = rng.integers(shape.vocabulary, size=document + question)
    pinned = torch.empty((1, shape.vocabulary), dtype=torch.float32, pin_memory=True).numpy()

    def run(first, last):
        """Positions [first, last) in chunks; logits for the last one. Returns seconds to the logits on the host."""
        torch.cuda.synchronize()
        begin = time.perf_counter()
        for start in range(first, last, chunk):
            stop = min(last, start + chunk)
            logits = model.forward([(0, int(tokens[p]), p, 0 if p == last - 1 else -1) for p in range(start, stop)],
                                   out=pinned)
        seconds = time.perf_counter() - begin
        assert np.isfinite(logits).all()
        return seconds

    run(0, 2048)  # warm-up (kernels, allocations)
    cold = [run(0, document) for _ in range(max(1, args.steps // 10))]
    warm_runs = [run(document, document + question) for _ in range(args.warmup)]
    warm = [run(document, document + question) for _ in range(args.steps)]
    del warm_runs
    model.close()
    cold_s = statistics.median(cold)
    warm_s = statistics.median(warm)
    return {
        "metric": "time to first token: 30,000-token document (cold), then a 32-token question over it (warm), "
                  "0.5B-shaped Q8_0 decoder, FP16 KV",
        "value": round(cold_s, 4), "unit": "s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(cold_s * 1e3, 3), "higher_is_better": False, "scaling": "strong", "vs_baseline": None,
        "dtype": "f32 (Q8_0 weights, FP16 KV)",
        "data": f"synthetic Q8_0 model (numpy seed {SEED + 9}), random token ids",
        "config": {"workload": "ttft: Qwen2.5-0.5B shape (24 layers, hidden 896, ffn 4,864, 14 q / 2 KV heads, "
                               "vocab 151,936), document 30,000 tokens in 512-token chunks, question 32 tokens",
                   "parallelism": "single GPU"},
        "cold_ttft_s": round(cold_s, 4), "cold_runs_s": [round(x, 4) for x in cold],
        "prompt_tokens_per_s": round(document / cold_s, 1),
        "warm_ttft_s": round(warm_s, 5), "warm_p95_s": round(sorted(warm)[min(len(warm) - 1, int(0.95 * len(warm)))], 5),
        "reference_published": {"cold_ttft_s": 23.8, "warm_ttft_s": 0.13,
                                "hardware": "Apple M2 Pro (Metal), real Qwen2.5-0.5B Q8_0",
                                "source": "reference README.md:51 (context only, not this metric's baseline)"},
    }


def config_decoder(args, torch) -> dict:
    """The whole decoder step (synapse_kv_decoder_forward) on a Qwen2.5-7B-shaped synthetic Q8_0 model: 16
    sequences at the C3 lengths decode one token each per step, every token's logits copied back. The KV cache is
    filled through the model's cache (random K/V rows, as C3) rather than by running the prompts, which would
    only take longer. Algorithmic bytes per step: every Q8_0 matrix once (QKV, O, gate, up, down, logits), the K/V
    of every attended position, the new K/V, the embedding rows and the logits written."""
    import ctypes

    sys.path.insert(0, str(ROOT / "tests"))
    from synapse_amd.decoder import Decoder, DecoderShape
    from synthetic_models import q4_k_m, synthetic_model
    from synapse_amd.kv_cache import batch_tokens
    from synapse_amd.projection import matrix_bytes

    mix = args.weights
    choose = q4_k_m if mix == "q4_k_m" else (lambda name: 8)

    lengths = lengths_for(SEED + CONFIG_OFFSET)
    total = args.warmup + args.steps
    context = int(-(-(int(lengths.max()) + total + 1) // GROWTH) * GROWTH)
    shape = DecoderShape(layers=LAYERS, hidden=HEADS * HEAD_DIM, feed_forward=18944, heads=HEADS, kv_heads=KV_HEADS,
                         head_dim=HEAD_DIM, vocabulary=152064, context=context, session_slots=SEQUENCES,
                         step_tokens=4096, logits_rows=SEQUENCES, kv_precision="f16", growth=GROWTH)
    started = time.perf_counter()
    blob, layout = synthetic_model(shape, seed=SEED + 8, encodings=choose)
    model = Decoder(blob, layout, shape)
    log(f"model {blob.nbytes / 2**30:.2f} GiB built and uploaded in {time.perf_counter() - started:.1f} s")
    del blob
    library = model.library
    cache = model.cache
    width = (HEADS + 2 * KV_HEADS) * HEAD_DIM
    source = Rows(torch, 8, HEADS, HEAD_DIM, width)
    chunk = 4096
    rows = torch.empty((chunk, width), device="cuda")
    for slot, length in enumerate(lengths.tolist()):
        library.check(library.c_reserve(cache, slot, length + total + 1))
        for first in range(0, length, chunk):
            count = min(chunk, length - first)
            tokens = batch_tokens([(slot, p) for p in range(first, first + count)])
            library.check(library.c_step(cache, tokens, count))
            for layer in range(LAYERS):
                source.fill(rows[:count], slot, layer, first)
                library.check(library.c_append_rope(cache, layer, rows.data_ptr(), width))
    torch.cuda.synchronize()
    log(f"KV filled: {model.kv_bytes / 2**30:.2f} GiB")
    if args.adaptive_split is not None:
        from synapse_amd.native import OPTION_ADAPTIVE_SPLIT

        model.set_option(OPTION_ADAPTIVE_SPLIT, args.adaptive_split)
    rng = np.random.default_rng(SEED + 8)
    # The logits land in a reused pinned host buffer (the caller's buffer; a fresh pageable array per step would
    # time page faults and a staged copy).
    pinned = torch.empty((SEQUENCES, shape.vocabulary), dtype=torch.float32, pin_memory=True).numpy()

    def step(index):
        return model.forward([(slot, int(rng.integers(shape.vocabulary)), int(lengths[slot]) + index, slot)
                              for slot in range(SEQUENCES)], out=pinned)

    for index in range(args.warmup):
        step(index)
    torch.cuda.synchronize()
    begin = time.perf_counter()
    for index in range(args.steps):
        logits = step(args.warmup + index)
    elapsed = time.perf_counter() - begin
    assert np.isfinite(logits).all()
    seconds = elapsed / args.steps
    s = shape
    kv = s.kv_width
    # Bytes of the matrices in their GGML encodings (the K-quants are read from a repacked form holding 4-bit (Q4_K)
    # or 8-bit (Q6_K) codes plus FP32 factors, more than these bytes; the roofline counts the model's own size).
    weight_bytes = s.layers * (matrix_bytes(choose("attn_q"), s.hidden, s.hidden) +
                               matrix_bytes(choose("attn_k"), kv, s.hidden) +
                               matrix_bytes(choose("attn_v"), kv, s.hidden) +
                               matrix_bytes(choose("attn_output"), s.hidden, s.hidden) +
                               matrix_bytes(choose("ffn_gate"), s.feed_forward, s.hidden) +
                               matrix_bytes(choose("ffn_up"), s.feed_forward, s.hidden) +
                               matrix_bytes(choose("ffn_down"), s.hidden, s.feed_forward)) + \
        matrix_bytes(choose("output"), s.vocabulary, s.hidden)
    keys = float(np.mean([(lengths + args.warmup + i + 1).sum() for i in range(args.steps)]))
    kv_bytes = keys * KV_BYTES_PER_TOKEN_LAYER * LAYERS + SEQUENCES * KV_BYTES_PER_TOKEN_LAYER * LAYERS
    other = SEQUENCES * (matrix_bytes(choose("token_embd"), 1, s.hidden) + s.vocabulary * 4)
    step_bytes = weight_bytes + kv_bytes + other
    model.close()
    achieved = step_bytes / seconds / 1e9
    return {
        "metric": f"decoder step tokens/s (embedding, 28 layers, logits), 7B-shaped {mix.upper()}, 16 sequences @ C3 "
                  "lengths",
        "value": round(SEQUENCES / seconds, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(seconds * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": f"f32 ({mix.upper()} weights, FP16 KV)",
        "data": f"synthetic {mix.upper()} model (numpy seed {SEED + 8}), random K/V prefill, random token ids",
        "config": {"workload": "decoder: Qwen2.5-7B shape (hidden 3,584, ffn 18,944, 28 q / 4 KV heads, vocab "
                               "152,064), 16 sequences decoding at lengths U[1024, 32768], logits for every token",
                   "layers": LAYERS, "lengths": lengths.tolist(), "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "whole step (all kernels)", "achieved": round(achieved, 1),
                     "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBPS, 4),
                     "traffic": None, "algorithmic_bytes_per_step": int(step_bytes),
                     "weight_bytes": int(weight_bytes), "kv_bytes": int(kv_bytes)},
    }


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--config", choices=["c1", "c2", "c3", "c4", "c5", "proj", "decoder", "ttft"], default="c3",
                        help="c3: the BASELINE metric (default); c1, c2, c4: the other decode configurations; "
                             "c5: chunked-prefill MFMA throughput; proj: the Q8_0 projections around the path; "
                             "decoder: the whole decoder step on a 7B-shaped synthetic model")
    parser.add_argument("--weights", choices=["q8_0", "q4_k_m"], default="q8_0",
                        help="decoder: the matrices' encodings (Q8_0, or the Q4_K_M mix of Q4_K and Q6_K)")
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--split-keys", type=int, default=None)
    parser.add_argument("--prefill-split-keys", type=int, default=None, help="c5: keys per prefill work item")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--prefetch", type=int, default=None, help="decode kernel variant (0 or 1)")
    parser.add_argument("--adaptive-split", type=int, default=None,
                        help="SYNAPSE_KV_OPTION_ADAPTIVE_SPLIT: 1 weights decode shares by measured XCD speed")
    parser.add_argument("--segment-cost", type=int, default=None,
                        help="decode split: quarter key steps charged per row start in a worker's range")
    parser.add_argument("--separate", action="store_true",
                        help="append_rope + attention as two launches instead of the fused append_attention")
    parser.add_argument("--cpu-threads", type=int, default=None)
    parser.add_argument("--kv-pages", default=None, metavar="BUDGET:WINDOW[:random[:SEED]]",
                        help="c3 under query-aware KV page activation (the reference CLI's --kv-pages)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "the decode shards by sequence with no exchange, so N GPUs would run N independent copies.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from synapse_amd import PagedKvCache

    if not torch.cuda.is_available():
        sys.exit("bench.py needs a HIP device")
    torch.cuda.set_device(0)
    if args.config != "c3":
        runner = {"c1": config_c1, "c2": config_c2, "c4": config_c4, "c5": prefill_config,
                  "proj": config_projection, "decoder": config_decoder, "ttft": config_ttft}[args.config]
        print(json.dumps(runner(args, torch)), flush=True)
        return
    lengths = lengths_for(SEED + CONFIG_OFFSET)
    total_steps = args.warmup + args.steps
    max_positions = int(-(-(int(lengths.max()) + total_steps + 1) // GROWTH) * GROWTH)
    reserved = [-(-(int(n) + total_steps + 1) // GROWTH) * GROWTH for n in lengths]
    pages = sum(-(-r // PAGE_TOKENS) for r in reserved)
    log(f"lengths {lengths.tolist()} sum {int(lengths.sum())}; pages {pages}")
    cache = PagedKvCache(layers=LAYERS, heads=HEADS, kv_heads=KV_HEADS, head_dim=HEAD_DIM,
                         max_positions=max_positions, growth_positions=GROWTH, page_tokens=PAGE_TOKENS,
                         precision="f16", session_slots=SEQUENCES, step_tokens=4096, max_pages=pages)
    stream = torch.cuda.current_stream()
    cache.set_stream(stream)
    apply_options(args, cache)
    activation = parse_kv_pages(args.kv_pages)
    for slot, length in enumerate(lengths.tolist()):
        cache.reserve(slot, length + total_steps + 1)
    width = (HEADS + 2 * KV_HEADS) * HEAD_DIM
    rows = Rows(torch, CONFIG_OFFSET, HEADS, HEAD_DIM, width)
    started = time.perf_counter()
    prefill(cache, torch, lengths, rows)
    log(f"prefill {time.perf_counter() - started:.1f} s; KV bytes {cache.allocated_bytes / 2**30:.2f} GiB")
    if activation is not None:
        cache.set_page_activation(activation["budget"], activation["window"], page_tokens=activation["page"],
                                  selection=activation["selection"], seed=activation["seed"])

    qkv = rows.decode(LAYERS, SEQUENCES)
    out = torch.empty((LAYERS, SEQUENCES, HEADS * HEAD_DIM), device="cuda")

    def step(index: int) -> None:
        cache.step([(slot, int(lengths[slot]) + index) for slot in range(SEQUENCES)])
        for layer in range(LAYERS):
            if args.separate:
                cache.append_rope(layer, qkv[layer])
                cache.attention(layer, qkv[layer], out[layer])
            else:
                cache.append_attention(layer, qkv[layer], out[layer])

    for index in range(args.warmup):
        step(index)
    torch.cuda.synchronize()
    # Kernel times come from the library's profile mode: sampled dispatches of the cache record HIP events around
    # themselves on the cache's stream (hipExtLaunchKernel), read back after the timed region. Every layer launches
    # identical work, so two launches of each kind per step are timed; timing all 56 would add queue time.
    from synapse_amd.native import OPTION_PROFILE_EVERY

    cache.set_option(OPTION_PROFILE_EVERY, LAYERS // 2)
    cache.profile_begin()
    elapsed, per_step = step_times(torch, stream, lambda index: step(args.warmup + index), args.steps)
    kernels = cache.profile_end()

    ms_per_step = elapsed * 1e3 / args.steps
    tokens_per_second = SEQUENCES * args.steps / elapsed
    # Algorithmic bytes: each step reads the K/V of every attended position once per layer and writes the new
    # token's K/V; q/out rows are read/written once (fp32).
    keys_per_step = [int((lengths + args.warmup + index + 1).sum()) for index in range(args.steps)]
    dense_keys_per_step = keys_per_step
    if activation is not None:
        keys_per_step = [sum(attended_keys(int(n) + args.warmup + index, activation) for n in lengths)
                         for index in range(args.steps)]
    q_bytes = SEQUENCES * HEADS * HEAD_DIM * 4
    kv_row_bytes = SEQUENCES * 2 * KV_HEADS * HEAD_DIM * 4  # the new token's fp32 K and V rows
    append_bytes = SEQUENCES * KV_BYTES_PER_TOKEN_LAYER  # the new token's FP16 K and V
    # Decode launch (fused append): every attended position's K/V read once, the new K/V written, Q and the new
    # K/V rows read. The step adds the output rows (written by the merge or directly).
    decode_bytes = [keys * KV_BYTES_PER_TOKEN_LAYER + append_bytes + q_bytes + kv_row_bytes for keys in keys_per_step]
    step_bytes = [LAYERS * (b + q_bytes) for b in decode_bytes]
    step_gbps = sum(step_bytes) / elapsed / 1e9
    decode_launches, decode_ms = kernels["decode"]
    decode_seconds = decode_ms * 1e-3 / decode_launches
    decode_gbps = statistics.mean(decode_bytes) / decode_seconds / 1e9
    merge_launches, merge_ms = kernels.get("merge", (0, 0.0))
    traffic = measured_traffic()

    result = {
        "metric": METRIC if activation is None else METRIC + ", KV page activation " + activation["name"],
        "value": round(tokens_per_second, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: N(0,1) fp32 rows from the splitmix64/Box-Muller generator, KV pre-filled through the "
                "append path; lengths 1024 + splitmix64 mod 31,745",
        "seeds": {**rows.seeds(), "lengths": SEED + CONFIG_OFFSET},
        "config": {
            "workload": "C3: Qwen2.5-7B-shaped batched decode, 16 sequences, ragged lengths U[1024, 32768], "
                        "FP16 paged KV (256-token pages), append + flash-decode per layer, 28 layers",
            "layers": LAYERS, "heads": HEADS, "kv_heads": KV_HEADS, "head_dim": HEAD_DIM, "sequences": SEQUENCES,
            "page_tokens": PAGE_TOKENS, "lengths": lengths.tolist(), "parallelism": "single GPU",
        },
        **({} if activation is None else {"kv_pages": {
            **activation, "attended_keys_per_step": int(statistics.mean(keys_per_step)),
            "dense_keys_per_step": int(statistics.mean(dense_keys_per_step)),
            "read_keys_per_step": int(statistics.mean(
                sum(read_keys(int(n) + args.warmup + index, activation) for n in lengths)
                for index in range(args.steps))),
            "page_select_us_per_layer": round(kernels["page_select"][1] * 1e3 / kernels["page_select"][0], 2)
            if "page_select" in kernels else None}}),
        **step_statistics(per_step),
        "hbm_gbps": round(step_gbps, 1),
        "hbm_frac_of_peak": round(step_gbps / PEAK_HBM_GBPS, 4),
        "roofline": {
            "bound": "hbm",
            "kernel": ("decode_kernel<128, true, true> (split-K decode)" if args.separate else
                       "decode_kernel<128, true, true> (fused append + split-K decode)"),
            "achieved": round(decode_gbps, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(decode_gbps / PEAK_HBM_GBPS, 4),
            "traffic": traffic["bytes_per_launch"] if traffic else None,
            # Not measured in this run: read from the committed PMC summary (FETCH_SIZE and WRITE_SIZE runs of their
            # own, scaled by a 1 GiB copy's counters).
            "traffic_source": ("profiles/decode_attention_c3_traffic.json (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; "
                               "committed summary, not this run)") if traffic else None,
            "algorithmic_bytes_per_launch": int(statistics.mean(decode_bytes)),
            "avg_launch_us": round(decode_seconds * 1e6, 2),
            "timed_launches": decode_launches,
            "merge_avg_launch_us": round(merge_ms * 1e3 / merge_launches, 2) if merge_launches else None,
            "kernels_ms": {kind: round(ms, 3) for kind, (count, ms) in kernels.items()},
        },
    }
    peaks = measured_peaks(read_bytes=int(statistics.mean(decode_bytes)))
    result["roofline"]["measured_peak"] = peaks
    result["roofline"]["frac_of_measured_read"] = round(decode_gbps / peaks["read_gbps"], 4)
    result["roofline"]["frac_of_measured_read_same_size"] = round(decode_gbps / peaks["read_gbps_same_size"], 4)
    if "pattern_gbps_same_size" in peaks:
        result["roofline"]["frac_of_decode_pattern"] = round(decode_gbps / peaks["pattern_gbps_same_size"], 4)
    result["hbm_frac_of_measured_read"] = round(step_gbps / peaks["read_gbps"], 4)
    if not args.no_cpu_baseline and activation is None:
        threads = cpu_threads(args)
        log(f"cpu baseline on {threads} threads")
        result["cpu_baseline"] = cpu_baseline(torch, lengths, rows, qkv, threads)
    cache.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
