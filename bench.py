"""Benchmark of the north-star workload: Qwen2.5-7B-shaped batched decode (config C3).

One step = one decode token for each of 16 sequences: for each of the 28 layers, the fused RoPE + FP16 KV append
and the GQA split-K flash-decode attention over the paged cache (the per-layer pairs run back to back; the
projections around them are outside this path). Lengths are drawn uniform in [1,024, 32,768] from the seed;
the KV cache is pre-filled through the same append path with N(0,1) fp32 K/V. Inputs are resident in HBM when
the timed region starts.

Prints one JSON line: the whole-job tokens/s, the step's algorithmic HBM GB/s, the dominant kernel's roofline
(decode attention, timed with HIP events on the cache's stream over the timed region) and the CPU baseline (the
restatement of Qwen2CpuAttention timed on host threads over one layer of the same workload).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode attn+KV-append tokens/s, HBM GB/s (% of peak), 7B shape @32k ctx"
PEAK_HBM_GBPS = 8000.0
SEED = 20261201
CONFIG_OFFSET = 3  # config C3
LAYERS, HEADS, KV_HEADS, HEAD_DIM = 28, 28, 4, 128
SEQUENCES = 16
PAGE_TOKENS = 256
GROWTH = 1024
KV_BYTES_PER_TOKEN_LAYER = 2 * KV_HEADS * HEAD_DIM * 2  # K + V, FP16
PROFILES = ROOT / "profiles"


def log(message: str) -> None:
    print(message, file=sys.stderr, flush=True)


def lengths_for(seed: int) -> np.ndarray:
    return np.random.default_rng(seed).integers(1024, 32768 + 1, size=SEQUENCES)


def measured_traffic() -> dict | None:
    """HBM bytes per decode launch from the committed rocprofv3 PMC summary, when it exists."""
    path = PROFILES / "decode_attention_c3_traffic.json"
    if not path.exists():
        return None
    return json.loads(path.read_text())


def prefill(cache, torch, lengths, generator, chunk=4096):
    """Fills every sequence through step + append_rope in prompt chunks (N(0,1) fp32 rows)."""
    width = (HEADS + 2 * KV_HEADS) * HEAD_DIM
    buffer = torch.empty((chunk, width), device="cuda")
    for slot, length in enumerate(lengths.tolist()):
        for first in range(0, length, chunk):
            count = min(chunk, length - first)
            cache.step([(slot, p) for p in range(first, first + count)])
            for layer in range(LAYERS):
                rows = buffer[:count]
                rows.normal_(generator=generator)
                cache.append_rope(layer, rows)
    torch.cuda.synchronize()


def parse_kv_pages(text: str | None) -> dict | None:
    """--kv-pages <budget>:<window>[:random[:seed]] (the reference CLI's option, ADR-016)."""
    if text is None:
        return None
    parts = text.split(":")
    if len(parts) < 2 or len(parts) > 4 or (len(parts) > 2 and parts[2] != "random"):
        sys.exit("--kv-pages takes <budget>:<window>[:random[:seed]]")
    budget, window = int(parts[0]), int(parts[1])
    random = len(parts) > 2
    seed = int(parts[3]) if len(parts) > 3 else 0
    name = f"kvpages{budget}w{window}" + ("r" if random else "")
    return {"budget": budget, "window": window, "selection": "random" if random else "key_bound", "seed": seed,
            "name": name}


def attended_keys(position: int, activation: dict) -> int:
    """Positions a decode token at `position` attends (KvPageSelector.Select with 64-position pages)."""
    count = position + 1
    window_page = max(0, count - activation["window"]) // 64
    if max(0, window_page - 1) <= activation["budget"]:
        return count
    return 64 + activation["budget"] * 64 + (count - window_page * 64)


def cpu_baseline(lengths, threads: int) -> dict:
    """The reference CPU attention restated in C++ (oracle/), timed on host threads: one layer of one decode step
    over the same lengths (FP16 pages widened exactly, Qwen2CpuAttention order), extrapolated to 28 layers."""
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_ffi import PagedCache, rope_table

    max_positions = int(lengths.max()) + 1024
    pages = int(sum(-(-(int(n) + 1) // PAGE_TOKENS) for n in lengths)) + SEQUENCES
    cache = PagedCache(1, HEADS, KV_HEADS, HEAD_DIM, max_positions, PAGE_TOKENS, PAGE_TOKENS, 1, SEQUENCES, pages,
                       4096)
    cos, sin = rope_table(HEAD_DIM, 1e6, max_positions)
    rng = np.random.default_rng(SEED + CONFIG_OFFSET)
    width = (HEADS + 2 * KV_HEADS) * HEAD_DIM
    start = time.perf_counter()
    for slot, length in enumerate(lengths.tolist()):
        assert cache.reserve(slot, length + 1) == 0
        for first in range(0, length, 4096):
            count = min(4096, length - first)
            rows = np.zeros((count, width), dtype=np.float32)
            rows[:, HEADS * HEAD_DIM:] = rng.standard_normal((count, 2 * KV_HEADS * HEAD_DIM), dtype=np.float32)
            assert cache.step([(slot, p) for p in range(first, first + count)]) == 0
            assert cache.append_rope(0, rows, cos, sin) == 0
    fill_seconds = time.perf_counter() - start
    tokens = [(slot, int(length)) for slot, length in enumerate(lengths)]
    assert cache.step(tokens) == 0
    rows = rng.standard_normal((SEQUENCES, width), dtype=np.float32)
    assert cache.append_rope(0, rows, cos, sin) == 0
    out = np.zeros((SEQUENCES, HEADS * HEAD_DIM), dtype=np.float32)
    cache.attention(0, rows, out, threads)  # warm-up
    times = [cache.attention(0, rows, out, threads) for _ in range(3)]
    layer_seconds = statistics.median(times)
    step_seconds = layer_seconds * LAYERS
    return {
        "value": SEQUENCES / step_seconds,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (
            f"decode attention of one layer for the 16 drawn lengths (sum {int(lengths.sum())} keys), median of 3 "
            f"after 1 warm-up, x28 layers; C++ restatement of Qwen2CpuAttention (4-lane dot, 3-pass softmax) over "
            f"FP16 pages widened per Fp16.ToSingle, {threads} std::threads; append excluded; fill took "
            f"{fill_seconds:.1f} s"
        ),
        "ms_per_layer": layer_seconds * 1e3,
    }


def prefill_config(args, torch) -> dict:
    """Config C5: a 2,048-token chunk attends causally over a 63,488-token FP16 cache plus itself (65,536 keys) in
    all 28 layers; one timed repetition = the chunk's 28 append_attention calls (append + MFMA prefill + merge)."""
    from synapse_amd import PagedKvCache

    cached, chunk = 63488, 2048
    cache = PagedKvCache(layers=LAYERS, heads=HEADS, kv_heads=KV_HEADS, head_dim=HEAD_DIM, max_positions=65536,
                         growth_positions=GROWTH, page_tokens=PAGE_TOKENS, precision="f16", session_slots=1,
                         step_tokens=4096, max_pages=256)
    cache.set_stream(torch.cuda.current_stream())
    if args.prefill_split_keys:
        cache.set_prefill_split_keys(args.prefill_split_keys)
    cache.reserve(0, cached + chunk)
    generator = torch.Generator(device="cuda")
    generator.manual_seed(SEED + 5)
    width = (HEADS + 2 * KV_HEADS) * HEAD_DIM
    buffer = torch.empty((4096, width), device="cuda")
    for first in range(0, cached, 4096):
        cache.step([(0, p) for p in range(first, first + 4096)])
        for layer in range(LAYERS):
            buffer.normal_(generator=generator)
            cache.append_rope(layer, buffer)
    qkv = torch.empty((LAYERS, chunk, width), device="cuda").normal_(generator=generator)
    out = torch.empty((LAYERS, chunk, HEADS * HEAD_DIM), device="cuda")
    cache.step([(0, cached + j) for j in range(chunk)])

    def run() -> None:
        for layer in range(LAYERS):
            cache.append_attention(layer, qkv[layer], out[layer])

    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    cache.profile_begin()
    begin = time.perf_counter()
    for _ in range(args.steps):
        run()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - begin
    kernels = cache.profile_end()
    cache.close()
    # Key visits per query head: each chunk token sees the whole cache plus the chunk up to itself.
    visits = chunk * cached + chunk * (chunk + 1) // 2
    flops_per_layer = HEADS * visits * 4 * HEAD_DIM
    seconds = elapsed / args.steps
    tflops = LAYERS * flops_per_layer / seconds / 1e12
    prefill_launches, prefill_ms = kernels["prefill"]
    kernel_tflops = flops_per_layer / (prefill_ms * 1e-3 / prefill_launches) / 1e12
    return {
        "metric": "chunked-prefill attention TFLOP/s (MFMA FP16), 7B shape, 2,048-token chunk over 63,488 cached",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(seconds * 1e3, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": f"synthetic N(0,1) fp32 rows, torch seed {SEED + 5}",
        "config": {"workload": "C5: 28 layers x (append + causal prefill, split-K merge when planned), 65,536 keys",
                   "flops_per_layer": flops_per_layer},
        "roofline": {"bound": "mfma", "kernel": "prefill_f16_kernel<128>", "achieved": round(kernel_tflops, 2),
                     "peak": 2500.0, "unit": "TFLOP/s", "frac": round(kernel_tflops / 2500.0, 4), "traffic": None,
                     "avg_launch_us": round(prefill_ms * 1e3 / prefill_launches, 2),
                     "kernels_ms": {kind: round(ms, 3) for kind, (count, ms) in kernels.items()}},
    }


def fill_slot(cache, torch, slot, first, count, chunk, layers, generator):
    """Appends positions [first, first + count) of `slot` through step + append_rope in prompt chunks."""
    buffer = torch.empty((chunk, cache.qkv_width), device="cuda")
    for start in range(first, first + count, chunk):
        size = min(chunk, first + count - start)
        cache.step([(slot, p) for p in range(start, start + size)])
        for layer in range(layers):
            rows = buffer[:size]
            rows.normal_(generator=generator)
            cache.append_rope(layer, rows)
    torch.cuda.synchronize()


def apply_options(args, cache) -> None:
    if args.split_keys:
        cache.set_split_keys(args.split_keys)
    if args.prefetch is not None:
        from synapse_amd.native import OPTION_DECODE_PREFETCH

        cache.set_option(OPTION_DECODE_PREFETCH, args.prefetch)


def timed(torch, cache, run, repetitions, profile_every=1):
    """Wall seconds per repetition of `run` (between synchronizations) and the cache's kernel profile."""
    from synapse_amd.native import OPTION_PROFILE_EVERY

    cache.set_option(OPTION_PROFILE_EVERY, profile_every)
    cache.profile_begin()
    torch.cuda.synchronize()
    begin = time.perf_counter()
    for index in range(repetitions):
        run(index)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - begin
    return elapsed / repetitions, cache.profile_end()


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
    generator = torch.Generator(device="cuda")
    generator.manual_seed(SEED + 1)
    fill_slot(cache, torch, 0, 0, cached, 512, layers, generator)
    qkv = torch.empty((layers, 1, cache.qkv_width), device="cuda").normal_(generator=generator)
    out = torch.empty((layers, 1, heads * d), device="cuda")

    def run(index):
        cache.step([(0, cached + index)])
        for layer in range(layers):
            cache.append_attention(layer, qkv[layer], out[layer])

    for index in range(args.warmup):
        run(index)
    seconds, kernels = timed(torch, cache, lambda i: run(args.warmup + i), args.steps, profile_every=layers // 2)
    row = 2 * kv_heads * d * 4  # K + V bytes per position per layer (FP32)
    keys = cached + args.warmup + (args.steps + 1) / 2
    launch_bytes = keys * row + row + heads * d * 4 + 2 * kv_heads * d * 4
    cache.close()
    return decode_line(args, metric="C1 decode attn+KV-append tokens/s, 0.5B FP32 KV @4k ctx",
                       workload="C1: Qwen2.5-0.5B-shaped single-sequence decode, FP32 KV, 4,096 cached tokens, "
                                "24 layers", tokens_per_step=1, seconds=seconds,
                       bytes_per_step=layers * (launch_bytes + heads * d * 4), layers=layers,
                       decode_bytes_per_launch=launch_bytes, kernels=kernels,
                       data=f"synthetic N(0,1) fp32 rows, torch seed {SEED + 1}")


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
    generator = torch.Generator(device="cuda")
    generator.manual_seed(SEED + 2)
    rows = torch.empty((64, 512, cache.qkv_width), device="cuda").normal_(generator=generator)
    torch.cuda.synchronize()

    # Fill: 64 chunks x 24 layers of append_rope (RoPE + FP16 RNE store), growth through the capacity policy.
    def fill_chunk(chunk):
        cache.step([(0, p) for p in range(chunk * 512, chunk * 512 + 512)])
        for layer in range(layers):
            cache.append_rope(layer, rows[chunk])

    fill_seconds, fill_kernels = timed(torch, cache, fill_chunk, 64)
    width = cache.qkv_width * 4
    fill_bytes = 512 * layers * (width + (heads + kv_heads) * d * 4 + 2 * kv_heads * d * 2)
    qkv = torch.empty((layers, 1, cache.qkv_width), device="cuda").normal_(generator=generator)
    out = torch.empty((layers, 1, heads * d), device="cuda")

    def run(index):
        cache.step([(0, filled + index)])
        for layer in range(layers):
            cache.append_attention(layer, qkv[layer], out[layer])

    for index in range(args.warmup):
        run(index)
    seconds, kernels = timed(torch, cache, lambda i: run(args.warmup + i), args.steps, profile_every=layers // 2)
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
        kernels=kernels, data=f"synthetic N(0,1) fp32 rows, torch seed {SEED + 2}",
        extra={"fill": {"ms": round(fill_seconds * 64 * 1e3, 3), "tokens_per_s": round(512 / fill_seconds, 1),
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
    generator = torch.Generator(device="cuda")
    generator.manual_seed(SEED + 4)
    cache.reserve(0, prefix)
    fill_slot(cache, torch, 0, 0, prefix, 4096, layers, generator)
    for target in range(1, forks + 1):
        cache.fork(0, target)
    suffix = torch.empty((64 * forks, cache.qkv_width), device="cuda").normal_(generator=generator)
    suffix_out = torch.empty((64 * forks, heads * d), device="cuda")

    def suffix_step(_):
        cache.step([(slot, prefix + j) for slot in range(1, forks + 1) for j in range(64)])
        for layer in range(layers):
            cache.append_attention(layer, suffix, suffix_out)

    suffix_seconds, suffix_kernels = timed(torch, cache, suffix_step, 1)
    qkv = torch.empty((layers, forks, cache.qkv_width), device="cuda").normal_(generator=generator)
    out = torch.empty((layers, forks, heads * d), device="cuda")

    def run(index):
        cache.step([(slot, prefix + 64 + index) for slot in range(1, forks + 1)])
        for layer in range(layers):
            cache.append_attention(layer, qkv[layer], out[layer])

    for index in range(args.warmup):
        run(index)
    seconds, kernels = timed(torch, cache, lambda i: run(args.warmup + i), args.steps, profile_every=layers // 2)
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
        decode_bytes_per_launch=launch_unique, kernels=kernels, data=f"synthetic N(0,1) fp32 rows, torch seed {SEED + 4}",
        extra={"suffix_step_ms": round(suffix_seconds * 1e3, 3),
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


def config_decoder(args, torch) -> dict:
    """The whole decoder step (synapse_kv_decoder_forward) on a Qwen2.5-7B-shaped synthetic Q8_0 model: 16
    sequences at the C3 lengths decode one token each per step, every token's logits copied back. The KV cache is
    filled through the model's cache (random K/V rows, as C3) rather than by running the prompts, which would
    only take longer. Algorithmic bytes per step: every Q8_0 matrix once (QKV, O, gate, up, down, logits), the K/V
    of every attended position, the new K/V, the embedding rows and the logits written."""
    import ctypes

    from synapse_amd.decoder import Decoder, DecoderShape, q4_k_m, synthetic_model
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
    generator = torch.Generator(device="cuda")
    generator.manual_seed(SEED + 8)
    width = (HEADS + 2 * KV_HEADS) * HEAD_DIM
    chunk = 4096
    rows = torch.empty((chunk, width), device="cuda")
    for slot, length in enumerate(lengths.tolist()):
        library.check(library.c_reserve(cache, slot, length + total + 1))
        for first in range(0, length, chunk):
            count = min(chunk, length - first)
            tokens = batch_tokens([(slot, p) for p in range(first, first + count)])
            library.check(library.c_step(cache, tokens, count))
            for layer in range(LAYERS):
                rows[:count].normal_(generator=generator)
                library.check(library.c_append_rope(cache, layer, rows.data_ptr(), width))
    torch.cuda.synchronize()
    log(f"KV filled: {model.kv_bytes / 2**30:.2f} GiB")
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
    parser.add_argument("--config", choices=["c1", "c2", "c3", "c4", "c5", "proj", "decoder"], default="c3",
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
                  "proj": config_projection, "decoder": config_decoder}[args.config]
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
    generator = torch.Generator(device="cuda")
    generator.manual_seed(SEED + CONFIG_OFFSET)
    started = time.perf_counter()
    prefill(cache, torch, lengths, generator)
    log(f"prefill {time.perf_counter() - started:.1f} s; KV bytes {cache.allocated_bytes / 2**30:.2f} GiB")
    if activation is not None:
        cache.set_page_activation(activation["budget"], activation["window"], selection=activation["selection"],
                                  seed=activation["seed"])

    width = (HEADS + 2 * KV_HEADS) * HEAD_DIM
    qkv = torch.empty((LAYERS, SEQUENCES, width), device="cuda").normal_(generator=generator)
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
    torch.cuda.synchronize()
    begin = time.perf_counter()
    for index in range(args.steps):
        step(args.warmup + index)
    host_seconds = time.perf_counter() - begin  # time to enqueue the timed steps (host side)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - begin
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
        "data": f"synthetic: N(0,1) fp32 q/k/v from torch seed {SEED + CONFIG_OFFSET}, KV pre-filled through the "
                f"append path; lengths from numpy default_rng({SEED + CONFIG_OFFSET})",
        "config": {
            "workload": "C3: Qwen2.5-7B-shaped batched decode, 16 sequences, ragged lengths U[1024, 32768], "
                        "FP16 paged KV (256-token pages), append + flash-decode per layer, 28 layers",
            "layers": LAYERS, "heads": HEADS, "kv_heads": KV_HEADS, "head_dim": HEAD_DIM, "sequences": SEQUENCES,
            "page_tokens": PAGE_TOKENS, "lengths": lengths.tolist(), "parallelism": "single GPU",
        },
        **({} if activation is None else {"kv_pages": {
            **activation, "attended_keys_per_step": int(statistics.mean(keys_per_step)),
            "dense_keys_per_step": int(statistics.mean(dense_keys_per_step)),
            "page_select_us_per_layer": round(kernels["page_select"][1] * 1e3 / kernels["page_select"][0], 2)
            if "page_select" in kernels else None}}),
        "hbm_gbps": round(step_gbps, 1),
        "host_ms_per_step": round(host_seconds * 1e3 / args.steps, 4),
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
            "algorithmic_bytes_per_launch": int(statistics.mean(decode_bytes)),
            "avg_launch_us": round(decode_seconds * 1e6, 2),
            "timed_launches": decode_launches,
            "merge_avg_launch_us": round(merge_ms * 1e3 / merge_launches, 2) if merge_launches else None,
            "kernels_ms": {kind: round(ms, 3) for kind, (count, ms) in kernels.items()},
        },
    }
    if not args.no_cpu_baseline and activation is None:
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        log(f"cpu baseline on {threads} threads")
        baseline = cpu_baseline(lengths, threads)
        result["cpu_baseline"] = baseline
    cache.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
