"""Device calibration: measured HBM and FP16 MFMA ceilings on the current device, timed with HIP events.

- read: 16-byte non-temporal loads over a large buffer, eight in flight per lane (bench_support/calibrate.hip);
  the practical ceiling of a streaming read, which the decode kernel is compared with beside the published 8 TB/s;
- pattern: the decode kernel's access pattern without its arithmetic (one wave per SIMD, each streaming its own
  run of 32 KiB steps through two register sets), over the decode launch's own byte count: the ceiling for that
  kernel's structure at that size;
- copy: the same with non-temporal stores (bytes read + written);
- torch copy and torch sum (library kernels, for reference); the torch copy is also the reference kernel for
  scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters (its counters against the bytes it is known to move);
- mfma: v_mfma_f32_16x16x32_f16 chains (8 independent per wave, 8 waves per CU), the measured ceiling of the FP16
  dense matrix rate beside the published 2.5 PFLOP/s.

``python bench_support/calibrate.py [--gib 4]`` prints one JSON line.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "_lib" / "libcalibrate.so"


def load() -> ctypes.CDLL:
    if not LIBRARY.exists():
        raise RuntimeError(f"{LIBRARY} is not built (run __graft_entry__.build())")
    library = ctypes.CDLL(str(LIBRARY))
    library.calibrate_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int,
                                       ctypes.c_void_p]
    library.calibrate_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                       ctypes.c_void_p]
    library.calibrate_mfma.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    library.calibrate_pattern.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int,
                                          ctypes.c_void_p]
    for function in (library.calibrate_read, library.calibrate_copy, library.calibrate_mfma,
                     library.calibrate_pattern):
        function.restype = ctypes.c_int
    return library


def _time(torch, stream, body, repeats: int) -> float:
    """Seconds per call of body() averaged over `repeats`, after two warm-up calls."""
    for _ in range(2):
        body()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(repeats):
        body()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e-3 / repeats


def measure(gib: float = 4.0, repeats: int = 10, mfma: bool = True, read_sizes: tuple = (),
            pattern_sizes: tuple = ()) -> dict:
    """Streaming read, copy and MFMA ceilings of this device.

    `read_sizes` adds the read rate over the first n bytes of the same buffer for each n (rounded down to
    8,192 bytes), as `read_gbps_at_bytes[n]`: a launch that moves a few hundred MB meets a lower ceiling than a
    multi-GiB stream, since the ramp-up and the drain of the grid are a larger share of its time.
    """
    import torch

    library = load()
    stream = torch.cuda.current_stream()
    handle = ctypes.c_void_p(stream.cuda_stream)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    nbytes = int(gib * 2**30) // 4096 * 4096
    source = torch.empty(nbytes // 2, dtype=torch.float16, device="cuda").normal_()
    target = torch.empty_like(source)
    sink = torch.zeros(1 << 20, dtype=torch.float32, device="cuda")
    blocks = cus * 4

    def check(status: int) -> None:
        if status != 0:
            raise RuntimeError(f"calibration launch failed: HIP error {status}")

    reads = {}
    for per_cu in (2, 4, 8):
        reads[per_cu] = _time(torch, stream, lambda: check(library.calibrate_read(
            source.data_ptr(), nbytes, sink.data_ptr(), cus * per_cu, handle)), repeats)
    read_s = min(reads.values())
    at_bytes = {}
    for size in read_sizes:
        size = min(int(size) // 8192 * 8192, nbytes)  # whole 8 KiB wave chunks: read_kernel reads no partial chunk
        best = min(_time(torch, stream, lambda: check(library.calibrate_read(
            source.data_ptr(), size, sink.data_ptr(), cus * per_cu, handle)), repeats * 4) for per_cu in (2, 4, 8))
        at_bytes[size] = round(size / best / 1e9, 1)
    pattern = {}
    for size in pattern_sizes:
        steps = max(1, int(size) // (32768 * cus * 4))
        moved = steps * 32768 * cus * 4
        if moved <= nbytes:
            seconds = _time(torch, stream, lambda: check(library.calibrate_pattern(
                source.data_ptr(), steps, sink.data_ptr(), cus, handle)), repeats * 4)
            pattern[moved] = round(moved / seconds / 1e9, 1)
    copy_s = _time(torch, stream, lambda: check(library.calibrate_copy(source.data_ptr(), target.data_ptr(), nbytes,
                                                                       blocks, handle)), repeats)
    torch_copy_s = _time(torch, stream, lambda: target.copy_(source), repeats)
    torch_sum_s = _time(torch, stream, lambda: source.sum(dtype=torch.float32), repeats)
    result = {
        "device_cus": cus,
        "bytes": nbytes,
        "read_gbps": round(nbytes / read_s / 1e9, 1),
        "read_gbps_by_waves_per_cu": {4 * k: round(nbytes / v / 1e9, 1) for k, v in reads.items()},
        "copy_gbps": round(2 * nbytes / copy_s / 1e9, 1),
        "torch_copy_gbps": round(2 * nbytes / torch_copy_s / 1e9, 1),
        "torch_sum_gbps": round(nbytes / torch_sum_s / 1e9, 1),
        "bytes_per_copy": 2 * nbytes,
    }
    if at_bytes:
        result["read_gbps_at_bytes"] = at_bytes
    if pattern:
        result["pattern_gbps_at_bytes"] = pattern
    if mfma:
        for wide, name in ((0, "16x16x32"), (1, "32x32x16")):
            for per_cu in (2, 4):
                mfma_blocks, iterations = cus * per_cu, 8000
                flops = mfma_blocks * 4 * iterations * 8 * 16 * 16 * 32 * 2
                mfma_s = _time(torch, stream, lambda: check(library.calibrate_mfma(
                    sink.data_ptr(), mfma_blocks, iterations, wide, handle)), 3)
                result[f"mfma_f16_{name}_{per_cu * 4}w_tflops"] = round(flops / mfma_s / 1e12, 1)
        result["mfma_f16_tflops"] = max(v for k, v in result.items() if k.startswith("mfma_f16_") and k.endswith("w_tflops"))
    del source, target, sink
    torch.cuda.empty_cache()
    return result


def main() -> None:
    parser = argparse.ArgumentParser()
    parser.add_argument("--gib", type=float, default=4.0)
    parser.add_argument("--repeats", type=int, default=10)
    args = parser.parse_args()
    sys.path.insert(0, str(HERE.parent))
    print(json.dumps(measure(args.gib, args.repeats)))


if __name__ == "__main__":
    main()
