"""HBM calibration on the current device: a plain copy and a plain read of known sizes, timed with HIP events.

The copy kernel (torch's elementwise copy) is also the reference kernel for scaling rocprofv3 FETCH_SIZE /
WRITE_SIZE counters: its counters are compared with the bytes it is known to move. Run:
``python -m synapse_amd.calibrate [--gib 4]``; prints one JSON line.
"""

from __future__ import annotations

import argparse
import json


def measure(gib: float = 4.0, repeats: int = 10) -> dict:
    import torch

    elements = int(gib * 2**30) // 2
    source = torch.empty(elements, dtype=torch.float16, device="cuda").normal_()
    target = torch.empty_like(source)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(2):
        target.copy_(source)
    torch.cuda.synchronize()
    start.record()
    for _ in range(repeats):
        target.copy_(source)
    end.record()
    torch.cuda.synchronize()
    copy_seconds = start.elapsed_time(end) * 1e-3 / repeats
    bytes_moved = 2 * source.numel() * source.element_size()
    for _ in range(2):
        source.sum(dtype=torch.float32)
    torch.cuda.synchronize()
    start.record()
    for _ in range(repeats):
        source.sum(dtype=torch.float32)
    end.record()
    torch.cuda.synchronize()
    read_seconds = start.elapsed_time(end) * 1e-3 / repeats
    return {
        "bytes_per_copy": bytes_moved,
        "copy_gbps": bytes_moved / copy_seconds / 1e9,
        "copy_us": copy_seconds * 1e6,
        "read_gbps": source.numel() * source.element_size() / read_seconds / 1e9,
        "read_us": read_seconds * 1e6,
    }


def main() -> None:
    parser = argparse.ArgumentParser()
    parser.add_argument("--gib", type=float, default=4.0)
    parser.add_argument("--repeats", type=int, default=10)
    args = parser.parse_args()
    print(json.dumps(measure(args.gib, args.repeats)))


if __name__ == "__main__":
    main()
