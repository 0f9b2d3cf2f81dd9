"""Writes tests/golden/fp16_rne.npz: FP32 inputs and their IEEE binary16 round-to-nearest-even bit patterns.

The expected bits come from numpy's float32 -> float16 cast (npy_floatbits_to_halfbits, round to nearest,
ties to even), a library routine independent of this repository and of the reference. The inputs cover
ties at every exponent, the subnormal range and its boundaries, the overflow threshold, zeros, infinities,
NaN, and a seeded sample across the whole finite range. Run: python tests/golden/make_fp16_golden.py
"""

from pathlib import Path

import numpy as np


def inputs() -> np.ndarray:
    values = []
    # Every binary16 value, and the exact midpoints between neighbours (ties) plus/minus one FP32 ulp.
    halves = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    pick = np.random.default_rng(7).choice(halves.size, 3000, replace=False)
    pick = np.union1d(pick, np.arange(0, 1100))  # every subnormal and the first normals
    halves = halves[pick]
    values.append(halves)
    upper = (pick + 1).astype(np.uint16).view(np.float16).astype(np.float32)
    mid = ((halves.astype(np.float64) + upper.astype(np.float64)) / 2).astype(np.float32)
    values += [mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0))]
    # Boundaries: 2^-25 (ties to zero), just above, 2^-24, max finite, 65519.996, 65520, huge, inf.
    specials = np.array(
        [0.0, 2.0**-25, np.nextafter(np.float32(2.0**-25), np.float32(1)), 2.0**-24, 2.0**-14,
         np.nextafter(np.float32(2.0**-14), np.float32(0)), 65504.0, np.nextafter(np.float32(65520.0), np.float32(0)),
         65520.0, 1e10, np.float32(np.finfo(np.float32).max), np.inf, 1e-30, np.finfo(np.float32).tiny,
         np.float32(1.4e-45)],
        dtype=np.float32,
    )
    values.append(specials)
    rng = np.random.default_rng(20261201)
    bits = rng.integers(0, 0x7F800000, size=4000, dtype=np.uint32)
    values.append(bits.view(np.float32))
    values.append(rng.standard_normal(4000).astype(np.float32))
    positive = np.concatenate(values)
    return np.concatenate([positive, -positive]).astype(np.float32)


def main() -> None:
    x = inputs()
    with np.errstate(over="ignore"):
        expected = x.astype(np.float16).view(np.uint16)
    nan_inputs = np.array([np.nan, -np.nan], dtype=np.float32)
    out = Path(__file__).with_name("fp16_rne.npz")
    np.savez_compressed(out, inputs=x, expected=expected, nan_inputs=nan_inputs)
    print(out, x.size)


if __name__ == "__main__":
    main()
