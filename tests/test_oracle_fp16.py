"""Pins the oracle's FP32 -> FP16 round-to-nearest-even and its exact FP16 -> FP32 widening.

The conversion is the Metal `(half)` cast of synapse_rope_kv (elementwise.metal:97-98, 116-117) and the
widening is Fp16.ToSingle (Fp16.cs:17-23). The golden vectors come from numpy's float16 cast
(tests/golden/make_fp16_golden.py), a routine independent of this repository.
"""

from pathlib import Path

import numpy as np

from oracle_ffi import f16_to_f32, f32_to_f16

GOLDEN = Path(__file__).resolve().parent / "golden" / "fp16_rne.npz"


def test_rne_matches_golden_vectors():
    data = np.load(GOLDEN)
    got = f32_to_f16(data["inputs"])
    mismatches = np.nonzero(got != data["expected"])[0]
    assert mismatches.size == 0, (data["inputs"][mismatches[:5]], got[mismatches[:5]])


def test_rne_exhaustive_neighbourhoods_match_numpy():
    # Every binary16 value, the ties between neighbours and one FP32 ulp either side.
    bits = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16)
    low = bits.view(np.float16).astype(np.float64)
    high = (bits + 1).view(np.float16).astype(np.float64)
    mid = ((low + high) / 2).astype(np.float32)
    x = np.concatenate([low.astype(np.float32), mid, np.nextafter(mid, np.float32(np.inf)),
                        np.nextafter(mid, np.float32(0))])
    x = np.concatenate([x, -x])
    with np.errstate(over="ignore"):
        expected = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(f32_to_f16(x), expected)


def test_rne_special_cases():
    cases = [
        (0.0, 0x0000), (-0.0, 0x8000), (1.0, 0x3C00), (65504.0, 0x7BFF), (65519.99, 0x7BFF), (65520.0, 0x7C00),
        (np.inf, 0x7C00), (-np.inf, 0xFC00), (2.0**-24, 0x0001), (2.0**-25, 0x0000), (3 * 2.0**-25, 0x0002),
        (2.0**-14, 0x0400), (1.0 + 2.0**-11, 0x3C00), (1.0 + 3 * 2.0**-11, 0x3C02),
    ]
    x = np.array([value for value, _ in cases], dtype=np.float32)
    assert [hex(v) for v in f32_to_f16(x)] == [hex(bits) for _, bits in cases]
    nan = f32_to_f16(np.array([np.nan, -np.nan], dtype=np.float32))
    assert all((v & 0x7C00) == 0x7C00 and (v & 0x3FF) != 0 for v in nan)


def test_widening_is_exact_for_every_finite_half():
    bits = np.arange(0, 0x10000, dtype=np.uint32).astype(np.uint16)
    reference = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(reference)
    got = f16_to_f32(bits)
    assert np.array_equal(got[finite].view(np.uint32), reference[finite].view(np.uint32))


def test_round_trip_is_identity_on_halves():
    bits = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16)
    bits = np.concatenate([bits, bits | 0x8000])
    assert np.array_equal(f32_to_f16(f16_to_f32(bits)), bits)
