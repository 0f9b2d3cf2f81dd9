"""The Q8_0 projection restatement (CPU): the GGML Q8_0 format, the FP64 anchor against an independent numpy
product, the reference's FP32 matrix-vector order against the anchor, and closed forms for bias, accumulation and
segment columns. The HIP kernels are checked against these in test_gpu_projection.py."""

import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle_ffi import q8_project
from ggml_blocks import dequantize_q8_0, quantize_q8_0

ROOT = Path(__file__).resolve().parent.parent


def random_q8(rng, rows, columns, scale=1.0):
    return quantize_q8_0(rng.standard_normal((rows, columns)).astype(np.float32) * np.float32(scale))


def test_q8_0_blocks_follow_the_ggml_format():
    # One block with max |x| = 127: d = 1.0 exactly (FP16 0x3C00), codes round half to even (TinyQwen2Gguf
    # QuantizeQ8Zero: Math.Round, ToEven).
    x = np.zeros((1, 32), dtype=np.float32)
    x[0, :6] = [127.0, -127.0, 2.5, 3.5, -2.5, 0.49]
    blocks = quantize_q8_0(x)
    assert blocks.shape == (1, 34)
    assert blocks[0, :2].view(np.uint16)[0] == 0x3C00
    assert blocks[0, 2:8].view(np.int8).tolist() == [127, -127, 2, 4, -2, 0]
    # An all-zero block has d = 0 and zero codes; dequantization is d * code, exactly.
    zero = quantize_q8_0(np.zeros((1, 32), dtype=np.float32))
    assert not zero.any()
    rng = np.random.default_rng(1)
    values = rng.standard_normal((8, 96)).astype(np.float32)
    blocks = quantize_q8_0(values)
    restored = dequantize_q8_0(blocks, 96)
    scale = blocks.reshape(8, 3, 34)[:, :, :2].copy().view(np.float16).astype(np.float32)
    # Each element is within half a quantum of the input (plus the FP16 rounding of d, below 2^-11 relative).
    quantum = np.repeat(scale[:, :, 0], 32, axis=1)
    assert np.all(np.abs(restored - values) <= 0.5 * quantum + np.abs(values) * 2.0 ** -10)


@pytest.mark.parametrize("rows,columns,tokens", [(7, 32, 1), (33, 96, 3), (48, 896, 5), (20, 4096, 2)])
def test_fp64_anchor_matches_an_independent_product(rows, columns, tokens):
    rng = np.random.default_rng(rows + columns)
    blocks = random_q8(rng, rows, columns, 0.05)
    bias = rng.standard_normal(rows).astype(np.float32)
    x = rng.standard_normal((tokens, columns)).astype(np.float32)
    out = np.zeros((tokens, rows), dtype=np.float32)
    magnitude = q8_project([(blocks, bias, 0)], x, out, exact=True)
    weights = dequantize_q8_0(blocks, columns).astype(np.float64)
    expected = x.astype(np.float64) @ weights.T + bias
    assert np.allclose(out, expected.astype(np.float32), rtol=1e-6, atol=1e-6)
    assert np.allclose(magnitude, np.abs(x.astype(np.float64)) @ np.abs(weights).T + np.abs(bias), rtol=1e-9)


@pytest.mark.parametrize("rows,columns,tokens", [(9, 64, 1), (40, 896, 4), (16, 3584, 2)])
def test_reference_matvec_order_is_within_fp32_error_of_the_anchor(rows, columns, tokens):
    rng = np.random.default_rng(3 * rows + columns)
    blocks = random_q8(rng, rows, columns, 0.02)
    x = rng.standard_normal((tokens, columns)).astype(np.float32)
    fp32 = np.zeros((tokens, rows), dtype=np.float32)
    q8_project([(blocks, None, 0)], x, fp32)
    exact = np.zeros_like(fp32)
    magnitude = q8_project([(blocks, None, 0)], x, exact, exact=True)
    assert np.all(np.abs(fp32 - exact) <= 2.0 ** -20 * magnitude + 1e-30)
    # Batch invariance (the reference's contract): one token alone gives the same bits, on any thread count.
    single = np.zeros((1, rows), dtype=np.float32)
    q8_project([(blocks, None, 0)], x[-1:], single, threads=4)
    assert np.array_equal(single[0].view(np.uint32), fp32[-1].view(np.uint32))


def test_segments_bias_and_accumulate_closed_forms():
    # Matrix 0: one code 5 at (row 1, column 40) with d = 0.5; matrix 1: one code -3 at (row 0, column 3), d = 2.
    first = np.zeros((2, 2 * 34), dtype=np.uint8)
    first[1, 34:36] = np.array([0.5], dtype=np.float16).view(np.uint8)
    first[1, 34 + 2 + 8] = np.uint8(5)
    second = np.zeros((1, 2 * 34), dtype=np.uint8)
    second[0, 0:2] = np.array([2.0], dtype=np.float16).view(np.uint8)
    second[0, 2 + 3] = np.int8(-3).view(np.uint8)
    x = np.arange(64, dtype=np.float32)[None, :] / 8
    bias = np.array([0.25, -1.0], dtype=np.float32)
    for exact in (False, True):
        out = np.full((1, 10), 7.0, dtype=np.float32)
        q8_project([(first, bias, 6), (second, None, 1)], x, out, accumulate=True, exact=exact)
        expected = np.full(10, 7.0, dtype=np.float32)
        expected[6] += 0.25  # row 0 of matrix 0: no codes, the bias only
        expected[7] += 0.5 * 5 * (40 / 8) - 1.0
        expected[1] += 2.0 * -3 * (3 / 8)
        assert out[0].tolist() == expected.tolist()


Q8_LAYOUT_PROGRAM = r'''
#include <cstdio>
#include <cstdlib>
#include <vector>
#include "q8_layout.h"
using namespace synapse_kv;
int main() {
    int failures = 0;
    for (int rows : {1, 16, 17, 40}) {
        for (int columns : {32, 64, 96, 896}) {
            const int chunks = q8_chunks(columns);
            const size_t codes_size = (size_t)q8_tiles(rows) * chunks * kQ8TileBytes;
            std::vector<int> seen(codes_size, 0);
            for (int row = 0; row < rows; ++row) {
                for (int column = 0; column < columns; ++column) {
                    const long long at = q8_code_offset(chunks, row, column);
                    if (at < 0 || at >= (long long)codes_size || seen[at]++) { ++failures; }
                }
            }
            std::vector<int> scale_seen((size_t)q8_tiles(rows) * chunks * kQ8TileScales, 0);
            for (int row = 0; row < rows; ++row) {
                for (int block = 0; block < columns / 32; ++block) {
                    const long long at = q8_scale_offset(chunks, row, block);
                    if (at < 0 || at >= (long long)scale_seen.size() || scale_seen[at]++) { ++failures; }
                }
            }
            // Round trip through the device layout.
            std::vector<unsigned char> blocks((size_t)rows * columns / 32 * 34), back(blocks.size());
            for (size_t i = 0; i < blocks.size(); ++i) { blocks[i] = (unsigned char)(rand() & 0xFF); }
            std::vector<unsigned char> codes(codes_size);
            std::vector<unsigned short> scales(scale_seen.size());
            q8_repack(blocks.data(), rows, columns, codes.data(), scales.data());
            q8_unpack(codes.data(), scales.data(), rows, columns, back.data());
            if (back != blocks) { ++failures; }
            // Padding stays zero.
            for (size_t i = 0; i < codes_size; ++i) { if (!seen[i] && codes[i]) { ++failures; } }
        }
    }
    // Fragment order: lane 16 g + r holds row r, columns 8 g .. 8 g + 7 of the chunk's first block, then of its
    // second block, 16 bytes at lane * 16.
    if (q8_code_offset(2, 3, 64 + 8 * 2 + 5) != (long long)(1 * 1024 + (16 * 2 + 3) * 16 + 5)) { ++failures; }
    if (q8_code_offset(2, 3, 64 + 32 + 8 * 1 + 7) != (long long)(1 * 1024 + (16 * 1 + 3) * 16 + 8 + 7)) { ++failures; }
    // Scales: row 18 is row 2 of tile 1 (row group 0); block 3 is the second block of chunk 1.
    if (q8_scale_offset(2, 18, 3) != (long long)((1 * 2 + 1) * 32 + 0 * 8 + 1 * 4 + 2)) { ++failures; }
    if (q8_scale_offset(2, 13, 0) != (long long)(3 * 8 + 0 * 4 + 1)) { ++failures; }
    std::printf("%d\n", failures);
    return failures != 0;
}
'''


def test_q8_device_layout_is_a_bijection_and_round_trips(tmp_path):
    source = tmp_path / "q8_layout.cpp"
    source.write_text(Q8_LAYOUT_PROGRAM)
    binary = tmp_path / "q8_layout"
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", str(ROOT / "synapse_amd" / "csrc"), str(source), "-o",
                    str(binary)], check=True)
    result = subprocess.run([str(binary)], capture_output=True, text=True)
    assert result.returncode == 0, result.stdout


Q6_LAYOUT_PROGRAM = r'''
#include <cstdio>
#include <cstdlib>
#include <vector>
#include "kquant_layout.h"
using namespace synapse_kv;
int main() {
    int failures = 0;
    for (int rows : {1, 16, 17, 40}) {
        for (int columns : {256, 512, 768}) {
            const int chunks = q8_chunks(columns);
            const size_t size = (size_t)q8_tiles(rows) * chunks * kQ6KTileBytes;
            std::vector<int> low_seen(size * 2, 0), high_seen(size * 4, 0);
            const int supers = columns / 256;
            std::vector<unsigned char> blocks((size_t)rows * supers * 210);
            for (auto& b : blocks) { b = (unsigned char)(rand() & 0xFF); }
            std::vector<unsigned char> codes(size), factors((size_t)q8_tiles(rows) * chunks * kKFactorBytes);
            kq_repack(kEncodingQ6K, blocks.data(), rows, columns, codes.data(), factors.data());
            for (int row = 0; row < rows; ++row) {
                for (int column = 0; column < columns; ++column) {
                    long long low = 0, high = 0;
                    int low_shift = 0, high_shift = 0;
                    int64_t l64 = 0, h64 = 0;
                    q6k_code_place(chunks, row, column, l64, low_shift, h64, high_shift);
                    low = l64;
                    high = h64;
                    if (low < 0 || low >= (long long)size || high < 0 || high >= (long long)size) { ++failures; continue; }
                    if (low_seen[low * 2 + low_shift / 4]++ || high_seen[high * 4 + high_shift / 2]++) { ++failures; }
                    const int q = ((codes[low] >> low_shift) & 15) | (((codes[high] >> high_shift) & 3) << 4);
                    const unsigned char* block = blocks.data() + ((size_t)row * supers + column / 256) * 210;
                    if (q != kq_code(kEncodingQ6K, block, column % 256) + 32) { ++failures; }
                }
            }
            // Slots no value owns stay zero (row padding); every byte is either all nibbles or all pairs.
            for (size_t byte = 0; byte < size; ++byte) {
                const bool is_high = byte % kQ6KTileBytes >= (size_t)kQ4KTileBytes;
                for (int s = 0; s < (is_high ? 4 : 2); ++s) {
                    const int seen = is_high ? high_seen[byte * 4 + s] : low_seen[byte * 2 + s];
                    const int bits = is_high ? (codes[byte] >> (2 * s)) & 3 : (codes[byte] >> (4 * s)) & 15;
                    if (!seen && bits) { ++failures; }
                }
                if ((is_high ? low_seen[byte * 2] : high_seen[byte * 4]) != 0) { ++failures; }
            }
        }
    }
    // Row 3, column 64 + 32 + 8 * 2 + 5 of a 4-chunk matrix: tile 0, chunk 1 (bytes 768..), lane 16 * 2 + 3, byte 5
    // of its nibbles (second block: high nibble), byte 1 of its pairs at p = 2 * 1 + 1.
    int64_t low = 0, high = 0;
    int low_shift = 0, high_shift = 0;
    q6k_code_place(4, 3, 64 + 32 + 16 + 5, low, low_shift, high, high_shift);
    if (low != 768 + 35 * 8 + 5 || low_shift != 4 || high != 768 + 512 + 35 * 4 + 1 || high_shift != 6) { ++failures; }
    std::printf("%d\n", failures);
    return failures != 0;
}
'''


def test_q6_k_device_layout_holds_every_code_once(tmp_path):
    """The six-bit Q6_K device layout (low nibbles, then high bit pairs): every value's two slots are distinct and
    inside the matrix, they hold GGML's code + 32 for random super-blocks, and slots no value owns stay zero."""
    source = tmp_path / "q6_layout.cpp"
    source.write_text(Q6_LAYOUT_PROGRAM)
    binary = tmp_path / "q6_layout"
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", str(ROOT / "synapse_amd" / "csrc"), str(source), "-o",
                    str(binary)], check=True)
    result = subprocess.run([str(binary)], capture_output=True, text=True)
    assert result.returncode == 0, result.stdout


HALF_PROGRAM = r'''
#include <cstdio>
#include "kquant_layout.h"
int main() {
    for (unsigned bits = 0; bits < 65536; ++bits) {
        const unsigned char p[2] = {(unsigned char)(bits & 0xFF), (unsigned char)(bits >> 8)};
        const float value = synapse_kv::kq_half(p);
        unsigned word;
        memcpy(&word, &value, 4);
        printf("%08x\n", word);
    }
    return 0;
}
'''


def test_host_half_conversion_matches_numpy_for_every_bit_pattern(tmp_path):
    """kq_half's host branch (used by the weight repack on the CPU) rebuilds FP16 factors as FP32 bits; for all
    65,536 patterns it must equal numpy's float16 -> float32 widening, NaN payloads, infinities and signed
    subnormals included."""
    source = tmp_path / "half.cpp"
    source.write_text(HALF_PROGRAM)
    binary = tmp_path / "half"
    subprocess.run(["g++", "-std=c++17", "-O2", "-I", str(ROOT / "synapse_amd" / "csrc"), str(source), "-o",
                    str(binary)], check=True)
    result = subprocess.run([str(binary)], capture_output=True, text=True, check=True)
    got = np.array([int(line, 16) for line in result.stdout.split()], dtype=np.uint32)
    expected = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32).view(np.uint32)
    assert got.shape == expected.shape and np.array_equal(got, expected)
