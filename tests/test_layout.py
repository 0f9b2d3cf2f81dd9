"""The page layout maps every (key, dim) of a region to its own element, inside the region (CPU, g++)."""

import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent

PROGRAM = r'''
#include <cstdio>
#include <vector>
#include "page_layout.h"
using namespace synapse_kv;
int main() {
    int failures = 0;
    for (int page : {64, 256, 1024}) {
        for (int d : {64, 128}) {
            for (int kind = 0; kind < 4; ++kind) {
                std::vector<int> seen(static_cast<size_t>(page) * d, 0);
                for (int key = 0; key < page; ++key) {
                    for (int dim = 0; dim < d; ++dim) {
                        long long at = kind == 0 ? key_offset_f16(d, key, dim) : kind == 1 ? value_offset_f16(d, key, dim)
                                     : kind == 2 ? key_offset_f32(d, key, dim) : value_offset_f32(d, key, dim);
                        if (at < 0 || at >= (long long)seen.size() || seen[at]++) { ++failures; }
                        // Every 64-key block stays inside its own block.
                        if (at / (64LL * d) != key / 64) { ++failures; }
                    }
                }
            }
        }
    }
    // Spot checks of the fragment order: FP16 K chunk (t=1, ks=0, lane 16g + r), index (1 * D/32 + 0) * 64 + lane,
    // holds key 4 + 8*(r/4) + r%4.
    if (key_offset_f16(128, 4, 0) != (1 * 4 + 0) * 64 * 8) { ++failures; }
    if (key_offset_f16(128, 0, 8) != 16 * 8) { ++failures; }
    // FP16 V chunk (h=0, mt=0, lane 16g + r) holds keys 8g..8g+7 of dim r, consecutive.
    if (value_offset_f16(128, 9, 3) != (16 * 1 + 3) * 8 + 1) { ++failures; }
    std::printf("%d\n", failures);
    return failures != 0;
}
'''


def test_layout_is_a_bijection(tmp_path):
    source = tmp_path / "layout.cpp"
    source.write_text(PROGRAM)
    binary = tmp_path / "layout"
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", str(ROOT / "synapse_amd" / "csrc"), str(source), "-o",
                    str(binary)], check=True)
    result = subprocess.run([str(binary)], capture_output=True, text=True)
    assert result.returncode == 0, result.stdout
