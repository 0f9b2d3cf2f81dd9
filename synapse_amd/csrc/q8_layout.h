// Device layout of one Q8_0 projection matrix, and the host conversions from and to GGML Q8_0 blocks.
//
// GGML Q8_0 (the model file, read by matmul.cu:87-121 / matmul.metal:88-128): each row is columns / 32 blocks of
// 34 bytes, an FP16 scale d followed by 32 int8 codes; element (row, k) = d(row, k / 32) * code(row, k).
//
// Device layout: the matrix is cut into tiles of 16 rows x 64 columns (two Q8_0 blocks; rows and columns padded
// with zero codes and zero scales), stored [row tile][column chunk]. A tile's codes are 1 KiB in the order the
// projection kernel loads its MFMA A operands: lane l = 16 g + r of a wave reads the 16 bytes at l * 16, the codes
// of row 16 * tile + r at columns 8 g .. 8 g + 7 of the chunk's first block, then the same columns of its second
// block (v_mfma_f32_16x16x32_bf16 takes k = 8 g .. 8 g + 7 of one 32-column block from lane group g). The tile's
// scales are 32 FP16 values (q8_scale_offset), kept in a separate array so the codes stay 1 KiB aligned.
#pragma once

#include <stddef.h>
#include <stdint.h>
#include <string.h>

namespace synapse_kv {

constexpr int kQ8BlockElements = 32;
constexpr int kQ8BlockBytes = 34;
constexpr int kQ8TileRows = 16;
constexpr int kQ8ChunkColumns = 64;
constexpr int kQ8TileBytes = kQ8TileRows * kQ8ChunkColumns;  // one byte per code
constexpr int kQ8TileScales = kQ8TileRows * (kQ8ChunkColumns / kQ8BlockElements);

#if defined(__HIPCC__)
#define SYNAPSE_Q8_HD __host__ __device__
#else
#define SYNAPSE_Q8_HD
#endif

SYNAPSE_Q8_HD inline int q8_tiles(int rows) { return (rows + kQ8TileRows - 1) / kQ8TileRows; }
SYNAPSE_Q8_HD inline int q8_chunks(int columns) { return (columns + kQ8ChunkColumns - 1) / kQ8ChunkColumns; }

// Byte offset of code (row, column) in the codes array of a matrix with `chunks` column chunks.
SYNAPSE_Q8_HD inline int64_t q8_code_offset(int chunks, int row, int column) {
    const int tile = row / kQ8TileRows;
    const int r = row % kQ8TileRows;
    const int chunk = column / kQ8ChunkColumns;
    const int block = (column % kQ8ChunkColumns) / kQ8BlockElements;
    const int g = (column % kQ8BlockElements) / 8;
    const int j = column % 8;
    return (static_cast<int64_t>(tile) * chunks + chunk) * kQ8TileBytes + (16 * g + r) * 16 + 8 * block + j;
}

// Element offset of the scale of (row, block) in the scales array (block = column / 32): per tile and chunk,
// [row group g = (row % 16) / 4][block of the chunk][row % 4], so the accumulator lanes of row group g read their
// eight scales (two blocks x four rows) with one 16-byte load.
SYNAPSE_Q8_HD inline int64_t q8_scale_offset(int chunks, int row, int block) {
    const int tile = row / kQ8TileRows;
    const int r = row % kQ8TileRows;
    const int chunk = block / 2;
    return (static_cast<int64_t>(tile) * chunks + chunk) * kQ8TileScales + (r / 4) * 8 + (block % 2) * 4 + r % 4;
}

// GGML blocks (rows x columns / 32 blocks of 34 bytes) -> device layout. `codes` holds
// q8_tiles(rows) * q8_chunks(columns) * kQ8TileBytes bytes and `scales` that many / 32 FP16 values (as raw
// uint16 bits); padding is zeroed.
inline void q8_repack(const uint8_t* blocks, int rows, int columns, uint8_t* codes, uint16_t* scales) {
    const int chunks = q8_chunks(columns);
    const size_t tiles = static_cast<size_t>(q8_tiles(rows));
    memset(codes, 0, tiles * chunks * kQ8TileBytes);
    memset(scales, 0, tiles * chunks * kQ8TileScales * sizeof(uint16_t));
    const int per_row = columns / kQ8BlockElements;
    for (int row = 0; row < rows; ++row) {
        for (int block = 0; block < per_row; ++block) {
            const uint8_t* source = blocks + (static_cast<size_t>(row) * per_row + block) * kQ8BlockBytes;
            uint16_t scale;
            memcpy(&scale, source, sizeof(scale));
            scales[q8_scale_offset(chunks, row, block)] = scale;
            // 32 codes = four runs of 8 consecutive columns, each contiguous in the tile.
            for (int g = 0; g < 4; ++g) {
                const int column = block * kQ8BlockElements + 8 * g;
                memcpy(codes + q8_code_offset(chunks, row, column), source + 2 + 8 * g, 8);
            }
        }
    }
}

// Device layout -> GGML blocks (the inverse of q8_repack on the unpadded part).
inline void q8_unpack(const uint8_t* codes, const uint16_t* scales, int rows, int columns, uint8_t* blocks) {
    const int chunks = q8_chunks(columns);
    const int per_row = columns / kQ8BlockElements;
    for (int row = 0; row < rows; ++row) {
        for (int block = 0; block < per_row; ++block) {
            uint8_t* target = blocks + (static_cast<size_t>(row) * per_row + block) * kQ8BlockBytes;
            const uint16_t scale = scales[q8_scale_offset(chunks, row, block)];
            memcpy(target, &scale, sizeof(scale));
            for (int g = 0; g < 4; ++g) {
                const int column = block * kQ8BlockElements + 8 * g;
                memcpy(target + 2 + 8 * g, codes + q8_code_offset(chunks, row, column), 8);
            }
        }
    }
}

}  // namespace synapse_kv
