// Device layout of GGML K-quant projection matrices (ADR-021) and the host conversion from GGML super-blocks.
//
// GGML Q4_K (144 bytes per 256 values; GgufKQuantBlocks.cs:99-153, matmul_kquant.metal:16-68): FP16 d at byte 0,
// FP16 dmin at byte 2, 12 bytes of packed 6-bit scales and minima (get_scale_min_k4), then 128 bytes of 4-bit
// codes: byte 32 p + l holds value l of sub-block 2 p in its low nibble and value l of sub-block 2 p + 1 in its high
// nibble. Value i of sub-block j is (d * sc_j) * q - (dmin * m_j).
// GGML Q6_K (210 bytes per 256 values; GgufKQuantBlocks.cs:155-177): ql[128] low nibbles, qh[64] high bit pairs,
// int8 scales[16] (one per 16 values) at byte 192, FP16 d at byte 208. Value i is (d * scale_{i/16}) * (q - 32) with
// q the six-bit code.
//
// On the device every 32-value block is an MFMA k-depth, as for Q8_0 (q8_layout.h), with the same 16-row x 64-column
// tiles [row tile][column chunk]:
//   * Q6_K codes are int8 (q - 32), exactly Q8_0's tile layout (1 KiB per tile);
//   * Q4_K codes stay four bits: 512 bytes per tile, lane l = 16 g + r owns the 8 bytes at l * 8, byte j holding
//     column 8 g + j of the chunk's first block (low nibble) and of its second block (high nibble) for row 16 t + r.
//     That pairing is GGML's own (sub-blocks 2 p and 2 p + 1 share bytes), and a chunk is always one such pair
//     because K-quant rows are whole 256-value super-blocks;
//   * scales are FP32, 64 per tile and chunk: [row group g = (row % 16) / 4][field][block of the chunk][row % 4].
//     For Q4_K field 0 is the block's scale d * sc and field 1 its offset dmin * m; for Q6_K field 0 is the scale of
//     the block's first 16 columns and field 1 that of its last 16. A wave reads a tile chunk's 64 factors with
//     one 4-byte load per lane: row group g's 16 land in the 16 lanes of that row group. FP16 x 6-bit and
//     FP16 x int8 products are exact in FP32, so these are the reference's per-block factors bit for bit.
#pragma once

#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include "q8_layout.h"

namespace synapse_kv {

constexpr uint32_t kEncodingQ8_0 = 8;
constexpr uint32_t kEncodingQ4K = 12;
constexpr uint32_t kEncodingQ6K = 14;
constexpr uint32_t kEncodingMixedK = 0xFFu;  // a decode launch over Q4_K and Q6_K segments together
constexpr int kSuperBlockValues = 256;
constexpr int kQ4KBlockBytes = 144;
constexpr int kQ6KBlockBytes = 210;
constexpr int kQ4KTileBytes = kQ8TileBytes / 2;
constexpr int kKTileScales = 64;  // FP32 values per tile and chunk

SYNAPSE_Q8_HD inline bool is_kquant(uint32_t encoding) { return encoding == kEncodingQ4K || encoding == kEncodingQ6K; }

// Bytes of one GGML block and values per block.
SYNAPSE_Q8_HD inline int ggml_block_bytes(uint32_t encoding) {
    return encoding == kEncodingQ4K ? kQ4KBlockBytes : (encoding == kEncodingQ6K ? kQ6KBlockBytes : kQ8BlockBytes);
}
SYNAPSE_Q8_HD inline int ggml_block_values(uint32_t encoding) {
    return is_kquant(encoding) ? kSuperBlockValues : kQ8BlockElements;
}

// Bytes of a rows x columns GGML matrix (columns a multiple of the block's values).
inline uint64_t ggml_matrix_bytes(uint32_t encoding, uint64_t rows, uint64_t columns) {
    return rows * (columns / ggml_block_values(encoding)) * ggml_block_bytes(encoding);
}

// Device bytes per tile and chunk: codes, then scales.
inline size_t tile_code_bytes(uint32_t encoding) { return encoding == kEncodingQ4K ? kQ4KTileBytes : kQ8TileBytes; }
inline size_t tile_scale_bytes(uint32_t encoding) {
    return is_kquant(encoding) ? kKTileScales * sizeof(float) : kQ8TileScales * sizeof(uint16_t);
}

SYNAPSE_Q8_HD inline float kq_half(const uint8_t* p) {
    const uint16_t bits = static_cast<uint16_t>(p[0] | (p[1] << 8));
#if defined(__HIP_DEVICE_COMPILE__)
    return static_cast<float>(__builtin_bit_cast(_Float16, bits));
#else
    _Float16 value;
    memcpy(&value, &bits, 2);
    return static_cast<float>(value);
#endif
}

// get_scale_min_k4: sub-block j's 6-bit scale and minimum from the 12 packed bytes.
SYNAPSE_Q8_HD inline void q4k_scale_min(const uint8_t* packed, int j, int& scale, int& minimum) {
    if (j < 4) {
        scale = packed[j] & 63;
        minimum = packed[j + 4] & 63;
    } else {
        scale = (packed[j + 4] & 0xF) | ((packed[j - 4] >> 6) << 4);
        minimum = (packed[j + 4] >> 4) | ((packed[j] >> 6) << 4);
    }
}

// Code of value i (0..255) of a super-block: Q4_K 0..15, Q6_K q - 32 in -32..31.
SYNAPSE_Q8_HD inline int kq_code(uint32_t encoding, const uint8_t* block, int i) {
    const int sub = i / 32;
    const int l = i % 32;
    if (encoding == kEncodingQ4K) {
        const uint8_t byte = block[16 + (sub / 2) * 32 + l];
        return (sub % 2 == 0) ? (byte & 0xF) : (byte >> 4);
    }
    const int half = sub / 4;
    const int quarter = sub % 4;
    const uint8_t low = block[half * 64 + ((quarter % 2 == 0) ? l : l + 32)];
    const int nibble = quarter < 2 ? (low & 0xF) : (low >> 4);
    const int high = (block[128 + half * 32 + l] >> (2 * quarter)) & 3;
    return (nibble | (high << 4)) - 32;
}

// Element offset of the scale-table entry (row, 32-column block, field) in the scales array.
SYNAPSE_Q8_HD inline int64_t kq_scale_offset(int chunks, int row, int block, int field) {
    const int tile = row / kQ8TileRows;
    const int r = row % kQ8TileRows;
    const int chunk = block / 2;
    return (static_cast<int64_t>(tile) * chunks + chunk) * kKTileScales + (r / 4) * 16 + field * 8 + (block % 2) * 4 +
           r % 4;
}

// GGML K-quant rows -> device layout. `codes` holds q8_tiles(rows) * q8_chunks(columns) * tile_code_bytes bytes,
// `scales` that many * 64 floats; padding is zeroed (zero codes and zero factors).
inline void kq_repack(uint32_t encoding, const uint8_t* blocks, int rows, int columns, uint8_t* codes, float* scales) {
    const int chunks = q8_chunks(columns);
    const size_t tiles = static_cast<size_t>(q8_tiles(rows)) * chunks;
    memset(codes, 0, tiles * tile_code_bytes(encoding));
    memset(scales, 0, tiles * kKTileScales * sizeof(float));
    const int supers = columns / kSuperBlockValues;
    const int block_bytes = ggml_block_bytes(encoding);
    for (int row = 0; row < rows; ++row) {
        for (int s = 0; s < supers; ++s) {
            const uint8_t* block = blocks + (static_cast<size_t>(row) * supers + s) * block_bytes;
            for (int sub = 0; sub < 8; ++sub) {
                const int b = s * 8 + sub;  // 32-column block of the row
                if (encoding == kEncodingQ4K) {
                    int sc = 0;
                    int m = 0;
                    q4k_scale_min(block + 4, sub, sc, m);
                    scales[kq_scale_offset(chunks, row, b, 0)] = kq_half(block) * static_cast<float>(sc);
                    scales[kq_scale_offset(chunks, row, b, 1)] = kq_half(block + 2) * static_cast<float>(m);
                } else {
                    const float d = kq_half(block + 208);
                    for (int h = 0; h < 2; ++h) {
                        const int8_t sc = static_cast<int8_t>(block[192 + 2 * sub + h]);
                        scales[kq_scale_offset(chunks, row, b, h)] = d * static_cast<float>(sc);
                    }
                }
                for (int l = 0; l < 32; ++l) {
                    const int code = kq_code(encoding, block, sub * 32 + l);
                    const int column = b * 32 + l;
                    if (encoding == kEncodingQ6K) {
                        codes[q8_code_offset(chunks, row, column)] = static_cast<uint8_t>(static_cast<int8_t>(code));
                    } else {
                        // The Q8_0 offset of (row, column) with the block bit dropped, halved: lane * 8 + j.
                        const int tile = row / kQ8TileRows;
                        const int r = row % kQ8TileRows;
                        const int chunk = column / kQ8ChunkColumns;
                        const int within = column % kQ8ChunkColumns;
                        const int g = (within % kQ8BlockElements) / 8;
                        const size_t at = (static_cast<size_t>(tile) * chunks + chunk) * kQ4KTileBytes +
                                          (16 * g + r) * 8 + within % 8;
                        codes[at] |= static_cast<uint8_t>(code << (within < kQ8BlockElements ? 0 : 4));
                    }
                }
            }
        }
    }
}

}  // namespace synapse_kv
