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
//   * Q6_K codes stay six bits (768 bytes per tile): the low nibbles in Q4_K's 512-byte layout (lane l owns the 8
//     bytes at l * 8, byte j holding column 8 g + j of the first block in its low nibble and of the second block in
//     its high nibble), then the high bit pairs, lane l owning the 4 bytes at 512 + l * 4: byte i holds, in bits
//     2 p .. 2 p + 1 with p = 2 b + w, column 4 w + i of block b. A lane turns its 12 bytes into four words of four
//     biased codes q (0..63) with a shift, a mask and one shift-or per word (q6k_code_place);
//   * Q4_K codes stay four bits: 512 bytes per tile, lane l = 16 g + r owns the 8 bytes at l * 8, byte j holding
//     column 8 g + j of the chunk's first block (low nibble) and of its second block (high nibble) for row 16 t + r.
//     That pairing is GGML's own (sub-blocks 2 p and 2 p + 1 share bytes), and a chunk is always one such pair
//     because K-quant rows are whole 256-value super-blocks;
//   * a tile chunk has 64 factors, [row group g = (row % 16) / 4][field][block of the chunk][row % 4]: for Q4_K
//     field 0 is the block's scale d * sc and field 1 its offset dmin * m; for Q6_K field 0 is the scale of the
//     block's first 16 columns and field 1 that of its last 16 (d * scale). They are stored as GGML has them, one
//     byte per factor (Q4_K's 6-bit sc or m, Q6_K's int8 scale) plus the FP16 multiplier (d, dmin or d) per tile
//     row and field of a 256-column super-block, and multiplied at use: FP16 x 6-bit and FP16 x int8 products are
//     exact in FP32, so these are the reference's per-block factors bit for bit. The factors of a tile's four
//     chunks of one super-block form a 320-byte group: 4 x 64 factor bytes (lane order), then the 16 rows' two
//     multipliers (FP16, [row][field]). A wave reads a chunk's factor bytes with one 1-byte load per lane and its
//     lane's multiplier with one 2-byte load: row group g's 16 factors land in the 16 lanes of that row group.
//     80 bytes per tile chunk (0.078 B per weight) against 256 for FP32 factors.
#pragma once

#include <math.h>
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
constexpr int kQ6KTileBytes = kQ8TileBytes * 3 / 4;  // low nibbles (kQ4KTileBytes), then high bit pairs
constexpr int kKTileScales = 64;        // factors per tile and chunk
constexpr int kKSuperFactorBytes = 320;  // a tile's factor group per super-block: 4 x 64 bytes + 16 x 2 FP16
constexpr int kKFactorBytes = kKSuperFactorBytes / 4;  // per tile chunk

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
inline size_t tile_code_bytes(uint32_t encoding) {
    return encoding == kEncodingQ4K ? kQ4KTileBytes : (encoding == kEncodingQ6K ? kQ6KTileBytes : kQ8TileBytes);
}

// Where the six-bit code q (= code + 32) of Q6_K value (row, column) sits in a matrix's device codes: its low nibble
// at byte `low`, bits low_shift .. + 3, and its high bit pair at byte `high`, bits high_shift .. + 1.
SYNAPSE_Q8_HD inline void q6k_code_place(int chunks, int row, int column, int64_t& low, int& low_shift, int64_t& high,
                                         int& high_shift) {
    const int tile = row / kQ8TileRows;
    const int r = row % kQ8TileRows;
    const int chunk = column / kQ8ChunkColumns;
    const int within = column % kQ8ChunkColumns;
    const int block = within / kQ8BlockElements;
    const int g = (within % kQ8BlockElements) / 8;
    const int j = within % 8;
    const int64_t base = (static_cast<int64_t>(tile) * chunks + chunk) * kQ6KTileBytes;
    const int lane = 16 * g + r;
    low = base + lane * 8 + j;
    low_shift = 4 * block;
    high = base + kQ4KTileBytes + lane * 4 + j % 4;
    high_shift = 2 * (2 * block + j / 4);
}
inline size_t tile_scale_bytes(uint32_t encoding) {
    return is_kquant(encoding) ? kKFactorBytes : kQ8TileScales * sizeof(uint16_t);
}

SYNAPSE_Q8_HD inline float kq_half(const uint8_t* p) {
    const uint16_t bits = static_cast<uint16_t>(p[0] | (p[1] << 8));
#if defined(__HIP_DEVICE_COMPILE__)
    return static_cast<float>(__builtin_bit_cast(_Float16, bits));
#else
    // IEEE binary16 to FP32, exact (host compilers without _Float16): subnormals scaled, the rest rebuilt as bits
    // (exponent rebiased by 112, infinities and NaNs kept), so no float arithmetic meets a non-finite value.
    const uint32_t sign = static_cast<uint32_t>(bits >> 15) << 31;
    const uint32_t exponent = (bits >> 10) & 31;
    const uint32_t mantissa = bits & 1023;
    if (exponent == 0) {
        const float magnitude = ldexpf(static_cast<float>(mantissa), -24);
        return sign != 0 ? -magnitude : magnitude;
    }
    const uint32_t word = sign | ((exponent == 31 ? 255 : exponent + 112) << 23) | (mantissa << 13);
    float value;
    memcpy(&value, &word, 4);
    return value;
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

// Byte offsets, in a matrix's factor array, of the factor byte of (row, 32-column block, field) and of the FP16
// multiplier of (row, super-block, field). Chunks per row are a multiple of 4 (whole super-blocks), so chunk c of a
// tile's first chunk t0 is in group (t0 + c) / 4.
SYNAPSE_Q8_HD inline int64_t kq_factor_offset(int chunks, int row, int block, int field) {
    const int tile = row / kQ8TileRows;
    const int r = row % kQ8TileRows;
    const int64_t tile_chunk = static_cast<int64_t>(tile) * chunks + block / 2;
    return (tile_chunk >> 2) * kKSuperFactorBytes + (tile_chunk & 3) * kKTileScales + (r / 4) * 16 + field * 8 +
           (block % 2) * 4 + r % 4;
}

SYNAPSE_Q8_HD inline int64_t kq_multiplier_offset(int chunks, int row, int super_block, int field) {
    const int tile = row / kQ8TileRows;
    const int r = row % kQ8TileRows;
    const int64_t tile_chunk = static_cast<int64_t>(tile) * chunks + super_block * 4;
    return (tile_chunk >> 2) * kKSuperFactorBytes + 4 * kKTileScales + (r * 2 + field) * 2;
}

// GGML K-quant rows -> device layout. `codes` holds q8_tiles(rows) * q8_chunks(columns) * tile_code_bytes bytes,
// `factors` that many * kKFactorBytes; padding is zeroed (zero codes and zero factors).
inline void kq_repack(uint32_t encoding, const uint8_t* blocks, int rows, int columns, uint8_t* codes,
                      uint8_t* factors) {
    const int chunks = q8_chunks(columns);
    const size_t tiles = static_cast<size_t>(q8_tiles(rows)) * chunks;
    memset(codes, 0, tiles * tile_code_bytes(encoding));
    memset(factors, 0, tiles * kKFactorBytes);
    const int supers = columns / kSuperBlockValues;
    const int block_bytes = ggml_block_bytes(encoding);
    for (int row = 0; row < rows; ++row) {
        for (int s = 0; s < supers; ++s) {
            const uint8_t* block = blocks + (static_cast<size_t>(row) * supers + s) * block_bytes;
            // The FP16 multipliers as GGML stores them (little endian): Q4_K d and dmin, Q6_K d for both fields.
            const uint8_t* multipliers[2] = {encoding == kEncodingQ4K ? block : block + 208,
                                             encoding == kEncodingQ4K ? block + 2 : block + 208};
            for (int field = 0; field < 2; ++field) {
                memcpy(factors + kq_multiplier_offset(chunks, row, s, field), multipliers[field], 2);
            }
            for (int sub = 0; sub < 8; ++sub) {
                const int b = s * 8 + sub;  // 32-column block of the row
                if (encoding == kEncodingQ4K) {
                    int sc = 0;
                    int m = 0;
                    q4k_scale_min(block + 4, sub, sc, m);
                    factors[kq_factor_offset(chunks, row, b, 0)] = static_cast<uint8_t>(sc);
                    factors[kq_factor_offset(chunks, row, b, 1)] = static_cast<uint8_t>(m);
                } else {
                    for (int h = 0; h < 2; ++h) {
                        factors[kq_factor_offset(chunks, row, b, h)] = block[192 + 2 * sub + h];  // int8 bits
                    }
                }
                for (int l = 0; l < 32; ++l) {
                    const int code = kq_code(encoding, block, sub * 32 + l);
                    const int column = b * 32 + l;
                    if (encoding == kEncodingQ6K) {
                        int64_t low = 0;
                        int64_t high = 0;
                        int low_shift = 0;
                        int high_shift = 0;
                        q6k_code_place(chunks, row, column, low, low_shift, high, high_shift);
                        const int q = code + 32;
                        codes[low] |= static_cast<uint8_t>((q & 0xF) << low_shift);
                        codes[high] |= static_cast<uint8_t>((q >> 4) << high_shift);
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
