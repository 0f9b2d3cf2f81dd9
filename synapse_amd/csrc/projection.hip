// Q8_0 and K-quant projections (QKV before the attention path, o_proj after it, the feed-forward and logits of the
// decoder step) on the matrix cores: bf16 with exact products for prompt runs, FP16 over a two-part input for decode.
//
// Semantics: synapse_q8_matvec_{1,2,4,8} and synapse_q8_gemm (native/synapse-gpu/src/Features/GpuKernels/cuda/
// kernels/matmul.cu:1-189, metal/shaders/matmul.metal:1-310): output[t][out_column + row] = (accumulate ? output : 0)
// + sum_blocks d * sum_k code[row][k] * input[t][k] + bias[row], rows of up to three matrices in one dispatch
// (locate_segment, common.metal:138-146). Weights stay Q8_0, activations FP32, sums FP32 (ADR-012).
//
// Prompt runs, exact products on the bf16 matrix cores: each FP32 input x is split into three bf16 parts with
// x = hi + mid + lo exactly (bf16 keeps FP32's exponent range; each part takes the next 8 significant bits, and the
// residuals x - hi and (x - hi) - mid are exact FP32 subtractions). A Q8_0 code is exact in bf16, and code * part
// is a product of at most 8 by 8 significant bits, exact in FP32. One Q8_0 block (32 columns) is one k-depth of
// v_mfma_f32_16x16x32_bf16: the block's three MFMAs (lo, mid, hi parts) sum its exact products in FP32 into a fresh
// accumulator, and the block's sum is then scaled and added as the reference does (sum = fma(block dot, d, sum),
// matmul.cu:101-104). Only the order of the FP32 additions differs from the reference's kernels.
//
// MI355X mapping, decode (at most 16 tokens): project_decode_kernel, one workgroup per eight 16-row tiles and one
// slice of at most eight 64-column chunks; the workgroup splits its input slice into LDS once, as two FP16 parts of
// the input scaled per token by a power of two (products exact in FP32; the parts hold the input to 2^-22), and every
// wave streams its tile's codes and scales against it on v_mfma_f32_16x16x32_f16 (see below); reduce_kernel adds the
// slices in order with bias and residual.
//
// K-quant matrices (Q4_K, Q6_K; kquant_layout.h) run the same kernels specialised on the encoding: a block's codes
// are exact in bf16 too (0..15, -32..31), and its factors (a factor byte times an FP16 multiplier, exact in FP32)
// are applied to the block's exact-product sum. Q4_K subtracts offset * sum(x) with the block's input sums (LDS in
// the decode kernel, written by split_kernel for prompt runs); Q6_K multiplies each 16-column half on its own (the
// other half's A fragments zeroed) and scales each.
//
// Prompt runs: split_kernel writes the three parts of the whole input once, in the B-operand fragment order of the
// MFMA, and project_gemm_kernel runs one workgroup per 128 rows x 64 (K-quants: 32) tokens. The tokens' split input
// goes through an LDS ring shared by the four waves; each wave streams the codes (one 16-byte load per lane per
// tile and chunk, fragment order, see q8_layout.h) and factors of its two row tiles, and writes its outputs with
// the bias and the residual.

#include "kv_internal.h"
#include <utility>

#include "kquant_layout.h"
#include "q8_layout.h"

namespace synapse_kv {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t uintx4 __attribute__((ext_vector_type(4)));
typedef uint32_t uintx2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kParts = 3;

// One thread per (token, 8 columns) in the order of split_thread: the three bf16 parts of input[token][8 j ..
// 8 j + 7] (zeros past `columns`); each thread reads 32 contiguous bytes of its row.
__global__ __launch_bounds__(256) void split_kernel(ProjectionArgs a) {
    int token;
    int column;
    if (!split_thread(blockIdx.x * 256 + threadIdx.x, a.chunks, a.tokens, token, column)) {
        return;
    }
    float values[8];
    if (column < a.columns) {
        const floatx4* source = reinterpret_cast<const floatx4*>(a.input + static_cast<size_t>(token) * a.in_stride + column);
        const floatx4 first = source[0];
        const floatx4 second = source[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            values[i] = first[i];
            values[i + 4] = second[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            values[i] = 0.0f;
        }
    }
    SplitInput split;
    split.parts = a.parts;
    split.sums = a.sums;
    split.chunks = a.chunks;
    store_split_group(split, token, column, values);
}

// Per token tile and block, the three parts of columns 8 g .. 8 g + 7 of token 16 c + r (B fragments).
template <int NT>
struct InputFragments {
    bf16x8 x[NT][2][kParts];
};

// One chunk of one 16-row tile as a lane loads it: its codes (16 bytes of int8 codes; Q4_K: 8 bytes of nibbles in
// .xy) and the factors of its accumulator rows (Q8_0: the row group's eight FP16 scales, wide or compact, see
// load_chunk). K-quant factors are loaded one per lane (its factor byte and its FP16 multiplier, multiplied at use):
// the chunk's 64 factors, [row group][field][block][row], so row group g's sixteen sit in DPP row g (lanes
// 16 g .. 16 g + 15), exactly the lanes whose accumulators need them; they are broadcast within the row at use
// (row_broadcast_factors) instead of every lane loading all sixteen.
template <uint32_t E>
struct ChunkWeights {
    uintx4 codes;
    uintx4 scales;        // Q8_0 with wide scales: the row group's eight FP16 scales
    uint32_t factor;      // Q8_0 otherwise: two FP16 scales (see load_chunk); K-quants: factor `lane`'s byte
                          // (Q4_K's 6-bit sc or m, Q6_K's int8 scale, sign-extended)
    uint32_t multiplier;  // K-quants: FP16 bits of factor `lane`'s multiplier (d, dmin or d)
};

// K-quant factor `lane` of a loaded chunk as FP32 bits: multiplier x factor byte, exact in FP32.
template <uint32_t E>
__device__ inline uint32_t kquant_factor_bits(const ChunkWeights<E>& w) {
    const float multiplier = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w.multiplier)));
    return __builtin_bit_cast(uint32_t, multiplier * static_cast<float>(static_cast<int32_t>(w.factor)));
}

// Loads chunk `tile_chunk` (tile * chunks + chunk) of a matrix for lane `lane` of row group g. Q8_0 scales come
// either wide (each lane loads its row group's eight scales, 16 bytes: no broadcast at use; the one-shot decode
// kernel, where it measured faster) or compact (lanes 16 g .. 16 g + 3 load the row group's four scale words, one
// register per lane, broadcast within the DPP row at use: the GEMM, where registers bound the occupancy).
template <uint32_t E, bool kWide = false>
__device__ inline ChunkWeights<E> load_chunk(const uint8_t* codes, const void* scales, size_t tile_chunk, int lane,
                                             int g) {
    ChunkWeights<E> w;
    if constexpr (E == kEncodingQ4K) {
        const uintx2 half = __builtin_nontemporal_load(reinterpret_cast<const uintx2*>(codes + tile_chunk * kQ4KTileBytes) + lane);
        w.codes = uintx4{half.x, half.y, 0u, 0u};
    } else if constexpr (E == kEncodingQ6K) {
        // Low nibbles in .xy, high bit pairs in .z (q6k_codes turns them into biased codes).
        const uint8_t* tile = codes + tile_chunk * kQ6KTileBytes;
        const uintx2 low = __builtin_nontemporal_load(reinterpret_cast<const uintx2*>(tile) + lane);
        const uint32_t high = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(tile + kQ4KTileBytes) + lane);
        w.codes = uintx4{low.x, low.y, high, 0u};
    } else {
        w.codes = __builtin_nontemporal_load(reinterpret_cast<const uintx4*>(codes + tile_chunk * kQ8TileBytes) + lane);
    }
    if constexpr (E == kEncodingQ8_0 && kWide) {
        w.scales = __builtin_nontemporal_load(
            reinterpret_cast<const uintx4*>(static_cast<const uint16_t*>(scales) + tile_chunk * kQ8TileScales) + g);
    } else if constexpr (E == kEncodingQ8_0) {
        // Row group g's eight scales (q8_scale_offset: [g][block][row % 4]) are four 32-bit words.
        w.factor = reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(scales) + tile_chunk * kQ8TileScales)
            [4 * g + (lane & 3)];
    } else {
        // The chunk's 320-byte factor group (kquant_layout.h): this lane's factor byte, and the FP16 multiplier of
        // its row (4 g + lane % 4) and field (lane / 8 % 2).
        const uint8_t* group = static_cast<const uint8_t*>(scales) + (tile_chunk >> 2) * kKSuperFactorBytes;
        const uint8_t* bytes = group + (tile_chunk & 3) * kKTileScales;
        if constexpr (E == kEncodingQ6K) {
            w.factor = static_cast<uint32_t>(static_cast<int32_t>(reinterpret_cast<const int8_t*>(bytes)[lane]));
        } else {
            w.factor = bytes[lane];
        }
        w.multiplier =
            reinterpret_cast<const uint16_t*>(group + 4 * kKTileScales)[(4 * g + (lane & 3)) * 2 + ((lane >> 3) & 1)];
    }
    return w;
}

// Word 2 b + w of a loaded Q6_K chunk (ChunkWeights::codes): the biased codes q = code + 32 of columns 4 w .. 4 w + 3
// of block b, one per byte (kquant_layout.h).
__device__ inline uint32_t q6k_word(uintx4 codes, int b, int w) {
    return ((codes[w] >> (4 * b)) & 0x0F0F0F0Fu) | (((codes[2] >> (2 * (2 * b + w))) & 0x03030303u) << 4);
}

// factors[n] = the value lane 16 g + n holds, for every lane of row group g (DPP row_newbcast:n).
template <int... N>
__device__ inline void broadcast_each(uint32_t bits, float (&factors)[16], std::integer_sequence<int, N...>) {
    ((factors[N] = __builtin_bit_cast(
          float, __builtin_amdgcn_update_dpp(0, static_cast<int>(bits), 0x150 + N, 0xF, 0xF, false))),
     ...);
}

__device__ inline void row_broadcast_factors(uint32_t bits, float (&factors)[16]) {
    broadcast_each(bits, factors, std::make_integer_sequence<int, 16>{});
}

// The chunk's two blocks of A fragments: eight codes of one row per block, exact in bf16.
template <uint32_t E>
__device__ inline void weight_fragments(uintx4 codes, bf16x8 (&weight)[2]) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int w = 0; w < 2; ++w) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int code;
                if constexpr (E == kEncodingQ4K) {
                    code = static_cast<int>((codes[w] >> (8 * i + 4 * b)) & 0xF);
                } else if constexpr (E == kEncodingQ6K) {
                    code = static_cast<int>((q6k_word(codes, b, w) >> (8 * i)) & 0xFF) - 32;
                } else {
                    code = static_cast<int8_t>((codes[2 * b + w] >> (8 * i)) & 0xFF);
                }
                weight[b][4 * w + i] = static_cast<__bf16>(static_cast<float>(code));
            }
        }
    }
}

// One chunk (two blocks): each block's three part products go to their own fresh accumulator, issued part by part
// across blocks and token tiles so a dependent MFMA is 2 NT MFMAs behind the one it needs, and the block sums are
// scaled into the running sums after all of them were issued.
//   Q8_0: acc += d * (codes . x) per block (matmul.cu:101-104).
//   Q4_K: acc += scale * (codes . x) - offset * sum(x) per block, with sum(x) the block's input sum per token in
//         `xsum` (kq_apply, matmul_kquant.metal:115-119).
//   Q6_K: the block's two 16-column halves have their own scales: the A fragments of lane groups 0-1 (columns
//         0-15) and 2-3 (columns 16-31) are multiplied separately (the other half zeroed) and each sum scaled.
template <uint32_t E, int NT, bool kWide = false>
__device__ inline void multiply_chunk(const ChunkWeights<E>& w, const InputFragments<NT>& input,
                                      const float (&xsum)[NT][2], floatx4 (&acc)[NT]) {
    bf16x8 weight[2];
    weight_fragments<E>(w.codes, weight);
    if constexpr (E == kEncodingQ8_0) {
        // The row group's four scale words: loaded wide, or broadcast within the DPP row from lanes
        // 16 g .. 16 g + 3.
        uint32_t words[4];
        if constexpr (kWide) {
            words[0] = w.scales[0];
            words[1] = w.scales[1];
            words[2] = w.scales[2];
            words[3] = w.scales[3];
        } else {
            const int bits = static_cast<int>(w.factor);
            words[0] = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, bits, 0x150, 0xF, 0xF, false));
            words[1] = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, bits, 0x151, 0xF, 0xF, false));
            words[2] = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, bits, 0x152, 0xF, 0xF, false));
            words[3] = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, bits, 0x153, 0xF, 0xF, false));
        }
        float d[2][4];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t pair = words[2 * b + h];
                d[b][2 * h] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(pair & 0xFFFF)));
                d[b][2 * h + 1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(pair >> 16)));
            }
        }
        floatx4 block[2][NT];
#pragma unroll
        for (int p = kParts - 1; p >= 0; --p) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
#pragma unroll
                for (int c = 0; c < NT; ++c) {
                    block[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        weight[b], input.x[c][b][p], p == kParts - 1 ? floatx4{0.0f, 0.0f, 0.0f, 0.0f} : block[b][c],
                        0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int c = 0; c < NT; ++c) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    acc[c][i] = __builtin_fmaf(block[b][c][i], d[b][i], acc[c][i]);
                }
            }
        }
    } else if constexpr (E == kEncodingQ4K) {
        floatx4 block[2][NT];
#pragma unroll
        for (int p = kParts - 1; p >= 0; --p) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
#pragma unroll
                for (int c = 0; c < NT; ++c) {
                    block[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        weight[b], input.x[c][b][p], p == kParts - 1 ? floatx4{0.0f, 0.0f, 0.0f, 0.0f} : block[b][c],
                        0, 0, 0);
                }
            }
        }
        float factors[16];
        row_broadcast_factors(kquant_factor_bits(w), factors);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int c = 0; c < NT; ++c) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float scale = factors[b * 4 + i];
                    const float offset = factors[8 + b * 4 + i];
                    acc[c][i] = __builtin_fmaf(block[b][c][i], scale, acc[c][i]);
                    acc[c][i] = __builtin_fmaf(-offset, xsum[c][b], acc[c][i]);
                }
            }
        }
    } else {
        const bool first_half = (threadIdx.x & 63) < 32;  // lane groups 0 and 1
        const bf16x8 zero = bf16x8{};
        bf16x8 halves[2][2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            halves[0][b] = first_half ? weight[b] : zero;
            halves[1][b] = first_half ? zero : weight[b];
        }
        floatx4 block[2][2][NT];
#pragma unroll
        for (int p = kParts - 1; p >= 0; --p) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int b = 0; b < 2; ++b) {
#pragma unroll
                    for (int c = 0; c < NT; ++c) {
                        block[h][b][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            halves[h][b], input.x[c][b][p],
                            p == kParts - 1 ? floatx4{0.0f, 0.0f, 0.0f, 0.0f} : block[h][b][c], 0, 0, 0);
                    }
                }
            }
        }
        float factors[16];
        row_broadcast_factors(kquant_factor_bits(w), factors);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
#pragma unroll
                for (int c = 0; c < NT; ++c) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        acc[c][i] = __builtin_fmaf(block[h][b][c][i], factors[h * 8 + b * 4 + i], acc[c][i]);
                    }
                }
            }
        }
    }
}

// ---- Decode (at most 16 tokens): row tiles share the split input through LDS ----------------------------------

// A workgroup of eight waves covers eight 16-row tiles (one per wave; tiles of different matrices may meet in one
// workgroup) over one slice of at most kDecodeSliceChunks column chunks. The workgroup first splits its slice of the
// input into two FP16 parts (scaled per token by a power of two), in B-fragment order, into LDS; then every wave
// streams its tile's codes and scales for the slice (its only vector-memory loads, all issued up front) and
// multiplies against the fragments in LDS. Each slice's 16 x 16 sums go to partial rows; reduce_kernel adds the
// slices in order with the bias and the residual. The input is read from L2 once per workgroup instead of once per
// tile. Eight waves share one 32 KiB staged input, so four workgroups fit a CU's LDS.
constexpr int kDecodeSliceChunks = 8;
constexpr int kDecodeWaves = 8;

__device__ inline int locate_tile(const ProjectionArgs& a, int tile, ProjectionSegment& seg) {
    int s = 0;
    while (s + 1 < a.segments && tile >= a.segment[s + 1].first_tile) {
        ++s;
    }
    seg = a.segment[s];
    return tile - seg.first_tile;
}

// ---- Prompt runs: two-dimensional workgroup tiles ----------------------------------------------------------------

// A workgroup covers 64 RT rows x 16 NT tokens: four waves of RT row tiles x NT token tiles each, against one copy
// of the tokens' split input per column chunk (6 NT KiB: NT token tiles x 3 parts x 2 blocks, 1 KiB each in
// fragment order) shared through LDS, while each wave streams its own rows' codes. Covering many rows per copy of
// the input is what matters: the input costs 6 bytes per value against 1 byte per code. launch_projection takes the
// largest tile (Q8_0: 4 x 2, then 2 x 2, then 2 x 1; K-quants: 2 x 2, then 2 x 1, their factors and Q4_K input
// sums taking more registers) that still gives two workgroups per CU.
//   - The chunk's split input goes through a three-deep LDS ring by global_load_lds, 1.5 NT copies of 1 KiB per
//     wave.
//   - Each wave's codes and factors (and, for Q4_K, its tokens' sums of 8 inputs) load into a ring of three
//     register sets.
//   - Per chunk a wave issues chunk + 2's loads, then its copies of chunk + 2 (scheduling barriers keep that
//     order). Loads complete in issue order, so waiting at the top of a chunk for all but the newest kOps
//     operations (the next chunk's) covers that chunk's loads and copy; the barrier after the wait also tells
//     every wave that the buffer the chunk's copy overwrites (read in the chunk before) is free. The loads are
//     never the newest operations when they are used, so the compiler's own waits stay partial too.
//   - The multiplies are multiply_chunk's, whose FP32 additions per output follow the reference's block order.
// Measured on the 7B QKV + o_proj pair at 2,048 tokens (Q8_0, split included): 269 TFLOP/s of exact-product work
// with 128 x 64 tiles, against 87.6 for one 16-row tile per workgroup.
constexpr int kGemmWaves = 4;
constexpr int kGemmDepth = 3;

// Per token-tile count: 1 KiB copies per chunk (and per wave) and tokens per workgroup.
template <int NT>
struct GemmShape {
    static constexpr int kSegments = NT * kParts * 2;
    static constexpr int kCopies = kSegments / kGemmWaves;
    static constexpr int kTokens = NT * 16;
    static_assert(kSegments % kGemmWaves == 0, "copies split evenly over the waves");
};

// This wave's LDS copies of one chunk's split input (a __device__ function: the copy builtin inside a lambda of the
// kernel, under a template-dependent loop, left the kernel's host launch stub undefined).
template <int NT>
__device__ inline void gemm_copy_chunk(const uint8_t* const* sources, size_t offset, bf16x8* stage, int wave) {
#pragma unroll
    for (int j = 0; j < GemmShape<NT>::kCopies; ++j) {
        __builtin_amdgcn_global_load_lds(sources[j] + offset,
                                         (__attribute__((address_space(3))) void*)(&stage[(wave + kGemmWaves * j) * 64]),
                                         16, 0, 0);
    }
}

template <uint32_t E, int NT, int RT>
struct GemmLoads {
    ChunkWeights<E> w[RT];
    floatx4 sums[NT][2];  // Q4_K
};

struct GemmTile {
    const uint8_t* codes;  // the tile's first chunk
    const void* scales;    // the tile's first chunk's factors
    int rows_left;         // rows of the segment from this tile's first row (0: past the last tile)
    int out_column;        // output column of the tile's first row
    const float* bias;     // at the tile's first row, or null
};

// NT token tiles per workgroup and RT row tiles per wave (launch_projection picks them per launch).
template <uint32_t E, int NT, int RT>
__global__ __launch_bounds__(kGemmWaves * 64, E == kEncodingQ6K ? 3 : 2) void project_gemm_kernel(ProjectionArgs a) {
    using Shape = GemmShape<NT>;
    __shared__ bf16x8 ring[kGemmDepth][Shape::kSegments * 64];
    // Vector-memory operations a wave issues per chunk: codes and factors per row tile (K-quants: factor bytes and
    // multipliers), Q4_K input sums per token tile and block, the LDS copies.
    constexpr int kOps = (E == kEncodingQ8_0 ? 2 : 3) * RT + (E == kEncodingQ4K ? 2 * NT : 0) + Shape::kCopies;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4;
    const int chunks = a.chunks;
    const int first_tile = (blockIdx.x * kGemmWaves + wave) * RT;

    // This wave's row tiles (a tile past the last reads the last; its outputs are not written).
    GemmTile tiles[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        ProjectionSegment seg;
        const int global_tile = first_tile + r;
        const int local = locate_tile(a, min(global_tile, a.total_tiles - 1), seg);
        const size_t first_chunk = static_cast<size_t>(local) * chunks;
        if constexpr (E == kEncodingQ8_0) {
            tiles[r].codes = seg.codes + first_chunk * kQ8TileBytes;
            tiles[r].scales = static_cast<const uint16_t*>(seg.scales) + first_chunk * kQ8TileScales;
        } else {
            tiles[r].codes = seg.codes + first_chunk * (E == kEncodingQ4K ? kQ4KTileBytes : kQ6KTileBytes);
            tiles[r].scales = static_cast<const uint8_t*>(seg.scales) + (first_chunk >> 2) * kKSuperFactorBytes;
        }
        tiles[r].rows_left = global_tile < a.total_tiles ? seg.rows - local * kQ8TileRows : 0;
        tiles[r].out_column = seg.out_column + local * kQ8TileRows;
        tiles[r].bias = seg.bias != nullptr ? seg.bias + local * kQ8TileRows : nullptr;
    }
    // Token tiles of this workgroup; tiles past the last token read tile 0 (their outputs are never written).
    int source_tile[NT];
#pragma unroll
    for (int c = 0; c < NT; ++c) {
        const int tile_index = blockIdx.y * NT + c;
        source_tile[c] = 16 * tile_index < a.tokens ? tile_index : 0;
    }
    // This wave's copies: segment s = wave + kGemmWaves * j is token tile s / 6, piece s % 6 (part, block).
    const uint8_t* copy_source[Shape::kCopies];
#pragma unroll
    for (int j = 0; j < Shape::kCopies; ++j) {
        const int segment = wave + kGemmWaves * j;
        copy_source[j] = reinterpret_cast<const uint8_t*>(a.parts) +
                         ((static_cast<size_t>(source_tile[segment / (kParts * 2)]) * chunks * kParts * 2 +
                           segment % (kParts * 2)) * 64 + lane) * 16;
    }
    constexpr size_t kCopyStride = kParts * 2 * 64 * 16;  // bytes per chunk of one token tile
    const float* sums[NT];
#pragma unroll
    for (int c = 0; c < NT; ++c) {
        sums[c] = a.sums != nullptr ? a.sums + static_cast<size_t>(16 * source_tile[c] + (lane & 15)) * (a.padded_columns / 8)
                                    : nullptr;
    }

    auto copy_chunk = [&](int chunk) __attribute__((always_inline)) {
        // Past the end: a harmless re-read of the last chunk.
        gemm_copy_chunk<NT>(copy_source, min(chunk, chunks - 1) * kCopyStride, ring[chunk % kGemmDepth], wave);
    };
    auto load = [&](int chunk, GemmLoads<E, NT, RT>& set) __attribute__((always_inline)) {
        const int source_chunk = min(chunk, chunks - 1);
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            set.w[r] = load_chunk<E>(tiles[r].codes, tiles[r].scales, source_chunk, lane, g);
        }
        if constexpr (E == kEncodingQ4K) {
#pragma unroll
            for (int c = 0; c < NT; ++c) {
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    set.sums[c][b] = reinterpret_cast<const floatx4*>(sums[c] + source_chunk * 8 + 4 * b)[0];
                }
            }
        }
    };

    floatx4 acc[RT][NT];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
#pragma unroll
        for (int c = 0; c < NT; ++c) {
            acc[r][c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }

    // Prologue: loads and copies of chunks 0 and 1, in the steady state's order.
    GemmLoads<E, NT, RT> set0;
    GemmLoads<E, NT, RT> set1;
    GemmLoads<E, NT, RT> set2;
    load(0, set0);
    __builtin_amdgcn_sched_barrier(0);
    copy_chunk(0);
    __builtin_amdgcn_sched_barrier(0);
    load(1, set1);
    __builtin_amdgcn_sched_barrier(0);
    copy_chunk(1);
    __builtin_amdgcn_sched_barrier(0);

    // The chunk's products from its LDS stage and the loads in `current`.
    auto multiply = [&](int chunk, const GemmLoads<E, NT, RT>& current) __attribute__((always_inline)) {
        const bf16x8* stage = ring[chunk % kGemmDepth];
        InputFragments<NT> input;
#pragma unroll
        for (int c = 0; c < NT; ++c) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
#pragma unroll
                for (int p = 0; p < kParts; ++p) {
                    input.x[c][b][p] = stage[(c * kParts * 2 + p * 2 + b) * 64 + lane];
                }
            }
        }
        float xsum[NT][2] = {};
        if constexpr (E == kEncodingQ4K) {
#pragma unroll
            for (int c = 0; c < NT; ++c) {
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const floatx4 four = current.sums[c][b];
                    xsum[c][b] = ((four[0] + four[1]) + four[2]) + four[3];
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            multiply_chunk<E, NT>(current.w[r], input, xsum, acc[r]);
        }
    };
    // One chunk of the loop: wait until only the next chunk's operations may be in flight, issue chunk + 2's,
    // multiply.
    auto step = [&](int chunk, const GemmLoads<E, NT, RT>& current, GemmLoads<E, NT, RT>& later) __attribute__((always_inline)) {
        barrier_after_copies<kOps>();
        load(chunk + 2, later);
        __builtin_amdgcn_sched_barrier(0);
        copy_chunk(chunk + 2);
        __builtin_amdgcn_sched_barrier(0);
        multiply(chunk, current);
    };
    // Whole rounds of three chunks (no conditional step inside the loop, so the compiler's waits stay partial),
    // then the one or two chunks left.
    // The tail issues nothing (its chunk + 2 is past the end; the compiler drops loads whose values are never used,
    // so kOps would no longer count the newest operations): its first chunk waits for all but the next chunk's
    // kOps operations, issued by the last full step or the prologue, its second chunk for everything. That count
    // holds only while the step issues set `later`'s loads beside its copies (kOps includes them); the first-call
    // tests on fresh weights cover tails of zero, one and two chunks for Q8_0 and K-quant matrices.
    int chunk = 0;
    for (; chunk + 3 <= chunks; chunk += 3) {
        step(chunk, set0, set2);
        step(chunk + 1, set1, set0);
        step(chunk + 2, set2, set1);
    }
    if (chunk < chunks) {
        barrier_after_copies<kOps>();
        multiply(chunk, set0);
        if (chunk + 1 < chunks) {
            barrier_after_copies<0>();
            multiply(chunk + 1, set1);
        }
    }
    wait_vector_memory<0>();  // the copies issued past the last chunk have landed before the wave ends

    // Lane (g, t) of MFMA tile (r, c) holds rows 4 g .. + 3 of token 16 c + t.
    const int t = lane & 15;
#pragma unroll
    for (int r = 0; r < RT; ++r) {
#pragma unroll
        for (int c = 0; c < NT; ++c) {
            const int token = blockIdx.y * Shape::kTokens + 16 * c + t;
            if (token >= a.tokens) {
                continue;
            }
            float* destination = a.output + static_cast<size_t>(token) * a.out_stride + tiles[r].out_column;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 4 * g + i;
                if (row < tiles[r].rows_left) {
                    const float total = acc[r][c][i] + (tiles[r].bias != nullptr ? tiles[r].bias[row] : 0.0f);
                    destination[row] = a.accumulate != 0 ? destination[row] + total : total;
                }
            }
        }
    }
}

// ---- Decode products on FP16 matrix cores: two input parts, scaled per token ---------------------------------

typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef _Float16 halfx2 __attribute__((ext_vector_type(2)));
constexpr int kDecodeParts = 2;

// Four int8 codes (a little-endian word) as exact FP16 values, into elements at .. at + 3 of `out`: each biased
// byte b = code + 128 becomes the FP16 bits 0x64bb = 1024 + b (one v_perm per pair), and one packed FP16
// subtraction of 1152 per pair leaves the code (an integer of at most 8 bits: exact).
__device__ inline void codes_to_half(uint32_t word, uint32_t bias_xor, _Float16 subtract, halfx8& out, int at) {
    const uint32_t biased = word ^ bias_xor;
    const uint32_t low = __builtin_amdgcn_perm(0x64646464u, biased, 0x04010400u);
    const uint32_t high = __builtin_amdgcn_perm(0x64646464u, biased, 0x04030402u);
    const halfx2 first = __builtin_bit_cast(halfx2, low) - halfx2{subtract, subtract};
    const halfx2 second = __builtin_bit_cast(halfx2, high) - halfx2{subtract, subtract};
    out[at] = first[0];
    out[at + 1] = first[1];
    out[at + 2] = second[0];
    out[at + 3] = second[1];
}

// The chunk's two blocks of A fragments in FP16: Q8_0 int8 codes, Q6_K six-bit codes biased by 32 (q6k_word), Q4_K
// nibbles (block 0 low, block 1 high).
template <uint32_t E>
__device__ inline void weight_fragments_f16(uintx4 codes, halfx8 (&weight)[2]) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            if constexpr (E == kEncodingQ4K) {
                codes_to_half((codes[w] >> (4 * b)) & 0x0F0F0F0Fu, 0u, static_cast<_Float16>(1024.0f), weight[b],
                              4 * w);
            } else if constexpr (E == kEncodingQ6K) {
                codes_to_half(q6k_word(codes, b, w), 0u, static_cast<_Float16>(1056.0f), weight[b], 4 * w);
            } else {
                codes_to_half(codes[2 * b + w], 0x80808080u, static_cast<_Float16>(1152.0f), weight[b], 4 * w);
            }
        }
    }
}

// One chunk of the decode kernel: as multiply_chunk, with the input as two FP16 parts (x' = hi + lo to 2^-22 of
// |x'|, x' the token's input scaled by a power of two) and FP16 codes. Each block's two part products go to a fresh
// accumulator; the block sums are then scaled into the running sums in the reference's block order.
template <uint32_t E, bool kWide = false>
__device__ inline void multiply_chunk_f16(const ChunkWeights<E>& w, const halfx8 (&input)[2][kDecodeParts],
                                          const float (&xsum)[2], floatx4& acc) {
    halfx8 weight[2];
    weight_fragments_f16<E>(w.codes, weight);
    if constexpr (E == kEncodingQ8_0) {
        uint32_t words[4];
        if constexpr (kWide) {
            words[0] = w.scales[0];
            words[1] = w.scales[1];
            words[2] = w.scales[2];
            words[3] = w.scales[3];
        } else {
            const int bits = static_cast<int>(w.factor);
            words[0] = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, bits, 0x150, 0xF, 0xF, false));
            words[1] = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, bits, 0x151, 0xF, 0xF, false));
            words[2] = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, bits, 0x152, 0xF, 0xF, false));
            words[3] = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, bits, 0x153, 0xF, 0xF, false));
        }
        floatx4 block[2];
#pragma unroll
        for (int p = kDecodeParts - 1; p >= 0; --p) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                block[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    weight[b], input[b][p], p == kDecodeParts - 1 ? floatx4{0.0f, 0.0f, 0.0f, 0.0f} : block[b], 0, 0,
                    0);
            }
        }
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const halfx2 pair = __builtin_bit_cast(halfx2, words[2 * b + h]);
                acc[2 * h] = __builtin_fmaf(block[b][2 * h], static_cast<float>(pair[0]), acc[2 * h]);
                acc[2 * h + 1] = __builtin_fmaf(block[b][2 * h + 1], static_cast<float>(pair[1]), acc[2 * h + 1]);
            }
        }
    } else if constexpr (E == kEncodingQ4K) {
        floatx4 block[2];
#pragma unroll
        for (int p = kDecodeParts - 1; p >= 0; --p) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                block[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    weight[b], input[b][p], p == kDecodeParts - 1 ? floatx4{0.0f, 0.0f, 0.0f, 0.0f} : block[b], 0, 0,
                    0);
            }
        }
        float factors[16];
        row_broadcast_factors(kquant_factor_bits(w), factors);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc[i] = __builtin_fmaf(block[b][i], factors[b * 4 + i], acc[i]);
                acc[i] = __builtin_fmaf(-factors[8 + b * 4 + i], xsum[b], acc[i]);
            }
        }
    } else {
        const bool first_half = (threadIdx.x & 63) < 32;  // lane groups 0 and 1: columns 0-15 of the block
        const halfx8 zero = halfx8{};
        halfx8 halves[2][2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            halves[0][b] = first_half ? weight[b] : zero;
            halves[1][b] = first_half ? zero : weight[b];
        }
        floatx4 block[2][2];
#pragma unroll
        for (int p = kDecodeParts - 1; p >= 0; --p) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    block[h][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        halves[h][b], input[b][p],
                        p == kDecodeParts - 1 ? floatx4{0.0f, 0.0f, 0.0f, 0.0f} : block[h][b], 0, 0, 0);
                }
            }
        }
        float factors[16];
        row_broadcast_factors(kquant_factor_bits(w), factors);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    acc[i] = __builtin_fmaf(block[h][b][i], factors[h * 8 + b * 4 + i], acc[i]);
                }
            }
        }
    }
}

// One row tile's codes and factors for a decode slice (a launch over both K-quant types keeps Q6_K-shaped registers
// and notes whether the tile is Q4_K; a Q4_K tile fills only the first half of each code vector).
template <uint32_t E>
struct DecodeTile {
    static constexpr uint32_t kStored = E == kEncodingMixedK ? kEncodingQ6K : E;
    ChunkWeights<kStored> w[kDecodeSliceChunks];
    bool q4k;
};

// Issues the loads of `tile`'s chunks k0 .. k0 + count - 1 (chunks past count re-read the last).
template <uint32_t E>
__device__ inline void load_decode_tile(const ProjectionArgs& a, int tile, int k0, int count, int lane, int g,
                                        DecodeTile<E>& out) {
    ProjectionSegment seg;
    const int local = locate_tile(a, tile, seg);
    const size_t first_chunk = static_cast<size_t>(local) * a.chunks + k0;
    out.q4k = E == kEncodingQ4K || (E == kEncodingMixedK && seg.encoding == kEncodingQ4K);
    if constexpr (E == kEncodingMixedK) {
        if (out.q4k) {
#pragma unroll
            for (int i = 0; i < kDecodeSliceChunks; ++i) {
                const ChunkWeights<kEncodingQ4K> w =
                    load_chunk<kEncodingQ4K>(seg.codes, seg.scales, first_chunk + min(i, count - 1), lane, g);
                out.w[i].codes = w.codes;
                out.w[i].factor = w.factor;
                out.w[i].multiplier = w.multiplier;
            }
        } else {
#pragma unroll
            for (int i = 0; i < kDecodeSliceChunks; ++i) {
                out.w[i] = load_chunk<kEncodingQ6K>(seg.codes, seg.scales, first_chunk + min(i, count - 1), lane, g);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < kDecodeSliceChunks; ++i) {
            out.w[i] = load_chunk<E, true>(seg.codes, seg.scales, first_chunk + min(i, count - 1), lane, g);
        }
    }
}

// Multiplies a loaded tile against the staged slice: lane (g, t) returns rows 4 g .. + 3 of token t, in the scaled
// input's units.
template <uint32_t E>
__device__ inline floatx4 multiply_decode_tile(const DecodeTile<E>& tile, int count, const halfx8* staged,
                                               const float* group_sums, int lane) {
    constexpr bool kSums = E == kEncodingQ4K || E == kEncodingMixedK;
    floatx4 acc = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < kDecodeSliceChunks; ++i) {
        if (i < count) {
            halfx8 input[2][kDecodeParts];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
#pragma unroll
                for (int p = 0; p < kDecodeParts; ++p) {
                    input[b][p] = staged[((i * kDecodeParts + p) * 2 + b) * 64 + lane];
                }
            }
            float xsum[2] = {};
            if constexpr (kSums) {
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const float* four = group_sums + (i * 8 + 4 * b) * 16 + (lane & 15);
                    xsum[b] = ((four[0] + four[16]) + four[32]) + four[48];
                }
            }
            if constexpr (E == kEncodingMixedK) {
                if (tile.q4k) {
                    ChunkWeights<kEncodingQ4K> w;
                    w.codes = tile.w[i].codes;
                    w.factor = tile.w[i].factor;
                    w.multiplier = tile.w[i].multiplier;
                    multiply_chunk_f16<kEncodingQ4K>(w, input, xsum, acc);
                } else {
                    multiply_chunk_f16<kEncodingQ6K>(tile.w[i], input, xsum, acc);
                }
            } else {
                multiply_chunk_f16<E, true>(tile.w[i], input, xsum, acc);
            }
        }
    }
    return acc;
}

// Writes a tile's 16 x 16 slice sums: partial[slice][t][16 * tile + 4 g + i], scaled back by the token's power of two
// (exact barring underflow; every lane's token t = lane % 16 is the token whose scale `shift` this lane holds).
__device__ inline void store_tile_sums(const ProjectionArgs& a, floatx4 acc, int tile_index, int slice, int shift,
                                       int lane, int g) {
    const int t = lane & 15;
    float* destination = a.partials + (static_cast<size_t>(slice) * 16 + t) * a.partial_stride +
                         static_cast<size_t>(tile_index) * kQ8TileRows + 4 * g;
    floatx4 value;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        value[i] = __builtin_ldexpf(acc[i], -shift);
    }
    *reinterpret_cast<floatx4*>(destination) = value;
}

// Input loads of a decode slice: item = threadIdx.x + 512 j is (token item % 16, 8-column group item / 16 of the
// slice); every item of a thread has token threadIdx.x % 16. Tokens past the last and columns past the matrix read
// nothing (zeros). With NORM the thread also loads the norm weights of its columns and its token's partial sums of
// squares.
constexpr int kDecodeItems = kDecodeSliceChunks * 128 / (kDecodeWaves * 64);  // split items per thread

template <bool NORM>
struct SliceInput {
    floatx4 raw[kDecodeItems][2];
    floatx4 weight[NORM ? kDecodeItems : 1][2];
    floatx4 squares[NORM ? kNormSquaresStride / 4 : 1];
};

template <bool NORM>
__device__ inline void load_slice_input(const ProjectionArgs& a, int k0, int count, SliceInput<NORM>& in) {
#pragma unroll
    for (int j = 0; j < kDecodeItems; ++j) {
        const int item = threadIdx.x + j * kDecodeWaves * 64;
        const int t = item & 15;
        const int group = item >> 4;
        const int column = (k0 + (group >> 3)) * kQ8ChunkColumns + 8 * (group & 7);
        const bool inside = (group >> 3) < count && t < a.tokens && column < a.columns;
        const floatx4* source = reinterpret_cast<const floatx4*>(
            a.input + static_cast<size_t>(inside ? t : 0) * a.in_stride + (inside ? column : 0));
        in.raw[j][0] = source[0];
        in.raw[j][1] = source[1];
        if (!inside) {
            in.raw[j][0] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            in.raw[j][1] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        if constexpr (NORM) {
            const floatx4* weight = reinterpret_cast<const floatx4*>(a.norm.weight + (inside ? column : 0));
            in.weight[j][0] = weight[0];
            in.weight[j][1] = weight[1];
        }
    }
    if constexpr (NORM) {
        const int t = min(static_cast<int>(threadIdx.x & 15), a.tokens - 1);
        const floatx4* squares = reinterpret_cast<const floatx4*>(a.norm.squares + t * kNormSquaresStride);
#pragma unroll
        for (int i = 0; i < kNormSquaresStride / 4; ++i) {
            in.squares[i] = 4 * i < a.norm.parts ? squares[i] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
}

// y = x * (1 / sqrt(total / columns + epsilon)) * w (normalize_values' arithmetic, decoder.hip), total the in-order
// sum of the token's partial sums of squares.
template <bool NORM>
__device__ inline void normalize_slice_input(const ProjectionArgs& a, SliceInput<NORM>& in) {
    if constexpr (NORM) {
#pragma clang fp contract(off)
        float total = in.squares[0][0];
#pragma unroll
        for (int i = 1; i < kNormSquaresStride; ++i) {
            if (i < a.norm.parts) {
                total += in.squares[i / 4][i % 4];
            }
        }
        const float scale = 1.0f / sqrtf(total / static_cast<float>(a.norm.columns) + a.norm.epsilon);
#pragma unroll
        for (int j = 0; j < kDecodeItems; ++j) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    in.raw[j][h][e] = in.raw[j][h][e] * scale * in.weight[j][h][e];
                }
            }
        }
    }
}

// LDS of a decode workgroup: the staged input parts, the waves' per-token maxima and (Q4_K) the input sums.
template <uint32_t E>
struct DecodeShared {
    static constexpr bool kSums = E == kEncodingQ4K || E == kEncodingMixedK;
    halfx8 staged[kDecodeSliceChunks * kDecodeParts * 2 * 64];
    float wave_maxima[kDecodeWaves][16];
    float group_sums[kSums ? kDecodeSliceChunks * 8 * 16 : 1];  // per chunk, 8-column group and token
};

// Stages the slice (the loaded `raw` inputs) and returns the token's power-of-two shift:
//   1. each token's largest |x| over the slice: this thread's items, the wave's four lanes of the token (lanes t,
//      t + 16, t + 32, t + 48), then the eight waves through LDS; the shift puts it in [2^14, 2^15) (exact; FP16 then
//      keeps every part of the scaled input in its normal range down to 2^-18 of that largest value);
//   2. each input is split into two FP16 parts, hi = fp16(x') and lo = fp16(x' - hi), in B-fragment order in LDS
//      (Q4_K: and the scaled sums of 8 inputs).
template <uint32_t E>
__device__ inline int stage_slice(const floatx4 (&raw)[kDecodeItems][2], DecodeShared<E>& shared, int wave,
                                  int lane) {
    float largest = 0.0f;
#pragma unroll
    for (int j = 0; j < kDecodeItems; ++j) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            largest = fmaxf(largest, fabsf(raw[j][i / 4][i % 4]));
        }
    }
    largest = fmaxf(largest, __shfl_xor(largest, 16));
    largest = fmaxf(largest, __shfl_xor(largest, 32));
    if (lane < 16) {
        shared.wave_maxima[wave][lane] = largest;
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) {
        largest = fmaxf(largest, shared.wave_maxima[w][lane & 15]);
    }
    int exponent = 0;
    (void)frexpf(largest, &exponent);  // largest = m 2^exponent, m in [0.5, 1) (0 for a zero slice)
    const int shift = 15 - exponent;
#pragma unroll
    for (int j = 0; j < kDecodeItems; ++j) {
        const int item = threadIdx.x + j * kDecodeWaves * 64;
        const int t = item & 15;
        const int group = item >> 4;
        const int chunk = group >> 3;
        const int within = 8 * (group & 7);  // column within the chunk
        const int block = within / kQ8BlockElements;
        const int lane_group = (within % kQ8BlockElements) / 8;
        halfx8 parts[kDecodeParts];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
#pragma clang fp contract(off)
            const float x = __builtin_ldexpf(raw[j][i / 4][i % 4], shift);
            const _Float16 hi = static_cast<_Float16>(x);
            parts[0][i] = hi;
            parts[1][i] = static_cast<_Float16>(x - static_cast<float>(hi));
        }
#pragma unroll
        for (int p = 0; p < kDecodeParts; ++p) {
            shared.staged[((chunk * kDecodeParts + p) * 2 + block) * 64 + 16 * lane_group + t] = parts[p];
        }
        if constexpr (DecodeShared<E>::kSums) {
            float sum = raw[j][0][0];
#pragma unroll
            for (int i = 1; i < 8; ++i) {
                sum += raw[j][i / 4][i % 4];
            }
            // Scaled like the parts, so the offset term matches the scaled products (exact: a power of two).
            shared.group_sums[(chunk * 8 + (group & 7)) * 16 + t] = __builtin_ldexpf(sum, shift);
        }
    }
    __syncthreads();
    return shift;
}

// Decode kernel (at most 16 tokens). Each workgroup covers eight 16-row tiles (one per wave) over one slice of at
// most eight 64-column chunks:
//   1. every thread loads its inputs (token, 8 columns), then its wave's codes and factors for the slice (the wave's
//      only other vector-memory loads, all in flight while the input is split);
//   2. the workgroup finds each token's largest |x| over the slice and scales the token's inputs by the power of two
//      that puts it in [2^14, 2^15) (exact; FP16 keeps every part of the scaled input in its normal range down to
//      2^-18 of that largest value);
//   3. each input is split into two FP16 parts, hi = fp16(x') and lo = fp16(x' - hi), in B-fragment order in LDS;
//   4. every wave multiplies its tile's chunks against the staged parts on v_mfma_f32_16x16x32_f16 (FP16 codes and
//      FP16 parts: products exact in FP32), and writes its 16 x 16 slice sums, scaled back by the power of two, to
//      the partial rows that reduce_kernel (or the consuming norm / SwiGLU kernel) adds in slice order.
// The products differ from FP32 x * FP32 code by the lo part's rounding, at most 2^-22 of |x| (FP32 products round
// at 2^-24): well inside the accumulation error of any FP32 order of the sums. Against the three-part bf16 split
// this takes two MFMAs per block instead of three, 1.25 VALU instructions per code instead of 1.5 and 32 KiB of
// LDS instead of 48 (decoder step, same box: Q8_0 5.70 -> 5.69 ms, Q4_K_M 6.11 -> 5.88).
// With NORM the input is a raw row that the kernel RMS-normalizes while staging (NormInput), in place of the norm
// kernel's launch and its normalized copy of the rows.
// A variant streaming 2-8 tiles per wave through two register sets (the next tile's loads in flight while the
// current one is multiplied; loads past a wave's last tile through empty-range buffer resources so the waits stay
// partial; sums stored after the last tile) measured slower: gate + up 38.3 against 34.2 us, logits 135.5 against
// 127.5. Its 182 VGPRs allow one workgroup per CU where the one-shot kernel runs two to four. With the multiplies
// skipped the one-shot kernel's loads alone take 26.2 us on gate + up (5.5 TB/s) and 89 us on the logits: the
// multiplies cost a quarter of the launch that they do not overlap. Compact Q8_0 scales (one register per chunk,
// broadcast at use: 73 VGPRs instead of 95) measured the same.
template <uint32_t E, bool NORM>
__global__ __launch_bounds__(kDecodeWaves * 64) void project_decode_kernel(ProjectionArgs a) {
    __shared__ DecodeShared<E> shared;
    const int slice = blockIdx.y;
    const int k0 = slice * a.chunks / a.slices;
    const int count = (slice + 1) * a.chunks / a.slices - k0;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4;
    const int tile = blockIdx.x * kDecodeWaves + wave;  // this wave's row tile (past the last: loads the last)

    SliceInput<NORM> input;
    load_slice_input<NORM>(a, k0, count, input);
    // This wave's codes and factors for the slice, issued after the input loads: loads complete in issue order, so
    // the staging waits for the input only, while the weight stream stays in flight.
    DecodeTile<E> weights;
    load_decode_tile<E>(a, min(tile, a.total_tiles - 1), k0, count, lane, g, weights);
    __builtin_amdgcn_sched_barrier(0);
    normalize_slice_input<NORM>(a, input);
    const int shift = stage_slice<E>(input.raw, shared, wave, lane);
    if (tile < a.total_tiles) {
        store_tile_sums(a, multiply_decode_tile<E>(weights, count, shared.staged, shared.group_sums, lane), tile,
                        slice, shift, lane, g);
    }
}

// output[t][out_column + row] = (accumulate ? output : 0) + (sum over slices in order) + bias, one thread per
// (token, row of all segments).
__global__ __launch_bounds__(256) void reduce_kernel(ProjectionArgs a) {
    const int index = blockIdx.x * 256 + threadIdx.x;
    const int rows = a.total_tiles * kQ8TileRows;
    if (index >= a.tokens * rows) {
        return;
    }
    const int t = index / rows;
    const int global_row = index % rows;
    ProjectionSegment seg;
    const int tile = locate_tile(a, global_row / kQ8TileRows, seg);
    const int row = tile * kQ8TileRows + global_row % kQ8TileRows;
    if (row >= seg.rows) {
        return;
    }
    const float* partial = a.partials + static_cast<size_t>(t) * a.partial_stride + global_row;
    const size_t stride = static_cast<size_t>(16) * a.partial_stride;
    // Slices summed in order; eight loads in flight at a time.
    float sum = partial[0];
    int slice = 1;
    for (; slice + 8 <= a.slices; slice += 8) {
        float values[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            values[i] = partial[(slice + i) * stride];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            sum += values[i];
        }
    }
    for (; slice < a.slices; ++slice) {
        sum += partial[slice * stride];
    }
    const float total = sum + (seg.bias != nullptr ? seg.bias[row] : 0.0f);
    float* destination = a.output + static_cast<size_t>(t) * a.out_stride + seg.out_column + row;
    *destination = a.accumulate != 0 ? *destination + total : total;
}

// The partial sum of squares of a workgroup's 256 values (one per thread, zeros past the row): each wave's 64 in a
// fixed butterfly, then the four waves in order.
__device__ inline float block_squares(float x) {
    __shared__ float waves[4];
    float square = x * x;
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        square += __shfl_xor(square, offset);
    }
    if ((threadIdx.x & 63) == 0) {
        waves[threadIdx.x >> 6] = square;
    }
    __syncthreads();
    return ((waves[0] + waves[1]) + waves[2]) + waves[3];
}

// reduce_kernel for a one-segment decode projection whose output rows feed an RMS norm: workgroup (part, token)
// writes output[t][out_column + row] for 256 rows exactly as reduce_kernel does, then the part's sum of squares of
// the written values into squares[t * kNormSquaresStride + part].
__global__ __launch_bounds__(256) void reduce_squares_kernel(ProjectionArgs a) {
    const int t = blockIdx.y;
    const int row = blockIdx.x * kNormSquaresColumns + threadIdx.x;
    const ProjectionSegment& seg = a.segment[0];
    float value = 0.0f;
    if (row < seg.rows) {
        const float* partial = a.partials + static_cast<size_t>(t) * a.partial_stride + row;
        const size_t stride = static_cast<size_t>(16) * a.partial_stride;
        float sum = partial[0];
        int slice = 1;
        for (; slice + 8 <= a.slices; slice += 8) {
            float values[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                values[i] = partial[(slice + i) * stride];
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                sum += values[i];
            }
        }
        for (; slice < a.slices; ++slice) {
            sum += partial[slice * stride];
        }
        const float total = sum + (seg.bias != nullptr ? seg.bias[row] : 0.0f);
        float* destination = a.output + static_cast<size_t>(t) * a.out_stride + seg.out_column + row;
        value = a.accumulate != 0 ? *destination + total : total;
        *destination = value;
    }
    const float squares = block_squares(value);
    if (threadIdx.x == 0) {
        a.squares[t * kNormSquaresStride + blockIdx.x] = squares;
    }
}

// Partial sums of squares of rows another kernel wrote (the embedding), as reduce_squares_kernel writes them.
__global__ __launch_bounds__(256) void row_squares_kernel(const float* rows, int columns, float* squares) {
    const int t = blockIdx.y;
    const int column = blockIdx.x * kNormSquaresColumns + threadIdx.x;
    const float value = column < columns ? rows[static_cast<size_t>(t) * columns + column] : 0.0f;
    const float sum = block_squares(value);
    if (threadIdx.x == 0) {
        squares[t * kNormSquaresStride + blockIdx.x] = sum;
    }
}

template <uint32_t E>
void launch_decode(const Launch& launch, const ProjectionArgs& args, int tiles) {
    const dim3 grid((tiles + kDecodeWaves - 1) / kDecodeWaves, args.slices);
    if (args.norm.weight != nullptr) {
        SYNAPSE_KV_LAUNCH((project_decode_kernel<E, true>), grid, dim3(kDecodeWaves * 64), launch, args);
    } else {
        SYNAPSE_KV_LAUNCH((project_decode_kernel<E, false>), grid, dim3(kDecodeWaves * 64), launch, args);
    }
}

}  // namespace

hipError_t launch_row_squares(hipStream_t stream, const float* rows, int columns, int tokens, float* squares) {
    hipLaunchKernelGGL(row_squares_kernel, dim3((columns + kNormSquaresColumns - 1) / kNormSquaresColumns, tokens),
                       dim3(256), 0, stream, rows, columns, squares);
    return hipGetLastError();
}

int projection_decode_slices(int chunks) { return (chunks + kDecodeSliceChunks - 1) / kDecodeSliceChunks; }

namespace {

// Compute units of the current device (cached per device).
int compute_units() {
    static int cached[64] = {};
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) {
        (void)hipGetLastError();
        return 256;
    }
    if (cached[device] == 0) {
        int count = 0;
        if (hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || count <= 0) {
            (void)hipGetLastError();
            count = 256;
        }
        cached[device] = count;
    }
    return cached[device];
}

template <uint32_t E, int NT, int RT>
hipError_t launch_gemm(const Launch& launch, const ProjectionArgs& args, int tiles) {
    const dim3 grid((tiles + kGemmWaves * RT - 1) / (kGemmWaves * RT), (args.tokens + 16 * NT - 1) / (16 * NT));
    SYNAPSE_KV_LAUNCH((project_gemm_kernel<E, NT, RT>), grid, dim3(kGemmWaves * 64), launch, args);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_projection(const Launch& launch, const ProjectionArgs& args, int tiles, bool reduce, bool split) {
    const Launch plain{launch.stream, nullptr, nullptr};
    if (args.tokens <= 16) {
        switch (args.encoding) {
            case kEncodingQ4K:
                launch_decode<kEncodingQ4K>(launch, args, tiles);
                break;
            case kEncodingQ6K:
                launch_decode<kEncodingQ6K>(launch, args, tiles);
                break;
            case kEncodingMixedK:
                launch_decode<kEncodingMixedK>(launch, args, tiles);
                break;
            default:
                launch_decode<kEncodingQ8_0>(launch, args, tiles);
                break;
        }
        if (reduce && args.squares != nullptr) {
            const dim3 grid((args.segment[0].rows + kNormSquaresColumns - 1) / kNormSquaresColumns, args.tokens);
            SYNAPSE_KV_LAUNCH(reduce_squares_kernel, grid, dim3(256), plain, args);
        } else if (reduce) {
            const int outputs = args.tokens * tiles * kQ8TileRows;
            SYNAPSE_KV_LAUNCH(reduce_kernel, dim3((outputs + 255) / 256), dim3(256), plain, args);
        }
        return hipGetLastError();
    }
    if (split) {
        const int splits = (args.tokens + 15) / 16 * 16 * (args.padded_columns / 8);
        SYNAPSE_KV_LAUNCH(split_kernel, dim3((splits + 255) / 256), dim3(256), plain, args);
    }
    // The largest workgroup tile that still gives two workgroups per CU (small matrices and short prompt runs
    // take the smaller tiles).
    const int64_t wanted = 2ll * compute_units();
    auto blocks = [&](int nt, int rt) {
        return static_cast<int64_t>((tiles + kGemmWaves * rt - 1) / (kGemmWaves * rt)) * ((args.tokens + 16 * nt - 1) / (16 * nt));
    };
    switch (args.encoding) {
        case kEncodingQ4K:
            return blocks(2, 2) >= wanted ? launch_gemm<kEncodingQ4K, 2, 2>(launch, args, tiles)
                                          : launch_gemm<kEncodingQ4K, 2, 1>(launch, args, tiles);
        case kEncodingQ6K:
            return blocks(2, 2) >= wanted ? launch_gemm<kEncodingQ6K, 2, 2>(launch, args, tiles)
                                          : launch_gemm<kEncodingQ6K, 2, 1>(launch, args, tiles);
        default:
            if (blocks(4, 2) >= wanted) {
                return launch_gemm<kEncodingQ8_0, 4, 2>(launch, args, tiles);
            }
            return blocks(2, 2) >= wanted ? launch_gemm<kEncodingQ8_0, 2, 2>(launch, args, tiles)
                                          : launch_gemm<kEncodingQ8_0, 2, 1>(launch, args, tiles);
    }
    return hipGetLastError();
}

}  // namespace synapse_kv
