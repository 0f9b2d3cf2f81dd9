// Q8_0 projections (QKV before the attention path, o_proj after it) on bf16 MFMA with exact products.
//
// Semantics: synapse_q8_matvec_{1,2,4,8} and synapse_q8_gemm (native/synapse-gpu/src/Features/GpuKernels/cuda/
// kernels/matmul.cu:1-189, metal/shaders/matmul.metal:1-310): output[t][out_column + row] = (accumulate ? output : 0)
// + sum_blocks d * sum_k code[row][k] * input[t][k] + bias[row], rows of up to three matrices in one dispatch
// (locate_segment, common.metal:138-146). Weights stay Q8_0, activations FP32, sums FP32 (ADR-012).
//
// Exact products on the bf16 matrix cores: each FP32 input x is split into three bf16 parts with
// x = hi + mid + lo exactly (bf16 keeps FP32's exponent range; each part takes the next 8 significant bits, and the
// residuals x - hi and (x - hi) - mid are exact FP32 subtractions). A Q8_0 code is exact in bf16, and code * part
// is a product of at most 8 by 8 significant bits, exact in FP32. One Q8_0 block (32 columns) is one k-depth of
// v_mfma_f32_16x16x32_bf16: the block's three MFMAs (lo, mid, hi parts) sum its exact products in FP32 into a fresh
// accumulator, and the block's sum is then scaled and added as the reference does (sum = fma(block dot, d, sum),
// matmul.cu:101-104). Only the order of the FP32 additions differs from the reference's kernels.
//
// MI355X mapping, decode (at most 16 tokens): project_decode_kernel, one workgroup per eight 16-row tiles and one
// slice of at most eight 64-column chunks; the workgroup splits its input slice into LDS once and every wave streams
// its tile's codes and scales against it (see below); reduce_kernel adds the slices in order with bias and residual.
//
// K-quant matrices (Q4_K, Q6_K; kquant_layout.h) run the same kernels specialised on the encoding: a block's codes
// are exact in bf16 too (0..15, -32..31), and its FP32 factors are applied to the block's exact-product sum. Q4_K
// subtracts offset * sum(x) with the block's input sums (LDS in the decode kernel, written by split_kernel for prompt
// runs); Q6_K multiplies each 16-column half on its own (the other half's A fragments zeroed) and scales each.
//
// Prompt runs: split_kernel writes the three parts of the whole input once, in the B-operand fragment order of the
// MFMA, and project_kernel<4> runs one workgroup per (16-row tile, 64 tokens); its four waves split the columns
// into contiguous ranges of 64-column chunks and load, per chunk, the tile's 1 KiB of codes (one 16-byte load per
// lane, fragment order, see q8_layout.h), the scales of their accumulator rows and, per token tile, the six 16-byte
// B fragments (part x block), in batches ahead of the multiplies. The waves' 16 x 64 sums meet in LDS and are added
// in wave order, then the bias and the residual.

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

// Waves per workgroup of project_kernel; each takes an equal contiguous range of the column chunks.
template <int NT>
constexpr int projection_waves() {
    return 4;
}
constexpr int kParts = 3;

// x = hi + mid + lo, each part rounded to nearest bf16; the residuals are exact in FP32 and lo holds the last (at
// most 8) significant bits exactly.
__device__ inline void split3(float x, __bf16& hi, __bf16& mid, __bf16& lo) {
#pragma clang fp contract(off)
    hi = static_cast<__bf16>(x);
    const float first = x - static_cast<float>(hi);
    mid = static_cast<__bf16>(first);
    lo = static_cast<__bf16>(first - static_cast<float>(mid));
}

// Element offset of the parts of (token, column) in the split input: [token tile][chunk][part][block][lane][8],
// lane = 16 g + t holding columns 8 g .. 8 g + 7 of the block for token 16 tile + t, so every B-fragment load of
// the projection kernel is one contiguous 1 KiB wave load. The tile's three parts follow each other per chunk.
__device__ inline size_t part_offset(int chunks, int token, int column, int part) {
    const int tile = token / 16;
    const int t = token % 16;
    const int chunk = column / kQ8ChunkColumns;
    const int block = (column % kQ8ChunkColumns) / kQ8BlockElements;
    const int g = (column % kQ8BlockElements) / 8;
    return ((((static_cast<size_t>(tile) * chunks + chunk) * kParts + part) * 2 + block) * 64 + 16 * g + t) * 8 +
           column % 8;
}

// One thread per (token, 8 columns): the three bf16 parts of input[token][8 j .. 8 j + 7] (zeros past `columns`),
// stored in fragment order.
__global__ __launch_bounds__(256) void split_kernel(ProjectionArgs a) {
    const int groups = a.padded_columns / 8;
    const int index = blockIdx.x * 256 + threadIdx.x;
    if (index >= a.tokens * groups) {
        return;
    }
    const int token = index / groups;
    const int column = (index % groups) * 8;
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
    bf16x8 parts[kParts];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        __bf16 hi;
        __bf16 mid;
        __bf16 lo;
        split3(values[i], hi, mid, lo);
        parts[0][i] = hi;
        parts[1][i] = mid;
        parts[2][i] = lo;
    }
#pragma unroll
    for (int p = 0; p < kParts; ++p) {
        *reinterpret_cast<bf16x8*>(a.parts + part_offset(a.chunks, token, column, p)) = parts[p];
    }
    if (a.sums != nullptr) {
        float sum = values[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) {
            sum += values[i];
        }
        a.sums[static_cast<size_t>(token) * groups + column / 8] = sum;
    }
}

// Per token tile and block, the three parts of columns 8 g .. 8 g + 7 of token 16 c + r (B fragments).
template <int NT>
struct InputFragments {
    bf16x8 x[NT][2][kParts];
};

// Chunks per batch: a batch's loads are all issued (in the order the multiplies use them: each chunk's input
// fragments, then its codes and scales) before its first multiply. Vector memory loads complete in issue order, so
// a batch is one round trip; another wave on the SIMD overlaps its own round trip with this wave's multiplies.
template <int NT>
constexpr int projection_batch() {
    return 2;
}

// One chunk of one 16-row tile as a lane loads it: its codes (16 bytes of int8 codes; Q4_K: 8 bytes of nibbles in
// .xy) and the factors of its accumulator rows (Q8_0: eight FP16 scales, [block][row]). K-quant factors are loaded
// one FP32 value per lane: the chunk's 64 factors, [row group][field][block][row], so row group g's sixteen sit in
// DPP row g (lanes 16 g .. 16 g + 15), exactly the lanes whose accumulators need them; they are broadcast within the
// row at use (row_broadcast_factors) instead of every lane loading all sixteen.
template <uint32_t E>
struct ChunkWeights {
    uintx4 codes;
    uintx4 scales;    // Q8_0
    uint32_t factor;  // K-quants: FP32 bits of factor `lane` of the chunk
};

// Loads chunk `tile_chunk` (tile * chunks + chunk) of a matrix for lane `lane` of row group g.
template <uint32_t E>
__device__ inline ChunkWeights<E> load_chunk(const uint8_t* codes, const void* scales, size_t tile_chunk, int lane,
                                             int g) {
    ChunkWeights<E> w;
    if constexpr (E == kEncodingQ4K) {
        const uintx2 half = __builtin_nontemporal_load(reinterpret_cast<const uintx2*>(codes + tile_chunk * kQ4KTileBytes) + lane);
        w.codes = uintx4{half.x, half.y, 0u, 0u};
    } else {
        w.codes = __builtin_nontemporal_load(reinterpret_cast<const uintx4*>(codes + tile_chunk * kQ8TileBytes) + lane);
    }
    if constexpr (E == kEncodingQ8_0) {
        w.scales = reinterpret_cast<const uintx4*>(static_cast<const uint16_t*>(scales) + tile_chunk * kQ8TileScales)[g];
    } else {
        w.factor = reinterpret_cast<const uint32_t*>(scales)[tile_chunk * kKTileScales + lane];
    }
    return w;
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
template <uint32_t E, int NT>
__device__ inline void multiply_chunk(const ChunkWeights<E>& w, const InputFragments<NT>& input,
                                      const float (&xsum)[NT][2], floatx4 (&acc)[NT]) {
    bf16x8 weight[2];
    weight_fragments<E>(w.codes, weight);
    if constexpr (E == kEncodingQ8_0) {
        float d[2][4];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t pair = w.scales[2 * b + h];
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
        row_broadcast_factors(w.factor, factors);
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
        row_broadcast_factors(w.factor, factors);
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

template <uint32_t E, int NT>
__global__ __launch_bounds__(projection_waves<NT>() * 64) void project_kernel(ProjectionArgs a) {
    constexpr int kWaves = projection_waves<NT>();
    constexpr int kBatch = projection_batch<NT>();
    int tile = blockIdx.x;
    int s = 0;
    while (s + 1 < a.segments && tile >= a.segment[s + 1].first_tile) {
        ++s;
    }
    const ProjectionSegment seg = a.segment[s];
    tile -= seg.first_tile;
    // Uniform per wave, so the chunk loop and its range tests are scalar branches.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4;
    const int token0 = blockIdx.y * 16 * NT;
    const int chunks = a.chunks;
    const int begin = wave * chunks / kWaves;
    const int end = (wave + 1) * chunks / kWaves;
    const size_t tile_chunks = static_cast<size_t>(tile) * chunks;

    // The split input's token tiles of this workgroup (a tile past the last token re-reads tile 0; never written).
    const bf16x8* tiles[NT];
    const float* sums[NT];
#pragma unroll
    for (int c = 0; c < NT; ++c) {
        const int tile_index = blockIdx.y * NT + c;
        const int source = 16 * tile_index < a.tokens ? tile_index : 0;
        tiles[c] = reinterpret_cast<const bf16x8*>(a.parts) + static_cast<size_t>(source) * chunks * (kParts * 2 * 64) + lane;
        sums[c] = a.sums + static_cast<size_t>(16 * source + (lane & 15)) * (a.padded_columns / 8);
    }

    floatx4 acc[NT];
#pragma unroll
    for (int c = 0; c < NT; ++c) {
        acc[c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    // A batch's loads are issued whether or not each chunk is in range (past the range they re-read the last chunk):
    // a load under a branch would leave the wait count at the join unknown. The scheduling barrier keeps them ahead
    // of the multiplies.
    for (int first = begin; first < end; first += kBatch) {
        InputFragments<NT> input[kBatch];
        ChunkWeights<E> weights[kBatch];
        floatx4 raw_sums[kBatch][NT][2];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int chunk = min(first + i, end - 1);
#pragma unroll
            for (int c = 0; c < NT; ++c) {
                const bf16x8* fragments = tiles[c] + static_cast<size_t>(chunk) * (kParts * 2 * 64);
#pragma unroll
                for (int b = 0; b < 2; ++b) {
#pragma unroll
                    for (int p = 0; p < kParts; ++p) {
                        input[i].x[c][b][p] = fragments[(p * 2 + b) * 64];
                    }
                }
            }
            weights[i] = load_chunk<E>(seg.codes, seg.scales, tile_chunks + chunk, lane, g);
            if constexpr (E == kEncodingQ4K) {
#pragma unroll
                for (int c = 0; c < NT; ++c) {
#pragma unroll
                    for (int b = 0; b < 2; ++b) {
                        raw_sums[i][c][b] = reinterpret_cast<const floatx4*>(sums[c] + chunk * 8 + 4 * b)[0];
                    }
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            if (first + i < end) {
                float xsum[NT][2] = {};
                if constexpr (E == kEncodingQ4K) {
#pragma unroll
                    for (int c = 0; c < NT; ++c) {
#pragma unroll
                        for (int b = 0; b < 2; ++b) {
                            const floatx4 four = raw_sums[i][c][b];
                            xsum[c][b] = ((four[0] + four[1]) + four[2]) + four[3];
                        }
                    }
                }
                multiply_chunk<E, NT>(weights[i], input[i], xsum, acc);
            }
        }
    }

    // Lane (g, t) of token tile c holds rows 4 g .. + 3 of token 16 c + t; the waves' column ranges meet here and
    // are added in wave order by the first 256 threads.
    __shared__ floatx4 partial[kWaves][NT][64];
#pragma unroll
    for (int c = 0; c < NT; ++c) {
        partial[wave][c][lane] = acc[c];
    }
    __syncthreads();
    if (threadIdx.x >= 256) {
        return;
    }
    const int source_lane = threadIdx.x >> 2;
    const int v = threadIdx.x & 3;
    const int row = tile * kQ8TileRows + 4 * (source_lane >> 4) + v;
    if (row >= seg.rows) {
        return;
    }
    const float bias = seg.bias != nullptr ? seg.bias[row] : 0.0f;
#pragma unroll
    for (int c = 0; c < NT; ++c) {
        const int token = token0 + 16 * c + (source_lane & 15);
        if (token >= a.tokens) {
            continue;
        }
        float sum = partial[0][c][source_lane][v];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) {
            sum += partial[w][c][source_lane][v];
        }
        const float total = sum + bias;
        float* destination = a.output + static_cast<size_t>(token) * a.out_stride + seg.out_column + row;
        *destination = a.accumulate != 0 ? *destination + total : total;
    }
}

// ---- Decode (at most 16 tokens): row tiles share the split input through LDS ----------------------------------

// A workgroup of eight waves covers eight 16-row tiles (one per wave; tiles of different matrices may meet in one
// workgroup) over one slice of at most kDecodeSliceChunks column chunks. The workgroup first splits its slice of the
// input into the three bf16 parts, in B-fragment order, into LDS; then every wave streams its tile's codes and
// scales for the slice (its only vector-memory loads, all issued up front) and multiplies against the fragments in
// LDS. Each slice's 16 x 16 sums go to partial rows; reduce_kernel adds the slices in order with the bias and the
// residual. The input is read from L2 once per workgroup instead of once per tile. Eight waves share one 48 KiB
// staged input (four did before: 16 resident waves per CU instead of 12; 3 % faster decoder steps). Streaming two
// or four tiles per wave instead changed nothing measurable.
constexpr int kDecodeSliceChunks = 8;
constexpr int kDecodeWaves = 8;

// Row tiles per wave of the decode kernel (each wave would stream this many tiles' codes and factors against the
// same staged input).
template <uint32_t E>
constexpr int decode_tiles_per_wave() {
    return 1;
}
template <uint32_t E>
constexpr int decode_tiles() {
    return kDecodeWaves * decode_tiles_per_wave<E>();
}

__device__ inline int locate_tile(const ProjectionArgs& a, int tile, ProjectionSegment& seg) {
    int s = 0;
    while (s + 1 < a.segments && tile >= a.segment[s + 1].first_tile) {
        ++s;
    }
    seg = a.segment[s];
    return tile - seg.first_tile;
}

template <uint32_t E>
__global__ __launch_bounds__(kDecodeWaves * 64) void project_decode_kernel(ProjectionArgs a) {
    constexpr int kItems = kDecodeSliceChunks * 128 / (kDecodeWaves * 64);  // split items per thread
    constexpr int TW = decode_tiles_per_wave<E>();
    __shared__ bf16x8 staged[kDecodeSliceChunks * kParts * 2 * 64];
    // Q4_K: per chunk, 8-column group and token, the sum of the 8 inputs.
    constexpr bool kSums = E == kEncodingQ4K || E == kEncodingMixedK;
    __shared__ float group_sums[kSums ? kDecodeSliceChunks * 8 * 16 : 1];
    const int slice = blockIdx.y;
    const int k0 = slice * a.chunks / a.slices;
    const int k1 = (slice + 1) * a.chunks / a.slices;
    const int count = k1 - k0;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4;
    const int first_tile = (blockIdx.x * kDecodeWaves + wave) * TW;  // this wave's tiles: first_tile + k, k < TW

    // 1. This thread's input loads for the split: item = threadIdx.x + 256 j is (token item % 16, 8-column group
    //    item / 16 of the slice). Tokens past the last and columns past the matrix read nothing (zeros).
    floatx4 raw[kItems][2];
#pragma unroll
    for (int j = 0; j < kItems; ++j) {
        const int item = threadIdx.x + j * kDecodeWaves * 64;
        const int t = item & 15;
        const int group = item >> 4;
        const int column = (k0 + (group >> 3)) * kQ8ChunkColumns + 8 * (group & 7);
        const bool inside = (group >> 3) < count && t < a.tokens && column < a.columns;
        const floatx4* source = reinterpret_cast<const floatx4*>(
            a.input + static_cast<size_t>(inside ? t : 0) * a.in_stride + (inside ? column : 0));
        raw[j][0] = source[0];
        raw[j][1] = source[1];
        if (!inside) {
            raw[j][0] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            raw[j][1] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    // 2. This wave's codes and scales for the slice, issued after the input loads: loads complete in issue order,
    //    so the split below waits for the input only, while the weight stream stays in flight.
    //    A tile past the last loads the last tile again.
    //    A launch over both K-quant types (kEncodingMixedK) keeps Q6_K-shaped registers and branches per wave on its
    //    tile's segment (uniform per wave); a Q4_K tile fills only the first half of each code vector.
    constexpr uint32_t kStored = E == kEncodingMixedK ? kEncodingQ6K : E;
    ChunkWeights<kStored> batch[TW][kDecodeSliceChunks];
    bool q4k_tile[TW];
#pragma unroll
    for (int k = 0; k < TW; ++k) {
        ProjectionSegment seg;
        const int tile = locate_tile(a, min(first_tile + k, a.total_tiles - 1), seg);
        const size_t first_chunk = static_cast<size_t>(tile) * a.chunks + k0;
        q4k_tile[k] = E == kEncodingQ4K || (E == kEncodingMixedK && seg.encoding == kEncodingQ4K);
        if constexpr (E == kEncodingMixedK) {
            if (q4k_tile[k]) {
#pragma unroll
                for (int i = 0; i < kDecodeSliceChunks; ++i) {
                    const ChunkWeights<kEncodingQ4K> w =
                        load_chunk<kEncodingQ4K>(seg.codes, seg.scales, first_chunk + min(i, count - 1), lane, g);
                    batch[k][i].codes = w.codes;
                    batch[k][i].factor = w.factor;
                }
            } else {
#pragma unroll
                for (int i = 0; i < kDecodeSliceChunks; ++i) {
                    batch[k][i] = load_chunk<kEncodingQ6K>(seg.codes, seg.scales, first_chunk + min(i, count - 1),
                                                           lane, g);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < kDecodeSliceChunks; ++i) {
                batch[k][i] = load_chunk<E>(seg.codes, seg.scales, first_chunk + min(i, count - 1), lane, g);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // 3. Split into the three bf16 parts, in B-fragment order, into LDS.
#pragma unroll
    for (int j = 0; j < kItems; ++j) {
        const int item = threadIdx.x + j * kDecodeWaves * 64;
        const int t = item & 15;
        const int group = item >> 4;
        const int chunk = group >> 3;
        const int within = 8 * (group & 7);  // column within the chunk
        const int block = within / kQ8BlockElements;
        const int lane_group = (within % kQ8BlockElements) / 8;
        bf16x8 parts[kParts];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            __bf16 hi;
            __bf16 mid;
            __bf16 lo;
            split3(raw[j][i / 4][i % 4], hi, mid, lo);
            parts[0][i] = hi;
            parts[1][i] = mid;
            parts[2][i] = lo;
        }
#pragma unroll
        for (int p = 0; p < kParts; ++p) {
            staged[((chunk * kParts + p) * 2 + block) * 64 + 16 * lane_group + t] = parts[p];
        }
        if constexpr (kSums) {
            float sum = raw[j][0][0];
#pragma unroll
            for (int i = 1; i < 8; ++i) {
                sum += raw[j][i / 4][i % 4];
            }
            group_sums[(chunk * 8 + (group & 7)) * 16 + t] = sum;
        }
    }
    __syncthreads();

    // 4. Multiply the slice against the staged input.
    floatx4 acc[TW][1];
#pragma unroll
    for (int k = 0; k < TW; ++k) {
        acc[k][0] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int i = 0; i < kDecodeSliceChunks; ++i) {
        if (i < count) {
            InputFragments<1> input;
#pragma unroll
            for (int b = 0; b < 2; ++b) {
#pragma unroll
                for (int p = 0; p < kParts; ++p) {
                    input.x[0][b][p] = staged[((i * kParts + p) * 2 + b) * 64 + lane];
                }
            }
            float xsum[1][2] = {};
            if constexpr (kSums) {
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const float* four = group_sums + (i * 8 + 4 * b) * 16 + (lane & 15);
                    xsum[0][b] = ((four[0] + four[16]) + four[32]) + four[48];
                }
            }
#pragma unroll
            for (int k = 0; k < TW; ++k) {
                if constexpr (E == kEncodingMixedK) {
                    if (q4k_tile[k]) {
                        ChunkWeights<kEncodingQ4K> w;
                        w.codes = batch[k][i].codes;
                        w.factor = batch[k][i].factor;
                        multiply_chunk<kEncodingQ4K, 1>(w, input, xsum, acc[k]);
                    } else {
                        multiply_chunk<kEncodingQ6K, 1>(batch[k][i], input, xsum, acc[k]);
                    }
                } else {
                    multiply_chunk<E, 1>(batch[k][i], input, xsum, acc[k]);
                }
            }
        }
    }
    // Lane (g, t) holds rows 4 g .. + 3 of token t: partial[slice][t][16 * tile + 4 g + i].
    const int t = lane & 15;
#pragma unroll
    for (int k = 0; k < TW; ++k) {
        if (first_tile + k < a.total_tiles) {
            float* destination = a.partials + (static_cast<size_t>(slice) * 16 + t) * a.partial_stride +
                                 static_cast<size_t>(first_tile + k) * kQ8TileRows + 4 * g;
            *reinterpret_cast<floatx4*>(destination) = acc[k][0];
        }
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

}  // namespace

int projection_token_tiles(int tokens) { return tokens <= 16 ? 1 : 4; }

int projection_decode_slices(int chunks) { return (chunks + kDecodeSliceChunks - 1) / kDecodeSliceChunks; }

hipError_t launch_projection(const Launch& launch, const ProjectionArgs& args, int tiles, bool reduce) {
    const Launch plain{launch.stream, nullptr, nullptr};
    if (args.tokens <= 16) {
        const dim3 block(kDecodeWaves * 64);
        switch (args.encoding) {
            case kEncodingQ4K:
                SYNAPSE_KV_LAUNCH(project_decode_kernel<kEncodingQ4K>,
                                  dim3((tiles + decode_tiles<kEncodingQ4K>() - 1) / decode_tiles<kEncodingQ4K>(), args.slices),
                                  block, launch, args);
                break;
            case kEncodingQ6K:
                SYNAPSE_KV_LAUNCH(project_decode_kernel<kEncodingQ6K>,
                                  dim3((tiles + decode_tiles<kEncodingQ6K>() - 1) / decode_tiles<kEncodingQ6K>(), args.slices),
                                  block, launch, args);
                break;
            case kEncodingMixedK:
                SYNAPSE_KV_LAUNCH(project_decode_kernel<kEncodingMixedK>,
                                  dim3((tiles + decode_tiles<kEncodingMixedK>() - 1) / decode_tiles<kEncodingMixedK>(),
                                       args.slices),
                                  block, launch, args);
                break;
            default:
                SYNAPSE_KV_LAUNCH(project_decode_kernel<kEncodingQ8_0>,
                                  dim3((tiles + decode_tiles<kEncodingQ8_0>() - 1) / decode_tiles<kEncodingQ8_0>(), args.slices),
                                  block, launch, args);
                break;
        }
        if (reduce) {
            const int outputs = args.tokens * tiles * kQ8TileRows;
            SYNAPSE_KV_LAUNCH(reduce_kernel, dim3((outputs + 255) / 256), dim3(256), plain, args);
        }
        return hipGetLastError();
    }
    const int splits = args.tokens * (args.padded_columns / 8);
    SYNAPSE_KV_LAUNCH(split_kernel, dim3((splits + 255) / 256), dim3(256), plain, args);
    const int per_block = 16 * projection_token_tiles(args.tokens);
    const dim3 grid(tiles, (args.tokens + per_block - 1) / per_block);
    const dim3 block(projection_waves<4>() * 64);
    switch (args.encoding) {
        case kEncodingQ4K:
            SYNAPSE_KV_LAUNCH((project_kernel<kEncodingQ4K, 4>), grid, block, launch, args);
            break;
        case kEncodingQ6K:
            SYNAPSE_KV_LAUNCH((project_kernel<kEncodingQ6K, 4>), grid, block, launch, args);
            break;
        default:
            SYNAPSE_KV_LAUNCH((project_kernel<kEncodingQ8_0, 4>), grid, block, launch, args);
            break;
    }
    return hipGetLastError();
}

}  // namespace synapse_kv
