// Q8_0 projections (QKV before the attention path, o_proj after it) on FP32 MFMA.
//
// Semantics: synapse_q8_matvec_{1,2,4,8} and synapse_q8_gemm (native/synapse-gpu/src/Features/GpuKernels/cuda/
// kernels/matmul.cu:1-189, metal/shaders/matmul.metal:1-310): output[t][out_column + row] = (accumulate ? output : 0)
// + sum_k (d * code)[row][k] * input[t][k] + bias[row], rows of up to three matrices in one dispatch
// (locate_segment, common.metal:138-146). Weights stay Q8_0, activations stay FP32 and every product and sum is
// FP32 (ADR-012): the weight element d * code is exact in FP32 (an 11-bit by 8-bit product) and the MFMA multiplies
// and accumulates in FP32, so only the summation order differs from the reference's kernels.
//
// MI355X mapping: one workgroup of four waves per (16-row tile, 16 * NT tokens). The waves split the columns into
// four contiguous ranges of 64-column chunks; per chunk a wave loads its tile's 1 KiB of codes (one 16-byte load per
// lane, fragment order, see q8_layout.h), the 16 rows' scales and, per token tile, 16 consecutive input values per
// lane, then runs 16 v_mfma_f32_16x16x4_f32 per token tile (lane g of the MFMA's k dimension takes columns
// 16 g + j of the chunk in MFMA j, for both operands). The next chunk's loads are in flight while the current one
// computes. The four waves' 16 x 16 * NT sums meet in LDS and are added in wave order.
//
// The same kernel serves decode (NT = 1: up to 16 tokens, the weight stream dominates) and prompt runs (NT = 4:
// 64 tokens per workgroup, each weight tile reused from registers for four token tiles).

#include "kv_internal.h"
#include "q8_layout.h"

namespace synapse_kv {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t uintx4 __attribute__((ext_vector_type(4)));

constexpr int kProjectionWaves = 4;

template <int NT>
struct ChunkOperands {
    uintx4 codes;        // 16 codes of row r, columns 16 g .. + 15 of the chunk
    float scale;         // d of row r for the block holding those columns
    floatx4 x[NT][4];    // per token tile: input[token 16 c + r][16 g .. + 15 of the chunk]
};

template <int NT>
__device__ inline void load_chunk(const ProjectionArgs& a, const uintx4* codes, const uint16_t* scales,
                                  const float* const (&rows)[NT], const bool (&valid)[NT], int chunk, int g,
                                  ChunkOperands<NT>& operands) {
    operands.codes = __builtin_nontemporal_load(codes + static_cast<size_t>(chunk) * 64);
    operands.scale = static_cast<float>(__builtin_bit_cast(_Float16, scales[static_cast<size_t>(chunk) * kQ8TileScales]));
    const int column = chunk * kQ8ChunkColumns + 16 * g;
    const bool inside = column < a.columns;  // columns are a multiple of 32: a 16-column group is all in or all out
#pragma unroll
    for (int c = 0; c < NT; ++c) {
        const floatx4* source = reinterpret_cast<const floatx4*>(rows[c] + column);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            operands.x[c][q] = valid[c] && inside ? source[q] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
}

template <int NT>
__device__ inline void multiply_chunk(const ChunkOperands<NT>& operands, floatx4 (&acc)[NT]) {
    float weight[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int code = static_cast<int>(static_cast<int8_t>((operands.codes[q] >> (8 * b)) & 0xFF));
            weight[4 * q + b] = static_cast<float>(code) * operands.scale;  // exact: |code| <= 128, d is FP16
        }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
#pragma unroll
        for (int c = 0; c < NT; ++c) {
            acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(weight[j], operands.x[c][j / 4][j % 4], acc[c], 0, 0, 0);
        }
    }
}

template <int NT>
__global__ __launch_bounds__(kProjectionWaves * 64) void project_kernel(ProjectionArgs a) {
    int tile = blockIdx.x;
    int s = 0;
    while (s + 1 < a.segments && tile >= a.segment[s + 1].first_tile) {
        ++s;
    }
    const ProjectionSegment seg = a.segment[s];
    tile -= seg.first_tile;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4;
    const int r = lane & 15;
    const int token0 = blockIdx.y * 16 * NT;
    const int chunks = a.chunks;
    const int begin = wave * chunks / kProjectionWaves;
    const int end = (wave + 1) * chunks / kProjectionWaves;

    const uintx4* codes = reinterpret_cast<const uintx4*>(seg.codes + static_cast<size_t>(tile) * chunks * kQ8TileBytes) + lane;
    const uint16_t* scales = seg.scales + static_cast<size_t>(tile) * chunks * kQ8TileScales + (g >> 1) * kQ8TileRows + r;
    const float* rows[NT];
    bool valid[NT];
#pragma unroll
    for (int c = 0; c < NT; ++c) {
        const int token = token0 + 16 * c + r;
        valid[c] = token < a.tokens;
        rows[c] = a.input + static_cast<size_t>(valid[c] ? token : 0) * a.in_stride;
    }

    floatx4 acc[NT];
#pragma unroll
    for (int c = 0; c < NT; ++c) {
        acc[c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    if (begin < end) {
        // Two operand sets: the next chunk's loads are in flight while the current chunk multiplies.
        ChunkOperands<NT> even;
        ChunkOperands<NT> odd;
        load_chunk<NT>(a, codes, scales, rows, valid, begin, g, even);
        for (int chunk = begin; chunk < end; chunk += 2) {
            if (chunk + 1 < end) {
                load_chunk<NT>(a, codes, scales, rows, valid, chunk + 1, g, odd);
            }
            multiply_chunk<NT>(even, acc);
            if (chunk + 1 >= end) {
                break;
            }
            if (chunk + 2 < end) {
                load_chunk<NT>(a, codes, scales, rows, valid, chunk + 2, g, even);
            }
            multiply_chunk<NT>(odd, acc);
        }
    }

    // Lane (g, t) of token tile c holds rows 4 g .. + 3 of token 16 c + t; the waves' column ranges meet here.
    __shared__ floatx4 partial[kProjectionWaves][NT][64];
#pragma unroll
    for (int c = 0; c < NT; ++c) {
        partial[wave][c][lane] = acc[c];
    }
    __syncthreads();
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
        const float sum = ((partial[0][c][source_lane][v] + partial[1][c][source_lane][v]) + partial[2][c][source_lane][v]) +
                          partial[3][c][source_lane][v];
        const float total = sum + bias;
        float* destination = a.output + static_cast<size_t>(token) * a.out_stride + seg.out_column + row;
        *destination = a.accumulate != 0 ? *destination + total : total;
    }
}

}  // namespace

int projection_token_tiles(int tokens) { return tokens <= 16 ? 1 : 4; }

hipError_t launch_projection(const Launch& launch, const ProjectionArgs& args, int tiles) {
    const int per_block = 16 * projection_token_tiles(args.tokens);
    const dim3 grid(tiles, (args.tokens + per_block - 1) / per_block);
    const dim3 block(kProjectionWaves * 64);
    if (per_block == 16) {
        SYNAPSE_KV_LAUNCH(project_kernel<1>, grid, block, launch, args);
    } else {
        SYNAPSE_KV_LAUNCH(project_kernel<4>, grid, block, launch, args);
    }
    return hipGetLastError();
}

}  // namespace synapse_kv
