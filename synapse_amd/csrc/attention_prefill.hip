// Chunked-prefill (prompt-run) attention on FP16 MFMA.
//
// Semantics: synapse_attention for prompt runs (native/synapse-gpu/src/Features/GpuKernels/metal/shaders/
// attention.metal:254-313; dispatch step/attention.rs:62-104): consecutive tokens of one slot at consecutive
// positions attend causally, token j sees keys 0..position_j (mask `key <= row_position`, attention.metal:80-81),
// after the run's K/V were appended (step/layers.rs:95-96). Long runs split their keys across work items and
// merge with the decode merge kernel (same (max, sum) partial rows).
//
// MI355X mapping: one workgroup per (KV head, block of kPrefillTokens tokens, key split) with one wave per query
// head of the GQA group; the group's waves share every K/V block through a double-buffered LDS stage. Each wave
// holds its head's queries for the block as kPrefillTiles MFMA column tiles of 16 tokens and runs the decode
// kernel's 64-key step:
// S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_16x16x32_f16, every K/V fragment loaded once and used by all
// column tiles. Causal masking is a per-element compare against the column's position.

#include "kv_internal.h"

namespace synapse_kv {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr float kNegativeInfinity = -__builtin_inff();
// 16-byte chunks of a staged block each thread carries in registers (a group of at least 4 waves covers the
// 2,048 chunks of a head_dim 128 block).
constexpr int kStageLoads = 8;

__device__ inline float fast_exp2(float value) { return __builtin_amdgcn_exp2f(value); }

// Qwen2RopeTable.Apply (Qwen2CpuState.cs:85-106) for one pair, products and sums rounded separately.
__device__ inline void rotate_pair(float x, float y, float c, float s, float& first, float& second) {
#pragma clang fp contract(off)
    first = x * c - y * s;
    second = x * s + y * c;
}

template <int D>
__global__ __launch_bounds__(512) void prefill_f16_kernel(AttentionArgs a) {
    constexpr int NT = kPrefillTiles;
    const PrefillItem item = a.prefill[blockIdx.x];
    const Geometry& geo = a.geo;
    const int wave = threadIdx.x >> 6;  // query head within the group
    const int lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int head = item.kv_head * geo.group + wave;
    const SynapseKvBatchToken first = a.tokens[item.first_token];
    const int first_position = first.position;

    // B operands of S^T = K Q^T: tile c, lane (g, r) holds dims 32*ks + 8*g .. +7 of token 16*c + r; the RoPE
    // partner of dim i < D/2 is in the same lane at ks + D/64.
    half8 query[NT][D / 32];
#pragma unroll
    for (int c = 0; c < NT; ++c) {
        const int j = 16 * c + r;
        const bool valid = j < item.count;
        const int token = item.first_token + (valid ? j : 0);
        const float* q = a.qkv + static_cast<size_t>(token) * a.qkv_stride + static_cast<size_t>(head) * D;
        float values[D / 32][8];
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            const floatx4 lo = *reinterpret_cast<const floatx4*>(q + 32 * ks + 8 * g);
            const floatx4 hi = *reinterpret_cast<const floatx4*>(q + 32 * ks + 8 * g + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                values[ks][e] = lo[e];
                values[ks][e + 4] = hi[e];
            }
        }
        if (a.rotate) {
            const int position = first_position + (valid ? j : 0);
            const float* cosines = a.cosines + static_cast<size_t>(position) * (D / 2);
            const float* sines = a.sines + static_cast<size_t>(position) * (D / 2);
#pragma unroll
            for (int ks = 0; ks < D / 64; ++ks) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int i = 32 * ks + 8 * g + e;
                    rotate_pair(values[ks][e], values[ks + D / 64][e], cosines[i], sines[i], values[ks][e],
                                values[ks + D / 64][e]);
                }
            }
        }
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                // The softmax scale (log2 e / sqrt(d)) is folded into Q before the FP16 conversion.
                query[c][ks][e] =
                    valid ? static_cast<_Float16>(values[ks][e] * a.scale_log2) : static_cast<_Float16>(0.0f);
            }
        }
    }

    floatx4 out[NT][D / 16];
    float maximum[NT];
    float sum[NT];
#pragma unroll
    for (int c = 0; c < NT; ++c) {
#pragma unroll
        for (int mt = 0; mt < D / 16; ++mt) {
            out[c][mt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        maximum[c] = kNegativeInfinity;
        sum[c] = 0.0f;
    }

    const int32_t* table = geo.block_table + static_cast<size_t>(first.slot) * geo.pages_per_slot;
    const size_t region = static_cast<size_t>(geo.page_tokens) * D;
    const size_t key_region = ((static_cast<size_t>(geo.layer) * 2) * geo.kv_heads + item.kv_head) * region;
    const size_t value_region = ((static_cast<size_t>(geo.layer) * 2 + 1) * geo.kv_heads + item.kv_head) * region;
    const int page_tokens = geo.page_tokens;
    // Keys past the block's last token are masked for every column.
    const int key_stop = min(item.key_end, first_position + item.count);
    const int unmasked_stop = min(item.key_end, first_position + 1);

    // The group's waves share each 64-key block through a double-buffered LDS stage: the block's K and V are two
    // contiguous runs of 16-byte chunks in the page (fragment order), copied with coalesced loads into registers
    // while the previous block is computed, then into LDS behind one barrier.
    constexpr int kKeyChunks = kStepKeys * D / 8;
    constexpr int kBlockChunks = 2 * kKeyChunks;
    __shared__ half8 stage[2][kBlockChunks];
    const int threads = blockDim.x;
    half8 staged[kStageLoads];
    auto block_source = [&](int key0, int chunk) {
        const int logical = key0 / page_tokens;
        const int within = key0 - logical * page_tokens;
        const _Float16* page = reinterpret_cast<const _Float16*>(
            geo.pool + static_cast<uint64_t>(table[logical]) * geo.page_bytes);
        const size_t base = chunk < kKeyChunks ? key_region : value_region;
        const int offset = chunk < kKeyChunks ? chunk : chunk - kKeyChunks;
        return reinterpret_cast<const half8*>(page + base + static_cast<size_t>(within) * D) + offset;
    };
    auto fetch_block = [&](int key0) {
#pragma unroll
        for (int k = 0; k < kStageLoads; ++k) {
            const int chunk = static_cast<int>(threadIdx.x) + k * threads;
            if (chunk < kBlockChunks) {
                staged[k] = *block_source(key0, chunk);
            }
        }
    };
    auto store_block = [&](int key0, int buffer) {
#pragma unroll
        for (int k = 0; k < kStageLoads; ++k) {
            const int chunk = static_cast<int>(threadIdx.x) + k * threads;
            if (chunk < kBlockChunks) {
                stage[buffer][chunk] = staged[k];
            }
        }
        // Groups too small to hold a block in kStageLoads chunks per thread copy the rest directly.
        for (int chunk = static_cast<int>(threadIdx.x) + kStageLoads * threads; chunk < kBlockChunks; chunk += threads) {
            stage[buffer][chunk] = *block_source(key0, chunk);
        }
    };
    const int steps = key_stop > item.key_begin ? (key_stop - item.key_begin + kStepKeys - 1) / kStepKeys : 0;
    if (steps > 0) {
        fetch_block(item.key_begin);
        store_block(item.key_begin, 0);
    }
    __syncthreads();

    for (int step = 0; step < steps; ++step) {
        const int key0 = item.key_begin + step * kStepKeys;
        const bool more = step + 1 < steps;
        if (more) {
            fetch_block(key0 + kStepKeys);
        }
        const half8* keys = stage[step & 1] + lane;
        const half8* values = stage[step & 1] + kKeyChunks + lane;

        floatx4 scores[NT][4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            half8 fragment[D / 32];
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) {
                fragment[ks] = keys[(t * (D / 32) + ks) * 64];
            }
#pragma unroll
            for (int c = 0; c < NT; ++c) {
                scores[c][t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks) {
                    scores[c][t] =
                        __builtin_amdgcn_mfma_f32_16x16x32_f16(fragment[ks], query[c][ks], scores[c][t], 0, 0, 0);
                }
            }
        }

        half8 probability[NT][2];
        float alpha[NT];
        // Steps that end at or before the block's first token (and inside the split) are visible to every column.
        const bool masked = key0 + kStepKeys > unmasked_stop;
#pragma unroll
        for (int c = 0; c < NT; ++c) {
            const int column_position = first_position + 16 * c + r;
            float tile_max = kNegativeInfinity;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (masked) {
                        const int key = key0 + 32 * (t >> 1) + 8 * g + 4 * (t & 1) + i;
                        if (key >= item.key_end || key > column_position) {
                            scores[c][t][i] = kNegativeInfinity;
                        }
                    }
                    tile_max = fmaxf(tile_max, scores[c][t][i]);
                }
            }
            tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 16));
            tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32));
            const float next = fmaxf(maximum[c], tile_max);
            // A column may see no key of this split yet; keep its state at (-inf, 0) without NaN.
            const float base = next == kNegativeInfinity ? 0.0f : next;
            alpha[c] = fast_exp2(maximum[c] - base);
            float tile_sum = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p = fast_exp2(scores[c][t][i] - base);
                    tile_sum += p;
                    probability[c][t >> 1][4 * (t & 1) + i] = static_cast<_Float16>(p);
                }
            }
            sum[c] = sum[c] * alpha[c] + tile_sum;
            maximum[c] = next;
        }
#pragma unroll
        for (int mt = 0; mt < D / 16; ++mt) {
            half8 value_fragment[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                value_fragment[h] = values[(h * (D / 16) + mt) * 64];
            }
#pragma unroll
            for (int c = 0; c < NT; ++c) {
                out[c][mt] *= alpha[c];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    out[c][mt] =
                        __builtin_amdgcn_mfma_f32_16x16x32_f16(value_fragment[h], probability[c][h], out[c][mt], 0, 0, 0);
                }
            }
        }
        if (more) {
            store_block(key0 + kStepKeys, (step + 1) & 1);
        }
        __syncthreads();
    }

    const int group = geo.group;
#pragma unroll
    for (int c = 0; c < NT; ++c) {
        float total = sum[c];
        total += __shfl_xor(total, 16);
        total += __shfl_xor(total, 32);
        const int j = 16 * c + r;
        if (j >= item.count) {
            continue;
        }
        const int token = item.first_token + j;
        if (item.row < 0) {
            float* destination = a.output + static_cast<size_t>(token) * a.out_stride + static_cast<size_t>(head) * D;
            const float inverse = 1.0f / total;
#pragma unroll
            for (int mt = 0; mt < D / 16; ++mt) {
                *reinterpret_cast<floatx4*>(destination + 16 * mt + 4 * g) = out[c][mt] * inverse;
            }
        } else {
            const size_t row = static_cast<size_t>(item.row + j * item.row_stride) * group + wave;
            float* destination = a.partial_out + row * D;
#pragma unroll
            for (int mt = 0; mt < D / 16; ++mt) {
                *reinterpret_cast<floatx4*>(destination + 16 * mt + 4 * g) = out[c][mt];
            }
            if (g == 0) {
                a.partial_ml[row * 2] = maximum[c];
                a.partial_ml[row * 2 + 1] = total;
            }
        }
    }
}

}  // namespace

hipError_t launch_prefill(const Launch& launch, const AttentionArgs& args, int items, bool fp16) {
    if (items == 0) {
        return hipSuccess;
    }
    if (!fp16) {
        return hipErrorNotSupported;  // the planner sends FP32 prompt runs through the decode kernel
    }
    const dim3 grid(items);
    const dim3 block(args.geo.group * 64);
    if (args.geo.head_dim == 128) {
        SYNAPSE_KV_LAUNCH(prefill_f16_kernel<128>, grid, block, launch, args);
    } else {
        SYNAPSE_KV_LAUNCH(prefill_f16_kernel<64>, grid, block, launch, args);
    }
    return hipGetLastError();
}

}  // namespace synapse_kv
