// GQA flash-decode attention with split-K over pages and a cross-split merge.
//
// Semantics: synapse_attention_decode (native/synapse-gpu/src/Features/GpuKernels/metal/shaders/
// attention.metal:319-355) and synapse_attention_reduce (attention_reduce.metal:5-40): each work item attends one
// token's query heads of one KV head (the GQA group) over keys [key_begin, key_end) of its slot with an online
// softmax; a token whose keys span several items writes unnormalized output plus (max, sum) rows that the merge
// kernel rescales by exp(m - max) and divides. Scores are q.k / sqrt(head_dim) over keys 0..position inclusive
// (Qwen2Attention.cs:5-25).
//
// MI355X mapping: one workgroup = 4 waves = one work item; each wave takes every fourth 64-key step. Per step a
// wave computes S^T = K Q^T and O^T = V^T P^T on MFMA with the group's query heads as the 16 columns (7 of 16
// used under GQA 7:1), so every K and V byte is read from HBM once per item and shared by all query heads:
//   FP16 KV: v_mfma_f32_16x16x32_f16. The A operand is 8 consecutive halves of one row: 8 dims of one key
//            (K, row-major) or 8 keys of one dim (V, stored transposed), i.e. one 128-bit load per lane.
//            The keys of the QK^T tiles are permuted so that the C layout of S^T (lane holds rows 4g..4g+3 of
//            two tiles) is exactly the B layout of P^T for the PV product: no shuffle between the two MFMAs.
//   FP32 KV: v_mfma_f32_16x16x4_f32 with float4 loads split across four k-steps.
// Softmax statistics are per lane (one query head per lane column); a row max needs two cross-lane steps.

#include "kv_internal.h"

namespace synapse_kv {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr float kNegativeInfinity = -__builtin_inff();

__device__ inline float wave_max_across_groups(float value) {
    value = fmaxf(value, __shfl_xor(value, 16));
    value = fmaxf(value, __shfl_xor(value, 32));
    return value;
}

__device__ inline float wave_sum_across_groups(float value) {
    value += __shfl_xor(value, 16);
    value += __shfl_xor(value, 32);
    return value;
}

__device__ inline float fast_exp2(float value) { return __builtin_amdgcn_exp2f(value); }

// Element offset of (layer, K|V, kv_head)'s region inside a page.
__device__ inline size_t region_offset(const Geometry& g, int which, int kv_head) {
    return ((static_cast<size_t>(g.layer) * 2 + which) * g.kv_heads + kv_head) * static_cast<size_t>(g.page_tokens) *
           g.head_dim;
}

template <int D>
struct WaveState {
    floatx4 out[D / 16];  // O^T: lane (g, r) holds dims 16*mt + 4*g + i of query head r
    float maximum;        // running max of head r in log2 units
    float sum;            // this lane's share of the running sum of head r
};

// Merges the waves of one workgroup and writes the item's result: normalized output for an unsplit token,
// otherwise the unnormalized output and (max, sum) of every head of the group into the partial row.
template <int D>
__device__ void finish_item(const AttentionArgs& a, const DecodeItem& item, WaveState<D>& state, int token_index) {
    __shared__ float stage_out[kWaves][16][D + 4];
    __shared__ float stage_max[kWaves][16];
    __shared__ float stage_sum[kWaves][16];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int g = lane >> 4;
    const float total = wave_sum_across_groups(state.sum);
#pragma unroll
    for (int mt = 0; mt < D / 16; ++mt) {
        *reinterpret_cast<floatx4*>(&stage_out[wave][r][16 * mt + 4 * g]) = state.out[mt];
    }
    if (g == 0) {
        stage_max[wave][r] = state.maximum;
        stage_sum[wave][r] = total;
    }
    __syncthreads();
    const Geometry& geo = a.geo;
    const int group = geo.group;
    for (int index = threadIdx.x; index < group * D; index += kWaves * 64) {
        const int head = index / D;
        const int dim = index - head * D;
        float maximum = kNegativeInfinity;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            if (stage_sum[w][head] > 0.0f) {
                maximum = fmaxf(maximum, stage_max[w][head]);
            }
        }
        float value = 0.0f;
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            if (stage_sum[w][head] > 0.0f) {
                const float factor = fast_exp2(stage_max[w][head] - maximum);
                value += stage_out[w][head][dim] * factor;
                sum += stage_sum[w][head] * factor;
            }
        }
        if (item.row < 0) {
            a.output[static_cast<size_t>(token_index) * a.out_stride +
                     static_cast<size_t>(item.kv_head * group + head) * D + dim] = value / sum;
        } else {
            const size_t row = static_cast<size_t>(item.row) * group + head;
            a.partial_out[row * D + dim] = value;
            if (dim == 0) {
                a.partial_ml[row * 2] = maximum;
                a.partial_ml[row * 2 + 1] = sum;
            }
        }
    }
}

template <int D>
__global__ __launch_bounds__(kWaves * 64) void decode_f16_kernel(AttentionArgs a) {
    const DecodeItem item = a.items[blockIdx.x];
    const Geometry& geo = a.geo;
    const SynapseKvBatchToken token = a.tokens[item.token];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int g = lane >> 4;

    // B operand of S^T = K Q^T: lane (g, r) holds dims 32*ks + 8*g .. +7 of query head r of the group.
    half8 query[D / 32];
    {
        const bool valid = r < geo.group;
        const float* q = a.qkv + static_cast<size_t>(item.token) * a.qkv_stride +
                         static_cast<size_t>(item.kv_head * geo.group + (valid ? r : 0)) * D;
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            const floatx4 lo = *reinterpret_cast<const floatx4*>(q + 32 * ks + 8 * g);
            const floatx4 hi = *reinterpret_cast<const floatx4*>(q + 32 * ks + 8 * g + 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                query[ks][j] = valid ? static_cast<_Float16>(lo[j]) : static_cast<_Float16>(0.0f);
                query[ks][j + 4] = valid ? static_cast<_Float16>(hi[j]) : static_cast<_Float16>(0.0f);
            }
        }
    }

    WaveState<D> state;
#pragma unroll
    for (int mt = 0; mt < D / 16; ++mt) {
        state.out[mt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    state.maximum = kNegativeInfinity;
    state.sum = 0.0f;

    const int32_t* table = geo.block_table + static_cast<size_t>(token.slot) * geo.pages_per_slot;
    const size_t key_region = region_offset(geo, 0, item.kv_head);
    const size_t value_region = region_offset(geo, 1, item.kv_head);
    const int page_tokens = geo.page_tokens;
    // Row of the A operand this lane loads for QK^T tile (h, u): the permutation that lands key 32h + 8g + 4u + i
    // of the C tile on this lane group's element 4u + i of the PV B operand.
    const int row_key = 8 * (r >> 2) + (r & 3);

    for (int key0 = item.key_begin + kStepKeys * wave; key0 < item.key_end; key0 += kStepKeys * kWaves) {
        const int logical = key0 / page_tokens;
        const int within = key0 - logical * page_tokens;
        const _Float16* page = reinterpret_cast<const _Float16*>(
            geo.pool + static_cast<uint64_t>(table[logical]) * geo.page_bytes);
        const _Float16* keys = page + key_region + static_cast<size_t>(within) * D;
        const _Float16* values = page + value_region + within;

        floatx4 scores[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int key = 32 * (t >> 1) + row_key + 4 * (t & 1);
            half8 fragment[D / 32];
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) {
                fragment[ks] = *reinterpret_cast<const half8*>(keys + static_cast<size_t>(key) * D + 32 * ks + 8 * g);
            }
            scores[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) {
                scores[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fragment[ks], query[ks], scores[t], 0, 0, 0);
            }
        }
        half8 value_fragment[2][D / 16];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int mt = 0; mt < D / 16; ++mt) {
                value_fragment[h][mt] = *reinterpret_cast<const half8*>(
                    values + static_cast<size_t>(16 * mt + r) * page_tokens + 32 * h + 8 * g);
            }
        }

        float tile_max = kNegativeInfinity;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = key0 + 32 * (t >> 1) + 8 * g + 4 * (t & 1) + i;
                const float s = key < item.key_end ? scores[t][i] * a.scale_log2 : kNegativeInfinity;
                scores[t][i] = s;
                tile_max = fmaxf(tile_max, s);
            }
        }
        tile_max = wave_max_across_groups(tile_max);
        const float next = fmaxf(state.maximum, tile_max);
        const float alpha = fast_exp2(state.maximum - next);
        float tile_sum = 0.0f;
        half8 probability[2];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p = fast_exp2(scores[t][i] - next);
                tile_sum += p;
                probability[t >> 1][4 * (t & 1) + i] = static_cast<_Float16>(p);
            }
        }
        state.sum = state.sum * alpha + tile_sum;
        state.maximum = next;
#pragma unroll
        for (int mt = 0; mt < D / 16; ++mt) {
            state.out[mt] *= alpha;
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int mt = 0; mt < D / 16; ++mt) {
                state.out[mt] =
                    __builtin_amdgcn_mfma_f32_16x16x32_f16(value_fragment[h][mt], probability[h], state.out[mt], 0, 0, 0);
            }
        }
    }
    finish_item<D>(a, item, state, item.token);
}

template <int D>
__global__ __launch_bounds__(kWaves * 64) void decode_f32_kernel(AttentionArgs a) {
    const DecodeItem item = a.items[blockIdx.x];
    const Geometry& geo = a.geo;
    const SynapseKvBatchToken token = a.tokens[item.token];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int g = lane >> 4;

    // B operand of S^T = K Q^T for k-step (c, i): dim 16*c + 4*g + i of query head r.
    floatx4 query[D / 16];
    {
        const bool valid = r < geo.group;
        const float* q = a.qkv + static_cast<size_t>(item.token) * a.qkv_stride +
                         static_cast<size_t>(item.kv_head * geo.group + (valid ? r : 0)) * D;
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
            const floatx4 v = *reinterpret_cast<const floatx4*>(q + 16 * c + 4 * g);
            query[c] = valid ? v : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }

    WaveState<D> state;
#pragma unroll
    for (int mt = 0; mt < D / 16; ++mt) {
        state.out[mt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    state.maximum = kNegativeInfinity;
    state.sum = 0.0f;

    const int32_t* table = geo.block_table + static_cast<size_t>(token.slot) * geo.pages_per_slot;
    const size_t key_region = region_offset(geo, 0, item.kv_head);
    const size_t value_region = region_offset(geo, 1, item.kv_head);
    const int page_tokens = geo.page_tokens;

    for (int key0 = item.key_begin + kStepKeys * wave; key0 < item.key_end; key0 += kStepKeys * kWaves) {
        const int logical = key0 / page_tokens;
        const int within = key0 - logical * page_tokens;
        const float* page =
            reinterpret_cast<const float*>(geo.pool + static_cast<uint64_t>(table[logical]) * geo.page_bytes);
        const float* keys = page + key_region + static_cast<size_t>(within) * D;
        const float* values = page + value_region + within;

        floatx4 scores[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            scores[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < D / 16; ++c) {
                const floatx4 k = *reinterpret_cast<const floatx4*>(keys + static_cast<size_t>(16 * t + r) * D + 16 * c + 4 * g);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    scores[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(k[i], query[c][i], scores[t], 0, 0, 0);
                }
            }
        }

        float tile_max = kNegativeInfinity;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = key0 + 16 * t + 4 * g + i;
                const float s = key < item.key_end ? scores[t][i] * a.scale_log2 : kNegativeInfinity;
                scores[t][i] = s;
                tile_max = fmaxf(tile_max, s);
            }
        }
        tile_max = wave_max_across_groups(tile_max);
        const float next = fmaxf(state.maximum, tile_max);
        const float alpha = fast_exp2(state.maximum - next);
        float tile_sum = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                scores[t][i] = fast_exp2(scores[t][i] - next);
                tile_sum += scores[t][i];
            }
        }
        state.sum = state.sum * alpha + tile_sum;
        state.maximum = next;
#pragma unroll
        for (int mt = 0; mt < D / 16; ++mt) {
            state.out[mt] *= alpha;
        }
        // O^T = V^T P^T: k-step (t, i) pairs lane group g with key 16*t + 4*g + i.
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int mt = 0; mt < D / 16; ++mt) {
                const floatx4 v = *reinterpret_cast<const floatx4*>(
                    values + static_cast<size_t>(16 * mt + r) * page_tokens + 16 * t + 4 * g);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    state.out[mt] = __builtin_amdgcn_mfma_f32_16x16x4f32(v[i], scores[t][i], state.out[mt], 0, 0, 0);
                }
            }
        }
    }
    finish_item<D>(a, item, state, item.token);
}

// Cross-split merge (attention_reduce.metal:5-40) with maxima in log2 units. Grid (merges, heads), head_dim
// threads.
template <int D>
__global__ __launch_bounds__(D) void merge_kernel(AttentionArgs a) {
    const MergeItem merge = a.merges[blockIdx.x];
    const int head = blockIdx.y;
    const int group = a.geo.group;
    const int kv_head = head / group;
    const int within = head - kv_head * group;
    const int dim = threadIdx.x;
    const int first = merge.first_row + kv_head * merge.splits;
    float maximum = kNegativeInfinity;
    for (int split = 0; split < merge.splits; ++split) {
        const size_t row = static_cast<size_t>(first + split) * group + within;
        if (a.partial_ml[row * 2 + 1] > 0.0f) {
            maximum = fmaxf(maximum, a.partial_ml[row * 2]);
        }
    }
    float sum = 0.0f;
    float value = 0.0f;
    for (int split = 0; split < merge.splits; ++split) {
        const size_t row = static_cast<size_t>(first + split) * group + within;
        const float weight = a.partial_ml[row * 2 + 1];
        if (weight > 0.0f) {
            const float factor = fast_exp2(a.partial_ml[row * 2] - maximum);
            sum += weight * factor;
            value += a.partial_out[row * D + dim] * factor;
        }
    }
    a.output[static_cast<size_t>(merge.token) * a.out_stride + static_cast<size_t>(head) * D + dim] = value / sum;
}

}  // namespace

hipError_t launch_decode(hipStream_t stream, const AttentionArgs& args, int items, bool fp16) {
    if (items == 0) {
        return hipSuccess;
    }
    const dim3 grid(items);
    const dim3 block(kWaves * 64);
    const int d = args.geo.head_dim;
    if (fp16) {
        if (d == 128) {
            hipLaunchKernelGGL(decode_f16_kernel<128>, grid, block, 0, stream, args);
        } else {
            hipLaunchKernelGGL(decode_f16_kernel<64>, grid, block, 0, stream, args);
        }
    } else {
        if (d == 128) {
            hipLaunchKernelGGL(decode_f32_kernel<128>, grid, block, 0, stream, args);
        } else {
            hipLaunchKernelGGL(decode_f32_kernel<64>, grid, block, 0, stream, args);
        }
    }
    return hipGetLastError();
}

hipError_t launch_merge(hipStream_t stream, const AttentionArgs& args, int merges) {
    if (merges == 0) {
        return hipSuccess;
    }
    const dim3 grid(merges, args.geo.heads);
    if (args.geo.head_dim == 128) {
        hipLaunchKernelGGL(merge_kernel<128>, grid, dim3(128), 0, stream, args);
    } else {
        hipLaunchKernelGGL(merge_kernel<64>, grid, dim3(64), 0, stream, args);
    }
    return hipGetLastError();
}

}  // namespace synapse_kv
