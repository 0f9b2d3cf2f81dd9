// Query-aware KV page activation (ADR-016) on the device: per-block key summaries and key-bound page selection.
//
// Semantics: KvPageSelector (src/Synapse.Runtime/Features/TextGeneration/KvPageSelector.cs:17-54) with 64-position
// pages. PageBound (:57-87): per channel the minimum and maximum of the page's keys (MathF.Min / MathF.Max from the
// first key on), then for each query head of the group bound = sum over channels, in order, of
// MathF.Max(q_c * min_c, q_c * max_c) (products and sums rounded separately), and the page's bound is the maximum
// over the heads. BestPages (:90-107): candidates 1..windowPage - 1 ranked by bound, highest first, ties to the
// earlier page (float.CompareTo order: NaN below every number), the first `budget` taken.
//
// MI355X mapping: summaries are kept per (pool page, layer, KV head, 64-key block) in the storage type (exact), so a
// bound reads 2 * head_dim values per block instead of its 64 keys. summary_kernel recomputes blocks from the
// stored keys (after a step's appends, and for everything cached when activation is switched on). select_kernel
// runs one workgroup per (decode token, KV head): the rotated query heads go to LDS, each thread bounds candidate
// blocks with the channel sum in the reference's order, the ranks come from pairwise comparison in LDS, and the
// selected blocks are written in ascending order into the row's block list.

#include "kv_internal.h"
#include "page_layout.h"

namespace synapse_kv {
namespace {

constexpr int kMaxGroup = 16;
constexpr int kMaxCandidates = kMaxSelectCandidates;

// MathF.Min / MathF.Max (IEEE 754-2019 minimum / maximum: NaN propagates, -0 < +0).
__device__ inline float math_min(float x, float y) {
    if (x != x) {
        return x;
    }
    if (y != y) {
        return y;
    }
    if (x == y) {
        return __builtin_signbit(x) ? x : y;
    }
    return x < y ? x : y;
}

__device__ inline float math_max(float x, float y) {
    if (x != x) {
        return x;
    }
    if (y != y) {
        return y;
    }
    if (x == y) {
        return __builtin_signbit(x) ? y : x;
    }
    return x > y ? x : y;
}

// float.CompareTo: -1, 0, 1 with NaN below every number and equal to NaN.
__device__ inline int compare_to(float x, float y) {
    const bool xn = x != x;
    const bool yn = y != y;
    if (xn || yn) {
        return xn == yn ? 0 : (xn ? -1 : 1);
    }
    return x < y ? -1 : (x > y ? 1 : 0);
}

__device__ inline void rotate_pair(float x, float y, float c, float s, float& first, float& second) {
#pragma clang fp contract(off)
    first = x * c - y * s;
    second = x * s + y * c;
}

template <typename T>
__device__ inline float widen(T value) {
    return static_cast<float>(value);
}

// Element offset of (layer, kv_head, block of the page, min|max, channel) in a summary page.
__device__ inline size_t summary_offset(const Geometry& g, int layer, int kv_head, int block, int which, int channel) {
    const int blocks = g.page_tokens / kBlockKeys;
    return ((((static_cast<size_t>(layer) * g.kv_heads + kv_head) * blocks + block) * 2 + which) * g.head_dim) + channel;
}

// Grid (pairs, layers, kv_heads) of head_dim threads: one channel of one block's minimum and maximum.
template <typename T>
__global__ __launch_bounds__(128) void summary_kernel(SummaryArgs a) {
    const Geometry& g = a.geo;
    const int channel = threadIdx.x;
    if (channel >= g.head_dim) {
        return;
    }
    const int page = a.blocks[2 * blockIdx.x];
    const int block = a.blocks[2 * blockIdx.x + 1];
    const int layer = a.first_layer + blockIdx.y;
    const int kv_head = blockIdx.z;
    const T* keys = reinterpret_cast<const T*>(g.pool + static_cast<uint64_t>(page) * g.page_bytes) +
                    ((static_cast<size_t>(layer) * 2) * g.kv_heads + kv_head) * static_cast<size_t>(g.page_tokens) *
                        g.head_dim;
    const int first = block * kBlockKeys;
    float minimum = widen(keys[key_offset<T>(g.head_dim, first, channel)]);
    float maximum = minimum;
    for (int key = first + 1; key < first + kBlockKeys; ++key) {
        const float value = widen(keys[key_offset<T>(g.head_dim, key, channel)]);
        minimum = math_min(minimum, value);
        maximum = math_max(maximum, value);
    }
    T* summary = reinterpret_cast<T*>(a.summaries + static_cast<uint64_t>(page) * a.summary_page_bytes);
    summary[summary_offset(g, layer, kv_head, block, 0, channel)] = static_cast<T>(minimum);
    summary[summary_offset(g, layer, kv_head, block, 1, channel)] = static_cast<T>(maximum);
}

// One workgroup per selection job.
template <typename T>
__global__ __launch_bounds__(256) void select_kernel(SelectArgs a) {
    __shared__ float query[kMaxGroup * 128];
    __shared__ float bound[kMaxCandidates];
    __shared__ int chosen[kMaxCandidates];
    const Geometry& g = a.geo;
    const SelectJob job = a.jobs[blockIdx.x];
    const SynapseKvBatchToken token = a.tokens[job.token];
    const int d = g.head_dim;
    const int group = g.group;
    // 1. The group's query heads, rotated at the token's position when the call asks for RoPE.
    const float* row = a.qkv + static_cast<size_t>(job.token) * a.qkv_stride + static_cast<size_t>(job.kv_head) * group * d;
    for (int item = threadIdx.x; item < group * (d / 2); item += 256) {
        const int h = item / (d / 2);
        const int i = item % (d / 2);
        float first = row[h * d + i];
        float second = row[h * d + i + d / 2];
        if (a.rotate) {
            const float c = a.cosines[static_cast<size_t>(token.position) * (d / 2) + i];
            const float s = a.sines[static_cast<size_t>(token.position) * (d / 2) + i];
            rotate_pair(first, second, c, s, first, second);
        }
        query[h * d + i] = first;
        query[h * d + i + d / 2] = second;
    }
    __syncthreads();
    // 2. Bounds of blocks 1..candidates.
    const int32_t* table = g.block_table + static_cast<size_t>(token.slot) * g.pages_per_slot;
    for (int index = threadIdx.x; index < job.candidates; index += 256) {
        const int block = index + 1;
        const int key = block * kBlockKeys;
        const int page = table[key / g.page_tokens];
        const T* summary = reinterpret_cast<const T*>(a.summaries + static_cast<uint64_t>(page) * a.summary_page_bytes);
        const T* minimum = summary + summary_offset(g, g.layer, job.kv_head, (key % g.page_tokens) / kBlockKeys, 0, 0);
        const T* maximum = minimum + d;
        float best = -__builtin_inff();
        for (int h = 0; h < group; ++h) {
            float sum = 0.0f;
            for (int c = 0; c < d; ++c) {
#pragma clang fp contract(off)
                const float q = query[h * d + c];
                sum += math_max(q * widen(minimum[c]), q * widen(maximum[c]));
            }
            best = math_max(best, sum);
        }
        bound[index] = best;
    }
    __syncthreads();
    // 3. Rank (higher bound first, the earlier block on ties) and mark the first `budget`.
    for (int index = threadIdx.x; index < job.candidates; index += 256) {
        const float mine = bound[index];
        int rank = 0;
        for (int other = 0; other < job.candidates && rank < a.budget; ++other) {
            const int order = compare_to(bound[other], mine);
            rank += order > 0 || (order == 0 && other < index) ? 1 : 0;
        }
        chosen[index] = rank < a.budget ? 1 : 0;
    }
    __syncthreads();
    // 4. The chosen blocks, ascending, after the sink entry.
    for (int index = threadIdx.x; index < job.candidates; index += 256) {
        if (chosen[index]) {
            int before = 0;
            for (int other = 0; other < index; ++other) {
                before += chosen[other];
            }
            a.lists[job.list + 1 + before] = index + 1;
        }
    }
}

}  // namespace

hipError_t launch_summaries(const Launch& launch, const SummaryArgs& args, bool fp16) {
    if (args.count == 0 || args.layers == 0) {
        return hipSuccess;
    }
    const dim3 grid(args.count, args.layers, args.geo.kv_heads);
    if (fp16) {
        SYNAPSE_KV_LAUNCH(summary_kernel<_Float16>, grid, dim3(128), launch, args);
    } else {
        SYNAPSE_KV_LAUNCH(summary_kernel<float>, grid, dim3(128), launch, args);
    }
    return hipGetLastError();
}

hipError_t launch_select(const Launch& launch, const SelectArgs& args, int jobs, bool fp16) {
    if (jobs == 0) {
        return hipSuccess;
    }
    if (fp16) {
        SYNAPSE_KV_LAUNCH(select_kernel<_Float16>, dim3(jobs), dim3(256), launch, args);
    } else {
        SYNAPSE_KV_LAUNCH(select_kernel<float>, dim3(jobs), dim3(256), launch, args);
    }
    return hipGetLastError();
}

}  // namespace synapse_kv
