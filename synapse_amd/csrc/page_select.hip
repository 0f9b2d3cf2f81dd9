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
// bound reads 2 * head_dim values per block instead of its 64 keys. The append kernel recomputes the summary of a
// block it alone writes in the step; summary_kernel covers the blocks several tokens of the step write (prompt
// runs) and everything cached when activation is switched on. Selection is one launch: select_kernel spreads
// (selection job, 64 candidate blocks) tiles over the whole device, staging the tile's summaries (widened) and the
// rotated query heads in LDS; one thread per (candidate, query head) sums the channels in the reference's order,
// so bounds are bit-identical with the CPU path. Each tile keeps its best min(budget, 64) candidates (rank keys:
// bound descending, then the earlier block); the last tile of a job to finish (an agent-scope counter per job,
// after a release fence) ranks the kept keys and writes the selected blocks, ascending, into the row's block list.

#include "page_summary.h"

namespace synapse_kv {
namespace {

constexpr int kMaxGroup = 8;
constexpr int kTileCandidates = 64;
constexpr int kExtremesStride = 130;  // float2 per channel; rows padded to 16-byte multiples (b128 reads, no conflicts)

__device__ inline void rotate_pair(float x, float y, float c, float s, float& first, float& second) {
#pragma clang fp contract(off)
    first = x * c - y * s;
    second = x * s + y * c;
}

// Grid (pairs, layers, kv_heads) of 256 threads: the summary of one (page, block) pair, layer and KV head.
template <typename T>
__global__ __launch_bounds__(256) void summary_kernel(SummaryArgs a) {
    __shared__ SummaryScratch<T> scratch;
    const int page = a.blocks[2 * blockIdx.x];
    const int block = a.blocks[2 * blockIdx.x + 1];
    summarize_block<T>(a.geo, a.first_layer + blockIdx.y, blockIdx.z, page, block, a.summaries, a.summary_page_bytes,
                       scratch);
}

// Sort key of a candidate, 44 bits: ascending order = bound descending (float.CompareTo: NaN below every number, -0
// equal to +0), then block ascending (KvPageSelector.cs:112-113). Keys are distinct (the block index is part).
__device__ inline uint64_t rank_key(float bound, int index) {
    uint32_t ordered = 0;  // NaN: after every number
    if (bound == bound) {
        const uint32_t bits = __float_as_uint(bound == 0.0f ? 0.0f : bound);
        ordered = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);  // ascending with the value, never 0
    }
    return (static_cast<uint64_t>(~ordered) << 12) | static_cast<uint32_t>(index);
}

struct TileScratch {
    float2 extremes[kTileCandidates * kExtremesStride];  // [candidate][channel] (min, max), widened
};

template <typename T>
constexpr size_t select_scratch_bytes() {
    return sizeof(TileScratch) > sizeof(SummaryScratch<T>) ? sizeof(TileScratch) : sizeof(SummaryScratch<T>);
}

struct MergeScratch {
    uint64_t keys[kMaxSelectCandidates];     // the tiles' kept keys
    int32_t chosen[kMaxSelectCandidates];    // block index of each rank below the budget
};

constexpr size_t kSelectScratch = sizeof(TileScratch) > sizeof(MergeScratch) ? sizeof(TileScratch) : sizeof(MergeScratch);

// MathF.Max of the candidate's head bounds, heads in order (KvPageSelector.cs:79-92).
__device__ inline float best_bound(const float* head_bounds, int group, int candidate) {
    float best = -__builtin_inff();
    for (int h = 0; h < group; ++h) {
        best = math_max(best, head_bounds[h * kTileCandidates + candidate]);
    }
    return best;
}

// Grid (tiles, jobs) of 64 * group threads: the bounds of candidate blocks 64 * tile + 1 .. 64 * tile + 64 of one
// job. Thread (head h = tid / 64, candidate c = tid % 64) sums MathF.Max(q * min, q * max) over channels in order
// (one rounding per product and per sum); the candidate's bound is the MathF.Max over heads in order
// (KvPageSelector.cs:79-92). Each tile keeps its best min(budget, 64) rank keys (the job's best `budget` are among
// them); the job's last tile merges them.
template <typename T>
__global__ __launch_bounds__(512) void select_kernel(SelectArgs a) {
    __shared__ __align__(16) float query[kMaxGroup * 128];
    __shared__ __align__(16) uint8_t scratch[kSelectScratch > select_scratch_bytes<T>() ? kSelectScratch
                                                                                       : select_scratch_bytes<T>()];
    __shared__ float head_bounds[kMaxGroup * kTileCandidates];
    __shared__ int32_t pages[kTileCandidates];
    __shared__ uint64_t tile_keys[kTileCandidates];
    __shared__ int32_t last_tile;
    TileScratch& tile = *reinterpret_cast<TileScratch*>(scratch);
    float2* extremes = tile.extremes;
    const Geometry& g = a.geo;
    if (static_cast<int>(blockIdx.y) >= a.job_count) {
        // Summary work: pair blockIdx.y - jobs of this layer, KV head blockIdx.x.
        if (static_cast<int>(blockIdx.x) < g.kv_heads) {
            const int pair = blockIdx.y - a.job_count;
            summarize_block<T>(g, g.layer, blockIdx.x, a.summary_blocks[2 * pair], a.summary_blocks[2 * pair + 1],
                               a.summary_out, a.summary_page_bytes, *reinterpret_cast<SummaryScratch<T>*>(scratch));
        }
        return;
    }
    const SelectJob job = a.jobs[blockIdx.y];
    const int first = blockIdx.x * kTileCandidates;
    if (first >= job.candidates) {
        return;
    }
    const int count = min(kTileCandidates, job.candidates - first);
    const SynapseKvBatchToken token = a.tokens[job.token];
    const int d = g.head_dim;
    const int group = g.group;
    // 1. The group's query heads, rotated at the token's position when Q in qkv is unrotated.
    const float* row = a.qkv + static_cast<size_t>(job.token) * a.qkv_stride + static_cast<size_t>(job.kv_head) * group * d;
    for (int item = threadIdx.x; item < group * (d / 2); item += blockDim.x) {
        const int h = item / (d / 2);
        const int i = item % (d / 2);
        float x = row[h * d + i];
        float y = row[h * d + i + d / 2];
        if (a.rotate) {
            const float c = a.cosines[static_cast<size_t>(token.position) * (d / 2) + i];
            const float s = a.sines[static_cast<size_t>(token.position) * (d / 2) + i];
            rotate_pair(x, y, c, s, x, y);
        }
        query[h * d + i] = x;
        query[h * d + i + d / 2] = y;
    }
    // 2. The tile's summaries, widened. The pool pages first (one table load per candidate), then the minimum and
    //    maximum rows of each candidate (2 * head_dim contiguous elements) with 16-byte loads, all issued together.
    const int32_t* table = g.block_table + static_cast<size_t>(token.slot) * g.pages_per_slot;
    if (threadIdx.x < count) {
        pages[threadIdx.x] = table[((first + threadIdx.x + 1) * kBlockKeys) / g.page_tokens];
    }
    __syncthreads();
    constexpr int kPerChunk = 16 / static_cast<int>(sizeof(T));
    const int row_chunks = 2 * d / kPerChunk;  // chunks of one candidate's minimum and maximum rows
    constexpr int kRounds = 4;  // loads in flight per thread
    const int items = count * row_chunks;
    for (int batch = 0; batch < items; batch += kRounds * blockDim.x) {
        uint4 loaded[kRounds];
#pragma unroll
        for (int round = 0; round < kRounds; ++round) {
            const int item = batch + threadIdx.x + round * blockDim.x;
            if (item < items) {
                const int candidate = item / row_chunks;
                const int key = (first + candidate + 1) * kBlockKeys;
                const T* summary = reinterpret_cast<const T*>(a.summaries +
                                                              static_cast<uint64_t>(pages[candidate]) * a.summary_page_bytes);
                const size_t at = summary_offset(g, g.layer, job.kv_head, (key % g.page_tokens) / kBlockKeys, 0, 0);
                loaded[round] = reinterpret_cast<const uint4*>(summary + at)[item % row_chunks];
            }
        }
#pragma unroll
        for (int round = 0; round < kRounds; ++round) {
            const int item = batch + threadIdx.x + round * blockDim.x;
            if (item < items) {
                const int candidate = item / row_chunks;
                const int element = (item % row_chunks) * kPerChunk;  // the chunk's first element in [min | max]
                const int which = element / d;
                const T* values = reinterpret_cast<const T*>(&loaded[round]);
                float* target = reinterpret_cast<float*>(extremes + candidate * kExtremesStride);
#pragma unroll
                for (int e = 0; e < kPerChunk; ++e) {
                    target[2 * (element % d + e) + which] = widen(values[e]);
                }
            }
        }
    }
    __syncthreads();
    // 3. One (candidate, head) sum per thread.
    const int candidate = threadIdx.x % kTileCandidates;
    const int head = threadIdx.x / kTileCandidates;
    if (candidate < count && head < group) {
        const float4* q = reinterpret_cast<const float4*>(query + head * d);
        const float4* e = reinterpret_cast<const float4*>(extremes + candidate * kExtremesStride);
        float sum = 0.0f;
        // Four channels per round, loaded before the serial sum so the LDS reads of a round overlap.
        for (int c4 = 0; c4 < d / 4; ++c4) {
#pragma clang fp contract(off)
            const float4 qv = q[c4];
            const float4 e01 = e[2 * c4];      // (min, max) of channels 4 c4, 4 c4 + 1
            const float4 e23 = e[2 * c4 + 1];  // (min, max) of channels 4 c4 + 2, 4 c4 + 3
            sum += math_max(qv.x * e01.x, qv.x * e01.y);
            sum += math_max(qv.y * e01.z, qv.y * e01.w);
            sum += math_max(qv.z * e23.x, qv.z * e23.y);
            sum += math_max(qv.w * e23.z, qv.w * e23.w);
        }
        head_bounds[head * kTileCandidates + candidate] = sum;
    }
    __syncthreads();
    // 4. The tile's best min(budget, 64) keys go to keys[job][tile * kept_stride + rank], in rank order.
    if (threadIdx.x < count) {
        tile_keys[threadIdx.x] = rank_key(best_bound(head_bounds, group, threadIdx.x), first + threadIdx.x);
    }
    __syncthreads();
    const int kept_stride = min(a.budget, kTileCandidates);
    uint64_t* job_keys = a.keys + static_cast<size_t>(blockIdx.y) * a.key_stride;
    if (threadIdx.x < count) {
        const uint64_t mine = tile_keys[threadIdx.x];
        int rank = 0;
        for (int other = 0; other < count; ++other) {
            rank += tile_keys[other] < mine ? 1 : 0;
        }
        if (rank < kept_stride) {
            job_keys[blockIdx.x * kept_stride + rank] = mine;
        }
    }
    // 5. The job's last tile to finish merges the tiles' keys: the `budget` smallest are the selected blocks.
    __syncthreads();
    if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const int tiles = (job.candidates + kTileCandidates - 1) / kTileCandidates;
        const int done = __hip_atomic_fetch_add(a.counters + blockIdx.y, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_tile = done == tiles - 1 ? 1 : 0;
        if (last_tile) {
            __hip_atomic_store(a.counters + blockIdx.y, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __syncthreads();
    if (!last_tile) {
        return;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    MergeScratch& merge = *reinterpret_cast<MergeScratch*>(scratch);
    const int tiles = (job.candidates + kTileCandidates - 1) / kTileCandidates;
    int merged = 0;
    for (int t = 0; t < tiles; ++t) {
        const int kept = min(kept_stride, min(kTileCandidates, job.candidates - t * kTileCandidates));
        for (int r = threadIdx.x; r < kept; r += blockDim.x) {
            merge.keys[merged + r] = job_keys[t * kept_stride + r];
        }
        merged += kept;
    }
    __syncthreads();
    for (int entry = threadIdx.x; entry < merged; entry += blockDim.x) {
        const uint64_t mine = merge.keys[entry];
        int rank = 0;
        for (int other = 0; other < merged; ++other) {
            rank += merge.keys[other] < mine ? 1 : 0;
        }
        if (rank < a.budget) {
            merge.chosen[rank] = static_cast<int32_t>(mine & 0xFFF);
        }
    }
    __syncthreads();
    // The chosen blocks in ascending order (KvPageSelector marks pages; the list is read in block order).
    for (int r = threadIdx.x; r < a.budget; r += blockDim.x) {
        const int index = merge.chosen[r];
        int before = 0;
        for (int other = 0; other < a.budget; ++other) {
            before += merge.chosen[other] < index ? 1 : 0;
        }
        a.lists[job.list + 1 + before] = index + 1;
    }
}

}  // namespace

hipError_t launch_summaries(const Launch& launch, const SummaryArgs& args, bool fp16) {
    if (args.count == 0 || args.layers == 0) {
        return hipSuccess;
    }
    const dim3 grid(args.count, args.layers, args.geo.kv_heads);
    if (fp16) {
        SYNAPSE_KV_LAUNCH(summary_kernel<_Float16>, grid, dim3(256), launch, args);
    } else {
        SYNAPSE_KV_LAUNCH(summary_kernel<float>, grid, dim3(256), launch, args);
    }
    return hipGetLastError();
}

hipError_t launch_select(const Launch& launch, const SelectArgs& args, int most_candidates, bool fp16) {
    if (args.job_count + args.summary_count == 0) {
        return hipSuccess;
    }
    const int tiles = (most_candidates + kTileCandidates - 1) / kTileCandidates;
    const dim3 grid(tiles > args.geo.kv_heads ? tiles : args.geo.kv_heads, args.job_count + args.summary_count);
    const dim3 block(kTileCandidates * args.geo.group);
    if (fp16) {
        SYNAPSE_KV_LAUNCH(select_kernel<_Float16>, grid, block, launch, args);
    } else {
        SYNAPSE_KV_LAUNCH(select_kernel<float>, grid, block, launch, args);
    }
    return hipGetLastError();
}

}  // namespace synapse_kv
