// Query-aware KV page activation (ADR-016) on the device: per-page key summaries and key-bound page selection.
//
// Semantics: KvPageSelector (src/Synapse.Runtime/Features/TextGeneration/KvPageSelector.cs:17-54) with pages of
// 16, 32 or 64 positions (KvPageActivation.PageTokens, KvPageActivation.cs:12-13, 33-36). PageBound (:57-87): per
// channel the minimum and maximum of the page's keys (MathF.Min / MathF.Max from the first key on), then for each query head of the group bound = sum over channels, in order, of
// MathF.Max(q_c * min_c, q_c * max_c) (products and sums rounded separately), and the page's bound is the maximum
// over the heads. BestPages (:90-107): candidates 1..windowPage - 1 ranked by bound, highest first, ties to the
// earlier page (float.CompareTo order: NaN below every number), the first `budget` taken.
//
// MI355X mapping: summaries are kept per (pool page, layer, KV head, activation page) in the storage type (exact),
// so a bound reads 2 * head_dim values per page instead of its keys. The append kernel folds a key into the summary
// of a page it alone writes in the step; summary_kernel covers the pages several tokens of the step write (prompt
// runs) and everything cached when activation is switched on. Selection is one launch: select_kernel spreads
// (selection job, 64 candidate pages) tiles over the whole device, staging the tile's summaries (widened) and the
// rotated query heads in LDS; one thread per (candidate, query head) sums the channels in the reference's order,
// so bounds are bit-identical with the CPU path. Each tile keeps its best min(budget, 64) candidates (rank keys:
// bound descending, then the earlier page); a second launch, one workgroup per job, sorts the kept keys in LDS and
// writes the selected pages' first keys, ascending, into the row's list. The decode kernel reads the 64-key block holding each listed page and masks the keys outside the page.

#include <algorithm>

#include "page_summary.h"

namespace synapse_kv {
namespace {

constexpr int kMaxGroup = 8;
constexpr int kTileCandidates = 64;

__device__ inline void rotate_pair(float x, float y, float c, float s, float& first, float& second) {
#pragma clang fp contract(off)
    first = x * c - y * s;
    second = x * s + y * c;
}

// Grid (items, layers, kv_heads) of 256 threads: the summary of one (pool page, activation page, keys) item's first
// keys, layer and KV head.
template <typename T>
__global__ __launch_bounds__(256) void summary_kernel(SummaryArgs a) {
    __shared__ SummaryScratch<T> scratch;
    const int32_t* item = a.blocks + 3 * blockIdx.x;
    summarize_block<T>(a.geo, a.first_layer + blockIdx.y, blockIdx.z, item[0], item[1], item[2], a.summaries,
                       a.summary_page_bytes, scratch);
}

// Sort key of a candidate: ascending order = bound descending (float.CompareTo: NaN below every number, -0 equal to
// +0), then page ascending (KvPageSelector.cs:112-113). Keys are distinct (the page index is the low 32 bits).
__device__ inline uint64_t rank_key(float bound, int index) {
    uint32_t ordered = 0;  // NaN: after every number
    if (bound == bound) {
        const uint32_t bits = __float_as_uint(bound == 0.0f ? 0.0f : bound);
        ordered = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);  // ascending with the value, never 0
    }
    return (static_cast<uint64_t>(~ordered) << 32) | static_cast<uint32_t>(index);
}

__host__ __device__ constexpr int next_power_of_two(int value) {
    int power = 1;
    while (power < value) {
        power <<= 1;
    }
    return power;
}

// Ascending bitonic sort of `count` (a power of two) keys in LDS by the whole workgroup; ends with a barrier.
__device__ void bitonic_sort(uint64_t* keys, int count) {
    for (int size = 2; size <= count; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int pair = threadIdx.x; pair < count / 2; pair += blockDim.x) {
                const int low = 2 * pair - (pair & (stride - 1));
                const int high = low + stride;
                const uint64_t first = keys[low];
                const uint64_t second = keys[high];
                if ((first > second) == ((low & size) == 0)) {
                    keys[low] = second;
                    keys[high] = first;
                }
            }
            __syncthreads();
        }
    }
}

// Elements of one staged candidate row: the page's minimum row, its maximum row, and 16 bytes of padding (rows at
// a 16-byte stride that spreads the lanes of a wave over the LDS banks).
template <typename T>
__host__ __device__ constexpr int staged_row(int head_dim) {
    return 2 * head_dim + 16 / static_cast<int>(sizeof(T));
}

// Dynamic LDS of the select kernel: the larger of the tile's staged summaries and a summary work item's scratch.
template <typename T>
size_t select_shared_bytes(int head_dim) {
    const size_t tile = static_cast<size_t>(kTileCandidates) * staged_row<T>(head_dim) * sizeof(T);
    const size_t bytes = sizeof(SummaryScratch<T>);
    return tile > bytes ? tile : bytes;
}

// MathF.Max of the candidate's head bounds, heads in order (KvPageSelector.cs:79-92). The head bounds are never
// -0 (see the bound sum), so the hardware maximum agrees with MathF.Max on them.
__device__ inline float best_bound(const float* head_bounds, int group, int candidate) {
    float best = -__builtin_inff();
    for (int h = 0; h < group; ++h) {
        best = __builtin_fmaxf(best, head_bounds[h * kTileCandidates + candidate]);
    }
    return best;
}

// Grid (tiles, jobs) of 64 * group threads: the bounds of candidate pages 64 * tile + 1 .. 64 * tile + 64 of one
// job. Thread (head h = tid / 64, candidate c = tid % 64) sums MathF.Max(q * min, q * max) over channels in order
// (one rounding per product and per sum); the candidate's bound is the MathF.Max over heads in order
// (KvPageSelector.cs:79-92). Each tile keeps its best min(budget, 64) rank keys (the job's best `budget` are among
// them); select_merge_kernel merges them per job.
template <typename T>
__global__ __launch_bounds__(512) void select_kernel(SelectArgs a) {
    extern __shared__ __align__(16) uint8_t scratch[];
    __shared__ __align__(16) float query[kMaxGroup * 128];
    __shared__ float head_bounds[kMaxGroup * kTileCandidates];
    __shared__ const T* summary_rows[kTileCandidates];
    __shared__ uint64_t tile_keys[kTileCandidates];
    const Geometry& g = a.geo;
    if (static_cast<int>(blockIdx.y) < a.summary_count) {
        // Summary work: pair blockIdx.y of this layer, KV head blockIdx.x.
        if (static_cast<int>(blockIdx.x) < g.kv_heads) {
            const int32_t* item = a.summary_blocks + 3 * blockIdx.y;
            summarize_block<T>(g, g.layer, blockIdx.x, item[0], item[1], item[2], a.summary_out, a.summary_page_bytes,
                               *reinterpret_cast<SummaryScratch<T>*>(scratch));
        }
        return;
    }
    const int job_index = blockIdx.y - a.summary_count;
    const SelectJob job = a.jobs[job_index];
    const int first = blockIdx.x * kTileCandidates;
    if (first >= job.candidates) {
        return;
    }
    const int count = min(kTileCandidates, job.candidates - first);
    const SynapseKvBatchToken token = a.tokens[job.token];
    const int d = g.head_dim;
    const int group = g.group;
    T* staged = reinterpret_cast<T*>(scratch);  // [candidate][staged_row]: minimum row, maximum row
    const int row_elements = staged_row<T>(d);
    const int32_t* table = g.block_table + static_cast<size_t>(token.slot) * g.pages_per_slot;
    // 1. The summary rows of the tile's candidates (a table load each): minimum and maximum rows, contiguous.
    if (threadIdx.x < count) {
        const int key = (first + threadIdx.x + 1) * g.summary_keys;
        const int page = table[key / g.page_tokens];
        summary_rows[threadIdx.x] =
            reinterpret_cast<const T*>(a.summaries + static_cast<uint64_t>(page) * a.summary_page_bytes) +
            summary_offset(g, g.layer, job.kv_head, (key % g.page_tokens) / g.summary_keys, 0, 0);
    }
    // 2. The group's query heads, rotated at the token's position when Q in qkv is unrotated.
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
    __syncthreads();
    // 3. The tile's summaries (each candidate's minimum and maximum rows, 2 * head_dim contiguous elements) copied
    //    to LDS with 16-byte loads, four in flight per thread.
    constexpr int kPerChunk = 16 / static_cast<int>(sizeof(T));
    const int row_chunks = 2 * d / kPerChunk;
    constexpr int kRounds = 4;
    const int items = count * row_chunks;
    // Every load is issued (items past the tile clamped to its last one), four into named registers, then stored.
    static_assert(kRounds == 4, "four named loads");
    for (int batch = 0; batch < items; batch += kRounds * blockDim.x) {
        auto load = [&](int round) __attribute__((always_inline)) {
            const int item = min(batch + static_cast<int>(threadIdx.x) + round * static_cast<int>(blockDim.x), items - 1);
            const int candidate = item / row_chunks;
            return reinterpret_cast<const uint4*>(summary_rows[candidate])[item - candidate * row_chunks];
        };
        auto store = [&](int round, const uint4& value) __attribute__((always_inline)) {
            const int item = batch + static_cast<int>(threadIdx.x) + round * static_cast<int>(blockDim.x);
            if (item < items) {
                const int candidate = item / row_chunks;
                reinterpret_cast<uint4*>(staged + candidate * row_elements)[item - candidate * row_chunks] = value;
            }
        };
        const uint4 loaded0 = load(0);
        const uint4 loaded1 = load(1);
        const uint4 loaded2 = load(2);
        const uint4 loaded3 = load(3);
        store(0, loaded0);
        store(1, loaded1);
        store(2, loaded2);
        store(3, loaded3);
    }
    __syncthreads();
    // 3. One (candidate, head) sum per thread.
    const int candidate = threadIdx.x % kTileCandidates;
    const int head = threadIdx.x / kTileCandidates;
    if (candidate < count && head < group) {
        const float* q = query + head * d;
        const T* minimum = staged + candidate * row_elements;
        const T* maximum = minimum + d;
        float sum = 0.0f;
        // The term MathF.Max(q * min, q * max) is q * max for q >= 0 and q * min otherwise: rounding is monotone
        // and min <= max, so the larger product is that one, bit for bit, except that two zero products may differ
        // in sign. A zero of either sign added to the running sum leaves it unchanged, since the sum starts at +0
        // and a round-to-nearest sum is -0 only when both addends are -0. Four channels per round, loaded before
        // the serial sum so the LDS reads of a round overlap.
        // Operands are held in vector registers (a local array written through a cast pointer would live in
        // scratch memory).
        typedef T Chunk __attribute__((ext_vector_type(kPerChunk)));
        typedef float Quad __attribute__((ext_vector_type(4)));
        for (int c0 = 0; c0 < d; c0 += kPerChunk) {
#pragma clang fp contract(off)
            const Chunk low = __builtin_bit_cast(Chunk, *reinterpret_cast<const uint4*>(minimum + c0));
            const Chunk high = __builtin_bit_cast(Chunk, *reinterpret_cast<const uint4*>(maximum + c0));
            Quad qv[kPerChunk / 4];
#pragma unroll
            for (int j = 0; j < kPerChunk / 4; ++j) {
                qv[j] = *reinterpret_cast<const Quad*>(q + c0 + 4 * j);
            }
#pragma unroll
            for (int j = 0; j < kPerChunk; ++j) {
                const float value = qv[j / 4][j % 4];
                sum += value * widen(value >= 0.0f ? high[j] : low[j]);
            }
        }
        head_bounds[head * kTileCandidates + candidate] = sum;
    }
    __syncthreads();
    // 4. The tile's best min(budget, 64) keys go to keys[job][tile * kept_stride + rank], in rank order (the job's
    //    best `budget` are among them; select_merge_kernel merges them).
    if (threadIdx.x < count) {
        tile_keys[threadIdx.x] = rank_key(best_bound(head_bounds, group, threadIdx.x), first + threadIdx.x);
    }
    __syncthreads();
    const int kept_stride = min(a.budget, kTileCandidates);
    uint64_t* job_keys = a.keys + static_cast<size_t>(job_index) * a.key_stride;
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
}

// Grid (jobs) of kMergeThreads threads, after select_kernel, for jobs of at most kSearchTiles tiles: selects the job's `budget` smallest rank keys among its
// tiles' kept keys and writes the selected pages' first keys, in ascending page order, to the row's list
// (KvPageSelector marks pages; the list is read in key order). Each tile's kept keys are sorted (select_kernel
// writes them by rank), so a key's rank among all of them is the sum over tiles of its lower bound in each (binary
// search in LDS; keys are distinct, so ranks are exact). A key of rank below `budget` sets its candidate's bit in
// an LDS bitmap; the bitmap's prefix counts give each selected page its place in the list. A launch of its own: the
// kernel boundary makes every tile's keys visible, where a last-tile merge inside select_kernel needed a
// device-scope release per tile and an acquire by the last one (measured: 46.5 against 14.8 us per launch without
// the merge at 64-position pages).
constexpr int kMergeThreads = 512;
constexpr int kBitmapWords = kMaxSelectCandidates / 32;

__global__ __launch_bounds__(kMergeThreads) void select_merge_kernel(SelectArgs a) {
    extern __shared__ __align__(16) uint8_t scratch[];
    __shared__ uint32_t bitmap[kBitmapWords];
    __shared__ uint32_t before[kBitmapWords];
    const SelectJob job = a.jobs[blockIdx.x];
    const int tiles = (job.candidates + kTileCandidates - 1) / kTileCandidates;
    const int kept_stride = min(a.budget, kTileCandidates);
    const int words = (job.candidates + 31) / 32;
    const uint64_t* job_keys = a.keys + static_cast<size_t>(blockIdx.x) * a.key_stride;
    uint64_t* keys = reinterpret_cast<uint64_t*>(scratch);  // [tile][kept_stride], each tile's run sorted
    auto kept_of = [&](int t) { return min(kept_stride, min(kTileCandidates, job.candidates - t * kTileCandidates)); };
    for (int e = threadIdx.x; e < tiles * kept_stride; e += blockDim.x) {
        keys[e] = e % kept_stride < kept_of(e / kept_stride) ? job_keys[e] : ~0ull;
    }
    for (int w = threadIdx.x; w < words; w += blockDim.x) {
        bitmap[w] = 0u;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < tiles * kept_stride; e += blockDim.x) {
        const uint64_t key = keys[e];
        if (key == ~0ull) {
            continue;
        }
        // Keys of each tile below `key`: a lower bound over its sorted run (padded with keys above every real one),
        // by binary decomposition of the count, eight runs at a time so that their LDS reads overlap.
        int rank = 0;
        for (int t0 = 0; t0 < tiles; t0 += 8) {
            int below[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                below[u] = 0;
            }
#pragma unroll
            for (int step = kTileCandidates; step > 0; step >>= 1) {
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int next = below[u] + step;
                    if (t0 + u < tiles && next <= kept_stride && keys[(t0 + u) * kept_stride + next - 1] < key) {
                        below[u] = next;
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                rank += below[u];
            }
        }
        if (rank < a.budget) {
            const uint32_t index = static_cast<uint32_t>(key & 0xFFFFFFFFull);
            atomicOr(&bitmap[index >> 5], 1u << (index & 31));
        }
    }
    __syncthreads();
    for (int w = threadIdx.x; w < words; w += blockDim.x) {
        uint32_t count = 0;
        for (int v = 0; v < w; ++v) {
            count += __builtin_popcount(bitmap[v]);
        }
        before[w] = count;
    }
    __syncthreads();
    for (int index = threadIdx.x; index < job.candidates; index += blockDim.x) {
        const uint32_t word = bitmap[index >> 5];
        const uint32_t bit = 1u << (index & 31);
        if ((word & bit) != 0) {
            const int position = static_cast<int>(before[index >> 5] + __builtin_popcount(word & (bit - 1)));
            a.lists[job.list + 1 + position] = (index + 1) * a.geo.summary_keys;
        }
    }
}

// The merge by sorting, for jobs of many tiles (where each key's rank would take many searches): one thread per pair
// of padded keys (64 to 1,024), the kept keys bitonic-sorted in LDS; the first `budget` are the selected pages,
// their indices sorted again in the same space (budget <= kept keys) give the list in ascending page order.
constexpr int kSortThreads = 1024;
constexpr int kSearchTiles = 16;  // jobs of more tiles take select_sort_kernel

__global__ __launch_bounds__(kSortThreads) void select_sort_kernel(SelectArgs a) {
    extern __shared__ __align__(16) uint8_t scratch[];
    const SelectJob job = a.jobs[blockIdx.x];
    const int tiles = (job.candidates + kTileCandidates - 1) / kTileCandidates;
    const int kept_stride = min(a.budget, kTileCandidates);
    const uint64_t* job_keys = a.keys + static_cast<size_t>(blockIdx.x) * a.key_stride;
    uint64_t* merged_keys = reinterpret_cast<uint64_t*>(scratch);
    int merged = 0;
    for (int t = 0; t < tiles; ++t) {
        const int kept = min(kept_stride, min(kTileCandidates, job.candidates - t * kTileCandidates));
        for (int r = threadIdx.x; r < kept; r += blockDim.x) {
            merged_keys[merged + r] = job_keys[t * kept_stride + r];
        }
        merged += kept;
    }
    const int padded = next_power_of_two(merged);
    for (int entry = merged + threadIdx.x; entry < padded; entry += blockDim.x) {
        merged_keys[entry] = ~0ull;
    }
    __syncthreads();
    bitonic_sort(merged_keys, padded);
    const int chosen = next_power_of_two(a.budget);
    for (int entry = threadIdx.x; entry < chosen; entry += blockDim.x) {
        merged_keys[entry] = entry < a.budget ? (merged_keys[entry] & 0xFFFFFFFFull) : ~0ull;
    }
    __syncthreads();
    bitonic_sort(merged_keys, chosen);
    for (int r = threadIdx.x; r < a.budget; r += blockDim.x) {
        a.lists[job.list + 1 + r] = (static_cast<int32_t>(merged_keys[r]) + 1) * a.geo.summary_keys;
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
    const dim3 grid(tiles > args.geo.kv_heads ? tiles : args.geo.kv_heads, args.summary_count + args.job_count);
    const dim3 block(kTileCandidates * args.geo.group);
    const int merged = tiles * (args.budget < kTileCandidates ? args.budget : kTileCandidates);
    // Dynamic LDS may exceed the 64 KiB default (an FP32 tile at head_dim 128 takes 66,560 bytes; the merge of
    // 8,192 kept keys 64 KiB).
    static const hipError_t configured = [] {
        constexpr int kMostDynamic = 96 * 1024;
        hipError_t status = hipFuncSetAttribute(reinterpret_cast<const void*>(select_kernel<_Float16>),
                                                hipFuncAttributeMaxDynamicSharedMemorySize, kMostDynamic);
        if (status == hipSuccess) {
            status = hipFuncSetAttribute(reinterpret_cast<const void*>(select_kernel<float>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, kMostDynamic);
        }
        if (status == hipSuccess) {
            status = hipFuncSetAttribute(reinterpret_cast<const void*>(select_merge_kernel),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, kMostDynamic);
        }
        if (status == hipSuccess) {
            status = hipFuncSetAttribute(reinterpret_cast<const void*>(select_sort_kernel),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, kMostDynamic);
        }
        return status;
    }();
    if (configured != hipSuccess) {
        return configured;
    }
    // Profile mode brackets both launches: the start event with the first, the stop event with the second.
    const Launch first{launch.stream, launch.start, args.job_count > 0 ? nullptr : launch.stop};
    if (fp16) {
        SYNAPSE_KV_LAUNCH_SHARED(select_kernel<_Float16>, grid, block, select_shared_bytes<_Float16>(args.geo.head_dim),
                                 first, args);
    } else {
        SYNAPSE_KV_LAUNCH_SHARED(select_kernel<float>, grid, block, select_shared_bytes<float>(args.geo.head_dim),
                                 first, args);
    }
    if (args.job_count > 0) {
        const Launch second{launch.stream, nullptr, launch.stop};
        if (tiles <= kSearchTiles) {
            const size_t shared = static_cast<size_t>(merged) * sizeof(uint64_t);
            SYNAPSE_KV_LAUNCH_SHARED(select_merge_kernel, dim3(args.job_count), dim3(kMergeThreads), shared, second,
                                     args);
        } else {
            const size_t shared = static_cast<size_t>(next_power_of_two(merged)) * sizeof(uint64_t);
            const int threads = std::min(kSortThreads, std::max(64, next_power_of_two(merged) / 2));
            SYNAPSE_KV_LAUNCH_SHARED(select_sort_kernel, dim3(args.job_count), dim3(threads), shared, second, args);
        }
    }
    return hipGetLastError();
}

}  // namespace synapse_kv
