// Internal interface between the host half of libsynapse_kv (cache.hip) and its kernels.
//
// Page layout (one page = page_tokens positions of one slot across every executed layer):
//   region(layer, which, kv_head) = ((layer * 2 + which) * kv_heads + kv_head) * page_tokens * head_dim elements
//   which = 0 (K): row-major [page_tokens][head_dim]   -- a 16-byte load holds 8 dims of one key
//   which = 1 (V): transposed [head_dim][page_tokens]  -- a 16-byte load holds 8 keys of one dim
// so both MFMA products of attention (S^T = K Q^T and O^T = V^T P^T) read their A operand straight from HBM
// with 128-bit loads. Elements are float (FP32 KV) or _Float16 (FP16 KV).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/synapse_kv.h"
#include "q8_layout.h"

namespace synapse_kv {

// A block-table operation, executed in order by the single-workgroup table kernel.
enum TableOpKind : int32_t {
    kOpResize = 1,  // slot, from pages, to pages, list offset (fresh pages on growth)
    kOpCow = 2,     // slot, logical page, list offset (copy pair)
    kOpFork = 3,    // source slot, target slot, pages
};

struct TableOp {
    int32_t kind;
    int32_t a;
    int32_t b;
    int32_t c;
    int32_t d;
    int32_t pad[3];
};
static_assert(sizeof(TableOp) == 32, "TableOp is 32 bytes");

struct TableArgs {
    const TableOp* ops;
    int32_t op_count;
    int32_t pages_per_slot;
    int32_t max_pages;
    int32_t* block_table;  // [slots][pages_per_slot]
    int32_t* refcount;     // [max_pages]
    int32_t* free_stack;   // [max_pages], bottom first
    int32_t* state;        // [0] free count, [1] status (0 = consistent)
    int32_t* fresh;        // pages to zero-fill
    int32_t* copies;       // (source, target) page pairs to copy
};

struct PageArgs {
    uint8_t* pool;
    uint64_t page_bytes;
    const int32_t* list;  // fresh pages, or (source, target) pairs
    int32_t count;
};

// A decode segment: keys [key_begin, key_end) of one (token, KV head) row. `row` >= 0 is the segment's partial
// row and `merge` the row's merge entry; row -1 writes the normalized output directly. With list >= 0 the row
// attends the activation pages whose first keys are lists[list + 0 ..] (KV page activation: a step reads the 64-key
// block holding the page and masks the keys outside it) and key_begin / key_end count list entries times 64. `last` marks the piece that holds the row's own position (the fused append writes it first).
struct DecodeSegment {
    int32_t token;
    int32_t kv_head;
    int32_t key_begin;
    int32_t key_end;
    int32_t row;       // partial row of a cut row, -1 for an uncut one
    int32_t list;      // block list (KV page activation), -1 for none
    int32_t last;      // 1: the segment ends at the token's own position (its wave appends the token)
    int32_t slot;      // the token's slot and position, copied from the step's tokens so that a wave starts with
    int32_t position;  // one descriptor read
    int32_t next;        // index of the same worker's next segment, -1 after its last (worker w's first is index w)
    int32_t first_page;   // pool page of the segment's first 64-key block (-1: read it from the block table)
    int32_t append_page;  // with `last`: pool page of the token's own position (-1: read it from the block table)
};
static_assert(sizeof(DecodeSegment) == 48, "DecodeSegment is 48 bytes");

// The partial rows first_row .. first_row + count - 1 of one (token, KV head), merged into the output.
struct MergeItem {
    int32_t token;
    int32_t kv_head;
    int32_t first_row;
    int32_t count;
    int32_t output_row;  // -1: normalize into the output; else write the combination as this partial row
    int32_t pad[3];
};

// A prefill work item: every query head of `kv_head` over keys [key_begin, key_end) for `count` (<= kPrefillTokens)
// columns. With listed == 0 the columns are consecutive tokens of one prompt run (consecutive positions of one
// slot) starting at step token `first_token`, masked causally. With listed == 1 they are the step tokens
// members[first_token .. first_token + count - 1], whose block tables all map the item's keys to the same pages
// (a copy-on-write prefix below every member's position): no mask, each column rotated at its own position.
// `row` >= 0: column j writes partial row `row + j * row_stride` (the decode merge layout); -1: the normalized
// output is written directly.
struct PrefillItem {
    int32_t first_token;
    int32_t count;
    int32_t kv_head;
    int32_t key_begin;
    int32_t key_end;
    int32_t row;
    int32_t row_stride;
    int32_t listed;
};
static_assert(sizeof(PrefillItem) == 32, "PrefillItem is 32 bytes");

struct Geometry {
    const uint8_t* pool;
    uint64_t page_bytes;
    const int32_t* block_table;
    int32_t pages_per_slot;
    int32_t page_tokens;
    int32_t heads;
    int32_t kv_heads;
    int32_t group;
    int32_t head_dim;
    int32_t layer;
    int32_t summary_keys;  // KV page activation: positions per activation page (16, 32 or 64), one summary each
};

struct AppendArgs {
    Geometry geo;
    uint8_t* pool;
    const SynapseKvBatchToken* tokens;
    float* qkv;
    int32_t qkv_stride;
    int32_t half_dim;
    const float* cosines;
    const float* sines;
    int32_t write_back;  // 1: rotated Q and K replace the qkv values; 0: qkv is left as it was
    // KV page activation: a token with extend[token] != 0 is alone in its activation page in the step and appends
    // right after its slot's keys, whose page summary covers exactly the keys below it, so the append kernel folds
    // the new key in (or starts the summary at a page's first position). Other written blocks are recomputed from
    // their keys below the slot's new length. Null: no summaries.
    uint8_t* summaries;
    uint64_t summary_page_bytes;
    const int32_t* extend;
};

struct AttentionArgs {
    Geometry geo;
    const SynapseKvBatchToken* tokens;
    const float* qkv;
    int32_t qkv_stride;
    float* output;
    int32_t out_stride;
    float scale_log2;  // log2(e) / sqrt(head_dim)
    int32_t rotate;    // 1: Q in qkv is unrotated; the decode kernel applies RoPE in registers
    int32_t append;    // 1: the decode kernel also appends each row's own K/V (fused step)
    const float* cosines;
    const float* sines;
    int32_t workers;                 // decode wave workers
    const DecodeSegment* segments;
    const int32_t* members;  // step token indices of listed prefill items' columns
    const int32_t* lists;    // block lists of rows under KV page activation (DecodeSegment::list)
    const MergeItem* merges;
    const PrefillItem* prefill;
    float* partial_out;  // [rows][group][head_dim]
    float* partial_ml;   // [rows][group][2] (maximum in log2 units, sum)
    uint32_t* timing;    // non-null: worker w writes its duration (s_memrealtime ticks) to timing[w]
};

// Waves per decode workgroup: worker w runs in workgroup w / kDecodeBlockWaves, which the dispatcher places on XCD
// (w / kDecodeBlockWaves) % kXcds.
constexpr int kDecodeBlockWaves = 4;
constexpr int kXcds = 8;

struct GatherArgs {
    Geometry geo;
    int32_t slot;
    int32_t first;
    int32_t count;
    uint8_t* keys;    // [count][kv_heads][head_dim] in the storage type
    uint8_t* values;  // [count][kv_heads][head_dim] in the storage type
};

// One matrix of a projection in the device layout of q8_layout.h: its row tiles are blockIdx.x values
// first_tile .. first_tile + q8_tiles(rows) - 1 of the launch.
struct ProjectionSegment {
    const uint8_t* codes;
    const void* scales;  // Q8_0: FP16 bits; K-quants: 320-byte factor groups (kquant_layout.h)
    const float* bias;       // null: no bias
    int32_t rows;
    int32_t first_tile;
    int32_t out_column;
    uint32_t encoding;  // GGML type of this segment's matrix
};

// A decode projection whose input is an RMS-normalized row (synapse_rms_norm, elementwise.cu:17-52): the kernel reads
// the raw row and normalizes it while staging, y = x * (1 / sqrt(total / columns + epsilon)) * weight, with total
// the in-order sum of the token's `parts` partial sums of squares (squares[token * kNormSquaresStride + part], part
// j covering columns 256 j .. 256 j + 255), written by the kernel that produced the row.
constexpr int kNormSquaresStride = 32;  // rows of up to 8,192 columns
constexpr int kNormSquaresColumns = 256;
struct NormInput {
    const float* weight = nullptr;  // null: the input is used as it is
    const float* squares = nullptr;
    int32_t parts = 0;
    int32_t columns = 0;
    float epsilon = 0.0f;
    int32_t pad = 0;
};

struct ProjectionArgs {
    ProjectionSegment segment[3];
    int32_t segments;
    int32_t columns;
    int32_t chunks;  // q8_chunks(columns)
    int32_t tokens;
    int32_t in_stride;
    int32_t out_stride;
    int32_t accumulate;
    int32_t padded_columns;  // chunks * 64
    const float* input;      // 16-byte aligned rows
    float* output;
    __bf16* parts;           // the exact 3-part bf16 split of the input in MFMA fragment order (scratch)
    int32_t total_tiles;     // row tiles over all segments
    int32_t slices;          // decode: column slices (projection_decode_slices)
    float* partials;         // decode: [slices][16][partial_stride] per-slice sums (scratch)
    int64_t partial_stride;  // total_tiles * 16
    uint32_t encoding;       // GGML type of every segment: 8 (Q8_0), 12 (Q4_K) or 14 (Q6_K); decode launches also
                             // take kEncodingMixedK: K-quant segments of both types (each segment's own field)
    int32_t pad;
    float* sums;             // prompt runs of Q4_K: [tokens][padded_columns / 8] sums of 8 inputs (scratch)
    NormInput norm;          // decode: normalize the input rows while staging (norm.weight non-null)
    float* squares;          // decode with reduce: also write the output rows' partial sums of squares (NormInput)
};

// KV page activation (ADR-016). Key summaries live in their own buffer, one summary page per pool page:
// [layer][kv_head][activation page of the pool page][min, max][head_dim] in the storage type (exact minima and
// maxima of the stored keys). An activation page is summary_keys (16, 32 or 64) consecutive positions.
inline uint64_t summary_page_elements(int layers, int kv_heads, int page_tokens, int head_dim, int summary_keys) {
    return static_cast<uint64_t>(layers) * kv_heads * (page_tokens / summary_keys) * 2 * head_dim;
}

// Recomputes the summaries of `count` (pool page, activation page of the pool page, keys 1..summary_keys) items for
// layers
// [first_layer, first_layer + layers) and every KV head from the block's first `keys` stored keys.
struct SummaryArgs {
    Geometry geo;  // geo.layer unused
    uint8_t* summaries;
    uint64_t summary_page_bytes;
    const int32_t* blocks;  // (page, block, keys) triples
    int32_t count;
    int32_t first_layer;
    int32_t layers;
    int32_t pad;
};

// One key-bound selection: the row (token, kv_head) ranks activation pages 1..candidates of its slot and writes the
// first keys of the `budget` best (ascending) to lists[list + 1 ..] (lists[list] is the sink page, the window pages
// follow the budget). The per-job merge holds up to 128 tiles' kept keys in LDS: 8,192 candidates (131,072
// positions with 16-position pages, 524,288 with 64).
constexpr int kMaxSelectCandidates = 8192;
struct SelectJob {
    int32_t token;
    int32_t kv_head;
    int32_t list;
    int32_t candidates;
};
static_assert(sizeof(SelectJob) == 16, "SelectJob is 16 bytes");

struct SelectArgs {
    Geometry geo;
    const SynapseKvBatchToken* tokens;
    const float* qkv;
    int32_t qkv_stride;
    int32_t rotate;  // 1: Q in qkv is unrotated (append_attention); the bound uses the rotated query
    const float* cosines;
    const float* sines;
    const uint8_t* summaries;
    uint64_t summary_page_bytes;
    const SelectJob* jobs;
    int32_t* lists;
    uint64_t* keys;      // [jobs][key_stride]: each tile's best min(budget, 64) rank keys, merged per job
    int32_t key_stride;  // tiles of the largest job * min(budget, 64)
    int32_t budget;
    int32_t job_count;
    // Summary work riding along (workgroups y < summary_count, x < kv_heads; the jobs follow): (page, block, keys)
    // triples of this layer whose summaries no job of the launch reads.
    uint8_t* summary_out;
    const int32_t* summary_blocks;
    int32_t summary_count;
    int32_t pad;
};

// Page regions are stored in MFMA-fragment order; see page_layout.h.

// Where a kernel goes: the cache's stream, and (when profiling) the events its dispatch records at start and end.
struct Launch {
    hipStream_t stream;
    hipEvent_t start;
    hipEvent_t stop;
};

// Dispatches `kernel` for `launch` (hipExtLaunchKernelGGL records the events around the dispatch itself).
#define SYNAPSE_KV_LAUNCH(kernel, grid, block, launch, ...)                                                       \
    hipExtLaunchKernelGGL(kernel, grid, block, 0, (launch).stream, (launch).start, (launch).stop, 0, __VA_ARGS__)
// The same with `shared` bytes of dynamic LDS.
#define SYNAPSE_KV_LAUNCH_SHARED(kernel, grid, block, shared, launch, ...)                                        \
    hipExtLaunchKernelGGL(kernel, grid, block, shared, (launch).stream, (launch).start, (launch).stop, 0, __VA_ARGS__)

// Launchers (each enqueues at most one kernel and returns the launch status).
// Copies `bytes` from coherent pinned host memory, addressed through its device view, to device memory on `stream`
// (a copy kernel, in place of hipMemcpyAsync for per-step uploads). Both addresses must be 16-byte aligned (the
// kernel moves 16-byte vectors); otherwise nothing is launched and the result is hipErrorInvalidValue.
hipError_t launch_upload(const void* source, void* target, size_t bytes, hipStream_t stream);
hipError_t launch_table(const Launch& launch, const TableArgs& args);
hipError_t launch_zero_pages(const Launch& launch, const PageArgs& args);
hipError_t launch_copy_pages(const Launch& launch, const PageArgs& args);
hipError_t launch_append(const Launch& launch, const AppendArgs& args, int tokens, bool fp16);
hipError_t launch_decode(const Launch& launch, const AttentionArgs& args, bool fp16, bool prefetch);
// Merges [first, first + count); `wide` items (more than kMergeRows partial rows) take a workgroup each.
hipError_t launch_merge(const Launch& launch, const AttentionArgs& args, int first, int count, bool wide);
// Waves of the decode kernel that are resident at once on `device` (the persistent worker count).
int decode_resident_waves(int device, bool fp16, int head_dim, bool prefetch);
// Prefill workgroups resident on the whole device at once (occupancy of the group's kernel times the CU count).
int prefill_resident_blocks(int device, int head_dim, int group);
// Prefill items [first, first + items) with `tiles` (1 or kPrefillTiles) column tiles of 16 tokens per wave.
hipError_t launch_prefill(const Launch& launch, const AttentionArgs& args, int first, int items, int tiles, bool fp16);
hipError_t launch_gather(const Launch& launch, const GatherArgs& args, bool fp16);
hipError_t launch_scatter(const Launch& launch, const GatherArgs& args, bool fp16);
hipError_t launch_summaries(const Launch& launch, const SummaryArgs& args, bool fp16);
// Key-bound selection (the largest job has `most_candidates` candidates), with args.summary_count summary items.
hipError_t launch_select(const Launch& launch, const SelectArgs& args, int most_candidates, bool fp16);
// A projection over `tiles` row tiles (all segments).
// `reduce` false (decode launches only): the slice sums stay in args.partials for the caller to add.
// `split`: prompt runs split the FP32 input first (split_kernel); false when args.parts already holds the split.
hipError_t launch_projection(const Launch& launch, const ProjectionArgs& args, int tiles, bool reduce = true,
                             bool split = true);
// Column slices of a decode projection (tokens <= 16) over `chunks` 64-column chunks.
int projection_decode_slices(int chunks);

// Read of a wave-uniform address in memory that no wave writes during the launch (block tables, step lists),
// through the constant address space: the compiler issues a scalar load, counted by lgkmcnt apart from the vector
// loads in flight. As a vector load it would complete in order behind every K/V fragment requested before it, and
// its use would wait for all of them (vmcnt 0), emptying the prefetch.
template <typename T>
__device__ inline T load_uniform(const T* pointer) {
    static_assert(sizeof(T) % 4 == 0, "read in 4-byte words");
    struct Words {
        uint32_t word[sizeof(T) / 4];
    } words;
    const auto* source = (const __attribute__((address_space(4))) uint32_t*)pointer;
#pragma unroll
    for (size_t i = 0; i < sizeof(T) / 4; ++i) {
        words.word[i] = source[i];
    }
    return __builtin_bit_cast(T, words);
}

// s_waitcnt vmcnt(N) with the other counters left alone (expcnt 7, lgkmcnt 15; vmcnt split over bits 3:0 and
// 15:14).
template <int N>
__device__ inline void wait_vector_memory() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

// Workgroup barrier after this wave's LDS reads and all but its newest N vector-memory operations (LDS copies)
// have completed. __syncthreads would also wait for every outstanding copy (its workgroup fence waits for
// vmcnt 0); the compiler-level memory clobbers keep LDS accesses on their side of the barrier.
template <int N>
__device__ inline void barrier_after_copies() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Query rows (tokens) per prefill work item: 16 per MFMA column tile, kPrefillTiles tiles per wave.
constexpr int kPrefillTiles = 2;
constexpr int kPrefillTokens = 16 * kPrefillTiles;
// Keys per decode/prefill inner step.
constexpr int kStepKeys = 64;
// Fewest keys per prefill work item when the split is chosen automatically.
constexpr int kMinPrefillChunk = 1024;
// Decode steps per worker that one merge launch is worth (the planner adds up to this many to avoid a second).
constexpr int kMergeSteps = 4;
// Most partial rows that merge_kernel combines with one wave (two rounds of 64 loads), and that merge_wide_kernel
// combines with a workgroup of kWideWaves such waves; rows of more pieces take two merge launches.
constexpr int kMergeRows = 128;
constexpr int kWideWaves = 8;
constexpr int kWideMergeRows = kMergeRows * kWideWaves;
// Fewest 64-key steps per listed (shared-prefix) prefill item.
constexpr int kMinSharedSteps = 4;

// A decode projection (at most 16 tokens, one encoding, no biases) whose slice sums are left for the caller:
// output[t][row of segment s] would be sum over slices, in order, of partials[(slice * 16 + t) * stride +
// first_row[s] + row] (plus 0.0f), added to the output when accumulating. Other projections run whole and return
// `deferred` false. The sums live in the weights' scratch until the next projection on its stream.
struct DeferredSums {
    const float* partials = nullptr;
    int64_t stride = 0;
    int32_t slices = 0;
    int32_t first_row[3] = {0, 0, 0};
    bool deferred = false;
};

// The prompt GEMM's split input: each input value x = hi + mid + lo in three bf16 parts (each rounded to nearest;
// the residuals are exact in FP32 and lo holds the last, at most 8, significant bits), stored in the MFMA's
// B-fragment order [token tile][chunk][part][block][lane][8] with lane = 16 g + t holding columns 8 g .. 8 g + 7
// of a 32-column block for token 16 tile + t, so every fragment load is one contiguous 1 KiB wave load. Columns
// past the input up to the last 64-column chunk hold zeros. For Q4_K matrices the sums of 8 inputs follow:
// [token][chunks * 8]. split_kernel writes it from an FP32 input; kernels that produce a projection's input can
// write it directly (store_split_group).
struct SplitInput {
    __bf16* parts = nullptr;
    float* sums = nullptr;  // null when no matrix of the projection needs them
    int32_t chunks = 0;     // 64-column chunks of the input
};

typedef __bf16 split_bf16x8 __attribute__((ext_vector_type(8)));

__device__ inline void split3(float x, __bf16& hi, __bf16& mid, __bf16& lo) {
#pragma clang fp contract(off)
    hi = static_cast<__bf16>(x);
    const float first = x - static_cast<float>(hi);
    mid = static_cast<__bf16>(first);
    lo = static_cast<__bf16>(first - static_cast<float>(mid));
}

// Element offset of part `part` of (token, column) in SplitInput::parts.
__device__ inline size_t split_part_offset(int chunks, int token, int column, int part) {
    const int tile = token / 16;
    const int t = token % 16;
    const int chunk = column / kQ8ChunkColumns;
    const int block = (column % kQ8ChunkColumns) / kQ8BlockElements;
    const int g = (column % kQ8BlockElements) / 8;
    return ((((static_cast<size_t>(tile) * chunks + chunk) * 3 + part) * 2 + block) * 64 + 16 * g + t) * 8 +
           column % 8;
}

// Writes the parts of input[token][column .. column + 7] (column a multiple of 8) and, when the split has sums,
// their sum in column order.
__device__ inline void store_split_group(const SplitInput& split, int token, int column, const float (&values)[8]) {
    split_bf16x8 parts[3];
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
    for (int p = 0; p < 3; ++p) {
        *reinterpret_cast<split_bf16x8*>(split.parts + split_part_offset(split.chunks, token, column, p)) = parts[p];
    }
    if (split.sums != nullptr) {
        float sum = values[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) {
            sum += values[i];
        }
        split.sums[static_cast<size_t>(token) * split.chunks * 8 + column / 8] = sum;
    }
}

// The (token, 8-column group) a thread of a split writer handles: thread = ((tile * chunks + chunk) * 2 + block) *
// 64 + 16 g + t, so each part's stores are contiguous 1 KiB runs. Threads run over (tokens rounded up to 16) x
// chunks x 64 columns / 8; false for a token past the last.
__device__ inline bool split_thread(int index, int chunks, int tokens, int& token, int& column) {
    const int lane = index & 63;
    const int block = (index >> 6) & 1;
    const int tile_chunk = index >> 7;
    const int chunk = tile_chunk % chunks;
    token = (tile_chunk / chunks) * 16 + (lane & 15);
    column = chunk * kQ8ChunkColumns + block * kQ8BlockElements + 8 * (lane >> 4);
    return token < tokens;
}

}  // namespace synapse_kv

struct SynapseKvWeights;

namespace synapse_kv {
// SYNAPSE_KV_OPTION_FUSED_SUMS of a cache (the decoder built on it reads it per step).
bool cache_fused_sums(const SynapseKvCache& cache);
DeferredSums project_deferred(SynapseKvWeights& weights, const SynapseKvProjection& p, const float* input,
                              float* output);
// Decode projections (at most 16 tokens) around the decoder's RMS norms. project_normalized projects the rows of
// `input` normalized per `norm` (the norm kernel's launch folded into the projection's staging);
// project_with_squares adds the projection into `output` (accumulate) and writes, per token, the partial sums of
// squares of the output row that a later project_normalized reads (one segment, no other output columns).
void project_normalized(SynapseKvWeights& weights, const SynapseKvProjection& p, const float* input, float* output,
                        const NormInput& norm);
void project_with_squares(SynapseKvWeights& weights, const SynapseKvProjection& p, const float* input, float* output,
                          float* squares);
// Partial sums of squares of `tokens` rows of `columns` floats (row stride `columns`) into squares.
hipError_t launch_row_squares(hipStream_t stream, const float* rows, int columns, int tokens, float* squares);
// A prompt run (more than 16 tokens) whose input the caller writes already split: prepare_split returns the
// weights' scratch sized for the projection (sums included when a matrix is Q4_K), valid until the next projection
// on the weights' stream; project_split runs the projection from it. Work queued on the weights' stream may be
// drained when the scratch grows.
SplitInput prepare_split(SynapseKvWeights& weights, const SynapseKvProjection& p);
void project_split(SynapseKvWeights& weights, const SynapseKvProjection& p, const SplitInput& split, float* output);
}  // namespace synapse_kv
