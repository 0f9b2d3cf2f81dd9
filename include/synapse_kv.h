/*
 * libsynapse_kv: the KV-cache and attention hot path of Synapse's decoder step on AMD Instinct MI355X (gfx950).
 *
 * A versioned C ABI with the conventions of Synapse's GPU library (native/synapse-gpu/src/Features/GpuKernels/
 * ffi.rs:1-263): every entry point validates its pointers, catches C++ exceptions, returns a status code and
 * records a thread-local message that synapse_kv_last_error copies out. A cache handle must not be used by two
 * threads at once (ffi.rs:177-180).
 *
 * Ownership: the caller owns the RoPE tables (copied to the device at create, as DecoderDesc.rope_cosines/sines,
 * decoder.rs:102-103), the token array and every qkv/output buffer. The cache owns its device page pool, block
 * tables, reference counts and free stack. qkv and output pointers are device pointers (HIP-resident step);
 * host-side arrays are passed only where noted. All device work is ordered on the cache's stream.
 *
 * Every struct below has its size pinned with a static assertion here and in the C# binding.
 */
#ifndef SYNAPSE_KV_H
#define SYNAPSE_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI version checked by the loader before any other call (ffi.rs:12 ABI_VERSION; NativeGpuLibrary.cs:14). */
#define SYNAPSE_KV_ABI_VERSION 4u

/* Status codes, identical to error.rs:4-16. */
#define SYNAPSE_KV_OK 0
#define SYNAPSE_KV_NULL_POINTER 1
#define SYNAPSE_KV_INVALID_ARGUMENT 2
#define SYNAPSE_KV_UNAVAILABLE 3
#define SYNAPSE_KV_DEVICE_ERROR 4
#define SYNAPSE_KV_OUT_OF_MEMORY 5
#define SYNAPSE_KV_PANIC 6

/* KV element types, values as KV_F32 / KV_F16 (decoder.rs:37-39). */
#define SYNAPSE_KV_F32 0u
#define SYNAPSE_KV_F16 1u

/* Tuning options for synapse_kv_set_option. */
#define SYNAPSE_KV_OPTION_SPLIT_KEYS 1u     /* fewest keys per decode wave worker; a multiple of 64 (default 64) */
#define SYNAPSE_KV_OPTION_PREFILL_RUNS 2u   /* 1: FP16 prompt runs use the MFMA prefill kernel (default); 0: decode path */
#define SYNAPSE_KV_OPTION_PREFILL_SPLIT_KEYS 3u /* keys per prefill split-K work item, a multiple of 64; 0 (default): fill the device */
#define SYNAPSE_KV_OPTION_DECODE_PREFETCH 4u /* 1: FP16 decode keeps the next step's loads in flight (two register sets) */
#define SYNAPSE_KV_OPTION_PROFILE_EVERY 5u   /* profile mode times every n-th launch of each kernel kind (default 1) */
#define SYNAPSE_KV_OPTION_SHARED_PREFIX 6u  /* 1 (default): FP16 decode reads pages shared by several step tokens once */
#define SYNAPSE_KV_OPTION_FUSED_SUMS 7u     /* decoder on this cache: 1 (default) adds the o_proj and gate/up slice sums
                                               inside the next RMS norm and SwiGLU (decode steps) and has the norms and
                                               SwiGLU write the next projection's split input (prompt steps); 0:
                                               separate reduce and split launches (same bits) */
#define SYNAPSE_KV_OPTION_SEGMENT_COST 8u   /* decode work split: what a row start in a worker's range costs, in quarter
                                               key steps (0..64, default 8); a key step costs 4 */
#define SYNAPSE_KV_OPTION_ADAPTIVE_SPLIT 9u /* 1: weight each decode worker's share of the steps by the measured speed of
                                               its XCD (worker durations of earlier steps); attention outputs then
                                               depend on timings in their last FP32 bits. 0 (default): equal shares,
                                               results repeat bit for bit */

/* GpuDeviceInfo (native/synapse-gpu/src/Features/GpuKernels/mod.rs:20-31), 152 bytes. */
typedef struct SynapseKvDeviceInfo {
    uint8_t name[128];
    uint64_t recommended_working_set_bytes;
    uint64_t max_buffer_bytes;
    uint32_t unified_memory;
    uint32_t apple_family;
} SynapseKvDeviceInfo;

/* BatchToken (decoder.rs:133-141), 16 bytes: the C# BatchToken array passes through unchanged. `slot` is the
 * sequence, `position` the KV position the token writes and attends up to (inclusive); token and logits_row are
 * carried but not read by this library. */
typedef struct SynapseKvBatchToken {
    int32_t slot;
    int32_t token;
    int32_t position;
    int32_t logits_row;
} SynapseKvBatchToken;

/* Cache description: the KV-relevant part of DecoderDesc (decoder.rs:95-128), 64 bytes.
 * layer_count counts executed layers only: dropped layers get no KV (ADR-019; Qwen2ModelComposition.cs:13-36).
 * page_tokens is a multiple of 64 in 64..1024; kv_growth_positions a positive multiple of page_tokens (the
 * reference requires a multiple of 64, decoder/checks.rs); max_pages sizes the device page pool. */
typedef struct SynapseKvDesc {
    const float* rope_cosines; /* host, [max_positions][head_dim / 2] */
    const float* rope_sines;   /* host, [max_positions][head_dim / 2] */
    uint32_t layer_count;
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t head_dim; /* 64 or 128 (METAL_HEAD_DIMS, decoder.rs:23) */
    uint32_t max_positions;
    uint32_t kv_growth_positions;
    uint32_t page_tokens;
    uint32_t kv_precision;
    uint32_t session_slots;
    uint32_t step_tokens;
    uint32_t max_pages;
    int32_t device;
} SynapseKvDesc;

/* Page pool occupancy, 40 bytes. */
typedef struct SynapseKvPageStats {
    uint32_t max_pages;
    uint32_t free_pages;
    uint32_t used_pages;
    uint32_t shared_pages; /* pages with a reference count above one */
    uint64_t page_bytes;
    uint64_t kv_bytes; /* used_pages * page_bytes */
    uint32_t device_status; /* 0, or the first inconsistency the table kernel found */
    uint32_t reserved;
} SynapseKvPageStats;

/* GPU time per kernel kind between synapse_kv_profile_begin and _end, 128 bytes. */
#define SYNAPSE_KV_KERNEL_TABLE 0   /* block-table operations */
#define SYNAPSE_KV_KERNEL_PAGES 1   /* page zero-fill and copy-on-write copies */
#define SYNAPSE_KV_KERNEL_APPEND 2  /* RoPE + KV append (and key summaries under KV page activation) */
#define SYNAPSE_KV_KERNEL_DECODE 3  /* split-K decode attention (with the fused append when used) */
#define SYNAPSE_KV_KERNEL_MERGE 4   /* split merge */
#define SYNAPSE_KV_KERNEL_PREFILL 5 /* prompt-run attention, and shared-prefix pages read once for their sharers */
#define SYNAPSE_KV_KERNEL_GATHER 6  /* KV read-back */
#define SYNAPSE_KV_KERNEL_PAGE_SELECT 7 /* KV page activation: key-bound page selection */
typedef struct SynapseKvProfile {
    uint64_t launches[8];
    double milliseconds[8];
} SynapseKvProfile;

typedef struct SynapseKvCache SynapseKvCache;

/* synapse_gpu_abi_version (ffi.rs:53-57). */
uint32_t synapse_kv_abi_version(void);

/* synapse_gpu_probe (ffi.rs:59-80) for the current HIP device. */
int32_t synapse_kv_probe(SynapseKvDeviceInfo* info);

/* synapse_gpu_last_error (ffi.rs:86-104): copies the calling thread's last message (UTF-8, not terminated) and
 * returns its full length. */
size_t synapse_kv_last_error(uint8_t* buffer, size_t capacity);

/* synapse_gpu_decoder_create (ffi.rs:106-142) for the KV path: validates the shape, copies the RoPE tables and
 * allocates the page pool. */
int32_t synapse_kv_cache_create(const SynapseKvDesc* desc, SynapseKvCache** cache);

/* synapse_gpu_decoder_destroy (ffi.rs:215-227); null is ignored. */
void synapse_kv_cache_destroy(SynapseKvCache* cache);

/* Orders all later device work of the cache on `stream` (a hipStream_t; null = the default stream). */
int32_t synapse_kv_set_stream(SynapseKvCache* cache, void* stream);

/* Tuning knobs (SYNAPSE_KV_OPTION_*). */
int32_t synapse_kv_set_option(SynapseKvCache* cache, uint32_t option, uint32_t value);

/* synapse_gpu_decoder_kv_bytes (ffi.rs:229-248): bytes of the pages in use, shared pages counted once;
 * 0 for null. */
uint64_t synapse_kv_bytes(const SynapseKvCache* cache);

/* synapse_gpu_decoder_reserve (ffi.rs:250-263) / MetalDecoder::reserve (metal/decoder.rs:164-179) with the
 * Qwen2KvCache.Reserve policy (Qwen2KvCache.cs:56-72): grow to the rounded need, or contract when the rounded
 * need is at most a quarter of the capacity; the prefix is kept. */
int32_t synapse_kv_reserve(SynapseKvCache* cache, uint32_t slot, uint32_t positions);

/* Qwen2KvCache.Release (Qwen2KvCache.cs:75-84) / Qwen2KvSlots.Release (Qwen2Vectors.cs:39-53) for one slot. */
int32_t synapse_kv_release(SynapseKvCache* cache, uint32_t slot);

/* Rollback to a shorter committed length (kv_pages.rs:158-177; DirectSessionPrefix.Claim forgetting,
 * DirectSessionPrefix.cs:16-27). Capacity is kept. */
int32_t synapse_kv_truncate(SynapseKvCache* cache, uint32_t slot, uint32_t length);

/* Prefix reuse across slots (ADR-018 extended to copy-on-write): the empty `target` shares every page that holds
 * `source`'s written positions. */
int32_t synapse_kv_fork(SynapseKvCache* cache, uint32_t source, uint32_t target);

/* Starts a step (MetalDecoder::forward's prepare_slots + plan_attention, metal/decoder.rs:106-156): validates
 * the tokens (validate_step, decoder.rs:303-335), grows slots and copies shared pages on write, and uploads the
 * tokens and the attention work plan. `tokens` is a host array. Appends are contiguous (PagedKvCache::append,
 * kv_pages.rs:98-100): per slot, the step's positions at or past the slot's length must fill [length, new length)
 * without a gap, else INVALID_ARGUMENT with nothing changed; positions below the length overwrite (rollback). */
int32_t synapse_kv_step(SynapseKvCache* cache, const SynapseKvBatchToken* tokens, size_t count);

/* synapse_kv_step with the step's prompt boundary (IBatchDecoder.Forward(tokens, promptStart),
 * BatchDecoding.cs:10-33): tokens from `prompt_start` on are prompt tokens and attend densely under KV page
 * activation. synapse_kv_step is this call with prompt_start = count. */
int32_t synapse_kv_step_prompt(SynapseKvCache* cache, const SynapseKvBatchToken* tokens, size_t count,
                               size_t prompt_start);

/* synapse_kv_step_prompt for callers that cannot allocate (tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference. The step's table operations, attention plan and attention
 * partial rows go to a static device array of SYNAPSE_KV_STATIC_SCRATCH_BYTES per GPU (held until the process
 * ends) instead of buffers the cache grows; the call makes no device or pinned-host allocation (its host planning
 * uses ordinary heap memory, as every step does) and uploads from pageable memory. The layer calls of the step
 * (append_rope, attention, append_attention) then read the scratch. A step that needs more scratch than there is
 * fails with INVALID_ARGUMENT and changes nothing; KV page activation is UNAVAILABLE here. Every cache on a GPU
 * shares that GPU's array, which keeps the last step's contents: from one cache's static step to the last layer
 * call of that step, no other static step may run on the same GPU (the two would race); calls of one cache on one
 * stream are ordered as usual. The call itself is not capturable into a HIP graph: it waits on host events for its
 * staging buffers and builds the plan on the host from the cache's state at call time. */
#define SYNAPSE_KV_STATIC_SCRATCH_BYTES (64u * 1024u * 1024u)
int32_t synapse_kv_step_static(SynapseKvCache* cache, const SynapseKvBatchToken* tokens, size_t count,
                               size_t prompt_start);

/* Query-aware KV page activation (ADR-016; KvPageActivation.cs, KvPageSelector.cs:17-54, Qwen2KvPageMasks.cs):
 * a decode unit (a token before the prompt boundary that is alone in its slot in the step) attends, per KV head,
 * to the sink page (positions 0..page_tokens-1), the pages overlapping its last window_tokens positions, and
 * budget_pages more pages: those with the highest bound max over the group's query heads of
 * sum_d max(q_d * min_d, q_d * max_d) over the page's per-channel key minimum and maximum (KEY_BOUND), or a seeded
 * random draw (RANDOM, the control; seed per (layer, KV head, position) as Qwen2KvPageMasks). Unselected pages
 * contribute nothing to that step's softmax. An approximation: off (enabled = 0) by default. Enabling (or changing
 * page_tokens while enabled) builds the per-page key summaries of everything already cached; later appends keep them
 * current. Key-bound selection ranks at most 8,192 candidate pages per row (UNAVAILABLE beyond). */
#define SYNAPSE_KV_SELECT_KEY_BOUND 0u
#define SYNAPSE_KV_SELECT_RANDOM 1u
typedef struct SynapseKvPageActivation {
    uint32_t enabled;       /* 0: dense attention (default) */
    uint32_t budget_pages;  /* BudgetPages */
    uint32_t window_tokens; /* WindowTokens */
    uint32_t page_tokens;   /* PageTokens: 16, 32 or 64 positions per activation page */
    uint32_t selection;     /* SYNAPSE_KV_SELECT_* */
    int32_t seed;           /* Seed of the random control */
} SynapseKvPageActivation;

int32_t synapse_kv_set_page_activation(SynapseKvCache* cache, const SynapseKvPageActivation* activation);

/* synapse_rope_kv[_f16] for one layer of the current step (elementwise.metal:73-126; dispatch step/layers.rs:
 * 111-148): `qkv` is a device [tokens][qkv_stride] FP32 block with Q at column 0, K at heads*head_dim and V at
 * (heads + kv_heads)*head_dim. Q and K rotate in place; K and V are appended to the pages (FP16: round to nearest
 * even). */
int32_t synapse_kv_append_rope(SynapseKvCache* cache, uint32_t layer, float* qkv, uint32_t qkv_stride);

/* Attention of the current step for one layer (step/attention.rs:9-145: synapse_attention for prompt runs,
 * synapse_attention_decode + synapse_attention_reduce for lone tokens): every token attends keys
 * 0..position of its slot. Reads Q from `qkv` (device), writes [tokens][out_stride] FP32 `output` (device)
 * at column head*head_dim. */
int32_t synapse_kv_attention(SynapseKvCache* cache, uint32_t layer, const float* qkv, uint32_t qkv_stride,
                             float* output, uint32_t out_stride);

/* synapse_kv_append_rope followed by synapse_kv_attention for one layer, as one decode launch when every token of
 * the step has its own slot (the decode wave that reads a token's own position rotates and stores its K/V first,
 * and every wave applies RoPE to Q in registers); otherwise the two launches run in order. `qkv` (device) is read
 * only: unlike synapse_kv_append_rope, the rotated Q and K are not written back (step/layers.rs:95-96 reads the
 * rotated rows only for this attention). */
int32_t synapse_kv_append_attention(SynapseKvCache* cache, uint32_t layer, const float* qkv, uint32_t qkv_stride,
                                    float* output, uint32_t out_stride);

/* Per-kernel GPU time, as SYNAPSE_GPU_PROFILE does for the Metal backend (metal/encoder.rs:161-182): between
 * _begin and _end every launch of the cache records HIP events around its own dispatch on the cache's stream;
 * _end waits for the stream and returns launch counts and summed milliseconds per SYNAPSE_KV_KERNEL_* kind.
 * With SYNAPSE_KV_OPTION_PROFILE_EVERY = n only every n-th launch of a kind is timed and counted (each timed
 * dispatch costs a few microseconds of queue time). */
int32_t synapse_kv_profile_begin(SynapseKvCache* cache);
int32_t synapse_kv_profile_end(SynapseKvCache* cache, SynapseKvProfile* profile);

/* Waits for the cache's stream. */
int32_t synapse_kv_synchronize(SynapseKvCache* cache);

/* Host-side view of a slot: capacity (positions), written length and mapped pages. */
int32_t synapse_kv_slot_info(const SynapseKvCache* cache, uint32_t slot, uint32_t* capacity, uint32_t* length,
                             uint32_t* pages);

/* Device state read-back for bit-exact checks (synchronous; host output arrays). */
int32_t synapse_kv_read_block_table(SynapseKvCache* cache, uint32_t slot, int32_t* pages, size_t capacity,
                                    size_t* count);
int32_t synapse_kv_read_refcounts(SynapseKvCache* cache, int32_t* counts, size_t capacity);
int32_t synapse_kv_read_free_list(SynapseKvCache* cache, int32_t* pages, size_t capacity, size_t* count);
int32_t synapse_kv_page_stats(SynapseKvCache* cache, SynapseKvPageStats* stats);

/* Copies positions [first, first + count) of one slot and layer into host arrays as [position][kv_head][head_dim]
 * in the storage type (float or uint16 FP16 bits): GetKey/GetValue (Qwen2KvCache.cs:86-88) in bulk. */
int32_t synapse_kv_read_kv(SynapseKvCache* cache, uint32_t slot, uint32_t layer, uint32_t first, uint32_t count,
                           void* keys, void* values);

/* ---- Persistent prefix payloads (the persistent prefix cache planned as ADR-018's next step) ----
 * A slot's first `length` positions serialized for a prefix cache outside the process: payloads keyed by model,
 * tokenizer, RoPE, KV type and prefix hash (ADR-018-prompt-prefix-reuse.md:42-44). The library writes and checks
 * the payload; where it is stored (the reference plans ZoneTree metadata and files on disk) is the caller's.
 *
 * Format, little-endian: a 128-byte SynapseKvPrefixHeader, then per layer the K rows and then the V rows of
 * positions 0..length-1, each [length][kv_heads][head_dim] in the storage type (FP16 or FP32; K already rotated).
 * payload_bytes counts those rows. checksum covers the header (its checksum field zero) and the rows, read as
 * little-endian 64-bit words with the tail zero-padded: h = 0xcbf29ce484222325; per word w,
 * h = rotl64(h ^ mix(w), 23) * 0x100000001b3; finally checksum = mix(h ^ total bytes), mix being the splitmix64
 * finalizer (z ^= z >> 30; z *= 0xbf58476d1ce4e5b9; z ^= z >> 27; z *= 0x94d049bb133111eb; z ^= z >> 31).
 * Importing into an empty slot reproduces the K/V bytes exactly, so attention over the imported prefix equals
 * attention over the original; a failed import leaves the slot empty. */
typedef struct SynapseKvPrefixKey {
    uint64_t model;     /* caller's hash of the model file / weights */
    uint64_t tokenizer; /* caller's hash of the tokenizer */
    uint64_t rope;      /* caller's hash of the RoPE parameters (theta, scaling) */
    uint64_t prefix;    /* synapse_kv_prefix_hash of the prefix's token ids */
} SynapseKvPrefixKey;

#define SYNAPSE_KV_PREFIX_MAGIC "SYNKVPX1"
#define SYNAPSE_KV_PREFIX_VERSION 2u

typedef struct SynapseKvPrefixHeader {
    char magic[8];           /* SYNAPSE_KV_PREFIX_MAGIC, not terminated */
    uint32_t version;        /* SYNAPSE_KV_PREFIX_VERSION */
    uint32_t header_bytes;   /* 128 */
    SynapseKvPrefixKey key;  /* the KV type and shape are checked from the fields below */
    uint32_t kv_precision;   /* SYNAPSE_KV_F32 or SYNAPSE_KV_F16 */
    uint32_t layer_count;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t length;         /* positions stored */
    uint32_t reserved0;      /* 0 */
    uint64_t payload_bytes;  /* 2 * layer_count * length * kv_heads * head_dim * element bytes */
    uint64_t checksum;       /* of the header (this field zero) and the rows, as above */
    uint8_t reserved[40];    /* 0 */
} SynapseKvPrefixHeader;

/* FNV-1a 64 (offset basis 0xcbf29ce484222325, prime 0x100000001b3) of `count` bytes: the prefix hash of a token
 * list is this over its int32 ids in little-endian order. */
uint64_t synapse_kv_prefix_hash(const uint8_t* bytes, size_t count);

/* Writes slot `slot`'s positions 0..length-1 (length at most the slot's written length) as a payload keyed by
 * `key` into `payload` (`capacity` bytes) and stores its size in `*bytes`. A null `payload` only reports the
 * size. Synchronizes the cache's stream. */
int32_t synapse_kv_export_prefix(SynapseKvCache* cache, uint32_t slot, uint32_t length, const SynapseKvPrefixKey* key,
                                 uint8_t* payload, uint64_t capacity, uint64_t* bytes);

/* Loads a payload into the empty slot `slot`: checks the magic, version, sizes, checksum, the cache's KV type and
 * shape, and that the payload's key equals `key` (status 2 otherwise, the slot untouched); reserves the slot with
 * the capacity policy, writes the K/V rows and sets the written length, stored in `*length`. Key summaries of
 * KV page activation are recomputed for the imported blocks. */
int32_t synapse_kv_import_prefix(SynapseKvCache* cache, uint32_t slot, const SynapseKvPrefixKey* key,
                                 const uint8_t* payload, uint64_t bytes, uint32_t* length);

/* RopeFrequencies (RopeFrequencies.cs:20-81) into host [positions][head_dim / 2] tables; yarn_factor <= 0 means
 * unscaled. The C# host builds the same tables itself (GpuDecoderExecutor.BuildRopeTables,
 * GpuDecoderExecutor.cs:183-192). */
int32_t synapse_kv_rope_table(uint32_t head_dim, float theta, float yarn_factor, uint32_t yarn_original,
                              uint32_t positions, float* cosines, float* sines);

/* ---- Q8_0 projections: the QKV and o_proj matrices that feed and consume the attention path ----
 * synapse_q8_matvec_{1,2,4,8} and synapse_q8_gemm (cuda/kernels/matmul.cu:1-189, metal/shaders/matmul.metal:1-310;
 * host step/projection.rs:1-141). Weights are GGML Q8_0 rows (34-byte blocks: FP16 scale d, then 32 int8 codes;
 * element = d * code) at byte offsets of a host blob (the mapped model file, GpuLayoutMapping.cs:14-32), with
 * optional FP32 biases. Activations and results are FP32 and every product accumulates in FP32 (ADR-012). */

/* No bias for a matrix (SYNAPSE_NO_BIAS, common.metal:11). */
#define SYNAPSE_KV_NO_BIAS UINT64_MAX

/* One matrix of the blob (the weight/bias/rows fields of matmul_segment, common.metal:54-59). */
typedef struct SynapseKvMatrix {
    uint64_t weight;  /* byte offset of rows x (columns / 32) Q8_0 blocks, row-major */
    uint64_t bias;    /* byte offset of `rows` FP32 biases, or SYNAPSE_KV_NO_BIAS */
    uint32_t rows;    /* positive */
    uint32_t columns; /* a positive multiple of 32 */
} SynapseKvMatrix;

typedef struct SynapseKvWeights SynapseKvWeights;

/* Uploads `count` matrices of a host blob to the current HIP device in the kernels' layout: 16-row x 64-column
 * tiles of codes in MFMA fragment order with their FP16 scales beside them, padded with zero codes (the weight
 * upload of synapse_gpu_decoder_create, ffi.rs:106-142, for the projection matrices). The blob is not kept. */
int32_t synapse_kv_weights_create(const uint8_t* blob, uint64_t blob_bytes, const SynapseKvMatrix* matrices,
                                  uint32_t count, SynapseKvWeights** weights);

/* The same for matrices in other GGML encodings (ADR-021; decoder/encoding.rs:5-73): encodings[i] is matrix i's
 * GGML type id, SYNAPSE_KV_ENCODING_Q8_0 (8), SYNAPSE_KV_ENCODING_Q4_K (12; 144-byte super-blocks of 256 values) or
 * SYNAPSE_KV_ENCODING_Q6_K (14; 210 bytes per 256 values); null means all Q8_0. K-quant matrices need columns that
 * are a multiple of 256 and keep 4-bit (Q4_K) or 8-bit (Q6_K) codes on the device with FP32 per-block factors;
 * other ids are SYNAPSE_KV_UNAVAILABLE. The segments of one projection may mix encodings. */
int32_t synapse_kv_weights_create_encoded(const uint8_t* blob, uint64_t blob_bytes, const SynapseKvMatrix* matrices,
                                          const uint32_t* encodings, uint32_t count, SynapseKvWeights** weights);

/* Null is ignored. */
void synapse_kv_weights_destroy(SynapseKvWeights* weights);

/* Device bytes held by the weights; 0 for null. */
uint64_t synapse_kv_weights_bytes(const SynapseKvWeights* weights);

/* Orders the projections on `stream` (a hipStream_t; null = the default stream). */
int32_t synapse_kv_weights_set_stream(SynapseKvWeights* weights, void* stream);

/* One projection (matmul_args, common.metal:61-71): the rows of up to three matrices with equal column counts,
 * in order (e.g. Q, K and V), matrix s written to output columns out_column[s] + row:
 *   output[t][out_column[s] + row] = (accumulate ? output[t][...] : 0) + sum_k W_s[row][k] * input[t][k] + bias_s[row]
 * for tokens t < tokens (accumulate adds the residual, as o_proj does, step/layers.rs:96-108). */
typedef struct SynapseKvProjection {
    uint32_t matrix[3];     /* matrix indices of synapse_kv_weights_create */
    uint32_t out_column[3]; /* first output column of each matrix's rows */
    uint32_t segments;      /* 1..3 */
    uint32_t tokens;        /* positive */
    uint32_t in_stride;     /* floats between input rows, at least columns */
    uint32_t out_stride;    /* floats between output rows */
    uint32_t accumulate;    /* 0 or 1 */
    uint32_t reserved;      /* 0 */
} SynapseKvProjection;

/* Runs a projection on the weights' stream (project() in step/projection.rs:51-72: up to 16 tokens take the
 * decode kernels, longer runs the tiled GEMM); input and output are device pointers and must not overlap. The
 * weights keep a scratch buffer for the call (per-slice sums or the split input), grown on demand. */
int32_t synapse_kv_project(SynapseKvWeights* weights, const SynapseKvProjection* projection, const float* input,
                           float* output);

/* Copies matrix `index` back in GGML Q8_0 block order (rows x columns / 32 blocks of 34 bytes) into host memory of
 * at least that many bytes (read-back for checks); K-quant matrices are SYNAPSE_KV_UNAVAILABLE. */
int32_t synapse_kv_weights_read(SynapseKvWeights* weights, uint32_t index, uint8_t* blocks, uint64_t bytes);

/* ---- The dense decoder step (libsynapse_gpu's model API, ffi.rs:106-271; decoder.rs:60-136) ----
 * A pre-norm decoder over caller-owned mapped weights: per layer RMS norm, Q/K/V projections with optional
 * biases, NeoX RoPE + KV append, grouped-query attention, the output projection added to the residual, RMS norm,
 * gate and up projections, SwiGLU, the down projection added to the residual; then the output norm and the logits
 * projection for the step's logits rows (step.rs:137-185, step/layers.rs). Built from the handles above: one KV
 * cache and one weights handle, on one stream. */

#define SYNAPSE_KV_NO_TENSOR 0xFFFFFFFFFFFFFFFFull /* NO_TENSOR: an optional tensor the model does not have */
#define SYNAPSE_KV_ENCODING_Q8_0 8u               /* GGML type IDs (ADR-021, decoder/encoding.rs:5-10) */
#define SYNAPSE_KV_ENCODING_Q4_K 12u
#define SYNAPSE_KV_ENCODING_Q6_K 14u
#define SYNAPSE_KV_ALL_Q8_0 0x08888888ull         /* DecoderLayerOffsets.encodings with every matrix in Q8_0 */
#define SYNAPSE_KV_ROPE_NEOX 0u
#define SYNAPSE_KV_ACTIVATION_SWIGLU 0u

/* DecoderLayerOffsets (decoder.rs:60-81): byte offsets of one block's tensors in the mapped weights. Norm weights
 * and biases are FP32; matrices are GGML blocks in the encoding packed four bits per matrix (Q, K, V, O, gate, up,
 * down from the lowest) in `encodings`. */
typedef struct SynapseKvLayerOffsets {
    uint64_t attention_norm;
    uint64_t query;
    uint64_t key;
    uint64_t value;
    uint64_t query_bias;        /* or SYNAPSE_KV_NO_TENSOR */
    uint64_t key_bias;          /* or SYNAPSE_KV_NO_TENSOR */
    uint64_t value_bias;        /* or SYNAPSE_KV_NO_TENSOR */
    uint64_t query_norm;        /* SYNAPSE_KV_NO_TENSOR (per-head Q/K norms are UNAVAILABLE, as in the reference) */
    uint64_t key_norm;          /* SYNAPSE_KV_NO_TENSOR */
    uint64_t attention_output;
    uint64_t feed_forward_norm;
    uint64_t gate;
    uint64_t up;
    uint64_t down;
    uint64_t encodings;
} SynapseKvLayerOffsets;

/* DecoderDesc (decoder.rs:85-116): pointers stay owned by the caller while the model lives. */
typedef struct SynapseKvDecoderDesc {
    const uint8_t* weights;
    uint64_t weights_length;
    const SynapseKvLayerOffsets* layers;
    const float* rope_cosines;  /* [context][head_dim / 2] */
    const float* rope_sines;
    uint64_t token_embedding;   /* vocabulary x hidden matrix */
    uint64_t output_norm;       /* FP32 [hidden] */
    uint64_t output;            /* vocabulary x hidden matrix */
    uint32_t layer_count;
    uint32_t hidden;            /* heads * head_dim */
    uint32_t feed_forward;
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t head_dim;          /* 64 or 128 */
    uint32_t vocabulary;
    uint32_t context;
    uint32_t session_slots;
    uint32_t step_tokens;
    uint32_t logits_rows;
    float rms_epsilon;
    uint32_t embedding_encoding;
    uint32_t rope_layout;       /* SYNAPSE_KV_ROPE_NEOX */
    uint32_t activation;        /* SYNAPSE_KV_ACTIVATION_SWIGLU */
    uint32_t kv_precision;      /* SYNAPSE_KV_F32 or SYNAPSE_KV_F16 */
    uint32_t kv_growth_positions;
    uint32_t output_encoding;
} SynapseKvDecoderDesc;

typedef struct SynapseKvDecoder SynapseKvDecoder;

/* synapse_gpu_decoder_create (ffi.rs:106-137) with DecoderPlan::new's validation (decoder/checks.rs): status 2
 * for inconsistent shapes and out-of-range or misaligned tensors, 3 for what the kernels do not implement
 * (encodings other than Q8_0, Q4_K and Q6_K, K-quant matrices whose columns are not whole 256-value super-blocks,
 * RoPE layouts other than NeoX, activations other than SwiGLU, per-head Q/K norms,
 * head dimensions other than 64 and 128, more than 8 query heads per KV head). Uploads the matrices (repacked), the
 * norms, biases and the embedding table to device memory on `device`; the KV page pool takes the pages every slot
 * needs at full context, or what fits in free device memory. */
int32_t synapse_kv_decoder_create(const SynapseKvDecoderDesc* desc, int32_t device, SynapseKvDecoder** model);

/* synapse_gpu_decoder_forward (ffi.rs:172-211): one batched step of `count` tokens; the tokens' logits rows must
 * be 0..k-1 in token order (BatchDecoding.cs:24-27) with k <= logits_rows, and `logits` (host memory) receives
 * k * vocabulary floats. Returns after the logits are copied. */
int32_t synapse_kv_decoder_forward(SynapseKvDecoder* model, const SynapseKvBatchToken* tokens, size_t count,
                                   float* logits, size_t logits_capacity);

/* synapse_kv_decoder_forward with the step's prompt boundary (IBatchDecoder.Forward(tokens, promptStart)), which
 * KV page activation uses; synapse_kv_decoder_forward passes prompt_start = count. */
int32_t synapse_kv_decoder_forward_prompt(SynapseKvDecoder* model, const SynapseKvBatchToken* tokens, size_t count,
                                          size_t prompt_start, float* logits, size_t logits_capacity);

/* synapse_gpu_decoder_destroy / _kv_bytes / _reserve (ffi.rs:213-271). */
void synapse_kv_decoder_destroy(SynapseKvDecoder* model);
uint64_t synapse_kv_decoder_kv_bytes(const SynapseKvDecoder* model);
int32_t synapse_kv_decoder_reserve(SynapseKvDecoder* model, uint32_t slot, uint32_t positions);

/* The model's KV cache and stream: options, KV page activation, fork/truncate/release and the read-backs work on
 * the returned cache (owned by the model). */
int32_t synapse_kv_decoder_cache(SynapseKvDecoder* model, SynapseKvCache** cache);
int32_t synapse_kv_decoder_set_stream(SynapseKvDecoder* model, void* stream);

#ifdef __cplusplus
} /* extern "C" */

static_assert(sizeof(SynapseKvDeviceInfo) == 152, "SynapseKvDeviceInfo is pinned at 152 bytes");
static_assert(sizeof(SynapseKvBatchToken) == 16, "SynapseKvBatchToken is pinned at 16 bytes");
static_assert(sizeof(SynapseKvDesc) == 64, "SynapseKvDesc is pinned at 64 bytes");
static_assert(sizeof(SynapseKvPageStats) == 40, "SynapseKvPageStats is pinned at 40 bytes");
static_assert(sizeof(SynapseKvProfile) == 128, "SynapseKvProfile is pinned at 128 bytes");
static_assert(sizeof(SynapseKvMatrix) == 24, "SynapseKvMatrix is pinned at 24 bytes");
static_assert(sizeof(SynapseKvPageActivation) == 24, "SynapseKvPageActivation is pinned at 24 bytes");
static_assert(sizeof(SynapseKvProjection) == 48, "SynapseKvProjection is pinned at 48 bytes");
static_assert(sizeof(SynapseKvLayerOffsets) == 120, "SynapseKvLayerOffsets is pinned at 120 bytes");
static_assert(sizeof(SynapseKvDecoderDesc) == 136, "SynapseKvDecoderDesc is pinned at 136 bytes");
static_assert(sizeof(SynapseKvPrefixKey) == 32, "SynapseKvPrefixKey is pinned at 32 bytes");
static_assert(sizeof(SynapseKvPrefixHeader) == 128, "SynapseKvPrefixHeader is pinned at 128 bytes");
#else
_Static_assert(sizeof(SynapseKvDeviceInfo) == 152, "SynapseKvDeviceInfo is pinned at 152 bytes");
_Static_assert(sizeof(SynapseKvBatchToken) == 16, "SynapseKvBatchToken is pinned at 16 bytes");
_Static_assert(sizeof(SynapseKvDesc) == 64, "SynapseKvDesc is pinned at 64 bytes");
_Static_assert(sizeof(SynapseKvPageStats) == 40, "SynapseKvPageStats is pinned at 40 bytes");
_Static_assert(sizeof(SynapseKvProfile) == 128, "SynapseKvProfile is pinned at 128 bytes");
_Static_assert(sizeof(SynapseKvMatrix) == 24, "SynapseKvMatrix is pinned at 24 bytes");
_Static_assert(sizeof(SynapseKvPageActivation) == 24, "SynapseKvPageActivation is pinned at 24 bytes");
_Static_assert(sizeof(SynapseKvProjection) == 48, "SynapseKvProjection is pinned at 48 bytes");
_Static_assert(sizeof(SynapseKvLayerOffsets) == 120, "SynapseKvLayerOffsets is pinned at 120 bytes");
_Static_assert(sizeof(SynapseKvDecoderDesc) == 136, "SynapseKvDecoderDesc is pinned at 136 bytes");
_Static_assert(sizeof(SynapseKvPrefixKey) == 32, "SynapseKvPrefixKey is pinned at 32 bytes");
_Static_assert(sizeof(SynapseKvPrefixHeader) == 128, "SynapseKvPrefixHeader is pinned at 128 bytes");
#endif

#endif /* SYNAPSE_KV_H */
