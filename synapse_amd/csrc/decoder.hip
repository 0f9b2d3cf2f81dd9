// The dense decoder step (libsynapse_gpu's model API; native/synapse-gpu/src/Features/GpuKernels/ffi.rs:106-271,
// decoder.rs:60-336, step.rs:137-185, step/layers.rs): validation of the model description, upload of the mapped
// weights, and one batched step as embedding -> per layer (RMS norm, Q/K/V projections, RoPE + KV append +
// attention, output projection into the residual, RMS norm, gate/up projections, SwiGLU, down projection into the
// residual) -> output norm of the logits rows -> logits projection.
//
// The model is composed from this library's own handles: a SynapseKvCache (pages, RoPE, attention) and a
// SynapseKvWeights (Q8_0, Q4_K and Q6_K matrices repacked for the MFMA projection kernels), on one stream. The kernels here are the
// elementwise ones (elementwise.cu / elementwise.metal): embedding lookup, RMS normalization and SwiGLU.

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../../include/synapse_gpu.h"
#include "abi_support.h"
#include "kquant_layout.h"
#include "kv_internal.h"

namespace synapse_kv {
namespace {

constexpr uint32_t kMatrices = 7;  // Q, K, V, O, gate, up, down (the packing order of `encodings`)

__device__ inline float half_bits_to_float(uint16_t bits) {
    _Float16 value;
    __builtin_memcpy(&value, &bits, 2);
    return static_cast<float>(value);
}

// synapse_embed_q8_0 (elementwise.cu:3-15): hidden[t][c] = d(token, c / 32) * code(token, c), one workgroup per
// token. Rows are GGML Q8_0 blocks of 34 bytes (an FP16 scale, 32 int8 codes).
__global__ __launch_bounds__(256) void embed_kernel(const uint8_t* table, uint32_t row_bytes, const int32_t* tokens,
                                                    uint32_t columns, float* hidden) {
    const int token = blockIdx.x;
    const uint8_t* row = table + static_cast<uint64_t>(tokens[token]) * row_bytes;
    float* out = hidden + static_cast<size_t>(token) * columns;
    for (uint32_t column = threadIdx.x; column < columns; column += blockDim.x) {
        const uint8_t* block = row + static_cast<size_t>(column / 32) * 34;
        const uint16_t scale = static_cast<uint16_t>(block[0] | (block[1] << 8));
        const int8_t code = static_cast<int8_t>(block[2 + column % 32]);
        out[column] = half_bits_to_float(scale) * static_cast<float>(code);
    }
}

// synapse_kq_embed (matmul_kquant.metal:293-308): hidden[t][c] is value c of the token's K-quant row, decoded as
// kq_values8 does ((d * sc) * q - dmin * m for Q4_K, (d * scale) * (q - 32) for Q6_K), one workgroup per token.
template <uint32_t E>
__global__ __launch_bounds__(256) void embed_kquant_kernel(const uint8_t* table, uint32_t row_bytes,
                                                           const int32_t* tokens, uint32_t columns, float* hidden) {
#pragma clang fp contract(off)
    const int token = blockIdx.x;
    const uint8_t* row = table + static_cast<uint64_t>(tokens[token]) * row_bytes;
    float* out = hidden + static_cast<size_t>(token) * columns;
    for (uint32_t column = threadIdx.x; column < columns; column += blockDim.x) {
        const uint8_t* block = row + static_cast<size_t>(column / kSuperBlockValues) * ggml_block_bytes(E);
        const int i = static_cast<int>(column % kSuperBlockValues);
        const float q = static_cast<float>(kq_code(E, block, i));
        if constexpr (E == kEncodingQ4K) {
            int sc = 0;
            int m = 0;
            q4k_scale_min(block + 4, i / 32, sc, m);
            out[column] = (kq_half(block) * static_cast<float>(sc)) * q - kq_half(block + 2) * static_cast<float>(m);
        } else {
            out[column] = (kq_half(block + 208) * static_cast<float>(static_cast<int8_t>(block[192 + i / 16]))) * q;
        }
    }
}

// synapse_rms_norm (elementwise.cu:17-52): y = x * (1 / sqrt(mean(x^2) + eps)) * w, one workgroup per row; with
// `gather` row r reads input row gather[r] (the logits rows). Each thread keeps its columns (16-byte groups, up to
// kNormGroups of them, i.e. hidden <= 8,192) in registers: all loads are issued before the sum, and the row is read
// once. The sum of squares is reduced per wave, then across the workgroup's 16 waves in order.
constexpr int kNormThreads = 1024;  // one workgroup of 16 waves per row: more loads in flight per row
constexpr int kNormGroups = 2;
#pragma clang fp contract(off)
// y = x * (1 / sqrt(mean(x^2) + eps)) * w for one row held by the workgroup (kNormThreads threads):
// thread i holds float4 groups i + kNormThreads j (zeros past the row).
__device__ inline void normalize_values(float4 (&values)[kNormGroups], const float* weight, uint32_t columns,
                                        float epsilon) {
    __shared__ float partial[kNormThreads / 64];
    const float4* w = reinterpret_cast<const float4*>(weight);
    const uint32_t groups = columns / 4;
    float4 scales[kNormGroups];
#pragma unroll
    for (int j = 0; j < kNormGroups; ++j) {
        const uint32_t index = threadIdx.x + kNormThreads * j;
        scales[j] = index < groups ? w[index] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < kNormGroups; ++j) {
        sum += values[j].x * values[j].x;
        sum += values[j].y * values[j].y;
        sum += values[j].z * values[j].z;
        sum += values[j].w * values[j].w;
    }
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        sum += __shfl_xor(sum, offset);
    }
    if ((threadIdx.x & 63) == 0) {
        partial[threadIdx.x >> 6] = sum;
    }
    __syncthreads();
    float total = partial[0];
#pragma unroll
    for (int wave = 1; wave < kNormThreads / 64; ++wave) {
        total += partial[wave];
    }
    const float scale = 1.0f / sqrtf(total / static_cast<float>(columns) + epsilon);
#pragma unroll
    for (int j = 0; j < kNormGroups; ++j) {
        const float4 v = values[j];
        const float4 c = scales[j];
        values[j] = make_float4(v.x * scale * c.x, v.y * scale * c.y, v.z * scale * c.z, v.w * scale * c.w);
    }
}

__device__ inline void normalize_row(float4 (&values)[kNormGroups], const float* weight, uint32_t columns,
                                     float epsilon, float* y_row) {
    normalize_values(values, weight, columns, epsilon);
    float4* y = reinterpret_cast<float4*>(y_row);
#pragma unroll
    for (int j = 0; j < kNormGroups; ++j) {
        const uint32_t index = threadIdx.x + kNormThreads * j;
        if (index < columns / 4) {
            y[index] = values[j];
        }
    }
}

// The same normalized row, written as the next projection's split input (SplitInput): lanes 2k and 2k + 1 hold the
// 8 columns of group k, which the even lane writes (zeros past the row, up to the last 64-column chunk).
__device__ inline void normalize_row_split(float4 (&values)[kNormGroups], const float* weight, uint32_t columns,
                                           float epsilon, const SplitInput& split, int token) {
    normalize_values(values, weight, columns, epsilon);
    const uint32_t padded_groups = static_cast<uint32_t>(split.chunks) * (kQ8ChunkColumns / 4);
#pragma unroll
    for (int j = 0; j < kNormGroups; ++j) {
        const uint32_t index = threadIdx.x + kNormThreads * j;
        float4 other;
        other.x = __shfl_xor(values[j].x, 1);
        other.y = __shfl_xor(values[j].y, 1);
        other.z = __shfl_xor(values[j].z, 1);
        other.w = __shfl_xor(values[j].w, 1);
        if ((index & 1) == 0 && index < padded_groups) {
            const float group[8] = {values[j].x, values[j].y, values[j].z, values[j].w,
                                    other.x,     other.y,     other.z,     other.w};
            store_split_group(split, token, static_cast<int>(4 * index), group);
        }
    }
}

__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(const float* input, const int32_t* gather,
                                                                const float* weight, uint32_t columns, float epsilon,
                                                                float* output) {
    const int row = blockIdx.x;
    const size_t source = gather != nullptr ? static_cast<size_t>(gather[row]) : static_cast<size_t>(row);
    const float4* x = reinterpret_cast<const float4*>(input + source * columns);
    const uint32_t groups = columns / 4;
    float4 values[kNormGroups];
#pragma unroll
    for (int j = 0; j < kNormGroups; ++j) {
        const uint32_t index = threadIdx.x + kNormThreads * j;
        values[j] = index < groups ? x[index] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    normalize_row(values, weight, columns, epsilon, output + static_cast<size_t>(row) * columns);
}

// rms_norm_kernel writing the next projection's split input instead of the FP32 row (prompt steps).
__global__ __launch_bounds__(kNormThreads) void rms_norm_split_kernel(const float* input, const float* weight,
                                                                      uint32_t columns, float epsilon,
                                                                      SplitInput split) {
    const int row = blockIdx.x;
    const float4* x = reinterpret_cast<const float4*>(input + static_cast<size_t>(row) * columns);
    const uint32_t groups = columns / 4;
    float4 values[kNormGroups];
#pragma unroll
    for (int j = 0; j < kNormGroups; ++j) {
        const uint32_t index = threadIdx.x + kNormThreads * j;
        values[j] = index < groups ? x[index] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    normalize_row_split(values, weight, columns, epsilon, split, row);
}

// Sum over slices, in order, of a deferred projection's partial sums at `offset` (element offset of (token, row) in
// slice 0), plus 0.0f: what reduce_kernel would have written (decode projections without biases).
__device__ inline float slice_sum(const DeferredSums& d, size_t offset) {
    const float* partial = d.partials + offset;
    const size_t stride = static_cast<size_t>(16) * d.stride;
    float sum = partial[0];
    for (int slice = 1; slice < d.slices; ++slice) {
        sum += partial[slice * stride];
    }
    return sum + 0.0f;
}

__device__ inline float4 slice_sum4(const DeferredSums& d, size_t offset) {
    const float4* partial = reinterpret_cast<const float4*>(d.partials + offset);
    const size_t stride = static_cast<size_t>(16) * d.stride / 4;
    float4 sum = partial[0];
    for (int slice = 1; slice < d.slices; ++slice) {
        const float4 v = partial[slice * stride];
        sum.x += v.x;
        sum.y += v.y;
        sum.z += v.z;
        sum.w += v.w;
    }
    return make_float4(sum.x + 0.0f, sum.y + 0.0f, sum.z + 0.0f, sum.w + 0.0f);
}

// The output projection's reduce fused with the next RMS norm (one launch instead of two): hidden[t] += the
// projection's slice sums (reduce_kernel with accumulate, in the same order), written back, then normalized into
// `output` as rms_norm_kernel does. One workgroup per token.
__global__ __launch_bounds__(kNormThreads) void residual_norm_kernel(float* hidden, DeferredSums o,
                                                                     const float* weight, uint32_t columns,
                                                                     float epsilon, float* output) {
    const int token = blockIdx.x;
    float4* x = reinterpret_cast<float4*>(hidden + static_cast<size_t>(token) * columns);
    const uint32_t groups = columns / 4;
    float4 values[kNormGroups];
#pragma unroll
    for (int j = 0; j < kNormGroups; ++j) {
        const uint32_t index = threadIdx.x + kNormThreads * j;
        values[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (index < groups) {
            const float4 h = x[index];
            const float4 add = slice_sum4(o, static_cast<size_t>(token) * o.stride + o.first_row[0] + 4 * index);
            values[j] = make_float4(h.x + add.x, h.y + add.y, h.z + add.z, h.w + add.w);
            x[index] = values[j];
        }
    }
    normalize_row(values, weight, columns, epsilon, output + static_cast<size_t>(token) * columns);
}

// The gate/up projection's reduce fused with SwiGLU: gate and up are their slice sums (reduce_kernel's values), out
// = gate / (1 + exp(-gate)) * up as swiglu_kernel computes it.
__global__ __launch_bounds__(256) void reduce_swiglu_kernel(DeferredSums gate_up, uint32_t columns, float* output) {
    const int token = blockIdx.y;
    const uint32_t column = blockIdx.x * blockDim.x + threadIdx.x;
    if (column >= columns) {
        return;
    }
    const size_t row0 = static_cast<size_t>(token) * gate_up.stride;
    const float gate = slice_sum(gate_up, row0 + gate_up.first_row[0] + column);
    const float up = slice_sum(gate_up, row0 + gate_up.first_row[1] + column);
    output[static_cast<size_t>(token) * columns + column] = gate / (1.0f + expf(-gate)) * up;
}

// synapse_swiglu (elementwise.cu:97-109): out = gate / (1 + exp(-gate)) * up, gate and up side by side in each row.
__global__ __launch_bounds__(256) void swiglu_kernel(const float* gate_up, uint32_t columns, float* output) {
    const int token = blockIdx.y;
    const uint32_t column = blockIdx.x * blockDim.x + threadIdx.x;
    if (column >= columns) {
        return;
    }
    const float* row = gate_up + static_cast<size_t>(token) * 2 * columns;
    const float gate = row[column];
    output[static_cast<size_t>(token) * columns + column] = gate / (1.0f + expf(-gate)) * row[columns + column];
}

// swiglu_kernel writing the down projection's split input (prompt steps): one thread per (token, 8 columns) in
// split_thread's order, zeros past `columns`.
__global__ __launch_bounds__(256) void swiglu_split_kernel(const float* gate_up, uint32_t columns, int tokens,
                                                           SplitInput split) {
    int token;
    int column;
    if (!split_thread(blockIdx.x * 256 + threadIdx.x, split.chunks, tokens, token, column)) {
        return;
    }
    const float* row = gate_up + static_cast<size_t>(token) * 2 * columns;
    float values[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t c = static_cast<uint32_t>(column + i);
        float value = 0.0f;
        if (c < columns) {
            const float gate = row[c];
            value = gate / (1.0f + expf(-gate)) * row[columns + c];
        }
        values[i] = value;
    }
    store_split_group(split, token, column, values);
}
#pragma clang fp contract(on)

template <typename T>
struct Buffer {
    T* pointer = nullptr;
    size_t count = 0;
    void allocate(size_t wanted, const char* what) {
        check_hip(hipMalloc(reinterpret_cast<void**>(&pointer), std::max<size_t>(wanted, 1) * sizeof(T)), what);
        count = wanted;
    }
    void reset() {
        if (pointer != nullptr) {
            (void)hipFree(pointer);
        }
        pointer = nullptr;
        count = 0;
    }
};

// The status a composed call recorded: raise it again with the message it left as the thread's last error.
void check_status(int32_t status) {
    if (status != SYNAPSE_KV_OK) {
        throw Failure{status, g_last_error};
    }
}

// A message without the "invalid argument: " prefix invalid() adds.
std::string strip_prefix(const std::string& message) {
    const std::string prefix = "invalid argument: ";
    return message.compare(0, prefix.size(), prefix) == 0 ? message.substr(prefix.size()) : message;
}

}  // namespace
}  // namespace synapse_kv

struct SynapseKvDecoder {
    SynapseKvDecoderDesc shape{};  // dimensions (pointers cleared)
    int device = 0;
    hipStream_t stream = nullptr;
    SynapseKvCache* cache = nullptr;
    SynapseKvWeights* weights = nullptr;
    uint32_t output_matrix = 0;  // index of the logits matrix in `weights`
    synapse_kv::Buffer<uint8_t> embedding;  // vocabulary rows of GGML blocks (Q8_0, Q4_K or Q6_K)
    synapse_kv::Buffer<float> norms;        // per layer [attention norm | feed-forward norm], then the output norm
    synapse_kv::Buffer<float> hidden;       // [step_tokens][hidden]: the residual stream
    synapse_kv::Buffer<float> normalized;   // [step_tokens][hidden]
    synapse_kv::Buffer<float> squares;      // decode steps: [16][kNormSquaresStride] partial sums of squares of hidden
    synapse_kv::Buffer<float> qkv;          // [step_tokens][hidden + 2 kv_width]
    synapse_kv::Buffer<float> attention;    // [step_tokens][hidden]
    synapse_kv::Buffer<float> gate_up;      // [step_tokens][2 feed_forward]
    synapse_kv::Buffer<float> feed_forward; // [step_tokens][feed_forward]
    synapse_kv::Buffer<float> logits_input; // [logits_rows][hidden]
    synapse_kv::Buffer<float> logits;       // [logits_rows][vocabulary]
    synapse_kv::Buffer<int32_t> indices;    // [step_tokens] token ids, then [logits_rows] gathered token indices
    int32_t* staging = nullptr;             // pinned host copy of `indices` (coherent, read by the upload kernel)
    void* staging_view = nullptr;           // `staging` as the device addresses it

    ~SynapseKvDecoder() {
        (void)hipSetDevice(device);
        if (stream != nullptr) {
            (void)hipStreamSynchronize(stream);
        }
        synapse_kv_cache_destroy(cache);
        synapse_kv_weights_destroy(weights);
        for (auto* buffer : {&hidden, &normalized, &squares, &qkv, &attention, &gate_up, &feed_forward, &logits_input,
                             &logits, &norms}) {
            buffer->reset();
        }
        embedding.reset();
        indices.reset();
        if (staging != nullptr) {
            (void)hipHostFree(staging);
        }
    }
};

namespace synapse_kv {
namespace {

// Encoding::from_id (decoder/encoding.rs:26-36).
void check_encoding(uint32_t id, const std::string& name) {
    if (id == SYNAPSE_KV_ENCODING_Q8_0 || is_kquant(id)) {
        return;
    }
    fail(SYNAPSE_KV_UNAVAILABLE, name + ": the GPU kernels implement Q8_0, Q4_K, and Q6_K matrices, not GGML type " +
                                     std::to_string(id));
}

// RangeCheck (decoder/checks.rs:169-225): the tensor lies inside the mapping and is aligned.
void check_span(const SynapseKvDecoderDesc& d, uint64_t offset, uint64_t bytes, uint64_t alignment,
                const std::string& name) {
    if (offset > d.weights_length || bytes > d.weights_length - offset || offset % alignment != 0) {
        invalid("tensor " + name + " at offset " + std::to_string(offset) + " is outside or misaligned");
    }
}

void check_matrix(const SynapseKvDecoderDesc& d, uint64_t offset, uint64_t rows, uint64_t columns, uint32_t encoding,
                  const std::string& name) {
    check_encoding(encoding, name);
    const uint64_t values = static_cast<uint64_t>(ggml_block_values(encoding));
    if (columns % values != 0) {
        fail(SYNAPSE_KV_UNAVAILABLE, "tensor " + name + " has " + std::to_string(columns) +
                                         " columns, not a multiple of its " + std::to_string(values) + "-value blocks");
    }
    check_span(d, offset, ggml_matrix_bytes(encoding, rows, columns), 2, name);
}

void check_f32(const SynapseKvDecoderDesc& d, uint64_t offset, uint64_t values, const std::string& name) {
    check_span(d, offset, values * 4, 4, name);
}

uint32_t encoding_of(const SynapseKvLayerOffsets& layer, uint32_t matrix) {
    return static_cast<uint32_t>((layer.encodings >> (4 * matrix)) & 0xF);
}

// DecoderPlan::new (decoder.rs:246-294; checks.rs:10-167).
void validate(const SynapseKvDecoderDesc& d) {
    if (d.weights == nullptr || d.layers == nullptr || d.rope_cosines == nullptr || d.rope_sines == nullptr) {
        fail(SYNAPSE_KV_NULL_POINTER, "null pointer: model description");
    }
    // check_variants (checks.rs:36-47).
    check_encoding(d.embedding_encoding, "token_embd");
    check_encoding(d.output_encoding, "output");
    if (d.rope_layout != SYNAPSE_KV_ROPE_NEOX || d.activation != SYNAPSE_KV_ACTIVATION_SWIGLU) {
        fail(SYNAPSE_KV_UNAVAILABLE, "the GPU kernels implement NeoX RoPE and SwiGLU; the model asks for RoPE layout " +
                                         std::to_string(d.rope_layout) + ", activation " +
                                         std::to_string(d.activation));
    }
    // check_dimensions (checks.rs:49-103).
    const uint32_t positive[] = {d.layer_count, d.hidden,       d.feed_forward, d.heads,       d.kv_heads,
                                 d.vocabulary,  d.context,      d.session_slots, d.step_tokens, d.logits_rows};
    if (std::find(std::begin(positive), std::end(positive), 0u) != std::end(positive) || !std::isfinite(d.rms_epsilon) ||
        d.rms_epsilon <= 0.0f) {
        invalid("every dimension must be positive and epsilon finite");
    }
    if (d.kv_growth_positions == 0 || d.kv_growth_positions % 64 != 0) {
        invalid("the KV growth unit must be a positive multiple of 64 positions");
    }
    if ((d.head_dim != 64 && d.head_dim != 128) || d.hidden != d.heads * d.head_dim) {
        fail(SYNAPSE_KV_UNAVAILABLE, "the GPU kernels implement head dimensions [64, 128] with hidden = heads x head; "
                                     "the model uses head " + std::to_string(d.head_dim) + " and hidden " +
                                         std::to_string(d.hidden));
    }
    if (d.heads % d.kv_heads != 0 || d.heads / d.kv_heads > 8) {
        fail(SYNAPSE_KV_UNAVAILABLE, "query heads per KV head must divide evenly and be at most 8");
    }
    if (d.hidden % 32 != 0 || d.feed_forward % 32 != 0) {
        invalid("hidden and feed-forward widths must be multiples of 32");
    }
    if (d.hidden > 4 * kNormThreads * kNormGroups) {
        fail(SYNAPSE_KV_UNAVAILABLE, "the RMS norm kernel keeps a row in registers: hidden widths up to " +
                                         std::to_string(4 * kNormThreads * kNormGroups) + " (the model has " +
                                         std::to_string(d.hidden) + ")");
    }
    if (d.kv_precision != SYNAPSE_KV_F32 && d.kv_precision != SYNAPSE_KV_F16) {
        invalid("unknown KV precision " + std::to_string(d.kv_precision));
    }
    // Ranges (decoder.rs:261-279).
    const uint64_t hidden = d.hidden;
    const uint64_t vocabulary = d.vocabulary;
    const uint64_t kv = static_cast<uint64_t>(d.kv_heads) * d.head_dim;
    const uint64_t ffn = d.feed_forward;
    check_matrix(d, d.token_embedding, vocabulary, hidden, d.embedding_encoding, "token_embd");
    check_matrix(d, d.output, vocabulary, hidden, d.output_encoding, "output");
    check_f32(d, d.output_norm, hidden, "output_norm");
    for (uint32_t index = 0; index < d.layer_count; ++index) {
        const SynapseKvLayerOffsets& l = d.layers[index];
        const std::string at = "layer " + std::to_string(index) + ": ";
        try {
            check_f32(d, l.attention_norm, hidden, "attn_norm");
            check_matrix(d, l.query, hidden, hidden, encoding_of(l, 0), "attn_q");
            check_matrix(d, l.key, kv, hidden, encoding_of(l, 1), "attn_k");
            check_matrix(d, l.value, kv, hidden, encoding_of(l, 2), "attn_v");
            if (l.query_bias != SYNAPSE_KV_NO_TENSOR) {
                check_f32(d, l.query_bias, hidden, "attn_q.bias");
            }
            if (l.key_bias != SYNAPSE_KV_NO_TENSOR) {
                check_f32(d, l.key_bias, kv, "attn_k.bias");
            }
            if (l.value_bias != SYNAPSE_KV_NO_TENSOR) {
                check_f32(d, l.value_bias, kv, "attn_v.bias");
            }
            if (l.query_norm != SYNAPSE_KV_NO_TENSOR || l.key_norm != SYNAPSE_KV_NO_TENSOR) {
                fail(SYNAPSE_KV_UNAVAILABLE, "per-head query/key normalization is not implemented by the GPU kernels yet");
            }
            check_matrix(d, l.attention_output, hidden, hidden, encoding_of(l, 3), "attn_output");
            check_f32(d, l.feed_forward_norm, hidden, "ffn_norm");
            check_matrix(d, l.gate, ffn, hidden, encoding_of(l, 4), "ffn_gate");
            check_matrix(d, l.up, ffn, hidden, encoding_of(l, 5), "ffn_up");
            check_matrix(d, l.down, hidden, ffn, encoding_of(l, 6), "ffn_down");
        } catch (const Failure& failure) {
            if (failure.status == SYNAPSE_KV_INVALID_ARGUMENT) {
                invalid(at + strip_prefix(failure.message));
            }
            throw;
        }
    }
}

void create_decoder(const SynapseKvDecoderDesc& d, int32_t device, SynapseKvDecoder** output) {
    auto model = std::make_unique<SynapseKvDecoder>();
    model->shape = d;
    model->shape.weights = nullptr;
    model->shape.layers = nullptr;
    model->shape.rope_cosines = nullptr;
    model->shape.rope_sines = nullptr;
    model->device = device;
    const uint64_t kv = static_cast<uint64_t>(d.kv_heads) * d.head_dim;

    // Matrices: per layer Q, K, V (with their biases), O, gate, up, down; then the logits matrix.
    std::vector<SynapseKvMatrix> matrices;
    std::vector<uint32_t> encodings;
    for (uint32_t index = 0; index < d.layer_count; ++index) {
        const SynapseKvLayerOffsets& l = d.layers[index];
        for (uint32_t matrix = 0; matrix < kMatrices; ++matrix) {
            encodings.push_back(encoding_of(l, matrix));
        }
        matrices.push_back({l.query, l.query_bias, d.hidden, d.hidden});
        matrices.push_back({l.key, l.key_bias, static_cast<uint32_t>(kv), d.hidden});
        matrices.push_back({l.value, l.value_bias, static_cast<uint32_t>(kv), d.hidden});
        matrices.push_back({l.attention_output, SYNAPSE_KV_NO_BIAS, d.hidden, d.hidden});
        matrices.push_back({l.gate, SYNAPSE_KV_NO_BIAS, d.feed_forward, d.hidden});
        matrices.push_back({l.up, SYNAPSE_KV_NO_BIAS, d.feed_forward, d.hidden});
        matrices.push_back({l.down, SYNAPSE_KV_NO_BIAS, d.hidden, d.feed_forward});
    }
    matrices.push_back({d.output, SYNAPSE_KV_NO_BIAS, d.vocabulary, d.hidden});
    encodings.push_back(d.output_encoding);
    model->output_matrix = static_cast<uint32_t>(matrices.size() - 1);
    check_hip(hipSetDevice(device), "set device");
    check_status(synapse_kv_weights_create_encoded(d.weights, d.weights_length, matrices.data(), encodings.data(),
                                                   static_cast<uint32_t>(matrices.size()), &model->weights));

    // Embedding table (GGML rows, looked up per token), norms.
    const size_t embedding_bytes = ggml_matrix_bytes(d.embedding_encoding, d.vocabulary, d.hidden);
    model->embedding.allocate(embedding_bytes, "token embedding");
    check_hip(hipMemcpy(model->embedding.pointer, d.weights + d.token_embedding, embedding_bytes, hipMemcpyHostToDevice),
              "token embedding upload");
    std::vector<float> norms(static_cast<size_t>(2 * d.layer_count + 1) * d.hidden);
    for (uint32_t index = 0; index < d.layer_count; ++index) {
        std::memcpy(&norms[(2 * index) * d.hidden], d.weights + d.layers[index].attention_norm, d.hidden * 4);
        std::memcpy(&norms[(2 * index + 1) * d.hidden], d.weights + d.layers[index].feed_forward_norm, d.hidden * 4);
    }
    std::memcpy(&norms[(2 * d.layer_count) * d.hidden], d.weights + d.output_norm, d.hidden * 4);
    model->norms.allocate(norms.size(), "norm weights");
    check_hip(hipMemcpy(model->norms.pointer, norms.data(), norms.size() * 4, hipMemcpyHostToDevice), "norm upload");

    // Activations.
    const size_t steps = d.step_tokens;
    model->hidden.allocate(steps * d.hidden, "hidden rows");
    model->normalized.allocate(steps * d.hidden, "normalized rows");
    model->squares.allocate(16 * kNormSquaresStride, "row squares");
    check_hip(hipMemset(model->squares.pointer, 0, 16 * kNormSquaresStride * sizeof(float)), "row squares");
    model->qkv.allocate(steps * (d.hidden + 2 * kv), "qkv rows");
    model->attention.allocate(steps * d.hidden, "attention rows");
    model->gate_up.allocate(steps * 2 * static_cast<size_t>(d.feed_forward), "gate/up rows");
    model->feed_forward.allocate(steps * d.feed_forward, "feed-forward rows");
    model->logits_input.allocate(static_cast<size_t>(d.logits_rows) * d.hidden, "logits input rows");
    model->logits.allocate(static_cast<size_t>(d.logits_rows) * d.vocabulary, "logits");
    model->indices.allocate(steps + d.logits_rows, "token indices");
    check_hip(hipHostMalloc(reinterpret_cast<void**>(&model->staging), (steps + d.logits_rows) * sizeof(int32_t),
                            hipHostMallocMapped | hipHostMallocCoherent),
              "token staging");
    check_hip(hipHostGetDevicePointer(&model->staging_view, model->staging, 0), "token staging device address");

    // KV cache: 256-position pages when the growth unit allows, every slot's full context or what fits.
    SynapseKvDesc cache{};
    cache.rope_cosines = d.rope_cosines;
    cache.rope_sines = d.rope_sines;
    cache.layer_count = d.layer_count;
    cache.heads = d.heads;
    cache.kv_heads = d.kv_heads;
    cache.head_dim = d.head_dim;
    cache.max_positions = d.context;
    cache.kv_growth_positions = d.kv_growth_positions;
    cache.page_tokens = d.kv_growth_positions % 256 == 0 ? 256 : 64;
    cache.kv_precision = d.kv_precision;
    cache.session_slots = d.session_slots;
    cache.step_tokens = d.step_tokens;
    cache.device = device;
    const uint64_t page_bytes = static_cast<uint64_t>(d.layer_count) * 2 * kv * cache.page_tokens *
                                (d.kv_precision == SYNAPSE_KV_F16 ? 2 : 4);
    const uint64_t wanted = static_cast<uint64_t>(d.session_slots) * ((d.context + cache.page_tokens - 1) / cache.page_tokens);
    size_t free_bytes = 0;
    size_t total_bytes = 0;
    check_hip(hipMemGetInfo(&free_bytes, &total_bytes), "device memory query");
    const uint64_t fits = static_cast<uint64_t>(static_cast<double>(free_bytes) * 0.85) / page_bytes;
    cache.max_pages = static_cast<uint32_t>(std::min<uint64_t>({wanted, fits, 1u << 30}));
    if (cache.max_pages == 0) {
        fail(SYNAPSE_KV_OUT_OF_MEMORY, "out of device memory: no KV page fits after the weights");
    }
    check_status(synapse_kv_cache_create(&cache, &model->cache));
    check_status(synapse_kv_set_stream(model->cache, nullptr));
    check_status(synapse_kv_weights_set_stream(model->weights, nullptr));
    *output = model.release();
}

// A projection of `tokens` rows through up to three matrices (indices), each writing from its output column.
SynapseKvProjection projection(std::initializer_list<std::pair<uint32_t, uint32_t>> parts, uint32_t tokens,
                               uint32_t in_stride, uint32_t out_stride, bool accumulate) {
    SynapseKvProjection p{};
    p.segments = 0;
    for (const auto& [matrix, column] : parts) {
        p.matrix[p.segments] = matrix;
        p.out_column[p.segments] = column;
        ++p.segments;
    }
    p.tokens = tokens;
    p.in_stride = in_stride;
    p.out_stride = out_stride;
    p.accumulate = accumulate ? 1 : 0;
    return p;
}

// Projects `tokens` rows of `input` through up to three matrices (indices) into `output`.
void project(SynapseKvDecoder& m, std::initializer_list<std::pair<uint32_t, uint32_t>> parts, uint32_t tokens,
             const float* input, uint32_t in_stride, float* output, uint32_t out_stride, bool accumulate) {
    const SynapseKvProjection p = projection(parts, tokens, in_stride, out_stride, accumulate);
    check_status(synapse_kv_project(m.weights, &p, input, output));
}

// The same, leaving a decode projection's slice sums to the caller's next kernel (DeferredSums).
DeferredSums project_deferred_sums(SynapseKvDecoder& m, std::initializer_list<std::pair<uint32_t, uint32_t>> parts,
                                   uint32_t tokens, const float* input, uint32_t in_stride, float* output,
                                   uint32_t out_stride, bool accumulate) {
    SynapseKvProjection p{};
    p.segments = 0;
    for (const auto& [matrix, column] : parts) {
        p.matrix[p.segments] = matrix;
        p.out_column[p.segments] = column;
        ++p.segments;
    }
    p.tokens = tokens;
    p.in_stride = in_stride;
    p.out_stride = out_stride;
    p.accumulate = accumulate ? 1 : 0;
    return project_deferred(*m.weights, p, input, output);
}

// DecoderPlan::validate_step (decoder.rs:303-335): returns the number of logits rows.
uint32_t validate_step(const SynapseKvDecoder& m, const SynapseKvBatchToken* tokens, size_t count) {
    const SynapseKvDecoderDesc& d = m.shape;
    if (count == 0 || count > d.step_tokens) {
        invalid("a step holds 1.." + std::to_string(d.step_tokens) + " tokens");
    }
    uint32_t rows = 0;
    for (size_t index = 0; index < count; ++index) {
        const SynapseKvBatchToken& t = tokens[index];
        auto in_range = [](int32_t value, uint32_t limit) { return value >= 0 && static_cast<uint32_t>(value) < limit; };
        if (!in_range(t.slot, d.session_slots) || !in_range(t.token, d.vocabulary) || !in_range(t.position, d.context)) {
            invalid("invalid batch token " + std::to_string(index) + " (slot " + std::to_string(t.slot) + ", token " +
                    std::to_string(t.token) + ", position " + std::to_string(t.position) + ")");
        }
        if (t.logits_row >= 0) {
            if (static_cast<uint32_t>(t.logits_row) != rows || rows >= d.logits_rows) {
                invalid("logits rows must be 0..k-1 in token order");
            }
            ++rows;
        }
    }
    return rows;
}

// MetalDecoder / CudaDecoder::forward (cuda/decoder.rs:97-146) over encode_step (step.rs:137-185).
void forward(SynapseKvDecoder& m, const SynapseKvBatchToken* tokens, size_t count, size_t prompt_start, float* logits,
             size_t logits_capacity) {
    const SynapseKvDecoderDesc& d = m.shape;
    const uint32_t rows = validate_step(m, tokens, count);
    if (logits_capacity < static_cast<size_t>(rows) * d.vocabulary) {
        invalid("the logits buffer is shorter than rows * vocabulary");
    }
    check_hip(hipSetDevice(m.device), "set device");
    check_status(synapse_kv_step_prompt(m.cache, tokens, count, prompt_start));
    // Token ids, then the step indices of the logits rows (the gather of the output norm).
    check_hip(hipStreamSynchronize(m.stream), "staging reuse");
    uint32_t gathered = 0;
    for (size_t index = 0; index < count; ++index) {
        m.staging[index] = tokens[index].token;
        if (tokens[index].logits_row >= 0) {
            m.staging[d.step_tokens + gathered++] = static_cast<int32_t>(index);
        }
    }
    check_hip(launch_upload(m.staging_view, m.indices.pointer, (d.step_tokens + rows) * sizeof(int32_t), m.stream),
              "token upload");
    const uint32_t n = static_cast<uint32_t>(count);
    const uint32_t hidden = d.hidden;
    const uint32_t kv = d.kv_heads * d.head_dim;
    const uint32_t qkv_width = hidden + 2 * kv;
    const uint32_t ffn = d.feed_forward;
    const uint32_t row_bytes = static_cast<uint32_t>(ggml_matrix_bytes(d.embedding_encoding, 1, hidden));
    switch (d.embedding_encoding) {
        case kEncodingQ4K:
            hipLaunchKernelGGL(embed_kquant_kernel<kEncodingQ4K>, dim3(n), dim3(256), 0, m.stream, m.embedding.pointer,
                               row_bytes, m.indices.pointer, hidden, m.hidden.pointer);
            break;
        case kEncodingQ6K:
            hipLaunchKernelGGL(embed_kquant_kernel<kEncodingQ6K>, dim3(n), dim3(256), 0, m.stream, m.embedding.pointer,
                               row_bytes, m.indices.pointer, hidden, m.hidden.pointer);
            break;
        default:
            hipLaunchKernelGGL(embed_kernel, dim3(n), dim3(256), 0, m.stream, m.embedding.pointer, row_bytes,
                               m.indices.pointer, hidden, m.hidden.pointer);
            break;
    }
    check_hip(hipGetLastError(), "embedding");
    // Decode steps (at most 16 tokens) fold the attention norms into the QKV projection's staging: the embedding and
    // each down projection's reduce leave the hidden rows' partial sums of squares (NormInput).
    const bool decode = n <= 16;
    const int32_t norm_parts = static_cast<int32_t>((hidden + kNormSquaresColumns - 1) / kNormSquaresColumns);
    if (decode) {
        check_hip(launch_row_squares(m.stream, m.hidden.pointer, static_cast<int>(hidden), static_cast<int>(n),
                                     m.squares.pointer),
                  "row squares");
    }
    // Prompt steps (more than 16 tokens) have the norms and SwiGLU write the next projection's split input
    // directly (three launches fewer per layer); SYNAPSE_KV_OPTION_FUSED_SUMS = 0 keeps FP32 rows and split_kernel.
    // Both give the same bits.
    const bool split_inputs = n > 16 && cache_fused_sums(*m.cache);
    for (uint32_t layer = 0; layer < d.layer_count; ++layer) {
        const uint32_t base = layer * kMatrices;
        const float* attention_norm = m.norms.pointer + static_cast<size_t>(2 * layer) * hidden;
        const float* ffn_norm = attention_norm + hidden;
        if (split_inputs) {
            const SynapseKvProjection p =
                projection({{base, 0}, {base + 1, hidden}, {base + 2, hidden + kv}}, n, hidden, qkv_width, false);
            const SplitInput split = prepare_split(*m.weights, p);
            hipLaunchKernelGGL(rms_norm_split_kernel, dim3(n), dim3(kNormThreads), 0, m.stream, m.hidden.pointer,
                               attention_norm, hidden, d.rms_epsilon, split);
            check_hip(hipGetLastError(), "attention norm");
            project_split(*m.weights, p, split, m.qkv.pointer);
        } else if (decode) {
            NormInput norm;
            norm.weight = attention_norm;
            norm.squares = m.squares.pointer;
            norm.parts = norm_parts;
            norm.columns = static_cast<int32_t>(hidden);
            norm.epsilon = d.rms_epsilon;
            project_normalized(*m.weights,
                               projection({{base, 0}, {base + 1, hidden}, {base + 2, hidden + kv}}, n, hidden,
                                          qkv_width, false),
                               m.hidden.pointer, m.qkv.pointer, norm);
        } else {
            hipLaunchKernelGGL(rms_norm_kernel, dim3(n), dim3(kNormThreads), 0, m.stream, m.hidden.pointer,
                               static_cast<const int32_t*>(nullptr), attention_norm, hidden, d.rms_epsilon,
                               m.normalized.pointer);
            check_hip(hipGetLastError(), "attention norm");
            project(m, {{base, 0}, {base + 1, hidden}, {base + 2, hidden + kv}}, n, m.normalized.pointer, hidden,
                    m.qkv.pointer, qkv_width, false);
        }
        check_status(synapse_kv_append_attention(m.cache, layer, m.qkv.pointer, qkv_width, m.attention.pointer, hidden));
        // Decode steps leave the output and gate/up projections' slice sums to the kernels that consume them: the
        // residual add runs inside the feed-forward norm and the gate/up sums inside SwiGLU (two launches fewer).
        const bool fused = cache_fused_sums(*m.cache);
        const DeferredSums o = fused ? project_deferred_sums(m, {{base + 3, 0}}, n, m.attention.pointer, hidden,
                                                             m.hidden.pointer, hidden, true)
                                     : DeferredSums{};
        if (!fused) {
            project(m, {{base + 3, 0}}, n, m.attention.pointer, hidden, m.hidden.pointer, hidden, true);
        }
        if (split_inputs) {
            // Prompt steps: the feed-forward norm, SwiGLU and the projections they feed through split inputs.
            const SynapseKvProjection up =
                projection({{base + 4, 0}, {base + 5, ffn}}, n, hidden, 2 * ffn, false);
            const SplitInput up_split = prepare_split(*m.weights, up);
            hipLaunchKernelGGL(rms_norm_split_kernel, dim3(n), dim3(kNormThreads), 0, m.stream, m.hidden.pointer,
                               ffn_norm, hidden, d.rms_epsilon, up_split);
            check_hip(hipGetLastError(), "feed-forward norm");
            project_split(*m.weights, up, up_split, m.gate_up.pointer);
            const SynapseKvProjection down = projection({{base + 6, 0}}, n, ffn, hidden, true);
            const SplitInput down_split = prepare_split(*m.weights, down);
            const int threads = static_cast<int>((n + 15) / 16 * 16) * down_split.chunks * (kQ8ChunkColumns / 8);
            hipLaunchKernelGGL(swiglu_split_kernel, dim3((threads + 255) / 256), dim3(256), 0, m.stream,
                               m.gate_up.pointer, ffn, static_cast<int>(n), down_split);
            check_hip(hipGetLastError(), "SwiGLU");
            project_split(*m.weights, down, down_split, m.hidden.pointer);
            continue;
        }
        if (o.deferred) {
            hipLaunchKernelGGL(residual_norm_kernel, dim3(n), dim3(kNormThreads), 0, m.stream, m.hidden.pointer, o,
                               ffn_norm, hidden, d.rms_epsilon, m.normalized.pointer);
        } else {
            hipLaunchKernelGGL(rms_norm_kernel, dim3(n), dim3(kNormThreads), 0, m.stream, m.hidden.pointer,
                               static_cast<const int32_t*>(nullptr), ffn_norm, hidden, d.rms_epsilon,
                               m.normalized.pointer);
        }
        check_hip(hipGetLastError(), "feed-forward norm");
        DeferredSums gate_up;
        if (fused) {
            gate_up = project_deferred_sums(m, {{base + 4, 0}, {base + 5, ffn}}, n, m.normalized.pointer, hidden,
                                            m.gate_up.pointer, 2 * ffn, false);
        } else {
            project(m, {{base + 4, 0}, {base + 5, ffn}}, n, m.normalized.pointer, hidden, m.gate_up.pointer, 2 * ffn,
                    false);
        }
        if (gate_up.deferred) {
            hipLaunchKernelGGL(reduce_swiglu_kernel, dim3((ffn + 255) / 256, n), dim3(256), 0, m.stream, gate_up, ffn,
                               m.feed_forward.pointer);
        } else {
            hipLaunchKernelGGL(swiglu_kernel, dim3((ffn + 255) / 256, n), dim3(256), 0, m.stream, m.gate_up.pointer,
                               ffn, m.feed_forward.pointer);
        }
        check_hip(hipGetLastError(), "SwiGLU");
        // The down projection's slice sums (a slice per 512 columns of 18,944: 37 at the 7B shape) are added by its
        // own reduce: one workgroup per token reading them all in the next norm measured slower than the launch.
        if (decode) {
            project_with_squares(*m.weights, projection({{base + 6, 0}}, n, ffn, hidden, true), m.feed_forward.pointer,
                                 m.hidden.pointer, m.squares.pointer);
        } else {
            project(m, {{base + 6, 0}}, n, m.feed_forward.pointer, ffn, m.hidden.pointer, hidden, true);
        }
    }
    if (rows > 0) {
        const float* output_norm = m.norms.pointer + static_cast<size_t>(2 * d.layer_count) * hidden;
        hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(kNormThreads), 0, m.stream, m.hidden.pointer,
                           static_cast<const int32_t*>(m.indices.pointer + d.step_tokens), output_norm, hidden,
                           d.rms_epsilon, m.logits_input.pointer);
        check_hip(hipGetLastError(), "output norm");
        project(m, {{m.output_matrix, 0}}, rows, m.logits_input.pointer, hidden, m.logits.pointer, d.vocabulary, false);
        check_hip(hipMemcpyAsync(logits, m.logits.pointer, static_cast<size_t>(rows) * d.vocabulary * sizeof(float),
                                 hipMemcpyDeviceToHost, m.stream),
                  "logits copy");
    }
    check_hip(hipStreamSynchronize(m.stream), "synchronize");
}

}  // namespace
}  // namespace synapse_kv

extern "C" {

int32_t synapse_kv_decoder_create(const SynapseKvDecoderDesc* desc, int32_t device, SynapseKvDecoder** model) {
    if (desc == nullptr || model == nullptr) {
        return synapse_kv::record(SYNAPSE_KV_NULL_POINTER, "null pointer: model description or output");
    }
    return synapse_kv::guarded([&] {
        synapse_kv::validate(*desc);  // DecoderPlan::new comes before the backend (ffi.rs:131-135)
        int devices = 0;
        if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0) {
            synapse_kv::fail(SYNAPSE_KV_UNAVAILABLE, "no HIP device is available");
        }
        if (device < 0 || device >= devices) {
            synapse_kv::invalid("device " + std::to_string(device) + " is outside 0.." + std::to_string(devices - 1));
        }
        synapse_kv::create_decoder(*desc, device, model);
    });
}

int32_t synapse_kv_decoder_forward_prompt(SynapseKvDecoder* model, const SynapseKvBatchToken* tokens, size_t count,
                                          size_t prompt_start, float* logits, size_t logits_capacity) {
    if (model == nullptr || tokens == nullptr || logits == nullptr) {
        return synapse_kv::record(SYNAPSE_KV_NULL_POINTER, "null pointer: model, tokens, or logits");
    }
    return synapse_kv::guarded(
        [&] { synapse_kv::forward(*model, tokens, count, prompt_start, logits, logits_capacity); });
}

int32_t synapse_kv_decoder_forward(SynapseKvDecoder* model, const SynapseKvBatchToken* tokens, size_t count,
                                   float* logits, size_t logits_capacity) {
    return synapse_kv_decoder_forward_prompt(model, tokens, count, count, logits, logits_capacity);
}

void synapse_kv_decoder_destroy(SynapseKvDecoder* model) { delete model; }

uint64_t synapse_kv_decoder_kv_bytes(const SynapseKvDecoder* model) {
    return model == nullptr ? 0 : synapse_kv_bytes(model->cache);
}

int32_t synapse_kv_decoder_reserve(SynapseKvDecoder* model, uint32_t slot, uint32_t positions) {
    if (model == nullptr) {
        return synapse_kv::record(SYNAPSE_KV_NULL_POINTER, "null pointer: model");
    }
    return synapse_kv_reserve(model->cache, slot, positions);
}

int32_t synapse_kv_decoder_cache(SynapseKvDecoder* model, SynapseKvCache** cache) {
    if (model == nullptr || cache == nullptr) {
        return synapse_kv::record(SYNAPSE_KV_NULL_POINTER, "null pointer: model or output");
    }
    *cache = model->cache;
    return SYNAPSE_KV_OK;
}

int32_t synapse_kv_decoder_set_stream(SynapseKvDecoder* model, void* stream) {
    if (model == nullptr) {
        return synapse_kv::record(SYNAPSE_KV_NULL_POINTER, "null pointer: model");
    }
    return synapse_kv::guarded([&] {
        synapse_kv::check_status(synapse_kv_set_stream(model->cache, stream));
        synapse_kv::check_status(synapse_kv_weights_set_stream(model->weights, stream));
        model->stream = static_cast<hipStream_t>(stream);
    });
}

// ---- libsynapse_gpu's ABI version 3 (include/synapse_gpu.h; ffi.rs:12-271) for the HIP backend ----

uint32_t synapse_gpu_abi_version(void) { return SYNAPSE_GPU_ABI_VERSION; }

// unsupported_backend (ffi.rs:46-51): Metal exists only on macOS; this build has no CUDA either.
static int32_t unsupported_backend(uint32_t backend) {
    if (backend == SYNAPSE_GPU_BACKEND_METAL) {
        return synapse_kv::record(SYNAPSE_KV_UNAVAILABLE, "the Metal backend exists only on macOS");
    }
    if (backend == SYNAPSE_GPU_BACKEND_CUDA) {
        return synapse_kv::record(SYNAPSE_KV_UNAVAILABLE, "the CUDA backend is not part of this HIP build");
    }
    return synapse_kv::record(SYNAPSE_KV_INVALID_ARGUMENT, "invalid argument: unknown GPU backend " +
                                                               std::to_string(backend));
}

int32_t synapse_gpu_probe(uint32_t backend, GpuDeviceInfo* info) {
    if (info == nullptr) {
        return synapse_kv::record(SYNAPSE_KV_NULL_POINTER, "null pointer: device info");
    }
    if (backend != SYNAPSE_GPU_BACKEND_HIP) {
        return unsupported_backend(backend);
    }
    return synapse_kv_probe(info);
}

size_t synapse_gpu_last_error(uint8_t* buffer, size_t capacity) { return synapse_kv_last_error(buffer, capacity); }

int32_t synapse_gpu_decoder_create(uint32_t backend, const DecoderDesc* desc, GpuModel** model) {
    if (desc == nullptr || model == nullptr) {
        return synapse_kv::record(SYNAPSE_KV_NULL_POINTER, "null pointer: model description or output");
    }
    // DecoderPlan::new runs before the backend is chosen (ffi.rs:122-137).
    const int32_t status = synapse_kv::guarded([&] { synapse_kv::validate(*desc); });
    if (status != SYNAPSE_KV_OK) {
        return status;
    }
    if (backend != SYNAPSE_GPU_BACKEND_HIP) {
        return unsupported_backend(backend);
    }
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) {
        (void)hipGetLastError();
        return synapse_kv::record(SYNAPSE_KV_UNAVAILABLE, "no HIP device is available");
    }
    return synapse_kv_decoder_create(desc, device, model);
}

int32_t synapse_gpu_decoder_forward(GpuModel* model, const BatchToken* tokens, size_t count, float* logits,
                                    size_t logits_capacity) {
    return synapse_kv_decoder_forward(model, tokens, count, logits, logits_capacity);
}

void synapse_gpu_decoder_destroy(GpuModel* model) { synapse_kv_decoder_destroy(model); }

uint64_t synapse_gpu_decoder_kv_bytes(const GpuModel* model) { return synapse_kv_decoder_kv_bytes(model); }

int32_t synapse_gpu_decoder_reserve(GpuModel* model, uint32_t slot, uint32_t positions) {
    return synapse_kv_decoder_reserve(model, slot, positions);
}

}  // extern "C"
