// Host half of the Q8_0 projections: the weights handle (upload and repack of GGML Q8_0 matrices), validation of a
// projection against matmul_args' rules (common.metal:54-71, locate_segment :138-146) and its launch.
//
// The reference binds the mapped model file and passes byte offsets per matrix (GpuLayoutMapping.cs:14-32,
// MatmulSegment params.rs); here the offsets select the matrices once, at upload, and a projection names them by
// index.

#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "abi_support.h"
#include "kv_internal.h"
#include "kquant_layout.h"
#include "q8_layout.h"

namespace synapse_kv {
namespace {

struct DeviceMatrix {
    uint32_t rows = 0;
    uint32_t columns = 0;
    size_t codes = 0;   // byte offsets into the weights' device memory
    size_t scales = 0;
    size_t bias = 0;
    bool has_bias = false;
    uint32_t encoding = kEncodingQ8_0;  // GGML type id
};

size_t align_to(size_t value, size_t alignment) { return (value + alignment - 1) / alignment * alignment; }

}  // namespace
}  // namespace synapse_kv

struct SynapseKvWeights {
    int device = 0;
    hipStream_t stream = nullptr;
    uint8_t* memory = nullptr;
    size_t bytes = 0;
    std::vector<synapse_kv::DeviceMatrix> matrices;
    std::vector<const void*> checked_pointers;  // device addresses that passed the check, most recent first
    __bf16* parts = nullptr;  // scratch: the split input (prompt runs) or the per-slice sums (decode)
    size_t parts_bytes = 0;

    ~SynapseKvWeights() {
        if (memory != nullptr) {
            (void)hipSetDevice(device);
            (void)hipStreamSynchronize(stream);
            (void)hipFree(memory);
        }
        if (parts != nullptr) {
            (void)hipFree(parts);
        }
    }
};

namespace synapse_kv {
namespace {

void check_device_pointer(SynapseKvWeights& weights, const void* pointer, const char* name) {
    if (pointer == nullptr) {
        fail(SYNAPSE_KV_NULL_POINTER, std::string("null pointer: ") + name);
    }
    auto& seen = weights.checked_pointers;
    if (std::find(seen.begin(), seen.end(), pointer) != seen.end()) {
        return;
    }
    hipPointerAttribute_t attributes{};
    if (hipPointerGetAttributes(&attributes, pointer) != hipSuccess || attributes.type != hipMemoryTypeDevice) {
        (void)hipGetLastError();
        invalid(std::string(name) + " must be device memory");
    }
    seen.insert(seen.begin(), pointer);
    if (seen.size() > 16) {
        seen.pop_back();
    }
}

void create_weights(const uint8_t* blob, uint64_t blob_bytes, const SynapseKvMatrix* matrices, const uint32_t* encodings,
                    uint32_t count, SynapseKvWeights** out) {
    if (count == 0) {
        invalid("at least one matrix");
    }
    std::vector<DeviceMatrix> layout(count);
    size_t total = 0;
    for (uint32_t index = 0; index < count; ++index) {
        const SynapseKvMatrix& m = matrices[index];
        const uint32_t encoding = encodings != nullptr ? encodings[index] : kEncodingQ8_0;
        const std::string name = "matrix " + std::to_string(index);
        if (encoding != kEncodingQ8_0 && !is_kquant(encoding)) {
            fail(SYNAPSE_KV_UNAVAILABLE, name + ": the kernels implement Q8_0, Q4_K, and Q6_K matrices, not GGML type " +
                                             std::to_string(encoding));
        }
        const uint32_t block_values = static_cast<uint32_t>(ggml_block_values(encoding));
        if (m.rows == 0 || m.columns == 0 || m.columns % block_values != 0) {
            invalid(name + ": rows must be positive and columns a positive multiple of " + std::to_string(block_values));
        }
        const uint64_t weight_bytes = ggml_matrix_bytes(encoding, m.rows, m.columns);
        if (m.weight > blob_bytes || weight_bytes > blob_bytes - m.weight) {
            invalid(name + ": its rows extend past the blob");
        }
        if (m.bias != SYNAPSE_KV_NO_BIAS &&
            (m.bias > blob_bytes || static_cast<uint64_t>(m.rows) * 4 > blob_bytes - m.bias || m.bias % 4 != 0)) {
            invalid(name + ": its biases extend past the blob or are not 4-byte aligned");
        }
        DeviceMatrix& d = layout[index];
        d.rows = m.rows;
        d.columns = m.columns;
        const size_t tiles = static_cast<size_t>(q8_tiles(static_cast<int>(m.rows))) * q8_chunks(static_cast<int>(m.columns));
        d.encoding = encoding;
        d.codes = total;
        total = align_to(total + tiles * tile_code_bytes(encoding), 256);
        d.scales = total;
        total = align_to(total + tiles * tile_scale_bytes(encoding), 256);
        d.has_bias = m.bias != SYNAPSE_KV_NO_BIAS;
        if (d.has_bias) {
            d.bias = total;
            total = align_to(total + static_cast<size_t>(m.rows) * 4, 256);
        }
    }
    std::vector<uint8_t> staging(total, 0);
    for (uint32_t index = 0; index < count; ++index) {
        const SynapseKvMatrix& m = matrices[index];
        const DeviceMatrix& d = layout[index];
        if (is_kquant(d.encoding)) {
            kq_repack(d.encoding, blob + m.weight, static_cast<int>(m.rows), static_cast<int>(m.columns),
                      staging.data() + d.codes, staging.data() + d.scales);
        } else {
            q8_repack(blob + m.weight, static_cast<int>(m.rows), static_cast<int>(m.columns), staging.data() + d.codes,
                      reinterpret_cast<uint16_t*>(staging.data() + d.scales));
        }
        if (d.has_bias) {
            std::memcpy(staging.data() + d.bias, blob + m.bias, static_cast<size_t>(m.rows) * 4);
        }
    }
    auto* weights = new SynapseKvWeights();
    try {
        check_hip(hipGetDevice(&weights->device), "current device");
        weights->bytes = total;
        weights->matrices = std::move(layout);
        check_hip(hipMalloc(reinterpret_cast<void**>(&weights->memory), std::max<size_t>(total, 1)), "weights");
        check_hip(hipMemcpy(weights->memory, staging.data(), total, hipMemcpyHostToDevice), "weights upload");
    } catch (...) {
        delete weights;
        throw;
    }
    *out = weights;
}

// Scratch bytes of a prompt run's split input (whole 16-token tiles: the GEMM reads every column of a tile, and a
// token past the last only feeds an output that is never written), without and with the Q4_K input sums.
size_t split_parts_bytes(uint32_t tokens, int32_t padded_columns) {
    return static_cast<size_t>((tokens + 15) / 16) * 16 * padded_columns * 3 * sizeof(__bf16);
}

size_t split_sums_bytes(uint32_t tokens, int32_t padded_columns) {
    return static_cast<size_t>((tokens + 15) / 16) * 16 * (padded_columns / 8) * sizeof(float);
}

// Grows the weights' scratch to at least `needed` bytes (contents not kept).
void ensure_scratch(SynapseKvWeights& weights, size_t needed) {
    if (needed <= weights.parts_bytes) {
        return;
    }
    // Work already queued may still read the old scratch.
    check_hip(hipStreamSynchronize(weights.stream), "drain before reallocation");
    if (weights.parts != nullptr) {
        check_hip(hipFree(weights.parts), "projection scratch");
        weights.parts = nullptr;
        weights.parts_bytes = 0;
    }
    check_hip(hipMalloc(reinterpret_cast<void**>(&weights.parts), needed), "projection scratch");
    weights.parts_bytes = needed;
}

// One launch over segments [first, first + count) of the projection, which share an encoding. With `presplit` (a
// prompt run) the input is already split in the scratch and `input` is not read.
DeferredSums launch_run(SynapseKvWeights& weights, const SynapseKvProjection& p, uint32_t first, uint32_t count,
                        const float* input, float* output, bool reduce = true, const SplitInput* presplit = nullptr,
                        const NormInput* norm = nullptr, float* squares = nullptr) {
    ProjectionArgs args{};
    if (norm != nullptr) {
        args.norm = *norm;
    }
    args.squares = squares;
    int tiles = 0;
    uint32_t columns = 0;
    for (uint32_t s = 0; s < count; ++s) {
        const DeviceMatrix& m = weights.matrices[p.matrix[first + s]];
        columns = m.columns;
        ProjectionSegment& seg = args.segment[s];
        seg.codes = weights.memory + m.codes;
        seg.scales = weights.memory + m.scales;
        seg.bias = m.has_bias ? reinterpret_cast<const float*>(weights.memory + m.bias) : nullptr;
        seg.rows = static_cast<int32_t>(m.rows);
        seg.first_tile = tiles;
        seg.out_column = static_cast<int32_t>(p.out_column[first + s]);
        seg.encoding = m.encoding;
        tiles += q8_tiles(static_cast<int>(m.rows));
    }
    uint32_t encoding = weights.matrices[p.matrix[first]].encoding;
    for (uint32_t s = 1; s < count; ++s) {
        if (args.segment[s].encoding != encoding) {
            encoding = kEncodingMixedK;  // a decode run over Q4_K and Q6_K segments
        }
    }
    args.encoding = encoding;
    args.segments = static_cast<int32_t>(count);
    args.columns = static_cast<int32_t>(columns);
    args.chunks = q8_chunks(static_cast<int>(columns));
    args.tokens = static_cast<int32_t>(p.tokens);
    args.in_stride = static_cast<int32_t>(p.in_stride);
    args.out_stride = static_cast<int32_t>(p.out_stride);
    args.accumulate = static_cast<int32_t>(p.accumulate);
    args.input = input;
    args.output = output;
    args.padded_columns = args.chunks * kQ8ChunkColumns;
    args.total_tiles = tiles;
    args.slices = projection_decode_slices(args.chunks);
    args.partial_stride = static_cast<int64_t>(tiles) * kQ8TileRows;
    // Scratch: decode keeps per-slice sums ([slices][16][rows]); prompt runs the input's bf16 split, followed for
    // Q4_K by the sums of 8 inputs (SplitInput).
    const size_t parts_bytes = split_parts_bytes(p.tokens, args.padded_columns);
    if (presplit != nullptr) {
        args.parts = presplit->parts;
        args.partials = nullptr;
        args.sums = encoding == kEncodingQ4K ? presplit->sums : nullptr;
        if (encoding == kEncodingQ4K && args.sums == nullptr) {
            invalid("a Q4_K prompt run needs the input sums in its split");
        }
    } else {
        ensure_scratch(weights, p.tokens <= 16 ? static_cast<size_t>(args.slices) * 16 * args.partial_stride * sizeof(float)
                                               : parts_bytes + (encoding == kEncodingQ4K
                                                                    ? split_sums_bytes(p.tokens, args.padded_columns)
                                                                    : 0));
        args.parts = weights.parts;
        args.partials = reinterpret_cast<float*>(weights.parts);
        args.sums = p.tokens > 16 && encoding == kEncodingQ4K
                        ? reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(weights.parts) + parts_bytes)
                        : nullptr;
    }
    check_hip(launch_projection(Launch{weights.stream, nullptr, nullptr}, args, tiles, reduce, presplit == nullptr),
              "projection");
    DeferredSums sums;
    sums.deferred = !reduce && p.tokens <= 16;
    sums.partials = args.partials;
    sums.stride = args.partial_stride;
    sums.slices = args.slices;
    for (uint32_t s = 0; s < count; ++s) {
        sums.first_row[s] = args.segment[s].first_tile * kQ8TileRows;
    }
    return sums;
}

void validate_projection(SynapseKvWeights& weights, const SynapseKvProjection& p, const float* input, float* output) {
    if (p.segments < 1 || p.segments > 3) {
        invalid("a projection has 1..3 segments");
    }
    if (p.tokens == 0 || p.accumulate > 1 || p.reserved != 0) {
        invalid("tokens must be positive, accumulate 0 or 1 and reserved 0");
    }
    uint32_t columns = 0;
    for (uint32_t s = 0; s < p.segments; ++s) {
        if (p.matrix[s] >= weights.matrices.size()) {
            invalid("segment " + std::to_string(s) + " names matrix " + std::to_string(p.matrix[s]) + " of " +
                    std::to_string(weights.matrices.size()));
        }
        const DeviceMatrix& m = weights.matrices[p.matrix[s]];
        if (s == 0) {
            columns = m.columns;
        } else if (m.columns != columns) {
            invalid("the segments' matrices must have equal column counts");
        }
        if (static_cast<uint64_t>(p.out_column[s]) + m.rows > p.out_stride) {
            invalid("segment " + std::to_string(s) + " writes past out_stride");
        }
    }
    if (p.in_stride < columns || p.in_stride % 4 != 0) {
        invalid("in_stride must be a multiple of 4 and hold the " + std::to_string(columns) + " input columns");
    }
    if (reinterpret_cast<uintptr_t>(input) % 16 != 0) {
        invalid("input must be 16-byte aligned");
    }
    check_hip(hipSetDevice(weights.device), "set device");
    check_device_pointer(weights, input, "input");
    check_device_pointer(weights, output, "output");
}

// Consecutive segments of one encoding share a launch (the kernels are specialised per encoding); decode runs
// (at most 16 tokens) also put Q4_K and Q6_K segments in one launch.
void project_runs(SynapseKvWeights& weights, const SynapseKvProjection& p, const float* input, float* output,
                  const SplitInput* presplit, const NormInput* norm = nullptr) {
    auto joins = [&](uint32_t a, uint32_t b) {
        const uint32_t x = weights.matrices[p.matrix[a]].encoding;
        const uint32_t y = weights.matrices[p.matrix[b]].encoding;
        return x == y || (p.tokens <= 16 && is_kquant(x) && is_kquant(y));
    };
    uint32_t first = 0;
    while (first < p.segments) {
        uint32_t count = 1;
        while (first + count < p.segments && joins(first, first + count)) {
            ++count;
        }
        launch_run(weights, p, first, count, input, output, true, presplit, norm);
        first += count;
    }
}

void project(SynapseKvWeights& weights, const SynapseKvProjection& p, const float* input, float* output) {
    validate_projection(weights, p, input, output);
    project_runs(weights, p, input, output, nullptr);
}

}  // namespace

DeferredSums project_deferred(SynapseKvWeights& weights, const SynapseKvProjection& p, const float* input,
                              float* output) {
    validate_projection(weights, p, input, output);
    bool single = p.tokens <= 16;
    for (uint32_t s = 0; s < p.segments; ++s) {
        const DeviceMatrix& m = weights.matrices[p.matrix[s]];
        const uint32_t first_encoding = weights.matrices[p.matrix[0]].encoding;
        single = single && !m.has_bias &&
                 (m.encoding == first_encoding || (is_kquant(m.encoding) && is_kquant(first_encoding)));
    }
    if (!single) {
        project(weights, p, input, output);
        return DeferredSums{};
    }
    return launch_run(weights, p, 0, p.segments, input, output, false);
}

void project_normalized(SynapseKvWeights& weights, const SynapseKvProjection& p, const float* input, float* output,
                        const NormInput& norm) {
    validate_projection(weights, p, input, output);
    if (p.tokens > 16 || norm.weight == nullptr || norm.squares == nullptr || norm.parts < 1 ||
        norm.parts > kNormSquaresStride || norm.columns != static_cast<int32_t>(weights.matrices[p.matrix[0]].columns) ||
        (norm.parts - 1) * kNormSquaresColumns >= norm.columns || norm.parts * kNormSquaresColumns < norm.columns) {
        invalid("a normalized projection takes at most 16 tokens and the squares of its input columns");
    }
    project_runs(weights, p, input, output, nullptr, &norm);
}

void project_with_squares(SynapseKvWeights& weights, const SynapseKvProjection& p, const float* input, float* output,
                          float* squares) {
    validate_projection(weights, p, input, output);
    const DeviceMatrix& m = weights.matrices[p.matrix[0]];
    if (p.tokens > 16 || p.segments != 1 || squares == nullptr || p.out_column[0] != 0 || m.rows != p.out_stride ||
        (m.rows + kNormSquaresColumns - 1) / kNormSquaresColumns > static_cast<uint32_t>(kNormSquaresStride)) {
        invalid("a projection with squares takes at most 16 tokens and one matrix filling its output rows");
    }
    launch_run(weights, p, 0, 1, input, output, true, nullptr, nullptr, squares);
}

SplitInput prepare_split(SynapseKvWeights& weights, const SynapseKvProjection& p) {
    if (p.tokens <= 16 || p.segments < 1 || p.segments > 3 || p.matrix[0] >= weights.matrices.size()) {
        invalid("a split input serves a prompt run (more than 16 tokens) of 1..3 valid segments");
    }
    bool sums = false;
    for (uint32_t s = 0; s < p.segments; ++s) {
        if (p.matrix[s] >= weights.matrices.size()) {
            invalid("segment " + std::to_string(s) + " names matrix " + std::to_string(p.matrix[s]) + " of " +
                    std::to_string(weights.matrices.size()));
        }
        sums = sums || weights.matrices[p.matrix[s]].encoding == kEncodingQ4K;
    }
    const int32_t chunks = q8_chunks(static_cast<int>(weights.matrices[p.matrix[0]].columns));
    const int32_t padded = chunks * kQ8ChunkColumns;
    const size_t parts_bytes = split_parts_bytes(p.tokens, padded);
    check_hip(hipSetDevice(weights.device), "set device");
    ensure_scratch(weights, parts_bytes + (sums ? split_sums_bytes(p.tokens, padded) : 0));
    SplitInput split;
    split.parts = weights.parts;
    split.sums = sums ? reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(weights.parts) + parts_bytes) : nullptr;
    split.chunks = chunks;
    return split;
}

void project_split(SynapseKvWeights& weights, const SynapseKvProjection& p, const SplitInput& split, float* output) {
    if (p.tokens <= 16) {
        invalid("a split input serves a prompt run (more than 16 tokens)");
    }
    // validate_projection checks the input pointer too: the split scratch stands in for it (it is not read).
    validate_projection(weights, p, reinterpret_cast<const float*>(split.parts), output);
    project_runs(weights, p, nullptr, output, &split);
}

}  // namespace synapse_kv

using namespace synapse_kv;

extern "C" {

int32_t synapse_kv_weights_create(const uint8_t* blob, uint64_t blob_bytes, const SynapseKvMatrix* matrices,
                                  uint32_t count, SynapseKvWeights** weights) {
    if (blob == nullptr || matrices == nullptr || weights == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: blob, matrices or output");
    }
    return guarded([&] { create_weights(blob, blob_bytes, matrices, nullptr, count, weights); });
}

int32_t synapse_kv_weights_create_encoded(const uint8_t* blob, uint64_t blob_bytes, const SynapseKvMatrix* matrices,
                                          const uint32_t* encodings, uint32_t count, SynapseKvWeights** weights) {
    if (blob == nullptr || matrices == nullptr || weights == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: blob, matrices or output");
    }
    return guarded([&] { create_weights(blob, blob_bytes, matrices, encodings, count, weights); });
}

void synapse_kv_weights_destroy(SynapseKvWeights* weights) { delete weights; }

uint64_t synapse_kv_weights_bytes(const SynapseKvWeights* weights) { return weights == nullptr ? 0 : weights->bytes; }

int32_t synapse_kv_weights_set_stream(SynapseKvWeights* weights, void* stream) {
    if (weights == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: weights");
    }
    return guarded([&] {
        check_hip(hipSetDevice(weights->device), "set device");
        check_hip(hipStreamSynchronize(weights->stream), "stream switch");
        weights->stream = static_cast<hipStream_t>(stream);
    });
}

int32_t synapse_kv_project(SynapseKvWeights* weights, const SynapseKvProjection* projection, const float* input,
                           float* output) {
    if (weights == nullptr || projection == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: weights or projection");
    }
    return guarded([&] { project(*weights, *projection, input, output); });
}

int32_t synapse_kv_weights_read(SynapseKvWeights* weights, uint32_t index, uint8_t* blocks, uint64_t bytes) {
    if (weights == nullptr || blocks == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: weights or blocks");
    }
    return guarded([&] {
        if (index >= weights->matrices.size()) {
            invalid("matrix " + std::to_string(index) + " of " + std::to_string(weights->matrices.size()));
        }
        const DeviceMatrix& m = weights->matrices[index];
        if (m.encoding != kEncodingQ8_0) {
            fail(SYNAPSE_KV_UNAVAILABLE, "matrix " + std::to_string(index) +
                                             " is a K-quant matrix; read-back returns Q8_0 blocks only");
        }
        const uint64_t needed = static_cast<uint64_t>(m.rows) * (m.columns / kQ8BlockElements) * kQ8BlockBytes;
        if (bytes < needed) {
            invalid("the matrix needs " + std::to_string(needed) + " bytes");
        }
        const size_t tiles = static_cast<size_t>(q8_tiles(static_cast<int>(m.rows))) * q8_chunks(static_cast<int>(m.columns));
        std::vector<uint8_t> codes(tiles * kQ8TileBytes);
        std::vector<uint16_t> scales(tiles * kQ8TileScales);
        check_hip(hipSetDevice(weights->device), "set device");
        check_hip(hipStreamSynchronize(weights->stream), "weights read");
        check_hip(hipMemcpy(codes.data(), weights->memory + m.codes, codes.size(), hipMemcpyDeviceToHost), "weights read");
        check_hip(hipMemcpy(scales.data(), weights->memory + m.scales, scales.size() * 2, hipMemcpyDeviceToHost),
                  "weights read");
        q8_unpack(codes.data(), scales.data(), static_cast<int>(m.rows), static_cast<int>(m.columns), blocks);
    });
}

}  // extern "C"
