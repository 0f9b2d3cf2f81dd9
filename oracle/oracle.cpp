// Test infrastructure only: a CPU restatement of Synapse's KV-cache and attention path, used as the parity
// oracle for the HIP library and as the CPU baseline in the benchmark. Nothing in the shipped library links,
// loads or calls this file. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it.
//
// Every function cites the reference file:line it restates (paths relative to the managedcode/Synapse tree).
// Pinning (how each part is checked against something other than itself) is in tests/test_oracle_*.py.
//
// Build: oracle/Makefile (g++ -O3 -ffp-contract=off; no fast-math, so float expressions round exactly as the
// reference's C# does: one rounding per operation, no fused multiply-add).

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <thread>
#include <vector>

namespace {

uint32_t float_bits(float value) {
    uint32_t bits;
    std::memcpy(&bits, &value, 4);
    return bits;
}

float bits_float(uint32_t bits) {
    float value;
    std::memcpy(&value, &bits, 4);
    return value;
}

// IEEE-754 binary32 -> binary16, round to nearest, ties to even. This is the Metal `(half)` cast the reference
// applies when it appends to an FP16 slot (native/synapse-gpu/src/Features/GpuKernels/metal/shaders/
// elementwise.metal:97-98, 116-117). NaN keeps the top mantissa bits and stays NaN.
uint16_t f32_to_f16(float value) {
    const uint32_t x = float_bits(value);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t magnitude = x & 0x7fffffffu;
    if (magnitude > 0x7f800000u) {
        uint32_t payload = 0x7c00u | ((magnitude & 0x7fffffu) >> 13);
        if (payload == 0x7c00u) {
            payload = 0x7c01u;
        }
        return static_cast<uint16_t>(sign | payload);
    }
    if (magnitude >= 0x477ff000u) {  // >= 65520 rounds to infinity
        return static_cast<uint16_t>(sign | 0x7c00u);
    }
    if (magnitude < 0x38800000u) {  // below 2^-14: binary16 subnormal or zero
        if (magnitude <= 0x33000000u) {  // <= 2^-25: ties to the even zero
            return static_cast<uint16_t>(sign);
        }
        const uint32_t exponent = magnitude >> 23;
        const uint32_t mantissa = (magnitude & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - exponent;  // value / 2^-24 = mantissa * 2^(exponent - 126)
        uint32_t result = mantissa >> shift;
        const uint32_t rest = mantissa & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rest > half || (rest == half && (result & 1u))) {
            ++result;
        }
        return static_cast<uint16_t>(sign | result);
    }
    uint32_t result = ((magnitude >> 23) - 112u) << 10 | ((magnitude >> 13) & 0x3ffu);
    const uint32_t rest = magnitude & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (result & 1u))) {
        ++result;  // a carry out of the mantissa correctly bumps the exponent
    }
    return static_cast<uint16_t>(sign | result);
}

// Fp16.ToSingle (src/Synapse.Runtime/Features/CpuKernels/Fp16.cs:17-23): shift the magnitude into FP32 position
// and rescale by 2^112; exact for every finite binary16 value including subnormals and zero.
float f16_to_f32(uint16_t bits) {
    const float magnitude = bits_float(static_cast<uint32_t>(bits & 0x7fffu) << 13) * bits_float(0x77800000u);
    return (bits & 0x8000u) == 0 ? magnitude : -magnitude;
}

// ADR-017 growth: Qwen2KvCache.NextCapacity (src/Synapse.Runtime/Features/TextGeneration/Qwen2/
// Qwen2KvCache.cs:91-95), identical to DecoderShape::next_capacity (native/synapse-gpu/src/Features/
// GpuKernels/decoder.rs:221-226).
int next_capacity(int needed, int current, int growth, int maximum) {
    const long long rounded_ll = (static_cast<long long>(needed) + growth - 1) / growth * growth;
    const int rounded = static_cast<int>(std::min<long long>(maximum, rounded_ll));
    return std::min(maximum, std::max(rounded, std::min(maximum, current * 2)));
}

// Reservation rounding of Qwen2KvCache.Reserve (Qwen2KvCache.cs:63).
int reserve_rounded(int positions, int growth, int maximum) {
    const long long rounded = (static_cast<long long>(positions) + growth - 1) / growth * growth;
    return static_cast<int>(std::min<long long>(maximum, rounded));
}

constexpr int kOk = 0;
constexpr int kNull = 1;
constexpr int kInvalid = 2;
constexpr int kOutOfMemory = 5;

// --- Dense growable cache: Qwen2KvCache (Qwen2KvCache.cs:8-134) -------------------------------------------------

struct DenseCache {
    int layers;
    int maximum;
    int kv_width;
    int growth;
    int allocated = 0;
    std::vector<std::vector<float>> keys;
    std::vector<std::vector<float>> values;
};

// Resize (Qwen2KvCache.cs:100-110): never shrinks an array on this path, publishes capacity last.
void dense_resize(DenseCache& cache, int positions) {
    const size_t length = static_cast<size_t>(positions) * cache.kv_width;
    for (int layer = 0; layer < cache.layers; ++layer) {
        cache.keys[layer].resize(std::max(length, cache.keys[layer].size()), 0.0f);
        cache.values[layer].resize(std::max(length, cache.values[layer].size()), 0.0f);
    }
    cache.allocated = positions;
}

// Contract (Qwen2KvCache.cs:113-133): fresh arrays of the smaller length holding the prefix.
void dense_contract(DenseCache& cache, int positions) {
    const size_t length = static_cast<size_t>(positions) * cache.kv_width;
    for (int layer = 0; layer < cache.layers; ++layer) {
        std::vector<float> keys(cache.keys[layer].begin(), cache.keys[layer].begin() + length);
        std::vector<float> values(cache.values[layer].begin(), cache.values[layer].begin() + length);
        cache.keys[layer].swap(keys);
        cache.values[layer].swap(values);
    }
    cache.allocated = positions;
}

// --- Paged FP16/FP32 cache: the a1/a3 policy at page granularity ------------------------------------------------
//
// The reference holds one contiguous buffer per slot (metal/decoder.rs:21-258); this restatement extends it to a
// pool of fixed-size pages with a block table per slot, page reference counts and a free stack, keeping:
//   * the capacity policy of Qwen2KvCache.Reserve/NextCapacity and MetalDecoder::reserve (grow when the need
//     exceeds the capacity; contract when the rounded need is at most a quarter; keep the prefix),
//   * batched growth per step, slots in ascending order (MetalDecoder::prepare_slots, metal/decoder.rs:192-223),
//   * zero-filled new storage (metal/decoder.rs:227-241),
//   * DirectSessionPrefix reuse (DirectSessionPrefix.cs:16-41) as copy-on-write page sharing,
//   * rollback truncation (native/synapse-core/src/Features/SessionState/kv_pages.rs:158-177).
// Determinism rules (the specification the GPU table kernels follow):
//   * the free stack starts as [max_pages-1, ..., 1, 0]; a pop takes the top, so the first pop is page 0;
//   * growth pops one page per new logical page, logical pages ascending;
//   * contraction walks logical pages descending, decrements each reference count and pushes a page whose
//     count reaches zero;
//   * a step grows slots in ascending slot order, then copies shared pages on write in token order: a token
//     whose page has a reference count above one pops a fresh page, copies the old page into it and drops
//     one reference from the old page;
//   * a fork shares the source's pages that hold its written positions, one reference each;
//   * any failing call leaves every table, count and page unchanged.

struct PagedCache {
    int layers;
    int heads;
    int kv_heads;
    int head_dim;
    int maximum;
    int growth;
    int page_tokens;
    int precision;  // 0 = FP32, 1 = FP16
    int max_sequences;
    int max_pages;
    int step_tokens;
    int pages_per_slot;
    size_t page_elements;
    std::vector<int> capacity;
    std::vector<int> length;
    std::vector<std::vector<int>> table;
    std::vector<int> refcount;
    std::vector<int> free_stack;
    std::vector<std::vector<float>> page_f32;
    std::vector<std::vector<uint16_t>> page_f16;
    std::vector<int32_t> step;  // last prepared step: 4 ints per token (slot, token, position, logits_row)
};

int pages_for(const PagedCache& cache, int positions) {
    return (positions + cache.page_tokens - 1) / cache.page_tokens;
}

void page_zero(PagedCache& cache, int page) {
    if (cache.precision == 0) {
        cache.page_f32[page].assign(cache.page_elements, 0.0f);
    } else {
        cache.page_f16[page].assign(cache.page_elements, 0);
    }
}

void page_copy(PagedCache& cache, int from, int to) {
    if (cache.precision == 0) {
        cache.page_f32[to] = cache.page_f32[from];
    } else {
        cache.page_f16[to] = cache.page_f16[from];
    }
}

int page_pop(PagedCache& cache) {
    const int page = cache.free_stack.back();
    cache.free_stack.pop_back();
    cache.refcount[page] = 1;
    return page;
}

// Pages a resize of `slot` to `positions` would take from the free stack (0 for a contraction).
int resize_need(const PagedCache& cache, int slot, int positions) {
    const int have = pages_for(cache, cache.capacity[slot]);
    const int want = pages_for(cache, positions);
    return std::max(0, want - have);
}

void paged_resize(PagedCache& cache, int slot, int positions) {
    const int have = pages_for(cache, cache.capacity[slot]);
    const int want = pages_for(cache, positions);
    for (int page = have; page < want; ++page) {
        const int id = page_pop(cache);
        page_zero(cache, id);
        cache.table[slot][page] = id;
    }
    for (int page = have - 1; page >= want; --page) {
        const int id = cache.table[slot][page];
        if (--cache.refcount[id] == 0) {
            cache.free_stack.push_back(id);
        }
        cache.table[slot][page] = -1;
    }
    cache.capacity[slot] = positions;
    cache.length[slot] = std::min(cache.length[slot], positions);
}

// Element index of (layer, key|value, kv_head, token in page, dim) inside a page, logical order.
size_t page_index(const PagedCache& cache, int layer, int which, int kv_head, int token, int dim) {
    return ((((static_cast<size_t>(layer) * 2 + which) * cache.kv_heads + kv_head) * cache.page_tokens + token) *
            cache.head_dim) + dim;
}

struct Token {
    int32_t slot;
    int32_t token;
    int32_t position;
    int32_t logits_row;
};

// --- Attention restatements ------------------------------------------------------------------------------------

// Qwen2Attention.Dot (Qwen2Attention.cs:225-234): sequential FP32 sum.
float dot_scalar(const float* left, const float* right, int count) {
    float sum = 0.0f;
    for (int index = 0; index < count; ++index) {
        sum += left[index] * right[index];
    }
    return sum;
}

// Qwen2CpuAttention.Dot (Qwen2CpuAttention.cs:116-132): four lanes, then a horizontal sum. The exact order of
// Vector128.Sum is not observable without running .NET; ((s0 + s1) + (s2 + s3)) is assumed (tolerance only).
float dot_lanes(const float* left, const float* right, int count) {
    float lane[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int index = 0;
    for (; index <= count - 4; index += 4) {
        for (int j = 0; j < 4; ++j) {
            lane[j] = lane[j] + left[index + j] * right[index + j];
        }
    }
    float total = (lane[0] + lane[1]) + (lane[2] + lane[3]);
    for (; index < count; ++index) {
        total += left[index] * right[index];
    }
    return total;
}

// Which key positions a query row sees: keys 0..position; `valid` masks individual keys when given.
struct KeyView {
    const float* keys;    // [positions][kv_heads][head_dim]
    const float* values;  // [positions][kv_heads][head_dim]
    int kv_heads;
    int head_dim;
};

const float* key_row(const KeyView& view, int position, int kv_head) {
    return view.keys + (static_cast<size_t>(position) * view.kv_heads + kv_head) * view.head_dim;
}

const float* value_row(const KeyView& view, int position, int kv_head) {
    return view.values + (static_cast<size_t>(position) * view.kv_heads + kv_head) * view.head_dim;
}

// Qwen2CpuAttention.Attend for one (token, head) item (Qwen2CpuAttention.cs:82-113) with its Softmax (:152-172,
// multiply by 1/sum) and MultiplyAdd (:135-149). `scores` must hold position + 1 floats. `attended` (null: every
// position) is a KV page mask: unattended positions score -infinity and add no value.
void attend_managed(const KeyView& view, const float* query, int kv_head, int position, float scale, float* scores,
                    float* destination, const uint8_t* attended = nullptr) {
    const int d = view.head_dim;
    for (int cached = 0; cached <= position; ++cached) {
        scores[cached] = attended == nullptr || attended[cached]
                             ? dot_lanes(query, key_row(view, cached, kv_head), d) * scale
                             : -std::numeric_limits<float>::infinity();
    }
    float maximum = scores[0];
    for (int index = 1; index <= position; ++index) {
        maximum = std::max(maximum, scores[index]);
    }
    float sum = 0.0f;
    for (int index = 0; index <= position; ++index) {
        scores[index] = std::exp(scores[index] - maximum);
        sum += scores[index];
    }
    const float inverse = 1.0f / sum;
    for (int index = 0; index <= position; ++index) {
        scores[index] *= inverse;
    }
    for (int dim = 0; dim < d; ++dim) {
        destination[dim] = 0.0f;
    }
    for (int cached = 0; cached <= position; ++cached) {
        if (attended != nullptr && !attended[cached]) {
            continue;
        }
        const float* value = value_row(view, cached, kv_head);
        const float weight = scores[cached];
        for (int dim = 0; dim < d; ++dim) {
            destination[dim] = destination[dim] + weight * value[dim];
        }
    }
}

struct Pool {
    // Runs body(worker, item) over items on `threads` std::threads in contiguous chunks, like CpuWorkerPool with
    // ChunkedRowWork (src/Synapse.Runtime/Features/CpuKernels/ChunkedRowWork.cs) at alignment 1.
    template <typename Body>
    static void run(int items, int threads, Body body) {
        if (threads <= 1 || items <= 1) {
            for (int item = 0; item < items; ++item) {
                body(0, item);
            }
            return;
        }
        std::atomic<int> next{0};
        const int chunk = std::max(1, items / (threads * 4));
        std::vector<std::thread> pool;
        for (int worker = 0; worker < threads; ++worker) {
            pool.emplace_back([&, worker] {
                for (;;) {
                    const int first = next.fetch_add(chunk);
                    if (first >= items) {
                        return;
                    }
                    const int last = std::min(items, first + chunk);
                    for (int item = first; item < last; ++item) {
                        body(worker, item);
                    }
                }
            });
        }
        for (auto& thread : pool) {
            thread.join();
        }
    }
};

}  // namespace

extern "C" {

// ---- FP16 -----------------------------------------------------------------------------------------------------

void orc_f32_to_f16(const float* input, uint16_t* output, size_t count) {
    for (size_t index = 0; index < count; ++index) {
        output[index] = f32_to_f16(input[index]);
    }
}

void orc_f16_to_f32(const uint16_t* input, float* output, size_t count) {
    for (size_t index = 0; index < count; ++index) {
        output[index] = f16_to_f32(input[index]);
    }
}

// ---- RoPE -----------------------------------------------------------------------------------------------------

// RopeFrequencies constructor + Compute (src/Synapse.Runtime/Features/TextGeneration/RopeFrequencies.cs:20-81) for
// positions 0..positions-1 into [position][head_dim / 2] tables. yarn_factor <= 0 means unscaled.
int orc_rope_table(int head_dim, float theta, float yarn_factor, int yarn_original, int positions, float* cosines,
                   float* sines) {
    if (head_dim <= 0 || (head_dim & 1) != 0 || !std::isfinite(theta) || theta <= 1 || positions < 0) {
        return kInvalid;
    }
    if (cosines == nullptr || sines == nullptr) {
        return kNull;
    }
    const int half = head_dim / 2;
    const float pi = 3.14159265358979323846f;  // MathF.PI
    std::vector<float> mix;
    float magnitude = 1.0f;
    if (yarn_factor > 0) {
        magnitude = 1.0f + (0.1f * std::log(yarn_factor));
        auto correction = [&](float rotations) {
            return static_cast<float>(head_dim) *
                   std::log(static_cast<float>(yarn_original) / (rotations * 2 * pi)) / (2 * std::log(theta));
        };
        const float low = std::max(0.0f, std::floor(correction(32.0f)));
        const float high = std::min(static_cast<float>(head_dim - 1), std::ceil(correction(1.0f)));
        mix.resize(half);
        for (int index = 0; index < half; ++index) {
            const float ramp = (static_cast<float>(index) - low) / std::max(0.001f, high - low);
            mix[index] = 1 - std::min(1.0f, std::max(0.0f, ramp));
        }
    }
    for (int position = 0; position < positions; ++position) {
        for (int index = 0; index < half; ++index) {
            const float exponent = 2.0f * static_cast<float>(index) / static_cast<float>(head_dim);
            const float angle = static_cast<float>(position) / std::pow(theta, exponent);
            const size_t at = static_cast<size_t>(position) * half + index;
            if (mix.empty()) {
                cosines[at] = std::cos(angle);
                sines[at] = std::sin(angle);
                continue;
            }
            const float scaled = (angle / yarn_factor * (1 - mix[index])) + (angle * mix[index]);
            cosines[at] = std::cos(scaled) * magnitude;
            sines[at] = std::sin(scaled) * magnitude;
        }
    }
    return kOk;
}

// Qwen2RopeTable.Apply (src/Synapse.Runtime/Features/TextGeneration/Qwen2/Qwen2CpuState.cs:85-106), also
// Qwen2Attention.ApplyRope (Qwen2Attention.cs:27-49): NeoX rotate-half, separate multiply and add/subtract.
void orc_rope_apply(float* values, int heads, int head_dim, const float* cosines, const float* sines) {
    const int half = head_dim / 2;
    for (int head = 0; head < heads; ++head) {
        float* row = values + static_cast<size_t>(head) * head_dim;
        for (int index = 0; index < half; ++index) {
            const float x = row[index];
            const float y = row[index + half];
            const float first = (x * cosines[index]) - (y * sines[index]);
            const float second = (x * sines[index]) + (y * cosines[index]);
            row[index] = first;
            row[index + half] = second;
        }
    }
}

// ---- Capacity policy ------------------------------------------------------------------------------------------

int orc_next_capacity(int needed, int current, int growth, int maximum) {
    return next_capacity(needed, current, growth, maximum);
}

// ---- Dense cache (Qwen2KvCache) -------------------------------------------------------------------------------

void* orc_dense_create(int layers, int maximum, int kv_width, int growth) {
    if (growth <= 0 || layers <= 0 || kv_width <= 0 || maximum < 0) {
        return nullptr;
    }
    auto* cache = new DenseCache{layers, maximum, kv_width, growth};
    cache->keys.resize(layers);
    cache->values.resize(layers);
    return cache;
}

void orc_dense_destroy(void* handle) { delete static_cast<DenseCache*>(handle); }

// Store (Qwen2KvCache.cs:39-53).
int orc_dense_store(void* handle, int layer, int position, const float* key, const float* value, int width) {
    auto& cache = *static_cast<DenseCache*>(handle);
    if (static_cast<unsigned>(position) >= static_cast<unsigned>(cache.maximum) || width != cache.kv_width ||
        layer < 0 || layer >= cache.layers) {
        return kInvalid;
    }
    if (position >= cache.allocated) {
        dense_resize(cache, next_capacity(position + 1, cache.allocated, cache.growth, cache.maximum));
    }
    std::memcpy(cache.keys[layer].data() + static_cast<size_t>(position) * width, key, width * sizeof(float));
    std::memcpy(cache.values[layer].data() + static_cast<size_t>(position) * width, value, width * sizeof(float));
    return kOk;
}

// Reserve (Qwen2KvCache.cs:56-72).
int orc_dense_reserve(void* handle, int positions) {
    auto& cache = *static_cast<DenseCache*>(handle);
    if (static_cast<unsigned>(positions) > static_cast<unsigned>(cache.maximum)) {
        return kInvalid;
    }
    const int rounded = reserve_rounded(positions, cache.growth, cache.maximum);
    if (positions > cache.allocated) {
        dense_resize(cache, rounded);
    } else if (rounded < cache.allocated && rounded <= cache.allocated / 4) {
        dense_contract(cache, rounded);
    }
    return kOk;
}

// Release (Qwen2KvCache.cs:75-84).
void orc_dense_release(void* handle) {
    auto& cache = *static_cast<DenseCache*>(handle);
    for (int layer = 0; layer < cache.layers; ++layer) {
        cache.keys[layer].clear();
        cache.values[layer].clear();
    }
    cache.allocated = 0;
}

int orc_dense_allocated(void* handle) { return static_cast<DenseCache*>(handle)->allocated; }

// AllocatedBytes (Qwen2KvCache.cs:37).
long long orc_dense_bytes(void* handle) {
    auto& cache = *static_cast<DenseCache*>(handle);
    return 2LL * cache.layers * cache.allocated * cache.kv_width * static_cast<long long>(sizeof(float));
}

// GetKey / GetValue (Qwen2KvCache.cs:86-88).
int orc_dense_get(void* handle, int layer, int position, int head, int head_dim, int value, float* output) {
    auto& cache = *static_cast<DenseCache*>(handle);
    if (layer < 0 || layer >= cache.layers || position < 0 || position >= cache.allocated ||
        (head + 1) * head_dim > cache.kv_width) {
        return kInvalid;
    }
    const auto& source = value ? cache.values[layer] : cache.keys[layer];
    std::memcpy(output, source.data() + static_cast<size_t>(position) * cache.kv_width + head * head_dim,
                head_dim * sizeof(float));
    return kOk;
}

// ---- Paged cache ----------------------------------------------------------------------------------------------

void* orc_paged_create(int layers, int heads, int kv_heads, int head_dim, int maximum, int growth, int page_tokens,
                       int precision, int max_sequences, int max_pages, int step_tokens) {
    if (layers <= 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0 || head_dim <= 0 || maximum <= 0 ||
        page_tokens <= 0 || growth <= 0 || growth % page_tokens != 0 || (precision != 0 && precision != 1) ||
        max_sequences <= 0 || max_pages <= 0 || step_tokens <= 0) {
        return nullptr;
    }
    auto* cache = new PagedCache{layers,        heads,     kv_heads,   head_dim,   maximum,    growth,
                                 page_tokens,   precision, max_sequences, max_pages, step_tokens, 0, 0};
    cache->pages_per_slot = pages_for(*cache, maximum);
    cache->page_elements = static_cast<size_t>(layers) * 2 * kv_heads * page_tokens * head_dim;
    cache->capacity.assign(max_sequences, 0);
    cache->length.assign(max_sequences, 0);
    cache->table.assign(max_sequences, std::vector<int>(cache->pages_per_slot, -1));
    cache->refcount.assign(max_pages, 0);
    for (int page = max_pages - 1; page >= 0; --page) {
        cache->free_stack.push_back(page);
    }
    if (precision == 0) {
        cache->page_f32.resize(max_pages);
    } else {
        cache->page_f16.resize(max_pages);
    }
    return cache;
}

void orc_paged_destroy(void* handle) { delete static_cast<PagedCache*>(handle); }

// Reservation: the Qwen2KvCache.Reserve policy (Qwen2KvCache.cs:56-72) as MetalDecoder::reserve applies it to a
// slot (metal/decoder.rs:164-179).
int orc_paged_reserve(void* handle, int slot, int positions) {
    auto& cache = *static_cast<PagedCache*>(handle);
    if (slot < 0 || slot >= cache.max_sequences || static_cast<unsigned>(positions) > static_cast<unsigned>(cache.maximum)) {
        return kInvalid;
    }
    const int current = cache.capacity[slot];
    const int rounded = reserve_rounded(positions, cache.growth, cache.maximum);
    if (positions > current || (rounded < current && rounded <= current / 4)) {
        if (resize_need(cache, slot, rounded) > static_cast<int>(cache.free_stack.size())) {
            return kOutOfMemory;
        }
        paged_resize(cache, slot, rounded);
    }
    return kOk;
}

// Release (Qwen2KvCache.cs:75-84) for one slot: every page back, capacity and length zero.
int orc_paged_release(void* handle, int slot) {
    auto& cache = *static_cast<PagedCache*>(handle);
    if (slot < 0 || slot >= cache.max_sequences) {
        return kInvalid;
    }
    paged_resize(cache, slot, 0);
    cache.length[slot] = 0;
    return kOk;
}

// Rollback to a shorter committed length (kv_pages.rs:158-177); capacity is kept (ADR-017 reuse).
int orc_paged_truncate(void* handle, int slot, int length) {
    auto& cache = *static_cast<PagedCache*>(handle);
    if (slot < 0 || slot >= cache.max_sequences || length < 0 || length > cache.length[slot]) {
        return kInvalid;
    }
    cache.length[slot] = length;
    return kOk;
}

// Copy-on-write fork: `target` (empty) shares the pages holding `source`'s written positions.
int orc_paged_fork(void* handle, int source, int target) {
    auto& cache = *static_cast<PagedCache*>(handle);
    if (source < 0 || source >= cache.max_sequences || target < 0 || target >= cache.max_sequences ||
        source == target || cache.capacity[target] != 0) {
        return kInvalid;
    }
    const int shared = pages_for(cache, cache.length[source]);
    for (int page = 0; page < shared; ++page) {
        const int id = cache.table[source][page];
        cache.table[target][page] = id;
        ++cache.refcount[id];
    }
    cache.capacity[target] = std::min(cache.maximum, shared * cache.page_tokens);
    cache.length[target] = cache.length[source];
    return kOk;
}

// A step's KV preparation: validate_step bounds (decoder.rs:303-335, without vocabulary and logits checks),
// batched growth per slot (MetalDecoder::prepare_slots, metal/decoder.rs:192-223), then copy-on-write in token
// order. `tokens` holds 4 int32 per token (slot, token, position, logits_row) as BatchToken (decoder.rs:136-141).
int orc_paged_step(void* handle, const int32_t* tokens, int count) {
    auto& cache = *static_cast<PagedCache*>(handle);
    if (tokens == nullptr) {
        return kNull;
    }
    if (count <= 0 || count > cache.step_tokens) {
        return kInvalid;
    }
    std::vector<int> needed(cache.max_sequences, 0);
    for (int index = 0; index < count; ++index) {
        const Token token = reinterpret_cast<const Token*>(tokens)[index];
        if (token.slot < 0 || token.slot >= cache.max_sequences || token.position < 0 ||
            token.position >= cache.maximum) {
            return kInvalid;
        }
        needed[token.slot] = std::max(needed[token.slot], token.position + 1);
    }
    // Dry run: pages the whole step takes, so a failure leaves everything unchanged.
    std::vector<int> grown(cache.max_sequences);
    int pops = 0;
    for (int slot = 0; slot < cache.max_sequences; ++slot) {
        grown[slot] = cache.capacity[slot];
        if (needed[slot] > cache.capacity[slot]) {
            grown[slot] = next_capacity(needed[slot], cache.capacity[slot], cache.growth, cache.maximum);
            pops += resize_need(cache, slot, grown[slot]);
        }
    }
    {
        std::vector<int> references(cache.refcount);
        std::vector<std::vector<char>> owned(cache.max_sequences);
        for (int index = 0; index < count; ++index) {
            const Token token = reinterpret_cast<const Token*>(tokens)[index];
            const int page = token.position / cache.page_tokens;
            if (page >= pages_for(cache, cache.capacity[token.slot])) {
                continue;  // grown this step: exclusive
            }
            auto& mine = owned[token.slot];
            if (mine.empty()) {
                mine.assign(cache.pages_per_slot, 0);
            }
            const int id = cache.table[token.slot][page];
            if (!mine[page] && references[id] > 1) {
                --references[id];
                ++pops;
                mine[page] = 1;
            }
        }
    }
    if (pops > static_cast<int>(cache.free_stack.size())) {
        return kOutOfMemory;
    }
    for (int slot = 0; slot < cache.max_sequences; ++slot) {
        if (grown[slot] != cache.capacity[slot]) {
            paged_resize(cache, slot, grown[slot]);
        }
    }
    for (int index = 0; index < count; ++index) {
        const Token token = reinterpret_cast<const Token*>(tokens)[index];
        const int page = token.position / cache.page_tokens;
        const int id = cache.table[token.slot][page];
        if (cache.refcount[id] > 1) {
            const int fresh = page_pop(cache);
            page_copy(cache, id, fresh);
            --cache.refcount[id];
            cache.table[token.slot][page] = fresh;
        }
    }
    for (int slot = 0; slot < cache.max_sequences; ++slot) {
        cache.length[slot] = std::max(cache.length[slot], needed[slot]);
    }
    cache.step.assign(tokens, tokens + 4 * count);
    return kOk;
}

// Fused RoPE + append of the prepared step for one layer: synapse_rope_kv (metal/shaders/elementwise.metal:73-126)
// over a [tokens][qkv_stride] FP32 row block whose Q heads start at column 0, K heads at heads*head_dim and V
// heads at (heads + kv_heads)*head_dim (DecoderShape::qkv_width, decoder.rs:185-187). Q and K rotate in place;
// K and V are stored in the slot's element type (FP16 round to nearest even). Rotation per Qwen2RopeTable.Apply.
int orc_paged_append_rope(void* handle, int layer, float* qkv, int qkv_stride, const float* cosines,
                          const float* sines) {
    auto& cache = *static_cast<PagedCache*>(handle);
    if (layer < 0 || layer >= cache.layers) {
        return kInvalid;
    }
    const int count = static_cast<int>(cache.step.size() / 4);
    const int d = cache.head_dim;
    const int half = d / 2;
    for (int index = 0; index < count; ++index) {
        const Token token = reinterpret_cast<const Token*>(cache.step.data())[index];
        float* row = qkv + static_cast<size_t>(index) * qkv_stride;
        const float* c = cosines + static_cast<size_t>(token.position) * half;
        const float* s = sines + static_cast<size_t>(token.position) * half;
        orc_rope_apply(row, cache.heads, d, c, s);
        float* keys = row + cache.heads * d;
        float* values = keys + cache.kv_heads * d;
        orc_rope_apply(keys, cache.kv_heads, d, c, s);
        const int page = cache.table[token.slot][token.position / cache.page_tokens];
        const int within = token.position % cache.page_tokens;
        for (int kv_head = 0; kv_head < cache.kv_heads; ++kv_head) {
            for (int dim = 0; dim < d; ++dim) {
                const size_t k_at = page_index(cache, layer, 0, kv_head, within, dim);
                const size_t v_at = page_index(cache, layer, 1, kv_head, within, dim);
                const float k = keys[kv_head * d + dim];
                const float v = values[kv_head * d + dim];
                if (cache.precision == 0) {
                    cache.page_f32[page][k_at] = k;
                    cache.page_f32[page][v_at] = v;
                } else {
                    cache.page_f16[page][k_at] = f32_to_f16(k);
                    cache.page_f16[page][v_at] = f32_to_f16(v);
                }
            }
        }
    }
    return kOk;
}

// Reads positions [first, first + count) of one slot and layer as FP32 [position][kv_head][head_dim] (FP16
// widened per Fp16.ToSingle), or as raw storage bits when `raw` is set (uint16 for FP16, float for FP32).
int orc_paged_gather(void* handle, int slot, int layer, int first, int count, void* keys, void* values, int raw) {
    auto& cache = *static_cast<PagedCache*>(handle);
    if (slot < 0 || slot >= cache.max_sequences || layer < 0 || layer >= cache.layers || first < 0 || count < 0 ||
        first + count > cache.capacity[slot]) {
        return kInvalid;
    }
    const int d = cache.head_dim;
    for (int position = first; position < first + count; ++position) {
        const int page = cache.table[slot][position / cache.page_tokens];
        const int within = position % cache.page_tokens;
        for (int kv_head = 0; kv_head < cache.kv_heads; ++kv_head) {
            for (int dim = 0; dim < d; ++dim) {
                const size_t out = (static_cast<size_t>(position - first) * cache.kv_heads + kv_head) * d + dim;
                const size_t k_at = page_index(cache, layer, 0, kv_head, within, dim);
                const size_t v_at = page_index(cache, layer, 1, kv_head, within, dim);
                if (cache.precision == 0) {
                    static_cast<float*>(keys)[out] = cache.page_f32[page][k_at];
                    static_cast<float*>(values)[out] = cache.page_f32[page][v_at];
                } else if (raw) {
                    static_cast<uint16_t*>(keys)[out] = cache.page_f16[page][k_at];
                    static_cast<uint16_t*>(values)[out] = cache.page_f16[page][v_at];
                } else {
                    static_cast<float*>(keys)[out] = f16_to_f32(cache.page_f16[page][k_at]);
                    static_cast<float*>(values)[out] = f16_to_f32(cache.page_f16[page][v_at]);
                }
            }
        }
    }
    return kOk;
}

int orc_paged_slot(void* handle, int slot, int* capacity, int* length, int* pages) {
    auto& cache = *static_cast<PagedCache*>(handle);
    if (slot < 0 || slot >= cache.max_sequences) {
        return kInvalid;
    }
    *capacity = cache.capacity[slot];
    *length = cache.length[slot];
    *pages = pages_for(cache, cache.capacity[slot]);
    return kOk;
}

// The slot's block table (pages_per_slot entries, -1 where unmapped).
int orc_paged_table(void* handle, int slot, int32_t* output) {
    auto& cache = *static_cast<PagedCache*>(handle);
    if (slot < 0 || slot >= cache.max_sequences) {
        return kInvalid;
    }
    std::copy(cache.table[slot].begin(), cache.table[slot].end(), output);
    return kOk;
}

void orc_paged_refcounts(void* handle, int32_t* output) {
    auto& cache = *static_cast<PagedCache*>(handle);
    std::copy(cache.refcount.begin(), cache.refcount.end(), output);
}

// The free stack bottom to top; returns its size.
int orc_paged_free_list(void* handle, int32_t* output) {
    auto& cache = *static_cast<PagedCache*>(handle);
    std::copy(cache.free_stack.begin(), cache.free_stack.end(), output);
    return static_cast<int>(cache.free_stack.size());
}

// Bytes of the pages in use (shared pages once).
long long orc_paged_kv_bytes(void* handle) {
    auto& cache = *static_cast<PagedCache*>(handle);
    const long long used = cache.max_pages - static_cast<long long>(cache.free_stack.size());
    return used * static_cast<long long>(cache.page_elements) * (cache.precision == 0 ? 4 : 2);
}

// ---- Attention ------------------------------------------------------------------------------------------------

// Qwen2Attention.Execute (Qwen2Attention.cs:5-25; FillScores :51-67, SoftmaxInPlace :102-121 dividing by the
// sum, AccumulateValues :69-89) for one query position: q [heads][head_dim], keys/values [positions][kv][d].
void orc_attention_scalar(const float* query, const float* keys, const float* values, int heads, int kv_heads,
                          int head_dim, int position, float* output) {
    const int group = heads / kv_heads;
    const float scale = 1.0f / std::sqrt(static_cast<float>(head_dim));
    const KeyView view{keys, values, kv_heads, head_dim};
    std::vector<float> scores(position + 1);
    for (int head = 0; head < heads; ++head) {
        const float* q = query + static_cast<size_t>(head) * head_dim;
        const int kv_head = head / group;
        for (int cached = 0; cached <= position; ++cached) {
            scores[cached] = dot_scalar(q, key_row(view, cached, kv_head), head_dim) * scale;
        }
        float maximum = scores[0];
        for (int index = 1; index <= position; ++index) {
            maximum = std::max(maximum, scores[index]);
        }
        float sum = 0.0f;
        for (int index = 0; index <= position; ++index) {
            scores[index] = std::exp(scores[index] - maximum);
            sum += scores[index];
        }
        for (int index = 0; index <= position; ++index) {
            scores[index] /= sum;
        }
        float* destination = output + static_cast<size_t>(head) * head_dim;
        for (int dim = 0; dim < head_dim; ++dim) {
            destination[dim] = 0.0f;
        }
        for (int cached = 0; cached <= position; ++cached) {
            const float* value = value_row(view, cached, kv_head);
            for (int dim = 0; dim < head_dim; ++dim) {
                destination[dim] += scores[cached] * value[dim];
            }
        }
    }
}

// Qwen2CpuAttention (Qwen2CpuAttention.cs:55-113) for one query position.
void orc_attention_managed(const float* query, const float* keys, const float* values, int heads, int kv_heads,
                           int head_dim, int position, float* output) {
    const int group = heads / kv_heads;
    const float scale = 1.0f / std::sqrt(static_cast<float>(head_dim));
    const KeyView view{keys, values, kv_heads, head_dim};
    std::vector<float> scores(position + 1);
    for (int head = 0; head < heads; ++head) {
        attend_managed(view, query + static_cast<size_t>(head) * head_dim, head / group, position, scale,
                       scores.data(), output + static_cast<size_t>(head) * head_dim);
    }
}

// ReferenceAttentionOperators.Execute (src/Synapse.Runtime/Features/GraphExecution/Reference/
// ReferenceAttentionOperators.cs:10-44; ComputeHead :108-141, NormalizeAndAccumulate :143-187): FP64
// accumulation, one rounding to FP32. `valid` may be null (all valid). Returns 0, 2 for a shape error, 7 for a
// non-finite visible input, 8 when every key is masked, 9 for an FP32 overflow; on failure `output` is
// untouched.
int orc_attention_fp64(const float* query, const float* keys, const float* values, const uint8_t* valid, int heads,
                       int kv_heads, int head_dim, int position, float scale, float* output) {
    if (kv_heads <= 0 || head_dim <= 0 || heads <= 0 || heads % kv_heads != 0 || position < 0 ||
        !std::isfinite(scale) || scale <= 0) {
        return kInvalid;
    }
    const int stride = kv_heads * head_dim;
    for (int index = 0; index < heads * head_dim; ++index) {
        if (!std::isfinite(query[index])) {
            return 7;
        }
    }
    bool visible = false;
    for (int current = 0; current <= position; ++current) {
        if (valid != nullptr && !valid[current]) {
            continue;
        }
        visible = true;
        for (int index = 0; index < stride; ++index) {
            if (!std::isfinite(keys[static_cast<size_t>(current) * stride + index]) ||
                !std::isfinite(values[static_cast<size_t>(current) * stride + index])) {
                return 7;
            }
        }
    }
    if (!visible) {
        return 8;
    }
    const int group = heads / kv_heads;
    std::vector<float> result(static_cast<size_t>(heads) * head_dim);
    std::vector<double> scores(position + 1);
    std::vector<double> weights(position + 1);
    for (int head = 0; head < heads; ++head) {
        const int kv_head = head / group;
        const float* q = query + static_cast<size_t>(head) * head_dim;
        double maximum = -std::numeric_limits<double>::infinity();
        for (int current = 0; current <= position; ++current) {
            if (valid != nullptr && !valid[current]) {
                continue;
            }
            const float* key = keys + (static_cast<size_t>(current) * kv_heads + kv_head) * head_dim;
            double score = 0.0;
            for (int index = 0; index < head_dim; ++index) {
                score += static_cast<double>(q[index]) * key[index];
            }
            scores[current] = score * scale;
            maximum = std::max(maximum, scores[current]);
        }
        double denominator = 0.0;
        for (int current = 0; current <= position; ++current) {
            if (valid == nullptr || valid[current]) {
                weights[current] = std::exp(scores[current] - maximum);
                denominator += weights[current];
            }
        }
        for (int coordinate = 0; coordinate < head_dim; ++coordinate) {
            double sum = 0.0;
            for (int current = 0; current <= position; ++current) {
                if (valid == nullptr || valid[current]) {
                    sum += weights[current] *
                           values[(static_cast<size_t>(current) * kv_heads + kv_head) * head_dim + coordinate];
                }
            }
            const double normalized = sum / denominator;
            if (!std::isfinite(normalized) || std::fabs(normalized) > std::numeric_limits<float>::max()) {
                return 9;
            }
            result[static_cast<size_t>(head) * head_dim + coordinate] = static_cast<float>(normalized);
        }
    }
    std::copy(result.begin(), result.end(), output);
    return kOk;
}

// Split-K attention with the merge of synapse_attention_reduce (native/synapse-gpu/src/Features/GpuKernels/metal/
// shaders/attention_reduce.metal:5-40): each split of `split_keys` keys keeps an FP32 running maximum, sum and
// unnormalized output (attend_tile/softmax_scores, attention.metal:67-167, one key at a time here); the merge
// takes the maximum over splits with a positive sum, rescales sums and outputs by exp(m - max) and divides.
void orc_attention_split(const float* query, const float* keys, const float* values, int heads, int kv_heads,
                         int head_dim, int position, int split_keys, float* output) {
    const int group = heads / kv_heads;
    const float scale = 1.0f / std::sqrt(static_cast<float>(head_dim));
    const KeyView view{keys, values, kv_heads, head_dim};
    const int key_end = position + 1;
    const int splits = (key_end + split_keys - 1) / split_keys;
    std::vector<float> maxima(splits);
    std::vector<float> sums(splits);
    std::vector<float> partial(static_cast<size_t>(splits) * head_dim);
    for (int head = 0; head < heads; ++head) {
        const float* q = query + static_cast<size_t>(head) * head_dim;
        const int kv_head = head / group;
        for (int split = 0; split < splits; ++split) {
            float running_max = -std::numeric_limits<float>::infinity();
            float running_sum = 0.0f;
            float* out = partial.data() + static_cast<size_t>(split) * head_dim;
            std::fill(out, out + head_dim, 0.0f);
            const int begin = split * split_keys;
            const int end = std::min(key_end, begin + split_keys);
            for (int key = begin; key < end; ++key) {
                const float score = dot_scalar(q, key_row(view, key, kv_head), head_dim) * scale;
                const float next = std::max(running_max, score);
                const float alpha = running_max == -std::numeric_limits<float>::infinity()
                                        ? 1.0f
                                        : std::exp(running_max - next);
                const float weight = std::exp(score - next);
                running_sum = running_sum * alpha + weight;
                const float* value = value_row(view, key, kv_head);
                for (int dim = 0; dim < head_dim; ++dim) {
                    out[dim] = out[dim] * alpha + weight * value[dim];
                }
                running_max = next;
            }
            maxima[split] = running_max;
            sums[split] = running_sum;
        }
        float maximum = -std::numeric_limits<float>::infinity();
        for (int split = 0; split < splits; ++split) {
            if (sums[split] > 0.0f) {
                maximum = std::max(maximum, maxima[split]);
            }
        }
        float* destination = output + static_cast<size_t>(head) * head_dim;
        for (int dim = 0; dim < head_dim; ++dim) {
            float sum = 0.0f;
            float value = 0.0f;
            for (int split = 0; split < splits; ++split) {
                if (sums[split] > 0.0f) {
                    const float factor = std::exp(maxima[split] - maximum);
                    sum += sums[split] * factor;
                    value += partial[static_cast<size_t>(split) * head_dim + dim] * factor;
                }
            }
            destination[dim] = value / sum;
        }
    }
}

}  // extern "C"

// ---- Query-aware KV page activation (ADR-016) ----------------------------------------------------------------

namespace {

// System.Random(int seed), the seeded generator .NET keeps for compatibility (dotnet/runtime
// src/libraries/System.Private.CoreLib/src/System/Random.Net5CompatImpl.cs, CompatPrng): Knuth's subtractive
// generator (TAOCP vol. 2, 3.6) as Numerical Recipes' ran3 seeds it, 55 words, lag 21 between the two indices.
// Not part of the reference tree; KvPageSelector.RandomPages (KvPageSelector.cs:118-129) draws from it.
struct CompatRandom {
    static constexpr int32_t kBig = 2147483647;  // int.MaxValue
    int32_t words[56];
    int first = 0;
    int second = 21;

    explicit CompatRandom(int32_t seed) {
        int32_t previous = 161803398 - (seed == INT32_MIN ? kBig : std::abs(seed));
        words[55] = previous;
        int32_t current = 1;
        for (int i = 1, at = 0; i < 55; ++i) {
            at = (at + 21) % 55;
            words[at] = current;
            current = previous - current;
            if (current < 0) {
                current += kBig;
            }
            previous = words[at];
        }
        for (int pass = 0; pass < 4; ++pass) {
            for (int i = 1; i < 56; ++i) {
                words[i] -= words[1 + (i + 30) % 55];
                if (words[i] < 0) {
                    words[i] += kBig;
                }
            }
        }
    }

    // InternalSample; Random.Next() returns it as is.
    int32_t sample() {
        first = first + 1 >= 56 ? 1 : first + 1;
        second = second + 1 >= 56 ? 1 : second + 1;
        int32_t value = words[first] - words[second];
        if (value == kBig) {
            value -= 1;
        }
        if (value < 0) {
            value += kBig;
        }
        words[first] = value;
        return value;
    }

    // Next(minValue, maxValue) for maxValue - minValue <= int.MaxValue: truncation of Sample() * range.
    int32_t next(int32_t low, int32_t high) {
        const double unit = sample() * (1.0 / kBig);
        return static_cast<int32_t>(unit * (static_cast<int64_t>(high) - low)) + low;
    }
};

// MathF.Min / MathF.Max (System.MathF): a NaN operand wins, and -0 < +0.
float math_f_min(float x, float y) {
    if (x != y) {
        return std::isnan(x) ? x : (x < y ? x : y);
    }
    return std::signbit(x) ? x : y;
}

float math_f_max(float x, float y) {
    if (x != y) {
        return std::isnan(x) ? x : (y < x ? x : y);
    }
    return std::signbit(y) ? x : y;
}

// float.CompareTo: NaN sorts below every number and equals NaN.
int float_compare(float x, float y) {
    if (x < y) {
        return -1;
    }
    if (x > y) {
        return 1;
    }
    if (x == y) {
        return 0;
    }
    return std::isnan(x) ? (std::isnan(y) ? 0 : -1) : 1;
}

struct Activation {
    int32_t budget_pages;
    int32_t window_tokens;
    int32_t page_tokens;
    int32_t selection;  // 0 key bound, 1 random
    int32_t seed;
};

// A key reader: keys of one KV head, row `position` at keys + position * stride.
struct Keys {
    const float* base;
    size_t stride;
    const float* at(int position) const { return base + static_cast<size_t>(position) * stride; }
};

// KvPageSelector.PageBound (KvPageSelector.cs:57-93).
float page_bound(const float* queries, int group, int head_dim, const Keys& keys, int first, int last) {
    std::vector<float> minimum(keys.at(first), keys.at(first) + head_dim);
    std::vector<float> maximum(minimum);
    for (int position = first + 1; position <= last; ++position) {
        const float* key = keys.at(position);
        for (int channel = 0; channel < head_dim; ++channel) {
            minimum[channel] = math_f_min(minimum[channel], key[channel]);
            maximum[channel] = math_f_max(maximum[channel], key[channel]);
        }
    }
    float best = -std::numeric_limits<float>::infinity();
    for (int head = 0; head < group; ++head) {
        const float* query = queries + static_cast<size_t>(head) * head_dim;
        float bound = 0.0f;
        for (int channel = 0; channel < head_dim; ++channel) {
            const float low = query[channel] * minimum[channel];
            const float high = query[channel] * maximum[channel];
            bound += math_f_max(low, high);
        }
        best = math_f_max(best, bound);
    }
    return best;
}

void mark_page(uint8_t* selected, int page, int size, int position) {
    const int first = page * size;
    const int last = std::min(first + size - 1, position);
    for (int index = first; index <= last; ++index) {
        selected[index] = 1;
    }
}

// KvPageSelector.Select (KvPageSelector.cs:17-54) with BestPages (:96-115) and RandomPages (:118-129).
void page_select(const Activation& activation, const float* queries, int group, int head_dim, const Keys& keys,
                 int position, int32_t seed, uint8_t* selected) {
    const int count = position + 1;
    const int size = activation.page_tokens;
    std::fill(selected, selected + count, 0);
    const int window_page = std::max(0, count - activation.window_tokens) / size;
    mark_page(selected, 0, size, position);
    for (int page = window_page; page <= position / size; ++page) {
        mark_page(selected, page, size, position);
    }
    const int candidates = std::max(0, window_page - 1);
    if (candidates <= activation.budget_pages) {
        for (int page = 1; page < window_page; ++page) {
            mark_page(selected, page, size, position);
        }
        return;
    }
    std::vector<int> chosen;
    if (activation.selection == 1) {
        std::vector<int> pages(candidates);
        for (int index = 0; index < candidates; ++index) {
            pages[index] = index + 1;
        }
        CompatRandom random(seed);
        for (int index = 0; index < activation.budget_pages; ++index) {
            std::swap(pages[index], pages[random.next(index, candidates)]);
        }
        chosen.assign(pages.begin(), pages.begin() + activation.budget_pages);
    } else {
        std::vector<std::pair<float, int>> ranked(candidates);
        for (int page = 1; page <= candidates; ++page) {
            const int first = page * size;
            ranked[page - 1] = {page_bound(queries, group, head_dim, keys, first, first + size - 1), page};
        }
        std::sort(ranked.begin(), ranked.end(), [](const auto& left, const auto& right) {
            const int order = float_compare(right.first, left.first);
            return order != 0 ? order < 0 : left.second < right.second;
        });
        for (int index = 0; index < activation.budget_pages; ++index) {
            chosen.push_back(ranked[index].second);
        }
    }
    for (int page : chosen) {
        mark_page(selected, page, size, position);
    }
}

}  // namespace

extern "C" {

// Random(seed).Next() `count` times (low == high == 0) or Next(low, high) `count` times.
void orc_dotnet_random(int32_t seed, int count, int32_t low, int32_t high, int32_t* out) {
    CompatRandom random(seed);
    for (int index = 0; index < count; ++index) {
        out[index] = low == 0 && high == 0 ? random.sample() : random.next(low, high);
    }
}

float orc_page_bound(const float* queries, int group, int head_dim, const float* keys, int first, int last) {
    return page_bound(queries, group, head_dim, Keys{keys, static_cast<size_t>(head_dim)}, first, last);
}

// KvPageSelector.Select over keys [positions][head_dim] of one KV head; selected[0..position].
void orc_page_select(int budget_pages, int window_tokens, int page_tokens, int selection, const float* queries,
                     int group, int head_dim, const float* keys, int position, int32_t seed, uint8_t* selected) {
    const Activation activation{budget_pages, window_tokens, page_tokens, selection, 0};
    page_select(activation, queries, group, head_dim, Keys{keys, static_cast<size_t>(head_dim)}, position, seed,
                selected);
}

}  // extern "C"

namespace {

// Qwen2KvPageMasks.Prepare (Qwen2KvPageMasks.cs:21-54): for each decode unit (a token before prompt_start alone in
// its slot) and KV head, the selected positions; masks[(token * kv_heads + kv_head) * stride + position], and
// units[token] = 1 for a decode unit.
void page_masks(const Activation& activation, int layer, const int32_t* step, int count, int prompt_start,
                const float* qkv, int qkv_stride, int kv_heads, int group, int head_dim,
                const std::vector<std::vector<float>>& keys, size_t stride, std::vector<uint8_t>& masks,
                std::vector<uint8_t>& units) {
    units.assign(count, 0);
    masks.assign(static_cast<size_t>(count) * kv_heads * stride, 0);
    for (int token = 0; token < count; ++token) {
        const int slot = step[4 * token];
        bool dense = token >= prompt_start;
        for (int other = 0; other < count && !dense; ++other) {
            dense = other != token && step[4 * other] == slot;
        }
        if (dense) {
            continue;
        }
        units[token] = 1;
        const int position = step[4 * token + 2];
        for (int kv_head = 0; kv_head < kv_heads; ++kv_head) {
            const uint32_t seed = static_cast<uint32_t>(activation.seed) * 1000003u +
                                  static_cast<uint32_t>(layer) * 7919u + static_cast<uint32_t>(kv_head) * 104729u +
                                  static_cast<uint32_t>(position);
            const Keys reader{keys[slot].data() + static_cast<size_t>(kv_head) * head_dim,
                              static_cast<size_t>(kv_heads) * head_dim};
            page_select(activation, qkv + static_cast<size_t>(token) * qkv_stride +
                                        static_cast<size_t>(kv_head) * group * head_dim,
                        group, head_dim, reader, position, static_cast<int32_t>(seed),
                        masks.data() + (static_cast<size_t>(token) * kv_heads + kv_head) * stride);
        }
    }
}

}  // namespace

extern "C" {

// Decode/prefill attention of the prepared step for one layer, read through the paged cache:
// Qwen2CpuAttention.Execute (Qwen2CpuAttention.cs:55-79) with its (token, head) work items spread over `threads`
// std::threads. q rows at qkv + token * qkv_stride (heads * head_dim floats), outputs at out + token * out_stride.
// With `activation` (budget, window, page_tokens, selection, seed; null: dense) the decode units of the step attend
// only their selected positions (Qwen2KvPageMasks; Qwen2CpuAttention.Attend, :94-110); `selected`, when not null,
// receives the masks as [token][kv_head][maximum positions] bytes (all zero for dense tokens).
// Returns the wall time of the attention in seconds (the gather of FP16 pages to FP32 is not timed).
double orc_paged_attention_pages(void* handle, int layer, const float* qkv, int qkv_stride, float* output,
                                 int out_stride, int threads, const int32_t* activation, int prompt_start,
                                 uint8_t* selected);

double orc_paged_attention(void* handle, int layer, const float* qkv, int qkv_stride, float* output, int out_stride,
                           int threads) {
    const auto& cache = *static_cast<PagedCache*>(handle);
    return orc_paged_attention_pages(handle, layer, qkv, qkv_stride, output, out_stride, threads, nullptr,
                                     static_cast<int>(cache.step.size() / 4), nullptr);
}

double orc_paged_attention_pages(void* handle, int layer, const float* qkv, int qkv_stride, float* output,
                                 int out_stride, int threads, const int32_t* activation, int prompt_start,
                                 uint8_t* selected) {
    auto& cache = *static_cast<PagedCache*>(handle);
    const int count = static_cast<int>(cache.step.size() / 4);
    const Token* tokens = reinterpret_cast<const Token*>(cache.step.data());
    const int d = cache.head_dim;
    const int group = cache.heads / cache.kv_heads;
    const float scale = 1.0f / std::sqrt(static_cast<float>(d));
    // Widen each distinct slot once into a dense [position][kv_head][d] view (Fp16.ToSingle per element).
    std::vector<std::vector<float>> keys(cache.max_sequences);
    std::vector<std::vector<float>> values(cache.max_sequences);
    std::vector<int> extent(cache.max_sequences, 0);
    for (int index = 0; index < count; ++index) {
        extent[tokens[index].slot] = std::max(extent[tokens[index].slot], tokens[index].position + 1);
    }
    for (int slot = 0; slot < cache.max_sequences; ++slot) {
        if (extent[slot] == 0) {
            continue;
        }
        const size_t elements = static_cast<size_t>(extent[slot]) * cache.kv_heads * d;
        keys[slot].resize(elements);
        values[slot].resize(elements);
        orc_paged_gather(handle, slot, layer, 0, extent[slot], keys[slot].data(), values[slot].data(), 0);
    }
    int longest = 0;
    for (int slot = 0; slot < cache.max_sequences; ++slot) {
        longest = std::max(longest, extent[slot]);
    }
    std::vector<uint8_t> masks;
    std::vector<uint8_t> units(count, 0);
    const size_t mask_stride = static_cast<size_t>(cache.maximum);
    if (activation != nullptr) {
        const Activation parsed{activation[0], activation[1], activation[2], activation[3], activation[4]};
        page_masks(parsed, layer, cache.step.data(), count, prompt_start, qkv, qkv_stride, cache.kv_heads, group, d,
                   keys, mask_stride, masks, units);
        if (selected != nullptr) {
            std::memcpy(selected, masks.data(), masks.size());
        }
    }
    const int workers = std::max(1, threads);
    std::vector<std::vector<float>> scores(workers, std::vector<float>(std::max(1, longest)));
    const auto start = std::chrono::steady_clock::now();
    Pool::run(count * cache.heads, workers, [&](int worker, int item) {
        const int index = item / cache.heads;
        const int head = item % cache.heads;
        const Token token = tokens[index];
        const KeyView view{keys[token.slot].data(), values[token.slot].data(), cache.kv_heads, d};
        const uint8_t* attended =
            units[index] ? masks.data() + (static_cast<size_t>(index) * cache.kv_heads + head / group) * mask_stride
                         : nullptr;
        attend_managed(view, qkv + static_cast<size_t>(index) * qkv_stride + static_cast<size_t>(head) * d,
                       head / group, token.position, scale, scores[worker].data(),
                       output + static_cast<size_t>(index) * out_stride + static_cast<size_t>(head) * d, attended);
    });
    return std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count();
}

// ---- Q8_0 projections ---------------------------------------------------------------------------------------

// One matrix of a projection: GGML Q8_0 rows (34-byte blocks: FP16 d, 32 int8 codes; common.metal:13-16) at
// `weight`, optional FP32 biases, and the first output column (matmul_segment, common.metal:54-59).
struct Q8Segment {
    const uint8_t* weight;
    const float* bias;  // null: none
    int rows;
    int out_column;
};

static float q8_scale(const uint8_t* block) {
    uint16_t bits;
    std::memcpy(&bits, block, 2);
    return f16_to_f32(bits);
}

// dot8 (matmul.cu:7-17): eight codes times eight activations, an explicit fma chain from the left.
static float q8_dot8(const int8_t* q, const float* x) {
    float acc = static_cast<float>(q[0]) * x[0];
    for (int i = 1; i < 8; ++i) {
        acc = std::fma(static_cast<float>(q[i]), x[i], acc);
    }
    return acc;
}

// q8_matvec<T> + matvec_finish (matmul.cu:45-111) for one (row, token): four warps of 32 lanes; lane l of warp w
// takes quarter l % 4 of blocks w * 8 + l / 4, w * 8 + l / 4 + 32, ...; sum = fma(dot8, d, sum); warp_sum
// (common.cuh:127-133: value += shfl_xor(value, 16, 8, 4, 2, 1)); the warps' totals added in order; then the bias.
static float q8_matvec_row(const uint8_t* row, int blocks, const float* x) {
    float warp_total[4];
    for (int warp = 0; warp < 4; ++warp) {
        float lane[32];
        for (int l = 0; l < 32; ++l) {
            float sum = 0.0f;
            const int quarter = l % 4;
            for (int block = warp * 8 + l / 4; block < blocks; block += 32) {
                const uint8_t* b = row + static_cast<size_t>(block) * 34;
                sum = std::fma(q8_dot8(reinterpret_cast<const int8_t*>(b + 2 + quarter * 8), x + block * 32 + quarter * 8),
                               q8_scale(b), sum);
            }
            lane[l] = sum;
        }
        for (int offset = 16; offset > 0; offset >>= 1) {
            float next[32];
            for (int l = 0; l < 32; ++l) {
                next[l] = lane[l] + lane[l ^ offset];
            }
            std::memcpy(lane, next, sizeof(lane));
        }
        warp_total[warp] = lane[0];
    }
    return ((warp_total[0] + warp_total[1]) + warp_total[2]) + warp_total[3];
}

// The reference's FP32 matrix-vector projection (matmul.cu:45-118) on `threads` std::threads over rows: output
// [t][out_column + row] = (accumulate ? output : 0) + (matvec sum + bias). Returns the wall time in seconds.
double orc_q8_project_f32(const uint8_t* const* weights, const float* const* biases, const int* rows,
                          const int* out_columns, int segments, int columns, int tokens, const float* input,
                          int in_stride, float* output, int out_stride, int accumulate, int threads) {
    const int blocks = columns / 32;
    std::vector<Q8Segment> list;
    int total_rows = 0;
    for (int s = 0; s < segments; ++s) {
        list.push_back(Q8Segment{weights[s], biases[s], rows[s], out_columns[s]});
        total_rows += rows[s];
    }
    const auto start = std::chrono::steady_clock::now();
    Pool::run(total_rows, std::max(1, threads), [&](int, int item) {
        int local = item;
        size_t s = 0;
        while (s + 1 < list.size() && local >= list[s].rows) {  // locate_segment (common.metal:138-146)
            local -= list[s].rows;
            ++s;
        }
        const Q8Segment& seg = list[s];
        const uint8_t* row = seg.weight + static_cast<size_t>(local) * blocks * 34;
        for (int t = 0; t < tokens; ++t) {
            float total = q8_matvec_row(row, blocks, input + static_cast<size_t>(t) * in_stride);
            if (seg.bias != nullptr) {
                total += seg.bias[local];
            }
            float& destination = output[static_cast<size_t>(t) * out_stride + seg.out_column + local];
            destination = accumulate != 0 ? destination + total : total;
        }
    });
    return std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count();
}

// The same projection accumulated in FP64 and rounded once (the tolerance anchor): output = (accumulate ? output
// : 0) + sum_k d * code * x + bias. `magnitude` (optional, [tokens][out_stride]) receives sum_k |d * code * x|
// + |bias| per written element, the scale of FP32 summation error.
void orc_q8_project_f64(const uint8_t* const* weights, const float* const* biases, const int* rows,
                        const int* out_columns, int segments, int columns, int tokens, const float* input, int in_stride,
                        float* output, int out_stride, int accumulate, double* magnitude) {
    const int blocks = columns / 32;
    for (int s = 0; s < segments; ++s) {
        for (int row = 0; row < rows[s]; ++row) {
            const uint8_t* w = weights[s] + static_cast<size_t>(row) * blocks * 34;
            for (int t = 0; t < tokens; ++t) {
                const float* x = input + static_cast<size_t>(t) * in_stride;
                double sum = 0.0;
                double size = 0.0;
                for (int block = 0; block < blocks; ++block) {
                    const double d = q8_scale(w + static_cast<size_t>(block) * 34);
                    const int8_t* q = reinterpret_cast<const int8_t*>(w + static_cast<size_t>(block) * 34 + 2);
                    for (int i = 0; i < 32; ++i) {
                        const double term = d * q[i] * static_cast<double>(x[block * 32 + i]);
                        sum += term;
                        size += std::fabs(term);
                    }
                }
                if (biases[s] != nullptr) {
                    sum += biases[s][row];
                    size += std::fabs(static_cast<double>(biases[s][row]));
                }
                const size_t at = static_cast<size_t>(t) * out_stride + out_columns[s] + row;
                output[at] = static_cast<float>(accumulate != 0 ? static_cast<double>(output[at]) + sum : sum);
                if (magnitude != nullptr) {
                    magnitude[at] = size + (accumulate != 0 ? std::fabs(static_cast<double>(output[at])) : 0.0);
                }
            }
        }
    }
}

// ---- Schedule -------------------------------------------------------------------------------------------------

// plan_attention + split_plan (native/synapse-gpu/src/Features/GpuKernels/schedule.rs:34-123). `blocks` receives
// 8 uint32 per block (first_token, token_count, kv_head, mode, slot, key_end, 0, 0) like AttentionBlock
// (params.rs:80-89). Returns the block count (or -1 when `capacity` is too small).
int orc_plan_attention(const int32_t* tokens, int count, int kv_heads, int run_tokens, uint32_t* blocks,
                       int capacity, uint32_t* summary /* run_blocks, single_blocks, split_keys, splits */) {
    const Token* t = reinterpret_cast<const Token*>(tokens);
    std::vector<std::pair<int, int>> runs;
    std::vector<int> singles;
    int start = 0;
    while (start < count) {
        int end = start + 1;
        while (end < count && t[end].slot == t[start].slot && t[end].position == t[end - 1].position + 1) {
            ++end;
        }
        if (end - start == 1) {
            singles.push_back(start);
        } else {
            for (int first = start; first < end;) {
                const int size = std::min(run_tokens, end - first);
                runs.emplace_back(first, size);
                first += size;
            }
        }
        start = end;
    }
    std::vector<uint32_t> out;
    auto push = [&](int first, int size, uint32_t mode, const Token& last) {
        for (int kv_head = 0; kv_head < kv_heads; ++kv_head) {
            const uint32_t block[8] = {static_cast<uint32_t>(first), static_cast<uint32_t>(size),
                                       static_cast<uint32_t>(kv_head), mode,
                                       static_cast<uint32_t>(std::abs(last.slot)),
                                       static_cast<uint32_t>(std::abs(last.position)) + 1, 0, 0};
            out.insert(out.end(), block, block + 8);
        }
    };
    for (auto [first, size] : runs) {
        push(first, size, 0, t[first + size - 1]);
    }
    const uint32_t run_blocks = static_cast<uint32_t>(out.size() / 8);
    for (int index : singles) {
        push(index, 1, 1, t[index]);
    }
    const uint32_t total = static_cast<uint32_t>(out.size() / 8);
    const uint32_t single_blocks = total - run_blocks;
    uint32_t longest = 0;
    for (uint32_t block = run_blocks; block < total; ++block) {
        longest = std::max(longest, out[block * 8 + 5]);
    }
    uint32_t split_keys = 32;
    uint32_t splits = 1;
    if (single_blocks != 0 && longest != 0) {
        auto div_ceil = [](uint32_t a, uint32_t b) { return (a + b - 1) / b; };
        const uint32_t wanted = div_ceil(256, single_blocks);
        const uint32_t by_keys = div_ceil(longest, 256);
        const uint32_t by_buffer = std::max(1u, 512 / single_blocks);
        const uint32_t chosen = std::max(1u, std::min(wanted, std::min(by_keys, by_buffer)));
        split_keys = div_ceil(div_ceil(longest, chosen), 32) * 32;
        splits = div_ceil(longest, split_keys);
    }
    summary[0] = run_blocks;
    summary[1] = single_blocks;
    summary[2] = split_keys;
    summary[3] = splits;
    if (static_cast<int>(total) > capacity) {
        return -1;
    }
    std::copy(out.begin(), out.end(), blocks);
    return static_cast<int>(total);
}

// ---- Prompt prefix reuse (DirectSessionPrefix.cs:7-42) --------------------------------------------------------

struct Prefix {
    bool enabled;
    std::vector<int> tokens;
};

void* orc_prefix_create(int enabled) { return new Prefix{enabled != 0, {}}; }

void orc_prefix_destroy(void* handle) { delete static_cast<Prefix*>(handle); }

// Claim (DirectSessionPrefix.cs:16-27).
int orc_prefix_claim(void* handle, const int32_t* prompt, int count) {
    auto& prefix = *static_cast<Prefix*>(handle);
    const int limit = std::min(static_cast<int>(prefix.tokens.size()), count - 1);
    int shared = 0;
    while (shared < limit && prefix.tokens[shared] == prompt[shared]) {
        ++shared;
    }
    prefix.tokens.resize(std::max(0, shared));
    return std::max(0, shared);
}

// Remember (DirectSessionPrefix.cs:30-38).
void orc_prefix_remember(void* handle, const int32_t* prompt, int count, const int32_t* generated, int produced) {
    auto& prefix = *static_cast<Prefix*>(handle);
    prefix.tokens.clear();
    if (prefix.enabled) {
        prefix.tokens.insert(prefix.tokens.end(), prompt, prompt + count);
        if (produced > 1) {
            prefix.tokens.insert(prefix.tokens.end(), generated, generated + produced - 1);
        }
    }
}

void orc_prefix_clear(void* handle) { static_cast<Prefix*>(handle)->tokens.clear(); }

}  // extern "C"

// ---- The dense decoder step ---------------------------------------------------------------------------------

// encode_step (native/synapse-gpu/src/Features/GpuKernels/step.rs:137-185) over the kernels' semantics: embedding
// lookup, RMS norm and SwiGLU as elementwise.cu:3-109, Q8_0 projections in matmul.cu's FP32 order
// (q8_matvec_row), NeoX RoPE + KV append and attention through the paged restatement above (orc_paged_*), the
// output and down projections added to the residual (step/layers.rs:62-206), and the logits rows normalized by
// the output norm and projected (step/layers.rs:208-228).
namespace {

struct DecoderOracle {
    const uint8_t* weights;
    std::vector<uint64_t> layers;  // layer_count x 15 offsets (DecoderLayerOffsets order)
    uint64_t token_embedding, output_norm, output;
    int embedding_encoding, output_encoding;
    int layer_count, hidden, feed_forward, heads, kv_heads, head_dim, vocabulary;
    float epsilon;
    std::vector<float> cosines, sines;
    void* cache;
};

constexpr uint64_t kNoTensor = ~0ull;

const float* f32_at(const DecoderOracle& m, uint64_t offset) {
    return reinterpret_cast<const float*>(m.weights + offset);
}

// synapse_rms_norm (elementwise.cu:17-52): the sum of squares, then x * (1 / sqrt(mean + eps)) * w.
void rms_norm_row(const float* x, const float* w, int columns, float epsilon, float* y) {
    float sum = 0.0f;
    for (int i = 0; i < columns; ++i) {
        sum += x[i] * x[i];
    }
    const float scale = 1.0f / std::sqrt(sum / static_cast<float>(columns) + epsilon);
    for (int i = 0; i < columns; ++i) {
        y[i] = x[i] * scale * w[i];
    }
}

// ---- K-quant matrices (ADR-021) ----
// GGML Q4_K: 144-byte super-blocks of 256 values (FP16 d, FP16 dmin, 12 packed 6-bit scale/minimum bytes, 128 bytes
// of nibbles); Q6_K: 210 bytes (ql[128], qh[64], int8 scales[16], FP16 d). GgufKQuantBlocks.cs:99-177 and
// matmul_kquant.metal:16-68 decode them; the functions below restate that decoding.
constexpr int kQ4K = 12;
constexpr int kQ6K = 14;

int kq_block_bytes(int encoding) { return encoding == kQ4K ? 144 : 210; }

float f16_at(const uint8_t* p) {
    uint16_t bits;
    std::memcpy(&bits, p, 2);
    return f16_to_f32(bits);
}

// Code of value i of a super-block: Q4_K q (0..15); Q6_K q - 32 (ScaleMinK4 :149-153, DecodeQ6K :155-177).
int kq_code(int encoding, const uint8_t* block, int i) {
    const int sub = i / 32;
    const int l = i % 32;
    if (encoding == kQ4K) {
        const uint8_t byte = block[16 + (sub / 2) * 32 + l];
        return sub % 2 == 0 ? (byte & 0xF) : (byte >> 4);
    }
    const int half = sub / 4;
    const int quarter = sub % 4;
    const uint8_t low = block[half * 64 + (quarter % 2 == 0 ? l : l + 32)];
    const int nibble = quarter < 2 ? (low & 0xF) : (low >> 4);
    const int high = (block[128 + half * 32 + l] >> (2 * quarter)) & 3;
    return (nibble | (high << 4)) - 32;
}

// The factors of value i: Q4_K scale d * sc_j and offset dmin * m_j of sub-block j = i / 32; Q6_K scale
// d * scales[i / 16] and offset 0 (kq_decode8, matmul_kquant.metal:76-113).
void kq_factors(int encoding, const uint8_t* block, int i, float& scale, float& offset) {
    if (encoding == kQ4K) {
        const int j = i / 32;
        const uint8_t* packed = block + 4;
        int sc;
        int mn;
        if (j < 4) {
            sc = packed[j] & 63;
            mn = packed[j + 4] & 63;
        } else {
            sc = (packed[j + 4] & 0xF) | ((packed[j - 4] >> 6) << 4);
            mn = (packed[j + 4] >> 4) | ((packed[j] >> 6) << 4);
        }
        scale = f16_at(block) * static_cast<float>(sc);
        offset = f16_at(block + 2) * static_cast<float>(mn);
    } else {
        scale = f16_at(block + 208) * static_cast<float>(static_cast<int8_t>(block[192 + i / 16]));
        offset = 0.0f;
    }
}

// One value of a K-quant row (kq_values8: d1 * q - m1, scale * (q - 32)).
float kq_value(int encoding, const uint8_t* row, int column) {
    const uint8_t* block = row + static_cast<size_t>(column / 256) * kq_block_bytes(encoding);
    float scale;
    float offset;
    kq_factors(encoding, block, column % 256, scale, offset);
    const float q = static_cast<float>(kq_code(encoding, block, column % 256));
    return encoding == kQ4K ? scale * q - offset : scale * q;
}

// synapse_kq_matvec (matmul_kquant.metal:153-210) for one (row, token): 32 lanes; lane (slot = l / 4, quarter =
// l % 4) walks 32-value chunks slot, slot + 8, ... and adds kq_apply = scale * (q0.x0 + q1.x1) - offset * (sum x0 +
// sum x1) for its 8 values; the lanes are added in a butterfly (simd_sum; restated in the xor-shuffle order).
float kq_matvec_row(int encoding, const uint8_t* row, int columns, const float* x) {
    float lane[32];
    for (int l = 0; l < 32; ++l) {
        const int slot = l / 4;
        const int quarter = l % 4;
        float sum = 0.0f;
        for (int chunk = slot; chunk < columns / 32; chunk += 8) {
            const uint8_t* block = row + static_cast<size_t>(chunk / 8) * kq_block_bytes(encoding);
            const int first = (chunk % 8) * 32 + quarter * 8;
            float scale;
            float offset;
            kq_factors(encoding, block, first, scale, offset);
            const float* v = x + chunk * 32 + quarter * 8;
            float dots[2];
            float sums[2];
            for (int h = 0; h < 2; ++h) {
                const float* q4 = v + 4 * h;
                float qv[4];
                for (int i = 0; i < 4; ++i) {
                    qv[i] = static_cast<float>(kq_code(encoding, block, first + 4 * h + i));
                }
                dots[h] = ((qv[0] * q4[0] + qv[1] * q4[1]) + qv[2] * q4[2]) + qv[3] * q4[3];
                sums[h] = ((q4[0] + q4[1]) + q4[2]) + q4[3];
            }
            const float qx = dots[0] + dots[1];
            const float sx = sums[0] + sums[1];
            sum += scale * qx - offset * sx;
        }
        lane[l] = sum;
    }
    for (int offset = 16; offset > 0; offset >>= 1) {
        float next[32];
        for (int l = 0; l < 32; ++l) {
            next[l] = lane[l] + lane[l ^ offset];
        }
        std::memcpy(lane, next, sizeof(lane));
    }
    return lane[0];
}

// Bytes of one row of a matrix in `encoding` (8: Q8_0, 12: Q4_K, 14: Q6_K).
size_t row_bytes_of(int encoding, int columns) {
    return encoding == 8 ? static_cast<size_t>(columns / 32) * 34
                         : static_cast<size_t>(columns / 256) * kq_block_bytes(encoding);
}

// Rows of one matrix (rows x columns at `offset`, GGML blocks of `encoding`) times input rows, plus an optional
// FP32 bias, into output[t * out_stride + out_column + row] (added to it when accumulating). Q8_0 follows
// matmul.cu's order, the K-quants matmul_kquant.metal's.
void project_rows(const DecoderOracle& m, uint64_t offset, uint64_t bias, int encoding, int rows, int columns,
                  int tokens, const float* input, int in_stride, float* output, int out_stride, int out_column,
                  bool accumulate, int threads) {
    const int blocks = columns / 32;
    const size_t row_bytes = row_bytes_of(encoding, columns);
    const float* biases = bias == kNoTensor ? nullptr : f32_at(m, bias);
    Pool::run(rows, threads, [&](int, int row) {
        const uint8_t* weights = m.weights + offset + row * row_bytes;
        for (int t = 0; t < tokens; ++t) {
            const float* x = input + static_cast<size_t>(t) * in_stride;
            float total = encoding == 8 ? q8_matvec_row(weights, blocks, x) : kq_matvec_row(encoding, weights, columns, x);
            if (biases != nullptr) {
                total += biases[row];
            }
            float& destination = output[static_cast<size_t>(t) * out_stride + out_column + row];
            destination = accumulate ? destination + total : total;
        }
    });
}

}  // namespace

extern "C" {

// dims: layer_count, hidden, feed_forward, heads, kv_heads, head_dim, vocabulary, context, session_slots,
// step_tokens, kv_precision, kv_growth_positions, page_tokens, max_pages. top: token_embedding, output_norm,
// output, embedding_encoding, output_encoding. layers: layer_count x 15 values (DecoderLayerOffsets: 14 offsets,
// then the packed encodings). The weights stay owned by the caller.
void* orc_decoder_create(const uint8_t* weights, const uint64_t* layers, const uint64_t* top, const int* dims,
                         float epsilon, const float* cosines, const float* sines) {
    auto* m = new DecoderOracle{};
    m->weights = weights;
    m->layer_count = dims[0];
    m->hidden = dims[1];
    m->feed_forward = dims[2];
    m->heads = dims[3];
    m->kv_heads = dims[4];
    m->head_dim = dims[5];
    m->vocabulary = dims[6];
    const int context = dims[7];
    m->layers.assign(layers, layers + static_cast<size_t>(m->layer_count) * 15);
    m->token_embedding = top[0];
    m->output_norm = top[1];
    m->output = top[2];
    m->embedding_encoding = static_cast<int>(top[3]);
    m->output_encoding = static_cast<int>(top[4]);
    m->epsilon = epsilon;
    m->cosines.assign(cosines, cosines + static_cast<size_t>(context) * (m->head_dim / 2));
    m->sines.assign(sines, sines + static_cast<size_t>(context) * (m->head_dim / 2));
    m->cache = orc_paged_create(m->layer_count, m->heads, m->kv_heads, m->head_dim, context, dims[11], dims[12], dims[10],
                                dims[8], dims[13], dims[9]);
    if (m->cache == nullptr) {
        delete m;
        return nullptr;
    }
    return m;
}

void orc_decoder_destroy(void* handle) {
    auto* m = static_cast<DecoderOracle*>(handle);
    orc_paged_destroy(m->cache);
    delete m;
}

void* orc_decoder_cache(void* handle) { return static_cast<DecoderOracle*>(handle)->cache; }

// One step of `count` tokens (4 ints each: slot, token, position, logits_row); logits rows 0..k-1 of
// `vocabulary` floats. Returns the paged cache's status (0 on success).
int orc_decoder_forward(void* handle, const int32_t* tokens, int count, float* logits, int threads) {
    auto& m = *static_cast<DecoderOracle*>(handle);
    const int status = orc_paged_step(m.cache, tokens, count);
    if (status != 0) {
        return status;
    }
    const int h = m.hidden;
    const int kv = m.kv_heads * m.head_dim;
    const int qkv_width = h + 2 * kv;
    const int ffn = m.feed_forward;
    std::vector<float> hidden(static_cast<size_t>(count) * h);
    std::vector<float> normalized(hidden.size());
    std::vector<float> qkv(static_cast<size_t>(count) * qkv_width);
    std::vector<float> attention(hidden.size());
    std::vector<float> gate_up(static_cast<size_t>(count) * 2 * ffn);
    std::vector<float> activated(static_cast<size_t>(count) * ffn);
    // synapse_embed_q8_0 (elementwise.cu:3-15); K-quant tables as synapse_kq_embed (matmul_kquant.metal:293-308).
    const size_t row_bytes = row_bytes_of(m.embedding_encoding, h);
    for (int t = 0; t < count; ++t) {
        const uint8_t* row = m.weights + m.token_embedding + static_cast<size_t>(tokens[4 * t + 1]) * row_bytes;
        for (int c = 0; c < h; ++c) {
            float& value = hidden[static_cast<size_t>(t) * h + c];
            if (m.embedding_encoding == 8) {
                const uint8_t* block = row + static_cast<size_t>(c / 32) * 34;
                value = q8_scale(block) * static_cast<float>(static_cast<int8_t>(block[2 + c % 32]));
            } else {
                value = kq_value(m.embedding_encoding, row, c);
            }
        }
    }
    for (int layer = 0; layer < m.layer_count; ++layer) {
        const uint64_t* o = &m.layers[static_cast<size_t>(layer) * 15];
        auto enc = [&](int matrix) { return static_cast<int>((o[14] >> (4 * matrix)) & 0xF); };
        // attention_half (step/layers.rs:62-108).
        for (int t = 0; t < count; ++t) {
            rms_norm_row(&hidden[static_cast<size_t>(t) * h], f32_at(m, o[0]), h, m.epsilon,
                         &normalized[static_cast<size_t>(t) * h]);
        }
        project_rows(m, o[1], o[4], enc(0), h, h, count, normalized.data(), h, qkv.data(), qkv_width, 0, false, threads);
        project_rows(m, o[2], o[5], enc(1), kv, h, count, normalized.data(), h, qkv.data(), qkv_width, h, false, threads);
        project_rows(m, o[3], o[6], enc(2), kv, h, count, normalized.data(), h, qkv.data(), qkv_width, h + kv, false, threads);
        const int appended = orc_paged_append_rope(m.cache, layer, qkv.data(), qkv_width, m.cosines.data(), m.sines.data());
        if (appended != 0) {
            return appended;
        }
        orc_paged_attention(m.cache, layer, qkv.data(), qkv_width, attention.data(), h, threads);
        project_rows(m, o[9], kNoTensor, enc(3), h, h, count, attention.data(), h, hidden.data(), h, 0, true, threads);
        // feed_forward_half (step/layers.rs:150-206).
        for (int t = 0; t < count; ++t) {
            rms_norm_row(&hidden[static_cast<size_t>(t) * h], f32_at(m, o[10]), h, m.epsilon,
                         &normalized[static_cast<size_t>(t) * h]);
        }
        project_rows(m, o[11], kNoTensor, enc(4), ffn, h, count, normalized.data(), h, gate_up.data(), 2 * ffn, 0, false, threads);
        project_rows(m, o[12], kNoTensor, enc(5), ffn, h, count, normalized.data(), h, gate_up.data(), 2 * ffn, ffn, false,
                     threads);
        for (int t = 0; t < count; ++t) {
            for (int c = 0; c < ffn; ++c) {
                const float gate = gate_up[static_cast<size_t>(t) * 2 * ffn + c];
                activated[static_cast<size_t>(t) * ffn + c] =
                    gate / (1.0f + std::exp(-gate)) * gate_up[static_cast<size_t>(t) * 2 * ffn + ffn + c];
            }
        }
        project_rows(m, o[13], kNoTensor, enc(6), h, ffn, count, activated.data(), ffn, hidden.data(), h, 0, true, threads);
    }
    // logits (step/layers.rs:208-228): the gathered rows in token order.
    int rows = 0;
    for (int t = 0; t < count; ++t) {
        if (tokens[4 * t + 3] >= 0) {
            rms_norm_row(&hidden[static_cast<size_t>(t) * h], f32_at(m, m.output_norm), h, m.epsilon,
                         &normalized[static_cast<size_t>(rows) * h]);
            ++rows;
        }
    }
    if (rows > 0) {
        project_rows(m, m.output, kNoTensor, m.output_encoding, m.vocabulary, h, rows, normalized.data(), h, logits, m.vocabulary, 0, false,
                     threads);
    }
    return 0;
}

}  // extern "C"
