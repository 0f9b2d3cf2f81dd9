// Fused RoPE + KV append (synapse_rope_kv, native/synapse-gpu/src/Features/GpuKernels/metal/shaders/
// elementwise.metal:73-126): rotate Q in place, rotate K in place and store it, store V, converting to the page's
// element type (FP16: round to nearest even, v_cvt_f16_f32 in the default rounding mode).
// The rotation follows Qwen2RopeTable.Apply (src/Synapse.Runtime/Features/TextGeneration/Qwen2/
// Qwen2CpuState.cs:85-106): x' = x*c - y*s, y' = x*s + y*c with every product and sum rounded separately (no
// fused multiply-add), so the result is bit-exact with the CPU path.
//
// One workgroup per token; every element goes to its MFMA-fragment slot of the page region (page_layout.h).

#include "kv_internal.h"
#include "page_layout.h"
#include "page_summary.h"

// hipcc contracts a*b - c*d into a fused multiply-add by default; the rotation must round every product.
#pragma clang fp contract(off)

namespace synapse_kv {
namespace {

template <typename T>
__device__ inline T to_storage(float value);

template <>
__device__ inline float to_storage<float>(float value) {
    return value;
}

template <>
__device__ inline _Float16 to_storage<_Float16>(float value) {
    return static_cast<_Float16>(value);
}

template <typename T>
__global__ __launch_bounds__(256) void append_kernel(AppendArgs a) {
    const Geometry& g = a.geo;
    const int index = blockIdx.x;
    const SynapseKvBatchToken token = a.tokens[index];
    float* row = a.qkv + static_cast<size_t>(index) * a.qkv_stride;
    const int half = a.half_dim;
    const int d = g.head_dim;
    const float* cosines = a.cosines + static_cast<size_t>(token.position) * half;
    const float* sines = a.sines + static_cast<size_t>(token.position) * half;
    const int logical = token.position / g.page_tokens;
    const int within = token.position - logical * g.page_tokens;
    const int page = g.block_table[static_cast<size_t>(token.slot) * g.pages_per_slot + logical];
    T* base = reinterpret_cast<T*>(a.pool + static_cast<uint64_t>(page) * g.page_bytes);
    const size_t region = static_cast<size_t>(g.page_tokens) * d;
    const size_t layer_base = static_cast<size_t>(g.layer) * 2 * g.kv_heads;

    // Without write-back only the K heads need rotating (Q is rotated where it is consumed).
    const int first_head = a.write_back ? 0 : g.heads;
    const int rotations = (g.heads + g.kv_heads - first_head) * half;
    for (int item = threadIdx.x; item < rotations; item += blockDim.x) {
        const int head = first_head + item / half;
        const int i = item % half;
        float* values = row + static_cast<size_t>(head) * d;  // K heads follow the Q heads in the row
        const float x = values[i];
        const float y = values[i + half];
        const float c = cosines[i];
        const float s = sines[i];
        const float first = x * c - y * s;   // contraction is off for this file: two products, one difference
        const float second = x * s + y * c;
        if (a.write_back) {
            values[i] = first;
            values[i + half] = second;
        }
        if (head >= g.heads) {
            const int kv_head = head - g.heads;
            T* keys = base + (layer_base + kv_head) * region;
            const T stored_first = to_storage<T>(first);
            const T stored_second = to_storage<T>(second);
            keys[key_offset<T>(d, within, i)] = stored_first;
            keys[key_offset<T>(d, within, i + half)] = stored_second;
            if (a.extend != nullptr && a.extend[index] != 0) {
                // The activation page's summary covers its keys below this position: fold the new key in
                // (MathF.Min / MathF.Max of KvPageSelector.PageBound), or start from it at the page's first position.
                T* summary = reinterpret_cast<T*>(a.summaries + static_cast<uint64_t>(page) * a.summary_page_bytes);
                const int block = within / g.summary_keys;
                const bool fresh = within % g.summary_keys == 0;
                const int channels[2] = {i, i + half};
                const float values[2] = {widen(stored_first), widen(stored_second)};
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    T& minimum = summary[summary_offset(g, g.layer, kv_head, block, 0, channels[c])];
                    T& maximum = summary[summary_offset(g, g.layer, kv_head, block, 1, channels[c])];
                    minimum = static_cast<T>(fresh ? values[c] : math_min(widen(minimum), values[c]));
                    maximum = static_cast<T>(fresh ? values[c] : math_max(widen(maximum), values[c]));
                }
            }
        }
    }

    const float* value_row = row + static_cast<size_t>(g.heads + g.kv_heads) * d;
    const int stores = g.kv_heads * d;
    for (int item = threadIdx.x; item < stores; item += blockDim.x) {
        const int kv_head = item / d;
        const int dim = item - kv_head * d;
        T* values = base + (layer_base + g.kv_heads + kv_head) * region;
        values[value_offset<T>(d, within, dim)] = to_storage<T>(value_row[item]);
    }
}

// Reads positions [first, first + count) of one slot/layer back into [position][kv_head][dim] order.
template <typename T>
__global__ __launch_bounds__(256) void gather_kernel(GatherArgs a) {
    const Geometry& g = a.geo;
    const int d = g.head_dim;
    const size_t per_position = static_cast<size_t>(g.kv_heads) * d;
    const size_t total = per_position * a.count;
    const size_t region = static_cast<size_t>(g.page_tokens) * d;
    const size_t layer_base = static_cast<size_t>(g.layer) * 2 * g.kv_heads;
    for (size_t index = blockIdx.x * 256ull + threadIdx.x; index < total; index += gridDim.x * 256ull) {
        const int position = a.first + static_cast<int>(index / per_position);
        const int kv_head = static_cast<int>((index % per_position) / d);
        const int dim = static_cast<int>(index % d);
        const int logical = position / g.page_tokens;
        const int within = position - logical * g.page_tokens;
        const int page = g.block_table[static_cast<size_t>(a.slot) * g.pages_per_slot + logical];
        const T* base = reinterpret_cast<const T*>(g.pool + static_cast<uint64_t>(page) * g.page_bytes);
        const T key = base[(layer_base + kv_head) * region + key_offset<T>(d, within, dim)];
        const T value = base[(layer_base + g.kv_heads + kv_head) * region + value_offset<T>(d, within, dim)];
        reinterpret_cast<T*>(a.keys)[index] = key;
        reinterpret_cast<T*>(a.values)[index] = value;
    }
}

// The inverse of gather_kernel: rows [count][kv_heads][head_dim] of K and V (the storage type) written into
// positions first.. of one slot and layer (prefix import).
template <typename T>
__global__ __launch_bounds__(256) void scatter_kernel(GatherArgs a) {
    const Geometry& g = a.geo;
    const int d = g.head_dim;
    const size_t per_position = static_cast<size_t>(g.kv_heads) * d;
    const size_t total = per_position * a.count;
    const size_t region = static_cast<size_t>(g.page_tokens) * d;
    const size_t layer_base = static_cast<size_t>(g.layer) * 2 * g.kv_heads;
    for (size_t index = blockIdx.x * 256ull + threadIdx.x; index < total; index += gridDim.x * 256ull) {
        const int position = a.first + static_cast<int>(index / per_position);
        const int kv_head = static_cast<int>((index % per_position) / d);
        const int dim = static_cast<int>(index % d);
        const int logical = position / g.page_tokens;
        const int within = position - logical * g.page_tokens;
        const int page = g.block_table[static_cast<size_t>(a.slot) * g.pages_per_slot + logical];
        T* base = reinterpret_cast<T*>(const_cast<uint8_t*>(g.pool) + static_cast<uint64_t>(page) * g.page_bytes);
        base[(layer_base + kv_head) * region + key_offset<T>(d, within, dim)] = reinterpret_cast<const T*>(a.keys)[index];
        base[(layer_base + g.kv_heads + kv_head) * region + value_offset<T>(d, within, dim)] =
            reinterpret_cast<const T*>(a.values)[index];
    }
}

}  // namespace

hipError_t launch_append(const Launch& launch, const AppendArgs& args, int tokens, bool fp16) {
    if (tokens == 0) {
        return hipSuccess;
    }
    if (fp16) {
        SYNAPSE_KV_LAUNCH(append_kernel<_Float16>, dim3(tokens), dim3(256), launch, args);
    } else {
        SYNAPSE_KV_LAUNCH(append_kernel<float>, dim3(tokens), dim3(256), launch, args);
    }
    return hipGetLastError();
}

hipError_t launch_gather(const Launch& launch, const GatherArgs& args, bool fp16) {
    const size_t total = static_cast<size_t>(args.geo.kv_heads) * args.geo.head_dim * args.count;
    if (total == 0) {
        return hipSuccess;
    }
    const size_t blocks = (total + 255) / 256;
    const dim3 grid(static_cast<unsigned>(blocks < 4096 ? blocks : 4096));
    if (fp16) {
        SYNAPSE_KV_LAUNCH(gather_kernel<_Float16>, grid, dim3(256), launch, args);
    } else {
        SYNAPSE_KV_LAUNCH(gather_kernel<float>, grid, dim3(256), launch, args);
    }
    return hipGetLastError();
}

hipError_t launch_scatter(const Launch& launch, const GatherArgs& args, bool fp16) {
    const size_t total = static_cast<size_t>(args.geo.kv_heads) * args.geo.head_dim * args.count;
    if (total == 0) {
        return hipSuccess;
    }
    const size_t blocks = (total + 255) / 256;
    const dim3 grid(static_cast<unsigned>(blocks < 4096 ? blocks : 4096));
    if (fp16) {
        SYNAPSE_KV_LAUNCH(scatter_kernel<_Float16>, grid, dim3(256), launch, args);
    } else {
        SYNAPSE_KV_LAUNCH(scatter_kernel<float>, grid, dim3(256), launch, args);
    }
    return hipGetLastError();
}

}  // namespace synapse_kv
