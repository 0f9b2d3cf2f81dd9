// Key summaries of KV page activation (ADR-016): per (pool page, layer, KV head, activation page of 16, 32 or 64
// positions) the per-channel minimum and maximum of the page's keys below the writing slot's length, kept in the
// storage type (exact). KvPageSelector.PageBound (src/Synapse.Runtime/Features/TextGeneration/KvPageSelector.cs:57-78) reduces the page's keys with MathF.Min and
// MathF.Max; both are exact and, for the non-NaN values keys hold, independent of the order of the keys.
#pragma once

#include "kv_internal.h"
#include "page_layout.h"

namespace synapse_kv {

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

template <typename T>
__device__ inline float widen(T value) {
    return static_cast<float>(value);
}

// Element offset of (layer, kv_head, activation page of the pool page, min|max, channel) in a summary page.
__device__ inline size_t summary_offset(const Geometry& g, int layer, int kv_head, int block, int which, int channel) {
    const int blocks = g.page_tokens / g.summary_keys;
    return ((((static_cast<size_t>(layer) * g.kv_heads + kv_head) * blocks + block) * 2 + which) * g.head_dim) + channel;
}

// LDS the block summary needs: one 64-key block of one KV head (fragment order, as stored) and the partial
// minima and maxima of up to 512 (channel, share) items.
template <typename T>
struct SummaryScratch {
    T keys[kBlockKeys * 128];
    float partial[2][512];
};

// Summary of the first `valid` (1..summary_keys) keys of activation page `block` of pool page `page` (layer,
// kv_head), by the whole workgroup (blockDim.x a multiple of 64, at most 512): the 64-key block holding the page is
// copied to LDS with 16-byte loads, the page's keys of each channel are reduced in shares, and the shares combined.
// Starts and ends with a barrier.
template <typename T>
__device__ void summarize_block(const Geometry& g, int layer, int kv_head, int page, int block, int valid,
                                uint8_t* summaries, uint64_t summary_page_bytes, SummaryScratch<T>& scratch) {
    const int d = g.head_dim;
    const T* region = reinterpret_cast<const T*>(g.pool + static_cast<uint64_t>(page) * g.page_bytes) +
                      ((static_cast<size_t>(layer) * 2) * g.kv_heads + kv_head) * static_cast<size_t>(g.page_tokens) * d;
    const int first_key = block * g.summary_keys;  // within the pool page
    const int offset = first_key % kBlockKeys;     // within its 64-key block
    const uint4* source =
        reinterpret_cast<const uint4*>(region + static_cast<size_t>(first_key / kBlockKeys) * kBlockKeys * d);
    uint4* staged = reinterpret_cast<uint4*>(scratch.keys);
    const int chunks = kBlockKeys * d * static_cast<int>(sizeof(T)) / 16;
    __syncthreads();
    for (int chunk = threadIdx.x; chunk < chunks; chunk += blockDim.x) {
        staged[chunk] = source[chunk];
    }
    __syncthreads();
    const int fit = static_cast<int>(blockDim.x) / d;  // the keys of a channel are split into 1, 2 or 4 runs
    const int shares = fit >= 4 ? 4 : (fit >= 2 ? 2 : 1);
    const int per_share = g.summary_keys / shares;
    for (int item = threadIdx.x; item < d * shares; item += blockDim.x) {
        const int channel = item % d;
        const int share = item / d;
        // Unwritten keys are left out; a share holding none keeps (+inf, -inf), which the combination ignores.
        float minimum = __builtin_inff();
        float maximum = -__builtin_inff();
        const int stop = min((share + 1) * per_share, valid);
        for (int key = share * per_share; key < stop; ++key) {
            const float value = widen(scratch.keys[key_offset<T>(d, offset + key, channel)]);
            minimum = math_min(minimum, value);
            maximum = math_max(maximum, value);
        }
        scratch.partial[0][item] = minimum;
        scratch.partial[1][item] = maximum;
    }
    __syncthreads();
    for (int channel = threadIdx.x; channel < d; channel += blockDim.x) {
        float minimum = scratch.partial[0][channel];
        float maximum = scratch.partial[1][channel];
        for (int share = 1; share < shares; ++share) {
            minimum = math_min(minimum, scratch.partial[0][share * d + channel]);
            maximum = math_max(maximum, scratch.partial[1][share * d + channel]);
        }
        T* summary = reinterpret_cast<T*>(summaries + static_cast<uint64_t>(page) * summary_page_bytes);
        summary[summary_offset(g, layer, kv_head, block, 0, channel)] = static_cast<T>(minimum);
        summary[summary_offset(g, layer, kv_head, block, 1, channel)] = static_cast<T>(maximum);
    }
    __syncthreads();
}

}  // namespace synapse_kv
