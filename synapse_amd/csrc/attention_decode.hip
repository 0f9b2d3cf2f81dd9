// GQA flash-decode attention: persistent wave workers over an evenly split key space, then a split merge.
//
// Semantics: synapse_attention_decode (native/synapse-gpu/src/Features/GpuKernels/metal/shaders/
// attention.metal:319-355) and synapse_attention_reduce (attention_reduce.metal:5-40): the query heads of one KV
// head (the GQA group) of one token attend keys 0..position of the token's slot (Qwen2Attention.cs:5-25) with an
// online softmax; a key range split across workers leaves unnormalized output plus (max, sum) per head, and the
// merge takes the max over splits with a positive sum, rescales by exp(m - max) and divides.
//
// Work split (MI355X): the host flattens every (token, KV head) row into 64-key steps and gives each resident wave
// an equal contiguous share of the steps (about the same bytes per wave whatever the ragged lengths). A wave walks
// its segments in order; a row that lies inside one wave is written normalized, a row cut by worker boundaries
// writes partial rows that the merge kernel combines. No tail of idle CUs, and each wave reads every K/V byte of
// its share once for all query heads of the group.
//
// Per 64-key step a wave computes S^T = K Q^T and O^T = V^T P^T on MFMA with the group's query heads as the 16
// columns (7 of 16 used under GQA 7:1):
//   FP16 KV: v_mfma_f32_16x16x32_f16. The A operand is 8 consecutive halves of one row: 8 dims of one key
//            (K, row-major) or 8 keys of one dim (V, stored transposed), one 128-bit load per lane. The keys of
//            the QK^T tiles are permuted so the C layout of S^T (lane holds rows 4g..4g+3 of two tiles) is exactly
//            the B layout of P^T for the PV product: no data movement between the two MFMAs.
//   FP32 KV: v_mfma_f32_16x16x4_f32 with float4 loads split across four k-steps.
// Softmax statistics live per lane (one query head per lane column); a row max needs two cross-lane steps.

#include "kv_internal.h"
#include "page_layout.h"

namespace synapse_kv {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = kDecodeBlockWaves;
constexpr float kNegativeInfinity = -__builtin_inff();

__device__ inline float fast_exp2(float value) { return __builtin_amdgcn_exp2f(value); }

// Qwen2RopeTable.Apply (Qwen2CpuState.cs:85-106) for one pair: separately rounded products and sums, so the
// rotated values are bit-exact with the CPU path.
__device__ inline void rotate_pair(float x, float y, float c, float s, float& first, float& second) {
#pragma clang fp contract(off)
    first = x * c - y * s;
    second = x * s + y * c;
}

template <typename T>
__device__ inline T load_fragment(const T* pointer) {
    return __builtin_nontemporal_load(pointer);  // K/V stream through once per launch
}

__device__ inline float max_across_groups(float value) {
    value = fmaxf(value, __shfl_xor(value, 16));
    return fmaxf(value, __shfl_xor(value, 32));
}

__device__ inline float sum_across_groups(float value) {
    value += __shfl_xor(value, 16);
    return value + __shfl_xor(value, 32);
}

__device__ inline size_t region_offset(const Geometry& g, int which, int kv_head) {
    return ((static_cast<size_t>(g.layer) * 2 + which) * g.kv_heads + kv_head) * static_cast<size_t>(g.page_tokens) *
           g.head_dim;
}

template <int D>
struct WaveState {
    floatx4 out[D / 16];  // O^T: lane (g, r) holds dims 16*mt + 4*g + i of query head r
    float maximum;        // running max of head r in log2 units
    float sum;            // this lane's share of the running sum of head r
};

template <int D>
__device__ inline void reset(WaveState<D>& state) {
#pragma unroll
    for (int mt = 0; mt < D / 16; ++mt) {
        state.out[mt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    state.maximum = kNegativeInfinity;
    state.sum = 0.0f;
}

// Online-softmax update of one 64-key step from its scaled, masked scores (4 tiles of 4 per lane). Returns the
// factor that rescales the earlier output and replaces the scores with probabilities.
__device__ inline float softmax_step(floatx4 (&scores)[4], float& maximum, float& sum) {
    float tile_max = kNegativeInfinity;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            tile_max = fmaxf(tile_max, scores[t][i]);
        }
    }
    tile_max = max_across_groups(tile_max);
    const float next = fmaxf(maximum, tile_max);
    const float alpha = fast_exp2(maximum - next);
    float tile_sum = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            scores[t][i] = fast_exp2(scores[t][i] - next);
            tile_sum += scores[t][i];
        }
    }
    sum = sum * alpha + tile_sum;
    maximum = next;
    return alpha;
}

template <int D>
struct Fragments16 {
    half8 key[4][D / 32];
    half8 value[2][D / 16];
};

// value + the value of the lane 8 places away in the same row of 16 lanes (DPP row_ror:8, a rotation by 8 within
// each row): lanes r and r + 8 exchange values, so both get the same sum (addition commutes bit-exactly).
__device__ inline float add_half_row(float value) {
    return value + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, value), 0x128, 0xF,
                                                                         0xF, false));
}

template <int D>
struct QueryLoads {
    float values[D / 32][8];
    float cosines[D / 64][8];
    float sines[D / 64][8];
};

template <int D>
__device__ inline void issue_query_f16(const AttentionArgs& a, int token, int position, int kv_head,
                                       QueryLoads<D>& loads) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4;
    const int column = lane & 7;
    const bool valid = column < a.geo.group;
    const float* q = a.qkv + static_cast<size_t>(token) * a.qkv_stride +
                     static_cast<size_t>(kv_head * a.geo.group + (valid ? column : 0)) * D;
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
        const floatx4 lo = *reinterpret_cast<const floatx4*>(q + 32 * ks + 8 * g);
        const floatx4 hi = *reinterpret_cast<const floatx4*>(q + 32 * ks + 8 * g + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            loads.values[ks][j] = lo[j];
            loads.values[ks][j + 4] = hi[j];
        }
    }
    if (a.rotate) {
        const float* cosines = a.cosines + static_cast<size_t>(position) * (D / 2);
        const float* sines = a.sines + static_cast<size_t>(position) * (D / 2);
#pragma unroll
        for (int ks = 0; ks < D / 64; ++ks) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = 32 * ks + 8 * g + j;
                loads.cosines[ks][j] = cosines[i];
                loads.sines[ks][j] = sines[i];
            }
        }
    }
}

// B operand of S^T = K Q^T for one lane (g, r): dims 32*ks + 8*g .. +7 of query head r % 8 of the group of
// `kv_head` of `token`, rotated (when the call asks for RoPE) at the token's position. The FP32 query is split
// exactly into FP16 parts q = hi + lo (hi = q rounded to FP16, lo = the remainder rounded to FP16; |q - hi - lo|
// <= 2^-22 |q| for normal parts): columns 0..7 carry hi and columns 8..15 lo of the same heads (a GQA group has at
// most 8 heads), so one MFMA gives both products and add_half_row joins them: the product of the FP16 keys with
// the FP32 query to about FP32 accuracy, at no extra MFMA. Zero for columns past the group. With D/2 = 32 * (D/64)
// the RoPE partner of dim i < D/2 (i + D/2) sits in the same lane at ks + D/64.
template <int D>
__device__ inline void finish_query_f16(const AttentionArgs& a, QueryLoads<D>& loads, half8 (&query)[D / 32]) {
    const int lane = threadIdx.x & 63;
    const bool low_part = (lane & 8) != 0;
    const bool valid = (lane & 7) < a.geo.group;
    if (a.rotate) {
#pragma unroll
        for (int ks = 0; ks < D / 64; ++ks) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                rotate_pair(loads.values[ks][j], loads.values[ks + D / 64][j], loads.cosines[ks][j],
                            loads.sines[ks][j], loads.values[ks][j], loads.values[ks + D / 64][j]);
            }
        }
    }
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float value = valid ? loads.values[ks][j] : 0.0f;
            const _Float16 high = static_cast<_Float16>(value);
            query[ks][j] = low_part ? static_cast<_Float16>(value - static_cast<float>(high)) : high;
        }
    }
}

template <int D>
__device__ inline void load_query_f16(const AttentionArgs& a, int token, int position, int kv_head,
                                      half8 (&query)[D / 32]) {
    QueryLoads<D> loads;
    issue_query_f16<D>(a, token, position, kv_head, loads);
    finish_query_f16<D>(a, loads, query);
}

// Loads the FP16 fragments of the 64-key block holding key0 (a multiple of 64) of one (slot table, KV head).
// `known_page` >= 0: the block's pool page (from the plan), else read from the block table.
template <int D>
__device__ inline void fetch_f16(const Geometry& geo, const int32_t* table, size_t key_region, size_t value_region,
                                 int key0, Fragments16<D>& fragments, int known_page = -1) {
    const int lane = threadIdx.x & 63;
    const int logical = key0 / geo.page_tokens;
    const int within = key0 - logical * geo.page_tokens;
    const int page_index = known_page >= 0 ? known_page : load_uniform(table + logical);
    const _Float16* page =
        reinterpret_cast<const _Float16*>(geo.pool + static_cast<uint64_t>(page_index) * geo.page_bytes);
    // 64-key blocks in fragment order: every load below is one contiguous 1 KiB wave load.
    const half8* keys = reinterpret_cast<const half8*>(page + key_region + static_cast<size_t>(within) * D) + lane;
    const half8* values = reinterpret_cast<const half8*>(page + value_region + static_cast<size_t>(within) * D) + lane;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            fragments.key[t][ks] = load_fragment(keys + (t * (D / 32) + ks) * 64);
        }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int mt = 0; mt < D / 16; ++mt) {
            fragments.value[h][mt] = load_fragment(values + (h * (D / 16) + mt) * 64);
        }
    }
}

// One 64-key step for one column tile: S^T = K Q^T, masked scale to log2 units, online softmax, O^T += V^T P^T.
// The A operand of QK^T tile t = 2h + u holds key 32h + 8*(r/4) + 4u + r%4 in row r (the page layout stores it
// there), so the C tile puts key 32h + 8g + 4u + i on this lane group's element 4u + i of the PV B operand.
// Columns r and r + 8 hold the hi and lo products of head r % 8; after add_half_row both hold the head's FP32 score
// and run the same softmax. The probabilities enter the PV product split the same way (column r: hi, column r + 8:
// lo), so the O^T columns r and r + 8 add up, at the end, to V times the FP32 probabilities the row sum adds up (to
// 2^-22 relative, or 2^-25 absolute).
template <int D>
__device__ inline void step_f16(const Fragments16<D>& fragments, const half8 (&query)[D / 32], WaveState<D>& state,
                                int key0, int key_low, int key_end, float scale_log2) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4;
    const bool low_part = (lane & 8) != 0;
    floatx4 scores[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        scores[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            scores[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fragments.key[t][ks], query[ks], scores[t], 0, 0, 0);
        }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // key_low <= key < key_end, as one unsigned compare.
            const int key = key0 + 32 * (t >> 1) + 8 * g + 4 * (t & 1) + i;
            const bool visible = static_cast<uint32_t>(key - key_low) < static_cast<uint32_t>(key_end - key_low);
            scores[t][i] = visible ? add_half_row(scores[t][i]) * scale_log2 : kNegativeInfinity;
        }
    }
    const float alpha = softmax_step(scores, state.maximum, state.sum);
    half8 probability[2];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p = scores[t][i];
            const _Float16 high = static_cast<_Float16>(p);
            probability[t >> 1][4 * (t & 1) + i] = low_part ? static_cast<_Float16>(p - static_cast<float>(high)) : high;
        }
    }
#pragma unroll
    for (int mt = 0; mt < D / 16; ++mt) {
        state.out[mt] *= alpha;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int mt = 0; mt < D / 16; ++mt) {
            state.out[mt] =
                __builtin_amdgcn_mfma_f32_16x16x32_f16(fragments.value[h][mt], probability[h], state.out[mt], 0, 0, 0);
        }
    }
}

// Steps [step_begin, step_end) of one KV head through the block table `table` against one column tile of queries,
// FP16 pages: step s covers the 64-key block of keys 64 s .. (list null), or under KV page activation the activation
// page of a.geo.summary_keys keys from key list[s] (the 64-key block holding it is read, its other keys masked); keys
// at or past `key_limit` are masked. The list is read with uniform (scalar) loads. With PREFETCH the next step's
// fragments are loaded before the current step is computed.
// With PREFETCH the caller has already requested the first step's block into `first` (attend_f16).
template <int D, bool PREFETCH>
__device__ void attend_blocks_f16(const AttentionArgs& a, const int32_t* table, int kv_head, int step_begin,
                                  int step_end, const int32_t* list, int key_limit, const half8 (&query)[D / 32],
                                  WaveState<D>& state, Fragments16<D>& first) {
    const Geometry& geo = a.geo;
    const size_t key_region = region_offset(geo, 0, kv_head);
    const size_t value_region = region_offset(geo, 1, kv_head);
    // A step's entry: its first visible key (a page's first key under activation, else the block's first key).
    auto first_key = [&](int step) __attribute__((always_inline)) {
        return list != nullptr ? load_uniform(list + step) : step * kStepKeys;
    };
    const int span = geo.summary_keys;
    auto attend = [&](const Fragments16<D>& fragments, int entry) __attribute__((always_inline)) {
        const int low = list != nullptr ? entry : 0;
        const int end = list != nullptr ? min(entry + span, key_limit) : key_limit;
        step_f16<D>(fragments, query, state, entry & ~(kStepKeys - 1), low, end, a.scale_log2);
    };
    if constexpr (!PREFETCH) {
        for (int step = step_begin; step < step_end; ++step) {
            Fragments16<D> fragments;
            const int key0 = first_key(step);
            fetch_f16<D>(geo, table, key_region, value_region, key0 & ~(kStepKeys - 1), fragments);
            attend(fragments, key0);
        }
    } else {
        // Two register sets: the loads of the next step are in flight while the current step computes. The loop
        // runs while at least two steps remain, so both of its fetches are unconditional and every step waits only
        // for its own fragments (a fetch under a branch would leave the number of loads in flight unknown at the
        // join, and the step after it would wait for the prefetched block too); the last one or two steps follow.
        Fragments16<D>& even = first;
        Fragments16<D> odd;
        constexpr int kBlock = ~(kStepKeys - 1);
        int step = step_begin;
        int key0 = first_key(step);
        while (step + 2 < step_end) {
            const int key1 = first_key(step + 1);
            const int key2 = first_key(step + 2);
            fetch_f16<D>(geo, table, key_region, value_region, key1 & kBlock, odd);
            attend(even, key0);
            fetch_f16<D>(geo, table, key_region, value_region, key2 & kBlock, even);
            attend(odd, key1);
            step += 2;
            key0 = key2;
        }
        if (step + 1 < step_end) {
            const int key1 = first_key(step + 1);
            fetch_f16<D>(geo, table, key_region, value_region, key1 & kBlock, odd);
            attend(even, key0);
            attend(odd, key1);
        } else {
            attend(even, key0);
        }
    }
}

// One token's segment for one KV head, FP16 pages.
// With PREFETCH the segment's first K/V block is requested between the query's loads and its use (the query and
// the block are one round trip, not two), from the plan's page of that block when it has one.
template <int D, bool PREFETCH>
__device__ void attend_f16(const AttentionArgs& a, const DecodeSegment& seg, WaveState<D>& state) {
    const Geometry& geo = a.geo;
    const int32_t* table = geo.block_table + static_cast<size_t>(seg.slot) * geo.pages_per_slot;
    const int32_t* list = seg.list >= 0 ? a.lists + seg.list : nullptr;
    const int step_begin = seg.key_begin / kStepKeys;
    const int step_end = (seg.key_end + kStepKeys - 1) / kStepKeys;
    half8 query[D / 32];
    Fragments16<D> first;
    if constexpr (PREFETCH) {
        QueryLoads<D> loads;
        issue_query_f16<D>(a, seg.token, seg.position, seg.kv_head, loads);
        __builtin_amdgcn_sched_barrier(0);
        const int key0 = list != nullptr ? load_uniform(list + step_begin) : step_begin * kStepKeys;
        fetch_f16<D>(geo, table, region_offset(geo, 0, seg.kv_head), region_offset(geo, 1, seg.kv_head),
                     key0 & ~(kStepKeys - 1), first, list != nullptr ? -1 : seg.first_page);
        __builtin_amdgcn_sched_barrier(0);
        finish_query_f16<D>(a, loads, query);
    } else {
        load_query_f16<D>(a, seg.token, seg.position, seg.kv_head, query);
    }
    attend_blocks_f16<D, PREFETCH>(a, table, seg.kv_head, step_begin, step_end, list,
                                   list != nullptr ? seg.position + 1 : seg.key_end, query, state, first);
}

// One token's segment for one KV head, FP32 pages. The first step's K and V are requested right after the query's
// loads (the plan carries the block's pool page), so the query and the first block are one round trip.
template <int D>
__device__ void attend_f32(const AttentionArgs& a, const DecodeSegment& seg, WaveState<D>& state) {
    const Geometry& geo = a.geo;
    const int lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int g = lane >> 4;
    // B operand of S^T = K Q^T for k-step (c, i): dim 16*c + 4*g + i of query head r. The RoPE partner of dim
    // i < D/2 sits in the same lane at c + D/32.
    floatx4 query[D / 16];
    float cosines[D / 32][4];
    float sines[D / 32][4];
    const bool valid = r < geo.group;
    {
        const float* q = a.qkv + static_cast<size_t>(seg.token) * a.qkv_stride +
                         static_cast<size_t>(seg.kv_head * geo.group + (valid ? r : 0)) * D;
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
            query[c] = *reinterpret_cast<const floatx4*>(q + 16 * c + 4 * g);
        }
        if (a.rotate) {
            const float* cos_row = a.cosines + static_cast<size_t>(seg.position) * (D / 2);
            const float* sin_row = a.sines + static_cast<size_t>(seg.position) * (D / 2);
#pragma unroll
            for (int c = 0; c < D / 32; ++c) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    cosines[c][i] = cos_row[16 * c + 4 * g + i];
                    sines[c][i] = sin_row[16 * c + 4 * g + i];
                }
            }
        }
    }
    const int32_t* table = geo.block_table + static_cast<size_t>(seg.slot) * geo.pages_per_slot;
    const size_t key_region = region_offset(geo, 0, seg.kv_head);
    const size_t value_region = region_offset(geo, 1, seg.kv_head);
    const int page_tokens = geo.page_tokens;
    // Step s covers keys 64 s .. of block s, or under KV page activation the activation page from key list[s] (the
    // 64-key block holding it is read, its other keys masked); keys at or past key_limit are masked.
    const int32_t* list = seg.list >= 0 ? a.lists + seg.list : nullptr;
    const int key_limit = list != nullptr ? seg.position + 1 : seg.key_end;
    const int step_begin = seg.key_begin / kStepKeys;
    const int step_end = (seg.key_end + kStepKeys - 1) / kStepKeys;

    // The step's K and V fragments are requested together: one memory round trip per step.
    floatx4 key_fragment[4][D / 16];
    floatx4 value_fragment[4][D / 16];
    auto fetch = [&](int step) __attribute__((always_inline)) {
        const int entry = list != nullptr ? load_uniform(list + step) : step * kStepKeys;
        const int key0 = entry & ~(kStepKeys - 1);
        const int logical = key0 / page_tokens;
        const int within = key0 - logical * page_tokens;
        // The first step's page comes with the plan (no table read before the wave's first request).
        const int page_index =
            step == step_begin && list == nullptr && seg.first_page >= 0 ? seg.first_page : load_uniform(table + logical);
        const float* page = reinterpret_cast<const float*>(geo.pool + static_cast<uint64_t>(page_index) * geo.page_bytes);
        const floatx4* keys =
            reinterpret_cast<const floatx4*>(page + key_region + static_cast<size_t>(within) * D) + lane;
        const floatx4* values =
            reinterpret_cast<const floatx4*>(page + value_region + static_cast<size_t>(within) * D) + lane;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int c = 0; c < D / 16; ++c) {
                key_fragment[t][c] = load_fragment(keys + (t * (D / 16) + c) * 64);
            }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int mt = 0; mt < D / 16; ++mt) {
                value_fragment[t][mt] = load_fragment(values + (t * (D / 16) + mt) * 64);
            }
        }
        return entry;
    };
    auto compute = [&](int entry) __attribute__((always_inline)) {
        const int key0 = entry & ~(kStepKeys - 1);
        const int key_low = list != nullptr ? entry : 0;
        const int key_end = list != nullptr ? min(entry + geo.summary_keys, key_limit) : key_limit;
        floatx4 scores[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            scores[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < D / 16; ++c) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    scores[t] =
                        __builtin_amdgcn_mfma_f32_16x16x4f32(key_fragment[t][c][i], query[c][i], scores[t], 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = key0 + 16 * t + 4 * g + i;
                const bool visible =
                    static_cast<uint32_t>(key - key_low) < static_cast<uint32_t>(key_end - key_low);
                scores[t][i] = visible ? scores[t][i] * a.scale_log2 : kNegativeInfinity;
            }
        }
        const float alpha = softmax_step(scores, state.maximum, state.sum);
#pragma unroll
        for (int mt = 0; mt < D / 16; ++mt) {
            state.out[mt] *= alpha;
        }
        // O^T = V^T P^T: k-step (t, i) pairs lane group g with key 16*t + 4*g + i.
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int mt = 0; mt < D / 16; ++mt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    state.out[mt] = __builtin_amdgcn_mfma_f32_16x16x4f32(value_fragment[t][mt][i], scores[t][i],
                                                                         state.out[mt], 0, 0, 0);
                }
            }
        }
    };

    // Keeps the scheduler from sinking the loads towards their uses (which would serialize the round trips).
    int entry = fetch(step_begin);
    __builtin_amdgcn_sched_barrier(0);
    if (a.rotate) {
#pragma unroll
        for (int c = 0; c < D / 32; ++c) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float first;
                float second;
                rotate_pair(query[c][i], query[c + D / 32][i], cosines[c][i], sines[c][i], first, second);
                query[c][i] = first;
                query[c + D / 32][i] = second;
            }
        }
    }
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
        if (!valid) {
            query[c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    compute(entry);
    for (int step = step_begin + 1; step < step_end; ++step) {
        entry = fetch(step);
        __builtin_amdgcn_sched_barrier(0);
        compute(entry);
    }
}

// Writes a wave's finished segment: the normalized output of an uncut row, or the segment's partial row (its
// unnormalized output and, per head, the running max and sum) for the merge kernel.
// With SPLIT_COLUMNS (FP16 pages) the output columns r and r + 8 hold the hi and lo parts of head r's product and
// are added first.
template <int D, bool SPLIT_COLUMNS>
__device__ void finish_segment(const AttentionArgs& a, const DecodeSegment& seg, WaveState<D>& state) {
    const int lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int group = a.geo.group;
    const float total = sum_across_groups(state.sum);
    if constexpr (SPLIT_COLUMNS) {
#pragma unroll
        for (int mt = 0; mt < D / 16; ++mt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                state.out[mt][i] = add_half_row(state.out[mt][i]);
            }
        }
    }
    if (r >= group) {
        return;
    }
    if (seg.row < 0) {
        float* destination = a.output + static_cast<size_t>(seg.token) * a.out_stride +
                             static_cast<size_t>(seg.kv_head * group + r) * D;
        const float inverse = 1.0f / total;
#pragma unroll
        for (int mt = 0; mt < D / 16; ++mt) {
            *reinterpret_cast<floatx4*>(destination + 16 * mt + 4 * g) = state.out[mt] * inverse;
        }
        return;
    }
    const size_t row = static_cast<size_t>(seg.row) * group + r;
    float* destination = a.partial_out + row * D;
#pragma unroll
    for (int mt = 0; mt < D / 16; ++mt) {
        *reinterpret_cast<floatx4*>(destination + 16 * mt + 4 * g) = state.out[mt];
    }
    if (g == 0) {
        a.partial_ml[row * 2] = state.maximum;
        a.partial_ml[row * 2 + 1] = total;
    }
}

// Fused append (synapse_rope_kv, elementwise.metal:73-126) of one (token, KV head) by the wave that owns the row's
// last segment, i.e. the only wave that reads the token's own position: rotate K, store K and V in the page's
// element type, then wait for the stores before this wave's loads. The qkv rows are read, not rewritten.
template <typename T, int D>
__device__ void append_row(const AttentionArgs& a, const DecodeSegment& seg) {
    const Geometry& geo = a.geo;
    const int lane = threadIdx.x & 63;
    const int logical = seg.position / geo.page_tokens;
    const int within = seg.position - logical * geo.page_tokens;
    const int32_t page =
        seg.append_page >= 0
            ? seg.append_page
            : load_uniform(geo.block_table + static_cast<size_t>(seg.slot) * geo.pages_per_slot + logical);
    T* base = reinterpret_cast<T*>(const_cast<uint8_t*>(geo.pool) + static_cast<uint64_t>(page) * geo.page_bytes);
    T* keys = base + region_offset(geo, 0, seg.kv_head);
    T* values = base + region_offset(geo, 1, seg.kv_head);
    const float* row = a.qkv + static_cast<size_t>(seg.token) * a.qkv_stride;
    const float* key = row + static_cast<size_t>(geo.heads + seg.kv_head) * D;
    const float* value = row + static_cast<size_t>(geo.heads + geo.kv_heads + seg.kv_head) * D;
    const float* cosines = a.cosines + static_cast<size_t>(seg.position) * (D / 2);
    const float* sines = a.sines + static_cast<size_t>(seg.position) * (D / 2);
    for (int i = lane; i < D / 2; i += 64) {
        float first;
        float second;
        rotate_pair(key[i], key[i + D / 2], cosines[i], sines[i], first, second);
        keys[key_offset<T>(D, within, i)] = static_cast<T>(first);
        keys[key_offset<T>(D, within, i + D / 2)] = static_cast<T>(second);
    }
    for (int dim = lane; dim < D; dim += 64) {
        values[value_offset<T>(D, within, dim)] = static_cast<T>(value[dim]);
    }
    // The stores reach this XCD's L2 before the wave's own loads of the block are issued; no other wave reads the
    // row's region in this launch, so no device-wide fence (L2 write-back) is needed.
    __builtin_amdgcn_s_waitcnt(0);
}

template <int D, bool F16, bool PREFETCH>
__global__ __launch_bounds__(kWaves * 64) void decode_kernel(AttentionArgs a) {
    // The segment descriptors are uniform reads of the step's plan (scalar loads): a descriptor carries everything
    // a segment needs before its query and first block can be requested, the block's pool page included.
    const int worker = __builtin_amdgcn_readfirstlane(blockIdx.x * kWaves + (threadIdx.x >> 6));
    if (worker >= a.workers) {
        return;
    }
    const uint64_t started = a.timing != nullptr ? __builtin_amdgcn_s_memrealtime() : 0;
    // Worker w's first segment is segment w; the later ones follow `next`.
    for (int index = worker; index >= 0;) {
        const DecodeSegment seg = load_uniform(a.segments + index);
        index = seg.next;
        if (seg.token < 0) {
            break;
        }
        if (a.append && seg.last) {
            if constexpr (F16) {
                append_row<_Float16, D>(a, seg);
            } else {
                append_row<float, D>(a, seg);
            }
        }
        WaveState<D> state;
        reset(state);
        if constexpr (F16) {
            attend_f16<D, PREFETCH>(a, seg, state);
        } else {
            attend_f32<D>(a, seg, state);
        }
        finish_segment<D, F16>(a, seg, state);
    }
    if (a.timing != nullptr && (threadIdx.x & 63) == 0) {
        a.timing[worker] = static_cast<uint32_t>(__builtin_amdgcn_s_memrealtime() - started);
    }
}

// The weighted sum of up to 64 * R splits in one round of loads: every split's row value and (max, sum) are
// requested before any is used. Lane l holds splits l, l + 64, ...; the max runs over splits with a positive sum
// and each split's weight is exp2(m - max). Returns the lane's share of the weighted sums in `sum` and the weighted
// row value in `value`, splits added in order.
template <int D, int R>
__device__ inline void merge_splits(const AttentionArgs& a, const MergeItem& merge, int head, int column,
                                    float& maximum, float& sum, float& value) {
    const int lane = threadIdx.x & 63;
    const int group = a.geo.group;
    const size_t stride = static_cast<size_t>(group) * D;
    const float* rows = a.partial_out + (static_cast<size_t>(merge.first_row) * group + head) * D + column;
    float values[R][64];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int split = 0; split < 64; ++split) {
            values[r][split] = 64 * r + split < merge.count ? rows[(64 * r + split) * stride] : 0.0f;
        }
    }
    float split_max[R];
    float split_sum[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        split_max[r] = kNegativeInfinity;
        split_sum[r] = 0.0f;
        if (64 * r + lane < merge.count) {
            const size_t row = static_cast<size_t>(merge.first_row + 64 * r + lane) * group + head;
            split_max[r] = a.partial_ml[row * 2];
            split_sum[r] = a.partial_ml[row * 2 + 1];
        }
    }
    maximum = kNegativeInfinity;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        maximum = fmaxf(maximum, split_sum[r] > 0.0f ? split_max[r] : kNegativeInfinity);
    }
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        maximum = fmaxf(maximum, __shfl_xor(maximum, offset));
    }
    sum = 0.0f;
    value = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float weight = split_sum[r] > 0.0f ? fast_exp2(split_max[r] - maximum) : 0.0f;
        sum += split_sum[r] * weight;
#pragma unroll
        for (int split = 0; split < 64; ++split) {
            const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, weight), split));
            value += values[r][split] * w;
        }
    }
}

// Writes a merged row: normalized into the output, or, at the first level of a two-level merge, as a partial row
// itself (unnormalized values relative to `maximum`, with their weighted sum).
template <int D>
__device__ inline void store_merged(const AttentionArgs& a, const MergeItem& merge, int head, int chunk,
                                    float maximum, float sum, float value) {
    const int lane = threadIdx.x & 63;
    const int group = a.geo.group;
    if (merge.output_row >= 0) {
        const size_t row = static_cast<size_t>(merge.output_row) * group + head;
        a.partial_out[row * D + 64 * chunk + lane] = value;
        if (chunk == 0 && lane == 0) {
            a.partial_ml[row * 2] = maximum;
            a.partial_ml[row * 2 + 1] = sum;
        }
        return;
    }
    a.output[static_cast<size_t>(merge.token) * a.out_stride +
             static_cast<size_t>(merge.kv_head * group + head) * D + 64 * chunk + lane] = value / sum;
}

// Split merge (attention_reduce.metal:5-40): one wave per (merge entry, query head of the group, 64 dims). The
// lanes first load the (max, sum) of 64 or 128 splits at once, reduce the max over splits with a positive sum and
// turn each split into its weight exp2(m - max); the output is then the weighted sum of the splits' rows over the
// weighted sums, every row load independent of the others. Rows of more than 128 splits go to merge_wide_kernel,
// or, past its limit, are merged in two launches: blocks of 64 splits into intermediate partial rows
// (output_row >= 0), then those.
template <int D>
__global__ __launch_bounds__(kWaves * 64) void merge_kernel(AttentionArgs a, int first, int count) {
    const int group = a.geo.group;
    const int chunks = D / 64;
    const int job = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (job >= count * group * chunks) {
        return;
    }
    const int lane = threadIdx.x & 63;
    // The wave's merge item is a uniform read of the step's plan (a scalar load: one vector round trip fewer
    // before the partial rows are requested).
    const MergeItem merge = load_uniform(a.merges + __builtin_amdgcn_readfirstlane(first + job / (group * chunks)));
    const int head = (job / chunks) % group;
    const int chunk = job % chunks;
    const float* ml = a.partial_ml;
    const size_t stride = static_cast<size_t>(group) * D;
    float sum = 0.0f;
    float value = 0.0f;
    float maximum = kNegativeInfinity;
    if (merge.count <= 64) {
        merge_splits<D, 1>(a, merge, head, 64 * chunk + lane, maximum, sum, value);
    } else if (merge.count <= 128) {
        merge_splits<D, 2>(a, merge, head, 64 * chunk + lane, maximum, sum, value);
    } else {
        for (int base = 0; base < merge.count; base += 64) {
            const int split = base + lane;
            if (split < merge.count) {
                const size_t row = static_cast<size_t>(merge.first_row + split) * group + head;
                if (ml[row * 2 + 1] > 0.0f) {
                    maximum = fmaxf(maximum, ml[row * 2]);
                }
            }
        }
#pragma unroll
        for (int offset = 32; offset > 0; offset >>= 1) {
            maximum = fmaxf(maximum, __shfl_xor(maximum, offset));
        }
        for (int base = 0; base < merge.count; base += 64) {
            const int split = base + lane;
            float weight = 0.0f;
            if (split < merge.count) {
                const size_t row = static_cast<size_t>(merge.first_row + split) * group + head;
                const float total = ml[row * 2 + 1];
                weight = total > 0.0f ? fast_exp2(ml[row * 2] - maximum) : 0.0f;
                sum += total * weight;
            }
            const int here = min(64, merge.count - base);
            const float* rows =
                a.partial_out + (static_cast<size_t>(merge.first_row + base) * group + head) * D + 64 * chunk + lane;
            for (int index = 0; index < here; ++index) {
                value += rows[index * stride] * __shfl(weight, index);
            }
        }
    }
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        sum += __shfl_xor(sum, offset);
    }
    store_merged<D>(a, merge, head, chunk, maximum, sum, value);
}

// Wide split merge: one workgroup of kWideWaves waves per (merge entry, query head, 64 dims) for rows of up to
// 128 * kWideWaves splits. Wave w merges its share of about count / kWideWaves consecutive splits as merge_kernel
// does (one round of loads), then wave 0 combines the waves' (max, sum, row) through LDS with the same rescaling: a
// row of any piece count up to the limit takes one launch and about the latency of a merge of count / kWideWaves
// splits.
template <int D>
__global__ __launch_bounds__(kWideWaves * 64) void merge_wide_kernel(AttentionArgs a, int first, int count) {
    __shared__ float rows[kWideWaves][64];
    __shared__ float stats[kWideWaves][2];
    const int group = a.geo.group;
    const int chunks = D / 64;
    const int job = blockIdx.x;
    if (job >= count * group * chunks) {
        return;
    }
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const MergeItem merge = load_uniform(a.merges + first + job / (group * chunks));
    const int head = (job / chunks) % group;
    const int chunk = job % chunks;
    // The splits are shared out evenly: wave w takes `per` consecutive splits (at most 128).
    const int per = (merge.count + kWideWaves - 1) / kWideWaves;
    MergeItem part = merge;
    part.first_row = merge.first_row + per * wave;
    part.count = min(per, max(0, merge.count - per * wave));
    float maximum = kNegativeInfinity;
    float sum = 0.0f;
    float value = 0.0f;
    if (part.count > 64) {
        merge_splits<D, 2>(a, part, head, 64 * chunk + lane, maximum, sum, value);
    } else if (part.count > 0) {
        merge_splits<D, 1>(a, part, head, 64 * chunk + lane, maximum, sum, value);
    }
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        sum += __shfl_xor(sum, offset);
    }
    rows[wave][lane] = value;
    if (lane == 0) {
        stats[wave][0] = maximum;
        stats[wave][1] = sum;
    }
    __syncthreads();
    if (wave != 0) {
        return;
    }
    float total_max = kNegativeInfinity;
#pragma unroll
    for (int w = 0; w < kWideWaves; ++w) {
        total_max = fmaxf(total_max, stats[w][1] > 0.0f ? stats[w][0] : kNegativeInfinity);
    }
    float total = 0.0f;
    float combined = 0.0f;
#pragma unroll
    for (int w = 0; w < kWideWaves; ++w) {
        const float scale = stats[w][1] > 0.0f ? fast_exp2(stats[w][0] - total_max) : 0.0f;
        total += stats[w][1] * scale;
        combined += rows[w][lane] * scale;
    }
    store_merged<D>(a, merge, head, chunk, total_max, total, combined);
}

template <int D, bool F16, bool PREFETCH>
int resident_blocks() {
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, decode_kernel<D, F16, PREFETCH>, kWaves * 64, 0) !=
        hipSuccess) {
        (void)hipGetLastError();
        return 1;
    }
    return blocks > 0 ? blocks : 1;
}

}  // namespace

int decode_resident_waves(int device, bool fp16, int head_dim, bool prefetch) {
    hipDeviceProp_t properties{};
    if (hipGetDeviceProperties(&properties, device) != hipSuccess) {
        (void)hipGetLastError();
        return 1024;
    }
    int blocks = 1;
    if (fp16 && prefetch) {
        blocks = head_dim == 128 ? resident_blocks<128, true, true>() : resident_blocks<64, true, true>();
    } else if (fp16) {
        blocks = head_dim == 128 ? resident_blocks<128, true, false>() : resident_blocks<64, true, false>();
    } else {
        blocks = head_dim == 128 ? resident_blocks<128, false, false>() : resident_blocks<64, false, false>();
    }
    return properties.multiProcessorCount * blocks * kWaves;
}

hipError_t launch_decode(const Launch& launch, const AttentionArgs& args, bool fp16, bool prefetch) {
    if (args.workers == 0) {
        return hipSuccess;
    }
    const dim3 grid((args.workers + kWaves - 1) / kWaves);
    const dim3 block(kWaves * 64);
    const int d = args.geo.head_dim;
    if (fp16 && prefetch) {
        if (d == 128) {
            SYNAPSE_KV_LAUNCH((decode_kernel<128, true, true>), grid, block, launch, args);
        } else {
            SYNAPSE_KV_LAUNCH((decode_kernel<64, true, true>), grid, block, launch, args);
        }
    } else if (fp16) {
        if (d == 128) {
            SYNAPSE_KV_LAUNCH((decode_kernel<128, true, false>), grid, block, launch, args);
        } else {
            SYNAPSE_KV_LAUNCH((decode_kernel<64, true, false>), grid, block, launch, args);
        }
    } else {
        if (d == 128) {
            SYNAPSE_KV_LAUNCH((decode_kernel<128, false, false>), grid, block, launch, args);
        } else {
            SYNAPSE_KV_LAUNCH((decode_kernel<64, false, false>), grid, block, launch, args);
        }
    }
    return hipGetLastError();
}

hipError_t launch_merge(const Launch& launch, const AttentionArgs& args, int first, int count, bool wide) {
    if (count == 0) {
        return hipSuccess;
    }
    const int jobs = count * args.geo.group * (args.geo.head_dim / 64);
    if (wide) {
        if (args.geo.head_dim == 128) {
            SYNAPSE_KV_LAUNCH(merge_wide_kernel<128>, dim3(jobs), dim3(kWideWaves * 64), launch, args, first, count);
        } else {
            SYNAPSE_KV_LAUNCH(merge_wide_kernel<64>, dim3(jobs), dim3(kWideWaves * 64), launch, args, first, count);
        }
        return hipGetLastError();
    }
    const dim3 grid((jobs + kWaves - 1) / kWaves);
    if (args.geo.head_dim == 128) {
        SYNAPSE_KV_LAUNCH(merge_kernel<128>, grid, dim3(kWaves * 64), launch, args, first, count);
    } else {
        SYNAPSE_KV_LAUNCH(merge_kernel<64>, grid, dim3(kWaves * 64), launch, args, first, count);
    }
    return hipGetLastError();
}

}  // namespace synapse_kv
