// Chunked-prefill (prompt-run) attention on FP16 MFMA.
//
// Semantics: synapse_attention for prompt runs (native/synapse-gpu/src/Features/GpuKernels/metal/shaders/
// attention.metal:254-313; dispatch step/attention.rs:62-104): consecutive tokens of one slot at consecutive
// positions attend causally, token j sees keys 0..position_j (mask `key <= row_position`, attention.metal:80-81),
// after the run's K/V were appended (step/layers.rs:95-96). Long runs split their keys across work items and
// merge with the decode merge kernel (same (max, sum) partial rows).
//
// MI355X mapping: one workgroup per (KV head, block of kPrefillTokens tokens, key split) with one wave per query
// head of the GQA group; the group's waves share every K/V block through a 4-deep LDS ring. Each wave
// holds its head's queries for the block as kPrefillTiles MFMA column tiles of 16 tokens and runs the decode
// kernel's 64-key step:
// S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_16x16x32_f16, every K/V fragment loaded once and used by all
// column tiles. Causal masking is a per-element compare against the column's position.
//
// The same kernel reads copy-on-write prefixes once for several sequences: a listed item's columns are the decode
// tokens of forks that share the item's pages (unmasked, each rotated at its own position), so every shared K/V
// block goes through HBM once per item instead of once per fork.

#include <type_traits>

#include "kv_internal.h"

namespace synapse_kv {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr float kNegativeInfinity = -__builtin_inff();
// Offsets trail the running maximum by less than this (log2 units), so probabilities stay below 256.
constexpr float kLazyRescale = 8.0f;

__device__ inline float fast_exp2(float value) { return __builtin_amdgcn_exp2f(value); }

// Cross-lane reductions without LDS. v_permlane16_swap (v_permlane32_swap) of a value with itself returns, in
// every lane, the value of the lane and of its partner lane ^ 16 (^ 32), one in each result.
__device__ inline float max_lanes16(float value) {
    const auto pair = __builtin_amdgcn_permlane16_swap(__float_as_uint(value), __float_as_uint(value), false, false);
    return fmaxf(__uint_as_float(pair[0]), __uint_as_float(pair[1]));
}
__device__ inline float max_lanes32(float value) {
    const auto pair = __builtin_amdgcn_permlane32_swap(__float_as_uint(value), __float_as_uint(value), false, false);
    return fmaxf(__uint_as_float(pair[0]), __uint_as_float(pair[1]));
}
__device__ inline float sum_lanes16(float value) {
    const auto pair = __builtin_amdgcn_permlane16_swap(__float_as_uint(value), __float_as_uint(value), false, false);
    return __uint_as_float(pair[0]) + __uint_as_float(pair[1]);
}
__device__ inline float sum_lanes32(float value) {
    const auto pair = __builtin_amdgcn_permlane32_swap(__float_as_uint(value), __float_as_uint(value), false, false);
    return __uint_as_float(pair[0]) + __uint_as_float(pair[1]);
}

// Qwen2RopeTable.Apply (Qwen2CpuState.cs:85-106) for one pair, products and sums rounded separately.
__device__ inline void rotate_pair(float x, float y, float c, float s, float& first, float& second) {
#pragma clang fp contract(off)
    first = x * c - y * s;
    second = x * s + y * c;
}

// The group's waves share each 64-key block through a 4-deep LDS ring. A block's K and V are two contiguous runs of
// 16-byte chunks in its page (fragment order); global_load_lds moves 64 of them per wave instruction, one per lane,
// into 1 KiB of LDS. Block b is copied during step b - 3 and completes by the end of step b - 2 (its K is read in
// step b - 1, its V in step b), so every copy has two steps to land. Page numbers of 64 consecutive logical pages
// are held one per lane and read with v_readlane, reloaded only when the copy position leaves the window, so the
// copies never wait on a table load.
template <int D, int WAVES>
struct KvRing {
    static constexpr int kKeyChunks = kStepKeys * D / 8;
    static constexpr int kBlockChunks = 2 * kKeyChunks;
    static constexpr int kBlockSegments = kBlockChunks / 64;
    static constexpr int kKeySegments = kKeyChunks / 64;
    static constexpr int kDepth = 4;
    static constexpr int kLoads = (kBlockSegments + WAVES - 1) / WAVES;

    half8 (*stage)[kBlockChunks];
    const int32_t* table;
    const uint8_t* pool;
    uint64_t page_bytes;
    size_t key_region;    // elements
    size_t value_region;  // elements
    int page_tokens;
    int last_page;
    int wave;
    int lane;
    bool full_share;  // this wave copies kLoads segments of a block (else kLoads - 1)
    int copy_logical;
    int copy_within;
    int window_first;
    int window;

    __device__ KvRing(half8 (*ring)[kBlockChunks], const Geometry& geo, const int32_t* slot_table, int kv_head,
                      int key_begin, int wave_index)
        : stage(ring),
          table(slot_table),
          pool(geo.pool),
          page_bytes(geo.page_bytes),
          key_region(((static_cast<size_t>(geo.layer) * 2) * geo.kv_heads + kv_head) *
                     (static_cast<size_t>(geo.page_tokens) * D)),
          value_region(((static_cast<size_t>(geo.layer) * 2 + 1) * geo.kv_heads + kv_head) *
                       (static_cast<size_t>(geo.page_tokens) * D)),
          page_tokens(geo.page_tokens),
          last_page(geo.pages_per_slot - 1),
          wave(wave_index),
          lane(threadIdx.x & 63),
          full_share(wave_index + (kLoads - 1) * WAVES < kBlockSegments),
          copy_logical(key_begin / geo.page_tokens),
          copy_within(key_begin - (key_begin / geo.page_tokens) * geo.page_tokens),
          window_first(key_begin / geo.page_tokens),
          window(slot_table[min(key_begin / geo.page_tokens + static_cast<int>(threadIdx.x & 63), last_page)]) {}

    // Copies the next block of the item's keys into ring buffer `buffer`.
    __device__ __forceinline__ void issue(int buffer) {
        if (copy_logical - window_first >= 64) {
            window_first = copy_logical;
            window = table[min(window_first + lane, last_page)];
            wait_vector_memory<0>();
        }
        const int page_index = __builtin_amdgcn_readlane(window, copy_logical - window_first);
        const uint8_t* page = pool + static_cast<uint64_t>(page_index) * page_bytes;
        const uint8_t* keys = page + (key_region + static_cast<size_t>(copy_within) * D) * sizeof(_Float16);
        const uint8_t* values = page + (value_region + static_cast<size_t>(copy_within) * D) * sizeof(_Float16);
#pragma unroll
        for (int k = 0; k < kLoads; ++k) {
            const int segment = wave + k * WAVES;
            if (segment < kBlockSegments) {
                const uint8_t* source =
                    (segment < kKeySegments ? keys + segment * 1024 : values + (segment - kKeySegments) * 1024) +
                    lane * 16;
                // Non-temporal (cache policy 2): C4's listed items stream the shared prefix 1.3 % faster, C5 the same.
                __builtin_amdgcn_global_load_lds(
                    source, (__attribute__((address_space(3))) void*)(&stage[buffer][segment * 64]), 16, 0, 2);
            }
        }
        copy_within += kStepKeys;
        if (copy_within == page_tokens) {
            copy_within = 0;
            ++copy_logical;
        }
    }

    // Waits for this wave's copies, except the newest block's when `newest_in_flight`, then for the group (whose
    // waves have then finished reading the buffer the next copy overwrites).
    __device__ __forceinline__ void ready(bool newest_in_flight) const {
        if (!newest_in_flight) {
            barrier_after_copies<0>();
        } else if (full_share) {
            barrier_after_copies<kLoads>();
        } else {
            barrier_after_copies<kLoads - 1>();
        }
    }
};

// NT column tiles of 16 tokens per wave: kPrefillTiles for prompt runs, 1 for listed items of at most 16 members.
template <int D, int WAVES, int NT>
__global__ __launch_bounds__(WAVES * 64) void prefill_f16_kernel(AttentionArgs a, int first_item) {
    const PrefillItem item = a.prefill[first_item + blockIdx.x];
    const Geometry& geo = a.geo;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // query head within the group
    const int lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int head = item.kv_head * geo.group + wave;
    const bool listed = item.listed != 0;
    // Step token of column j: the run's j-th token, or the j-th listed member.
    auto column_token = [&](int j) { return listed ? a.members[item.first_token + j] : item.first_token + j; };
    const SynapseKvBatchToken first = a.tokens[column_token(0)];
    const int first_position = first.position;

    // B operands of S^T = K Q^T: tile c, lane (g, r) holds dims 32*ks + 8*g .. +7 of token 16*c + r; the RoPE
    // partner of dim i < D/2 is in the same lane at ks + D/64.
    half8 query[NT][D / 32];
    half8 query_lo[NT][D / 32];
    // With room in the register budget (two waves per SIMD: 256 registers), a step computes the next step's scores
    // while its softmax runs (two score sets trading roles); two tiles of head_dim 128 leave no room for the
    // second set, and a step then scores its own block before its softmax.
    constexpr bool kLookahead = NT * D <= 128;
#pragma unroll
    for (int c = 0; c < NT; ++c) {
        const int j = 16 * c + r;
        const bool valid = j < item.count;
        const int token = column_token(valid ? j : 0);
        const float* q = a.qkv + static_cast<size_t>(token) * a.qkv_stride + static_cast<size_t>(head) * D;
        float values[D / 32][8];
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            const floatx4 lo = *reinterpret_cast<const floatx4*>(q + 32 * ks + 8 * g);
            const floatx4 hi = *reinterpret_cast<const floatx4*>(q + 32 * ks + 8 * g + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                values[ks][e] = lo[e];
                values[ks][e + 4] = hi[e];
            }
        }
        if (a.rotate) {
            const int position = listed ? a.tokens[token].position : first_position + (valid ? j : 0);
            const float* cosines = a.cosines + static_cast<size_t>(position) * (D / 2);
            const float* sines = a.sines + static_cast<size_t>(position) * (D / 2);
#pragma unroll
            for (int ks = 0; ks < D / 64; ++ks) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int i = 32 * ks + 8 * g + e;
                    rotate_pair(values[ks][e], values[ks + D / 64][e], cosines[i], sines[i], values[ks][e],
                                values[ks + D / 64][e]);
                }
            }
        }
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                // The softmax scale (log2 e / sqrt(d)) is folded into Q, which is then split exactly into FP16
                // parts hi + lo: K hi + K lo is the product with the FP32 query to about FP32 accuracy.
                const float value = valid ? values[ks][e] * a.scale_log2 : 0.0f;
                const _Float16 high = static_cast<_Float16>(value);
                query[c][ks][e] = high;
                query_lo[c][ks][e] = static_cast<_Float16>(value - static_cast<float>(high));
            }
        }
    }

    // Running state per column tile: O^T accumulators, the column's log2-domain offset (-inf until the column has
    // seen a key) and the lane's partial sum of probabilities (its 16 keys of each step; lanes g = 0..3 of a
    // column are added at the end).
    floatx4 out[NT][D / 16];
    float base[NT];
    float total[NT];
#pragma unroll
    for (int c = 0; c < NT; ++c) {
#pragma unroll
        for (int mt = 0; mt < D / 16; ++mt) {
            out[c][mt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        base[c] = kNegativeInfinity;
        total[c] = 0.0f;
    }

    const int32_t* table = geo.block_table + static_cast<size_t>(first.slot) * geo.pages_per_slot;
    // Keys past the block's last token are masked for every column; steps ending at or before the block's first
    // token (and inside the split) are visible to every column. A listed item's keys are visible to every column.
    const int key_stop = listed ? item.key_end : min(item.key_end, first_position + item.count);
    const int unmasked_stop = listed ? item.key_end : min(item.key_end, first_position + 1);
    const int steps = key_stop > item.key_begin ? (key_stop - item.key_begin + kStepKeys - 1) / kStepKeys : 0;
    const int clean = unmasked_stop > item.key_begin ? min(steps, (unmasked_stop - item.key_begin) / kStepKeys) : 0;

    using Ring = KvRing<D, WAVES>;
    constexpr int kKeyChunks = Ring::kKeyChunks;
    constexpr int kRing = Ring::kDepth;
    __shared__ half8 stage[kRing][Ring::kBlockChunks];
    Ring ring(stage, geo, table, item.kv_head, item.key_begin, wave);

    // S^T - offset for one staged block: the accumulators start at -offset of their column, so the scores come out
    // of the MFMA already relative to the column's offset.
    auto score_block = [&](const half8* keys, floatx4 (&scores)[NT][4]) __attribute__((always_inline)) {
        float start[NT];
#pragma unroll
        for (int c = 0; c < NT; ++c) {
            start[c] = base[c] == kNegativeInfinity ? 0.0f : -base[c];
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            half8 fragment[D / 32];
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) {
                fragment[ks] = keys[(t * (D / 32) + ks) * 64 + lane];
            }
#pragma unroll
            for (int c = 0; c < NT; ++c) {
                scores[c][t] = floatx4{start[c], start[c], start[c], start[c]};
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks) {
                    scores[c][t] =
                        __builtin_amdgcn_mfma_f32_16x16x32_f16(fragment[ks], query_lo[c][ks], scores[c][t], 0, 0, 0);
                }
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks) {
                    scores[c][t] =
                        __builtin_amdgcn_mfma_f32_16x16x32_f16(fragment[ks], query[c][ks], scores[c][t], 0, 0, 0);
                }
            }
        }
    };

    // Softmax half of a step: scores of block `step` are in `current`; it leaves block step+1's in `upcoming` and
    // the step's probabilities as exact FP16 pairs: p = probability + probability_lo to about FP32 accuracy.
    half8 probability[NT][2];
    half8 probability_lo[NT][2];
    auto softmax_phase = [&](int step, auto masked_tag, floatx4(&current)[NT][4], floatx4(&upcoming)[NT][4]) __attribute__((always_inline)) {
        constexpr bool kMasked = decltype(masked_tag)::value;
        const int key0 = item.key_begin + step * kStepKeys;
        // The VALU-heavy half issues ahead of the SIMD's other wave, whose PV MFMAs fill the matrix pipe meanwhile.
        __builtin_amdgcn_s_setprio(1);
        if constexpr (kLookahead) {
            // The last step scores a stale buffer too (unused) so that the step has no data-dependent branches.
            score_block(stage[(step + 1) % kRing], upcoming);
        } else {
            score_block(stage[step % kRing], current);
        }
        float tile_max[NT];
        bool rescale = false;
#pragma unroll
        for (int c = 0; c < NT; ++c) {
            if (kMasked) {
                const int column_position = first_position + 16 * c + r;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int key = key0 + 32 * (t >> 1) + 8 * g + 4 * (t & 1) + i;
                        current[c][t][i] =
                            key >= item.key_end || key > column_position ? kNegativeInfinity : current[c][t][i];
                    }
                }
            }
            float m = kNegativeInfinity;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                m = fmaxf(m, fmaxf(fmaxf(current[c][t][0], current[c][t][1]), fmaxf(current[c][t][2], current[c][t][3])));
            }
            tile_max[c] = m;  // this lane's 16 keys; the column's maximum is taken only when the offset moves
            // Probabilities relative to a stale offset stay below 2^kLazyRescale; the offset moves only past that
            // (or when the column sees its first key). A lane's part exceeds the bound exactly when the column's
            // maximum does, so the wave-wide vote needs no cross-lane maximum.
            rescale |= m > kLazyRescale || (base[c] == kNegativeInfinity && m != kNegativeInfinity);
        }
        if (__builtin_amdgcn_ballot_w64(rescale) != 0) {
#pragma unroll
            for (int c = 0; c < NT; ++c) {
                tile_max[c] = max_lanes32(max_lanes16(tile_max[c]));
            }
#pragma unroll
            for (int c = 0; c < NT; ++c) {
                const float old_offset = base[c] == kNegativeInfinity ? 0.0f : base[c];
                const float next = fmaxf(base[c], old_offset + tile_max[c]);
                const float delta = (next == kNegativeInfinity ? 0.0f : next) - old_offset;
                const float alpha = base[c] == kNegativeInfinity ? 0.0f : fast_exp2(base[c] - next);
                base[c] = next;
                total[c] *= alpha;
#pragma unroll
                for (int mt = 0; mt < D / 16; ++mt) {
                    out[c][mt] *= alpha;
                }
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    current[c][t] -= delta;
                    if constexpr (kLookahead) {
                        upcoming[c][t] -= delta;
                    }
                }
            }
        }
#pragma unroll
        for (int c = 0; c < NT; ++c) {
            // p < 2^kLazyRescale, so the high part is finite. The FP32 probabilities' sum is the row total: numerator
            // and denominator carry the same weights (hi + lo = p to about 2^-22 relative).
            float sums[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                float p[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    p[i] = fast_exp2(current[c][t][i]);
                    const _Float16 high = static_cast<_Float16>(p[i]);
                    probability[c][t >> 1][4 * (t & 1) + i] = high;
                    probability_lo[c][t >> 1][4 * (t & 1) + i] = static_cast<_Float16>(p[i] - static_cast<float>(high));
                }
                sums[t] = (p[0] + p[1]) + (p[2] + p[3]);
            }
            total[c] += (sums[0] + sums[1]) + (sums[2] + sums[3]);
        }
        __builtin_amdgcn_s_setprio(0);
    };
    // PV half of a step: O^T += V^T P^T for block `step` with the probabilities the step's softmax left.
    auto pv_phase = [&](int step) __attribute__((always_inline)) {
        const half8* values = stage[step % kRing] + kKeyChunks;
#pragma unroll
        for (int mt = 0; mt < D / 16; ++mt) {
            half8 value_fragment[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                value_fragment[h] = values[(h * (D / 16) + mt) * 64 + lane];
            }
#pragma unroll
            for (int c = 0; c < NT; ++c) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    out[c][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(value_fragment[h], probability_lo[c][h],
                                                                        out[c][mt], 0, 0, 0);
                }
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    out[c][mt] =
                        __builtin_amdgcn_mfma_f32_16x16x32_f16(value_fragment[h], probability[c][h], out[c][mt], 0, 0, 0);
                }
            }
        }
    };
    // Two barriers per step. Waves 0-3 (one per SIMD) run softmax then PV of each step; the waves sharing a SIMD
    // with them (4-7) run half a step behind: PV of the previous step, then the softmax. Each SIMD then has one
    // wave in the MFMA-only PV half while the other is in the VALU-heavy softmax half. In the first half of step i
    // the group reads K(i+1) and V(i-1), in the second K(i+1) and V(i); block i+3 is copied in the second half,
    // into the buffer V(i-1) held.
    auto run_step = [&](int step, auto late_tag, auto masked_tag, floatx4(&current)[NT][4],
                        floatx4(&upcoming)[NT][4]) __attribute__((always_inline)) {
        constexpr bool kLate = decltype(late_tag)::value;
        const bool copying = step + 3 < steps;
        if (kLate) {
            if (step > 0) {
                pv_phase(step - 1);
            }
        } else {
            softmax_phase(step, masked_tag, current, upcoming);
        }
        if (WAVES > 4) {
            barrier_after_copies<63>();
        }
        if (copying) {
            ring.issue((step + 3) % kRing);
        }
        if (kLate) {
            softmax_phase(step, masked_tag, current, upcoming);
        } else {
            pv_phase(step);
        }
        ring.ready(copying);
    };
    auto advance = [&](floatx4(&current)[NT][4], const floatx4(&upcoming)[NT][4]) __attribute__((always_inline)) {
        if constexpr (!kLookahead) {
            return;
        }
#pragma unroll
        for (int c = 0; c < NT; ++c) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                current[c][t] = upcoming[c][t];
            }
        }
    };

    floatx4 scores_a[NT][4];
    floatx4 scores_b[NT][4];
    for (int block = 0; block < min(steps, kRing - 1); ++block) {
        ring.issue(block);
    }
    ring.ready(false);
    if (kLookahead && steps > 0) {
        score_block(stage[0], scores_a);
    }
    auto run_steps = [&](auto late_tag) __attribute__((always_inline)) {
        // Unmasked steps in pairs, the two score sets trading roles; masked steps (at most three) copy instead.
        int step = 0;
        for (; step + 1 < clean; step += 2) {
            run_step(step, late_tag, std::false_type{}, scores_a, scores_b);
            run_step(step + 1, late_tag, std::false_type{}, scores_b, scores_a);
        }
        if (step < clean) {
            run_step(step, late_tag, std::false_type{}, scores_a, scores_b);
            advance(scores_a, scores_b);
            ++step;
        }
        for (; step < steps; ++step) {
            run_step(step, late_tag, std::true_type{}, scores_a, scores_b);
            advance(scores_a, scores_b);
        }
        if (decltype(late_tag)::value && steps > 0) {
            pv_phase(steps - 1);
        }
    };
    if (WAVES > 4 && wave >= 4) {
        run_steps(std::true_type{});
    } else {
        run_steps(std::false_type{});
    }

    const int group = geo.group;
#pragma unroll
    for (int c = 0; c < NT; ++c) {
        const float sum = sum_lanes32(sum_lanes16(total[c]));
        const int j = 16 * c + r;
        if (j >= item.count) {
            continue;
        }
        const int token = column_token(j);
        if (item.row < 0) {
            float* destination = a.output + static_cast<size_t>(token) * a.out_stride + static_cast<size_t>(head) * D;
            const float inverse = 1.0f / sum;
#pragma unroll
            for (int mt = 0; mt < D / 16; ++mt) {
                *reinterpret_cast<floatx4*>(destination + 16 * mt + 4 * g) = out[c][mt] * inverse;
            }
        } else {
            const size_t row = static_cast<size_t>(item.row + j * item.row_stride) * group + wave;
            float* destination = a.partial_out + row * D;
#pragma unroll
            for (int mt = 0; mt < D / 16; ++mt) {
                *reinterpret_cast<floatx4*>(destination + 16 * mt + 4 * g) = out[c][mt];
            }
            if (g == 0) {
                a.partial_ml[row * 2] = base[c];
                a.partial_ml[row * 2 + 1] = sum;
            }
        }
    }
}

template <int WAVES, int NT>
hipError_t launch_prefill_for(const Launch& launch, const AttentionArgs& args, int first, dim3 grid, dim3 block) {
    if (args.geo.head_dim == 128) {
        SYNAPSE_KV_LAUNCH((prefill_f16_kernel<128, WAVES, NT>), grid, block, launch, args, first);
    } else {
        SYNAPSE_KV_LAUNCH((prefill_f16_kernel<64, WAVES, NT>), grid, block, launch, args, first);
    }
    return hipGetLastError();
}

template <int NT>
hipError_t launch_prefill_tiles(const Launch& launch, const AttentionArgs& args, int first, int items) {
    const dim3 grid(items);
    const dim3 block(args.geo.group * 64);
    // One wave per query head of the group (validated at cache creation: 1..8).
    switch (args.geo.group) {
        case 1: return launch_prefill_for<1, NT>(launch, args, first, grid, block);
        case 2: return launch_prefill_for<2, NT>(launch, args, first, grid, block);
        case 3: return launch_prefill_for<3, NT>(launch, args, first, grid, block);
        case 4: return launch_prefill_for<4, NT>(launch, args, first, grid, block);
        case 5: return launch_prefill_for<5, NT>(launch, args, first, grid, block);
        case 6: return launch_prefill_for<6, NT>(launch, args, first, grid, block);
        case 7: return launch_prefill_for<7, NT>(launch, args, first, grid, block);
        case 8: return launch_prefill_for<8, NT>(launch, args, first, grid, block);
        default: return hipErrorInvalidValue;
    }
}

template <int D>
int prefill_blocks_per_cu(int group) {
    int blocks = 0;
    hipError_t status = hipErrorInvalidValue;
    switch (group) {
        case 1: status = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, prefill_f16_kernel<D, 1, kPrefillTiles>, 64, 0); break;
        case 2: status = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, prefill_f16_kernel<D, 2, kPrefillTiles>, 128, 0); break;
        case 3: status = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, prefill_f16_kernel<D, 3, kPrefillTiles>, 192, 0); break;
        case 4: status = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, prefill_f16_kernel<D, 4, kPrefillTiles>, 256, 0); break;
        case 5: status = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, prefill_f16_kernel<D, 5, kPrefillTiles>, 320, 0); break;
        case 6: status = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, prefill_f16_kernel<D, 6, kPrefillTiles>, 384, 0); break;
        case 7: status = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, prefill_f16_kernel<D, 7, kPrefillTiles>, 448, 0); break;
        case 8: status = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, prefill_f16_kernel<D, 8, kPrefillTiles>, 512, 0); break;
        default: break;
    }
    if (status != hipSuccess) {
        (void)hipGetLastError();
        return 1;
    }
    return blocks > 0 ? blocks : 1;
}

}  // namespace

int prefill_resident_blocks(int device, int head_dim, int group) {
    hipDeviceProp_t properties{};
    if (hipGetDeviceProperties(&properties, device) != hipSuccess) {
        (void)hipGetLastError();
        return 256;
    }
    const int per_cu = head_dim == 128 ? prefill_blocks_per_cu<128>(group) : prefill_blocks_per_cu<64>(group);
    return properties.multiProcessorCount * per_cu;
}

hipError_t launch_prefill(const Launch& launch, const AttentionArgs& args, int first, int items, int tiles, bool fp16) {
    if (items == 0) {
        return hipSuccess;
    }
    if (!fp16) {
        return hipErrorNotSupported;  // the planner sends FP32 prompt runs through the decode kernel
    }
    return tiles == 1 ? launch_prefill_tiles<1>(launch, args, first, items)
                      : launch_prefill_tiles<kPrefillTiles>(launch, args, first, items);
}

}  // namespace synapse_kv
