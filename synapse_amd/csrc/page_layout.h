// Element layout of one (layer, K|V, KV head) region of a page: page_tokens keys of head_dim elements, stored as
// blocks of 64 keys, each block in MFMA-fragment order so that every operand load of the attention kernels is
// one contiguous 1 KiB wave load (lane l reads 16 bytes at chunk * 16 + l * 16):
//
// FP16 (8 halves per 16-byte chunk), MFMA v_mfma_f32_16x16x32_f16:
//   K chunk (t, ks, lane), t < 4, ks < D/32, lane = 16g + r:  dims 32ks + 8g .. +7 of key
//       32*(t/2) + 8*(r/4) + 4*(t%2) + r%4            (S^T = K Q^T, A operand of tile t, k-step ks)
//   V chunk (h, mt, lane), h < 2, mt < D/16:                 keys 32h + 8g .. +7 of dim 16mt + r
//                                                            (O^T = V^T P^T, A operand of k-step h, tile mt)
// FP32 (4 floats per chunk), MFMA v_mfma_f32_16x16x4_f32:
//   K chunk (t, c, lane), t < 4, c < D/16:  dims 16c + 4g .. +3 of key 16t + r
//   V chunk (t, mt, lane), t < 4, mt < D/16: keys 16t + 4g .. +3 of dim 16mt + r
// The key permutation of the FP16 K tiles makes the C layout of S^T equal the B layout of P^T (see
// attention_decode.hip), so scores never move between lanes.
#pragma once

#include <stdint.h>

namespace synapse_kv {

constexpr int kBlockKeys = 64;

#if defined(__HIPCC__)
#define SYNAPSE_KV_HD __host__ __device__
#else
#define SYNAPSE_KV_HD
#endif

// Element offset of (key, dim) inside a region, FP16.
SYNAPSE_KV_HD inline int64_t key_offset_f16(int head_dim, int key, int dim) {
    const int block = key / kBlockKeys;
    const int k = key % kBlockKeys;
    const int t = 2 * (k >> 5) + ((k >> 2) & 1);
    const int r = 4 * ((k >> 3) & 3) + (k & 3);
    const int ks = dim >> 5;
    const int g = (dim >> 3) & 3;
    const int chunk = (t * (head_dim / 32) + ks) * 64 + 16 * g + r;
    return static_cast<int64_t>(block) * kBlockKeys * head_dim + static_cast<int64_t>(chunk) * 8 + (dim & 7);
}

SYNAPSE_KV_HD inline int64_t value_offset_f16(int head_dim, int key, int dim) {
    const int block = key / kBlockKeys;
    const int k = key % kBlockKeys;
    const int h = k >> 5;
    const int g = (k >> 3) & 3;
    const int mt = dim >> 4;
    const int r = dim & 15;
    const int chunk = (h * (head_dim / 16) + mt) * 64 + 16 * g + r;
    return static_cast<int64_t>(block) * kBlockKeys * head_dim + static_cast<int64_t>(chunk) * 8 + (k & 7);
}

// Element offset of (key, dim) inside a region, FP32.
SYNAPSE_KV_HD inline int64_t key_offset_f32(int head_dim, int key, int dim) {
    const int block = key / kBlockKeys;
    const int k = key % kBlockKeys;
    const int t = k >> 4;
    const int r = k & 15;
    const int c = dim >> 4;
    const int g = (dim >> 2) & 3;
    const int chunk = (t * (head_dim / 16) + c) * 64 + 16 * g + r;
    return static_cast<int64_t>(block) * kBlockKeys * head_dim + static_cast<int64_t>(chunk) * 4 + (dim & 3);
}

SYNAPSE_KV_HD inline int64_t value_offset_f32(int head_dim, int key, int dim) {
    const int block = key / kBlockKeys;
    const int k = key % kBlockKeys;
    const int t = k >> 4;
    const int g = (k >> 2) & 3;
    const int mt = dim >> 4;
    const int r = dim & 15;
    const int chunk = (t * (head_dim / 16) + mt) * 64 + 16 * g + r;
    return static_cast<int64_t>(block) * kBlockKeys * head_dim + static_cast<int64_t>(chunk) * 4 + (k & 3);
}

template <typename T>
SYNAPSE_KV_HD inline int64_t key_offset(int head_dim, int key, int dim);
template <typename T>
SYNAPSE_KV_HD inline int64_t value_offset(int head_dim, int key, int dim);

template <>
SYNAPSE_KV_HD inline int64_t key_offset<float>(int head_dim, int key, int dim) {
    return key_offset_f32(head_dim, key, dim);
}
template <>
SYNAPSE_KV_HD inline int64_t value_offset<float>(int head_dim, int key, int dim) {
    return value_offset_f32(head_dim, key, dim);
}
#if defined(__HIPCC__)
template <>
SYNAPSE_KV_HD inline int64_t key_offset<_Float16>(int head_dim, int key, int dim) {
    return key_offset_f16(head_dim, key, dim);
}
template <>
SYNAPSE_KV_HD inline int64_t value_offset<_Float16>(int head_dim, int key, int dim) {
    return value_offset_f16(head_dim, key, dim);
}
#endif

}  // namespace synapse_kv
