// Device calibration kernels for the benchmark (not part of libsynapse_kv): a streaming read and a copy of a
// large buffer with 16-byte non-temporal accesses (the measured HBM ceilings the decode kernel is compared with),
// and an FP16 MFMA loop (the measured v_mfma_f32_16x16x32_f16 ceiling the prefill kernel is compared with).

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t uint4v __attribute__((ext_vector_type(4)));

constexpr int kUnroll = 8;

// Each wave streams contiguous 8 KiB chunks (chunk = wave, wave + waves, ...): eight 1 KiB wave loads in flight.
__global__ __launch_bounds__(256) void read_kernel(const uint4v* source, size_t count, uint32_t* sink) {
    const size_t waves = static_cast<size_t>(gridDim.x) * (blockDim.x / 64);
    const size_t wave = static_cast<size_t>(blockIdx.x) * (blockDim.x / 64) + threadIdx.x / 64;
    const int lane = threadIdx.x & 63;
    const size_t chunks = count / (64 * kUnroll);
    uint4v acc = {0u, 0u, 0u, 0u};
    for (size_t chunk = wave; chunk < chunks; chunk += waves) {
        const uint4v* base = source + chunk * (64 * kUnroll) + lane;
        uint4v values[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            values[u] = __builtin_nontemporal_load(base + u * 64);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            acc ^= values[u];
        }
    }
    const uint32_t folded = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    if (folded == 0x9E3779B9u) {  // keeps the loads; practically never taken
        sink[0] = folded;
    }
}

// The decode kernel's access pattern without its arithmetic: every wave streams its own contiguous run of 32 KiB
// steps (32 wave loads of 1 KiB), two register sets in turn, the next step's loads in flight while the current
// step's values are folded (64 loads in flight at most: the 6-bit vector memory counter holds 63, so a third set
// cannot be tracked and measured slower). One wave per SIMD (four per 256-thread workgroup, one workgroup per CU).
__global__ __launch_bounds__(256) void pattern_kernel(const uint4v* source, size_t steps_per_wave, uint32_t* sink) {
    const int lane = threadIdx.x & 63;
    const size_t wave = static_cast<size_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const uint4v* base = source + wave * steps_per_wave * 2048 + lane;  // 2,048 x 16 B = 32 KiB per step
    uint4v sets[2][32];
    uint4v acc = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        sets[0][i] = __builtin_nontemporal_load(base + i * 64);
    }
    for (size_t step = 0; step < steps_per_wave; step += 2) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const size_t next = step + k + 1 < steps_per_wave ? step + k + 1 : steps_per_wave - 1;
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                sets[(k + 1) % 2][i] = __builtin_nontemporal_load(base + next * 2048 + i * 64);
            }
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                acc ^= sets[k][i];
            }
        }
    }
    const uint32_t folded = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    if (folded == 0x9E3779B9u) {  // keeps the loads; practically never taken
        sink[0] = folded;
    }
}

__global__ __launch_bounds__(256) void copy_kernel(const uint4v* source, uint4v* target, size_t count) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    size_t index = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    for (; index + (kUnroll - 1) * stride < count; index += kUnroll * stride) {
        uint4v values[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            values[u] = __builtin_nontemporal_load(source + index + u * stride);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            __builtin_nontemporal_store(values[u], target + index + u * stride);
        }
    }
    for (; index < count; index += stride) {
        __builtin_nontemporal_store(__builtin_nontemporal_load(source + index), target + index);
    }
}

// Each wave runs `iterations` rounds of 8 independent MFMA chains: v_mfma_f32_16x16x32_f16 (WIDE false) or
// v_mfma_f32_32x32x16_f16 (WIDE true).
template <bool WIDE>
__global__ __launch_bounds__(256) void mfma_kernel(float* sink, int iterations) {
    const int lane = threadIdx.x & 63;
    half8 a;
    half8 b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = static_cast<_Float16>(0.001f * (lane + i));
        b[i] = static_cast<_Float16>(0.002f * (lane - i));
    }
    float total = 0.0f;
    if constexpr (WIDE) {
        typedef float floatx16 __attribute__((ext_vector_type(16)));
        floatx16 acc[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            acc[c] = floatx16{};
        }
        for (int it = 0; it < iterations; ++it) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[c], 0, 0, 0);
            }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                total += acc[c][e];
            }
        }
    } else {
        floatx4 acc[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            acc[c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        for (int it = 0; it < iterations; ++it) {
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[c], 0, 0, 0);
            }
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            total += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
        }
    }
    sink[blockIdx.x * blockDim.x + threadIdx.x] = total;
}

}  // namespace

extern "C" {

int calibrate_read(const void* source, size_t bytes, uint32_t* sink, int blocks, void* stream) {
    hipLaunchKernelGGL(read_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4v*>(source), bytes / 16, sink);
    return static_cast<int>(hipGetLastError());
}

// Streams `steps_per_wave` 32 KiB steps per wave over 4 * blocks waves (the bytes read: 32 KiB x both).
int calibrate_pattern(const void* source, size_t steps_per_wave, uint32_t* sink, int blocks, void* stream) {
    hipLaunchKernelGGL(pattern_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4v*>(source), steps_per_wave, sink);
    return static_cast<int>(hipGetLastError());
}

int calibrate_copy(const void* source, void* target, size_t bytes, int blocks, void* stream) {
    hipLaunchKernelGGL(copy_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4v*>(source), static_cast<uint4v*>(target), bytes / 16);
    return static_cast<int>(hipGetLastError());
}

// FLOPs of one launch: blocks * 4 waves * iterations * (8 x 16x16x32 or 4 x 32x32x16 MFMAs) * 16,384 or 32,768 * 2.
int calibrate_mfma(float* sink, int blocks, int iterations, int wide, void* stream) {
    if (wide != 0) {
        hipLaunchKernelGGL(mfma_kernel<true>, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), sink,
                           iterations);
    } else {
        hipLaunchKernelGGL(mfma_kernel<false>, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), sink,
                           iterations);
    }
    return static_cast<int>(hipGetLastError());
}

}  // extern "C"
