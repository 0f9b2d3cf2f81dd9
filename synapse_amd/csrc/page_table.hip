// Block-table management on the device: growth, contraction, copy-on-write and fork run as kernels over the
// HBM-resident block table, reference counts and free stack, so no table ever round-trips through the host.
//
// Order rules (bit-exact with the CPU restatement):
//   growth pops one page per new logical page, logical pages ascending, from the top of the free stack;
//   contraction walks logical pages descending, drops one reference each and pushes pages that reach zero;
//   copy-on-write pops a fresh page for a shared page and drops one reference from the shared page;
//   fork shares the first `pages` pages of the source with one more reference each.
// The host decides which operations a call needs (capacity policy of Qwen2KvCache.Reserve/NextCapacity,
// Qwen2KvCache.cs:56-95, and MetalDecoder::reserve/prepare_slots, metal/decoder.rs:164-223); the page ids come
// from the device stack. The kernel runs as one workgroup: table work is a few thousand integers at most.

#include "kv_internal.h"

namespace synapse_kv {
namespace {

constexpr int kTableThreads = 256;

// Exclusive prefix sum of one flag per thread across the workgroup; returns the total through `total`.
__device__ int block_exclusive_scan(int flag, int* scratch, int& total) {
    const int tid = threadIdx.x;
    scratch[tid] = flag;
    __syncthreads();
    for (int offset = 1; offset < kTableThreads; offset <<= 1) {
        const int add = tid >= offset ? scratch[tid - offset] : 0;
        __syncthreads();
        scratch[tid] += add;
        __syncthreads();
    }
    const int inclusive = scratch[tid];
    total = scratch[kTableThreads - 1];
    __syncthreads();
    return inclusive - flag;
}

__global__ __launch_bounds__(kTableThreads) void table_kernel(TableArgs a) {
    __shared__ int scan[kTableThreads];
    const int tid = threadIdx.x;
    int free_count = a.state[0];
    for (int index = 0; index < a.op_count; ++index) {
        const TableOp op = a.ops[index];
        if (op.kind == kOpResize) {
            int32_t* row = a.block_table + static_cast<size_t>(op.a) * a.pages_per_slot;
            const int from = op.b;
            const int to = op.c;
            if (to > from) {
                const int count = to - from;
                if (count > free_count && tid == 0) {
                    a.state[1] = 1;  // the host shadow promised pages the device does not have
                }
                for (int j = tid; j < count && j < free_count; j += kTableThreads) {
                    const int page = a.free_stack[free_count - 1 - j];
                    row[from + j] = page;
                    a.refcount[page] = 1;
                    a.fresh[op.d + j] = page;
                }
                free_count -= min(count, free_count);
            } else {
                const int count = from - to;
                for (int base = 0; base < count; base += kTableThreads) {
                    const int j = base + tid;
                    int page = -1;
                    int released = 0;
                    if (j < count) {
                        const int logical = from - 1 - j;
                        page = row[logical];
                        released = (--a.refcount[page] == 0) ? 1 : 0;
                        row[logical] = -1;
                    }
                    int total = 0;
                    const int at = block_exclusive_scan(released, scan, total);
                    if (released) {
                        a.free_stack[free_count + at] = page;
                    }
                    free_count += total;
                }
            }
        } else if (op.kind == kOpCow) {
            if (tid == 0) {
                int32_t* row = a.block_table + static_cast<size_t>(op.a) * a.pages_per_slot;
                const int shared = row[op.b];
                if (a.refcount[shared] <= 1 || free_count == 0) {
                    a.state[1] = 2;  // nothing to copy, or no page: the host shadow disagrees
                } else {
                    const int page = a.free_stack[--free_count];
                    a.refcount[page] = 1;
                    --a.refcount[shared];
                    row[op.b] = page;
                    a.copies[op.c * 2] = shared;
                    a.copies[op.c * 2 + 1] = page;
                }
            }
            if (tid == 0) {
                scan[0] = free_count;
            }
            __syncthreads();
            free_count = scan[0];
        } else if (op.kind == kOpFork) {
            const int32_t* source = a.block_table + static_cast<size_t>(op.a) * a.pages_per_slot;
            int32_t* target = a.block_table + static_cast<size_t>(op.b) * a.pages_per_slot;
            for (int j = tid; j < op.c; j += kTableThreads) {
                const int page = source[j];
                target[j] = page;
                atomicAdd(&a.refcount[page], 1);
            }
        }
        __syncthreads();
    }
    if (tid == 0) {
        a.state[0] = free_count;
    }
}

// Zero-fills whole pages, 16 bytes per store; grid-stride over (page, chunk).
__global__ __launch_bounds__(256) void zero_pages_kernel(PageArgs a) {
    const uint64_t chunks = a.page_bytes / 16;
    const uint64_t total = chunks * static_cast<uint64_t>(a.count);
    const uint4 zero = make_uint4(0, 0, 0, 0);
    for (uint64_t index = blockIdx.x * 256ull + threadIdx.x; index < total; index += gridDim.x * 256ull) {
        const uint64_t page = a.list[index / chunks];
        reinterpret_cast<uint4*>(a.pool + page * a.page_bytes)[index % chunks] = zero;
    }
}

// Copies whole pages (copy-on-write), 16 bytes per load and store.
__global__ __launch_bounds__(256) void copy_pages_kernel(PageArgs a) {
    const uint64_t chunks = a.page_bytes / 16;
    const uint64_t total = chunks * static_cast<uint64_t>(a.count);
    for (uint64_t index = blockIdx.x * 256ull + threadIdx.x; index < total; index += gridDim.x * 256ull) {
        const uint64_t pair = index / chunks;
        const uint64_t source = a.list[pair * 2];
        const uint64_t target = a.list[pair * 2 + 1];
        const uint64_t chunk = index % chunks;
        reinterpret_cast<uint4*>(a.pool + target * a.page_bytes)[chunk] =
            reinterpret_cast<const uint4*>(a.pool + source * a.page_bytes)[chunk];
    }
}

unsigned page_grid(const PageArgs& a) {
    const uint64_t total = a.page_bytes / 16 * static_cast<uint64_t>(a.count);
    const uint64_t blocks = (total + 255) / 256;
    return static_cast<unsigned>(blocks < 8192 ? blocks : 8192);
}

}  // namespace

hipError_t launch_table(const Launch& launch, const TableArgs& args) {
    if (args.op_count == 0) {
        return hipSuccess;
    }
    SYNAPSE_KV_LAUNCH(table_kernel, dim3(1), dim3(kTableThreads), launch, args);
    return hipGetLastError();
}

hipError_t launch_zero_pages(const Launch& launch, const PageArgs& args) {
    if (args.count == 0) {
        return hipSuccess;
    }
    SYNAPSE_KV_LAUNCH(zero_pages_kernel, dim3(page_grid(args)), dim3(256), launch, args);
    return hipGetLastError();
}

hipError_t launch_copy_pages(const Launch& launch, const PageArgs& args) {
    if (args.count == 0) {
        return hipSuccess;
    }
    SYNAPSE_KV_LAUNCH(copy_pages_kernel, dim3(page_grid(args)), dim3(256), launch, args);
    return hipGetLastError();
}

}  // namespace synapse_kv
