// Host half of libsynapse_kv: the C ABI, argument validation, the capacity policy, a host shadow of the page
// allocator (used to reject a call before any device work and to size launches without reading the device back),
// the per-step attention plan, and the kernel launches.
//
// ABI conventions follow native/synapse-gpu/src/Features/GpuKernels/ffi.rs: status codes (error.rs:4-16), a
// thread-local last error copied out by length (ffi.rs:19, 86-104), every entry point guarded (ffi.rs:34-45,
// C++ exceptions here instead of Rust panics), opaque handles, null-safe destroy and kv_bytes.

#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "abi_support.h"
#include "kv_internal.h"

// Device memory of synapse_kv_step_static: the step's table operations, attention plan and attention partial rows,
// for callers that cannot allocate. One array per GPU the library runs on, held until the process ends. In host
// code `scratch` names a host-side stand-in, not a device address: host code uses only the address that
// hipGetSymbolAddress returned on each device (scratch_address below).
static __device__ __align__(256) uint8_t scratch[SYNAPSE_KV_STATIC_SCRATCH_BYTES];

namespace synapse_kv {
namespace {

// Copies `bytes` from coherent pinned host memory (mapped into the device's address space) to device memory: 16-byte
// vector loads and stores, grid-stride, then the last bytes % 16 one by one. Uploads go through this kernel rather
// than hipMemcpyAsync, whose host call was measured stalling 5-7 ms once per process (at a varying step, the device
// running dry meanwhile).
__global__ __launch_bounds__(256) void upload_kernel(const uint8_t* source, uint8_t* target, size_t bytes) {
    const size_t vectors = bytes / 16;
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < vectors; i += stride) {
        reinterpret_cast<uint4*>(target)[i] = reinterpret_cast<const uint4*>(source)[i];
    }
    if (blockIdx.x == 0 && threadIdx.x < bytes % 16) {
        target[vectors * 16 + threadIdx.x] = source[vectors * 16 + threadIdx.x];
    }
}

}  // namespace

hipError_t launch_upload(const void* source, void* target, size_t bytes, hipStream_t stream) {
    if (bytes == 0) {
        return hipSuccess;
    }
    if (((reinterpret_cast<uintptr_t>(source) | reinterpret_cast<uintptr_t>(target)) & 15) != 0) {
        return hipErrorInvalidValue;  // the kernel moves 16-byte vectors
    }
    const size_t vectors = (bytes + 15) / 16;
    const unsigned blocks = static_cast<unsigned>(std::min<size_t>((vectors + 255) / 256, 1024));
    hipLaunchKernelGGL(upload_kernel, dim3(blocks), dim3(256), 0, stream, static_cast<const uint8_t*>(source),
                       static_cast<uint8_t*>(target), bytes);
    return hipGetLastError();
}

namespace {

// Qwen2KvCache.NextCapacity (Qwen2KvCache.cs:91-95) = DecoderShape::next_capacity (decoder.rs:221-226).
uint32_t next_capacity(uint32_t needed, uint32_t current, uint32_t growth, uint32_t maximum) {
    const uint64_t rounded = std::min<uint64_t>(maximum, (static_cast<uint64_t>(needed) + growth - 1) / growth * growth);
    return static_cast<uint32_t>(
        std::min<uint64_t>(maximum, std::max<uint64_t>(rounded, std::min<uint64_t>(maximum, 2ull * current))));
}

// Reservation rounding (Qwen2KvCache.cs:63; DecoderShape::reserve_capacity, decoder.rs:207-216).
uint32_t reserve_rounded(uint32_t positions, uint32_t growth, uint32_t maximum) {
    return static_cast<uint32_t>(
        std::min<uint64_t>(maximum, (static_cast<uint64_t>(positions) + growth - 1) / growth * growth));
}

template <typename T>
struct DeviceBuffer {
    T* pointer = nullptr;
    size_t count = 0;

    void reset() {
        if (pointer != nullptr) {
            (void)hipFree(pointer);
        }
        pointer = nullptr;
        count = 0;
    }

    // Grows to at least `wanted` elements (contents are not kept), and by at least half its size, so that a plan
    // that grows a little every few steps reallocates only a few times. Work already queued may still read the
    // old buffer, so the device is drained before it is freed.
    void ensure(size_t wanted, const char* what) {
        if (wanted <= count) {
            return;
        }
        if (pointer != nullptr) {
            check_hip(hipDeviceSynchronize(), "drain before reallocation");
        }
        const size_t grown = std::max(wanted, count + count / 2);
        reset();
        check_hip(hipMalloc(reinterpret_cast<void**>(&pointer), std::max<size_t>(grown, 1) * sizeof(T)), what);
        count = grown;
    }
};

// Two pinned host staging buffers used alternately for host-to-device uploads; an event per buffer tells when
// its last copy finished, so a buffer is never rewritten while the device may still read it.
struct Uploader {
    void* host[2] = {nullptr, nullptr};
    void* device_view[2] = {nullptr, nullptr};  // the same memory as the device addresses it
    size_t size[2] = {0, 0};
    hipEvent_t done[2] = {nullptr, nullptr};
    int next = 0;

    void release() {
        for (int index = 0; index < 2; ++index) {
            if (done[index] != nullptr) {
                (void)hipEventSynchronize(done[index]);
                (void)hipEventDestroy(done[index]);
                done[index] = nullptr;
            }
            if (host[index] != nullptr) {
                (void)hipHostFree(host[index]);
                host[index] = nullptr;
                device_view[index] = nullptr;
            }
            size[index] = 0;
        }
    }

    // Returns a pinned buffer of at least `bytes` that is safe to write now.
    void* acquire(size_t bytes) {
        const int index = next;
        if (done[index] == nullptr) {
            check_hip(hipEventCreateWithFlags(&done[index], hipEventDisableTiming), "upload event");
        } else {
            check_hip(hipEventSynchronize(done[index]), "upload wait");
        }
        if (size[index] < bytes) {
            if (host[index] != nullptr) {
                check_hip(hipHostFree(host[index]), "free staging");
                host[index] = nullptr;
            }
            const size_t rounded = std::max<size_t>({bytes, size[index] + size[index] / 2, 64 * 1024});
            // Coherent: the upload kernel's reads see the host's writes made before its launch.
            check_hip(hipHostMalloc(&host[index], rounded, hipHostMallocMapped | hipHostMallocCoherent),
                      "staging buffer");
            check_hip(hipHostGetDevicePointer(&device_view[index], host[index], 0), "staging device address");
            size[index] = rounded;
        }
        return host[index];
    }

    // The copy kernel beats hipMemcpyAsync up to about 1 MiB (5.9 against 13.5 us at 64 KiB, 28.6 against 31.4 us
    // at 1 MiB); from 4 MiB on the DMA copy is 5-15 % faster, so large one-off uploads (a page-activation summary
    // rebuild over many pages) take it.
    static constexpr size_t kDmaBytes = 2u << 20;

    void copy(void* device, size_t bytes, hipStream_t stream) {
        const int index = next;
        if (bytes >= kDmaBytes) {
            check_hip(hipMemcpyAsync(device, host[index], bytes, hipMemcpyHostToDevice, stream), "upload");
        } else {
            check_hip(launch_upload(device_view[index], device, bytes, stream), "upload");
        }
        check_hip(hipEventRecord(done[index], stream), "upload record");
        next ^= 1;
    }
};

// The static-scratch step's uploads: two pageable host buffers used alternately (no pinned allocation), each
// rewritten only after the event recorded behind its previous copy has completed.
struct PageableUploader {
    std::vector<uint8_t> host[2];
    hipEvent_t done[2] = {nullptr, nullptr};
    int next = 0;

    void release() {
        for (int index = 0; index < 2; ++index) {
            if (done[index] != nullptr) {
                (void)hipEventSynchronize(done[index]);
                (void)hipEventDestroy(done[index]);
                done[index] = nullptr;
            }
        }
    }

    uint8_t* acquire(size_t bytes) {
        const int index = next;
        if (done[index] == nullptr) {
            check_hip(hipEventCreateWithFlags(&done[index], hipEventDisableTiming), "upload event");
        } else {
            check_hip(hipEventSynchronize(done[index]), "upload wait");
        }
        host[index].resize(std::max<size_t>(bytes, 1));
        return host[index].data();
    }

    void copy(void* device, size_t bytes, hipStream_t stream) {
        const int index = next;
        check_hip(hipMemcpyAsync(device, host[index].data(), bytes, hipMemcpyHostToDevice, stream), "upload");
        check_hip(hipEventRecord(done[index], stream), "upload record");
        next ^= 1;
    }
};

// System.Random(int seed) as .NET seeds it (the runtime's compatible seeded generator, Random.Net5CompatImpl.cs:
// Knuth's subtractive generator, Seminumerical Algorithms 3.6, in the Numerical Recipes "ran3" form with the
// second index starting at 21), which KvPageSelector.RandomPages (KvPageSelector.cs:118-129) draws from. Only the
// calls that path makes: the constructor and Next(minValue, maxValue) for ranges below 2^31.
class SeededRandom {
public:
    explicit SeededRandom(int32_t seed) {
        constexpr int32_t kSeed = 161803398;
        const int32_t subtraction = seed == INT32_MIN ? INT32_MAX : (seed < 0 ? -seed : seed);
        int32_t mj = kSeed - subtraction;
        state_[55] = mj;
        int32_t mk = 1;
        int ii = 0;
        for (int i = 1; i < 55; ++i) {
            ii += 21;
            if (ii >= 55) {
                ii -= 55;
            }
            state_[ii] = mk;
            mk = mj - mk;
            if (mk < 0) {
                mk += INT32_MAX;
            }
            mj = state_[ii];
        }
        for (int round = 1; round < 5; ++round) {
            for (int i = 1; i < 56; ++i) {
                int n = i + 30;
                if (n >= 55) {
                    n -= 55;
                }
                state_[i] -= state_[1 + n];
                if (state_[i] < 0) {
                    state_[i] += INT32_MAX;
                }
            }
        }
    }

    // Next(minValue, maxValue): minValue + (int)(Sample() * (maxValue - minValue)).
    int32_t next(int32_t minimum, int32_t maximum) {
        const double sample = static_cast<double>(internal_sample()) * (1.0 / INT32_MAX);
        return static_cast<int32_t>(sample * (static_cast<int64_t>(maximum) - minimum)) + minimum;
    }

private:
    int32_t internal_sample() {
        if (++next_ >= 56) {
            next_ = 1;
        }
        if (++next_p_ >= 56) {
            next_p_ = 1;
        }
        int32_t value = state_[next_] - state_[next_p_];
        if (value == INT32_MAX) {
            --value;
        }
        if (value < 0) {
            value += INT32_MAX;
        }
        state_[next_] = value;
        return value;
    }

    int32_t state_[56] = {};
    int next_ = 0;
    int next_p_ = 21;
};

struct Dims {
    uint32_t layers;
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t max_positions;
    uint32_t growth;
    uint32_t page_tokens;
    uint32_t precision;
    uint32_t slots;
    uint32_t step_tokens;
    uint32_t max_pages;
    uint32_t pages_per_slot;
    uint64_t page_bytes;
};

}  // namespace
}  // namespace synapse_kv

namespace synapse_kv {
// Worker durations of a step's first kLaunches decode launches (SYNAPSE_KV_OPTION_ADAPTIVE_SPLIT): coherent pinned
// memory the decode kernel writes through its device view (kWorkers entries per launch), the planned cost of each
// worker, and an event after the last timed launch.
struct SplitTiming {
    static constexpr int kWorkers = 16384;
    static constexpr int kLaunches = 4;
    int launches = 0;            // timed launches of the step so far
    uint32_t* host = nullptr;
    uint32_t* device = nullptr;
    hipEvent_t done = nullptr;
    bool pending = false;        // launched, not yet read
    std::vector<int64_t> costs;  // per worker of the timed plan

    void allocate() {
        if (host == nullptr) {
            check_hip(hipHostMalloc(reinterpret_cast<void**>(&host), kLaunches * kWorkers * sizeof(uint32_t),
                                    hipHostMallocMapped | hipHostMallocCoherent),
                      "split timing buffer");
            check_hip(hipHostGetDevicePointer(reinterpret_cast<void**>(&device), host, 0), "split timing address");
            check_hip(hipEventCreateWithFlags(&done, hipEventDisableTiming), "split timing event");
        }
    }
    void release() {
        if (done != nullptr) {
            (void)hipEventSynchronize(done);
            (void)hipEventDestroy(done);
            done = nullptr;
        }
        if (host != nullptr) {
            (void)hipHostFree(host);
            host = nullptr;
            device = nullptr;
        }
        pending = false;
    }
};
}  // namespace synapse_kv

struct SynapseKvCache {
    synapse_kv::Dims dims{};
    int device = 0;
    hipStream_t stream = nullptr;
    uint32_t split_keys = 64;  // fewest keys per decode wave worker
    uint32_t prefill_runs = 1;
    uint32_t prefill_split_keys = 0;     // 0: chosen per step (plan_step)
    int32_t prefill_slots = 256;         // resident prefill workgroups on the device
    uint32_t prefetch = 1;  // decode kernel variant: 1 = two register sets, next step's loads in flight
    uint32_t shared_prefix = 1;  // 1: decode reads copy-on-write pages shared by several step tokens once
    uint32_t fused_sums = 1;     // decoder: 1 adds deferred slice sums in the consuming kernels
    uint32_t segment_cost = 8;   // quarter key steps a decode worker's range pays for each row start in it
    // Adaptive decode split: relative speed of each XCD's decode workers (1 = the mean), from timed launches.
    uint32_t adaptive_split = 0;
    double xcd_speed[synapse_kv::kXcds] = {1, 1, 1, 1, 1, 1, 1, 1};
    synapse_kv::SplitTiming timing[2];
    int timing_next = 0;     // buffer the next timed step uses
    int timing_armed = -1;   // buffer the current step's first decode launch writes (-1: none)
    SynapseKvPageActivation activation{};  // KV page activation (enabled = 0: dense)
    synapse_kv::DeviceBuffer<uint8_t> summaries;  // per pool page: key minima and maxima of its activation pages
    uint64_t summary_page_bytes = 0;
    int32_t summary_keys = 64;  // positions per activation page the summaries are kept for

    // Host shadow of the allocator (same rules as the table kernel).
    std::vector<uint32_t> capacity;
    std::vector<uint32_t> length;
    std::vector<int32_t> table;  // [slots][pages_per_slot]
    std::vector<int32_t> refcount;
    std::vector<int32_t> free_stack;

    // Device state.
    uint8_t* pool = nullptr;
    synapse_kv::DeviceBuffer<int32_t> block_table;
    synapse_kv::DeviceBuffer<int32_t> device_refcount;
    synapse_kv::DeviceBuffer<int32_t> device_free;
    synapse_kv::DeviceBuffer<int32_t> device_state;
    synapse_kv::DeviceBuffer<int32_t> fresh;
    synapse_kv::DeviceBuffer<int32_t> copies;
    synapse_kv::DeviceBuffer<float> cosines;
    synapse_kv::DeviceBuffer<float> sines;
    synapse_kv::DeviceBuffer<uint8_t> op_blob;  // table operations of the last call
    synapse_kv::DeviceBuffer<uint8_t> blob;     // the step: tokens, decode items, merges, prefill items
    synapse_kv::DeviceBuffer<float> partial_out;
    synapse_kv::DeviceBuffer<float> partial_ml;
    synapse_kv::Uploader uploader;
    synapse_kv::PageableUploader pageable;  // uploads of synapse_kv_step_static

    // Device memory of the current step: the cache's own buffers, or the static scratch.
    uint8_t* step_blob = nullptr;
    float* step_partial_out = nullptr;
    float* step_partial_ml = nullptr;

    // Pending table operations of the current call and the list offsets they use.
    std::vector<synapse_kv::TableOp> ops;
    int32_t fresh_count = 0;
    int32_t copy_count = 0;

    // Profiling (synapse_kv_profile_begin/end): an event pair per launch, reused from a pool.
    bool profiling = false;
    uint32_t profile_every = 1;       // time every n-th launch of each kind
    uint64_t profile_seen[8] = {};    // launches of each kind since profiling began
    std::vector<std::pair<hipEvent_t, hipEvent_t>> event_pool;
    std::vector<std::pair<int, size_t>> profiled;  // (kernel kind, event pair index)

    // Device addresses that passed the device-memory check, most recent first.
    std::vector<const void*> checked_pointers;

    // The current step.
    bool step_ready = false;
    int32_t step_count = 0;
    int32_t decode_workers = 0;
    int32_t first_level_merges = 0;  // merges[0, first_level_merges) run before the rest
    int32_t wide_merges = 0;         // the last wide_merges merges take a workgroup each
    int32_t merges = 0;
    int32_t prefill_items = 0;  // prompt-run items, followed in the blob by listed_items shared-prefix items
    int32_t listed_items = 0;
    int32_t listed_tiles = 1;   // column tiles the listed items need (1 when every set has at most 16 members)
    int32_t decode_waves = 1024;  // resident decode waves on the device
    bool fusable = false;         // the step can append and attend in one decode launch
    size_t tokens_offset = 0;
    size_t workers_offset = 0;
    size_t members_offset = 0;
    size_t segments_offset = 0;
    size_t merges_offset = 0;
    size_t prefill_offset = 0;
    int32_t prompt_start = 0;        // tokens from here on are prompt tokens (dense under page activation)
    size_t lists_offset = 0;         // block lists of page-activated rows
    size_t list_layer_entries = 0;   // entries per layer in the blob (random lists differ per layer), else 0
    size_t select_offset = 0;        // key-bound selection jobs
    int32_t select_jobs = 0;
    size_t touched_offset = 0;       // (page, block) pairs whose summaries are recomputed after each append
    int32_t touched_blocks = 0;
    size_t extend_offset = 0;        // per token: 1 when the append kernel folds the key into its block's summary
    // Per slot: the length up to which the summary of the slot's last block is exact, where the next append may
    // fold its key in (-1: not known; the next write recomputes).
    std::vector<int64_t> fold_next;
    bool select_reads_touched = false;  // a selection ranks a block the step writes (window 0 at a block's end)
    int32_t most_candidates = 0;     // largest key-bound selection job
    synapse_kv::DeviceBuffer<uint64_t> select_keys;

    ~SynapseKvCache() {
        (void)hipSetDevice(device);
        (void)hipStreamSynchronize(stream);
        uploader.release();
        pageable.release();
        timing[0].release();
        timing[1].release();
        for (auto& pair : event_pool) {
            (void)hipEventDestroy(pair.first);
            (void)hipEventDestroy(pair.second);
        }
        block_table.reset();
        device_refcount.reset();
        device_free.reset();
        device_state.reset();
        fresh.reset();
        copies.reset();
        cosines.reset();
        sines.reset();
        op_blob.reset();
        blob.reset();
        partial_out.reset();
        partial_ml.reset();
        summaries.reset();
        select_keys.reset();
        if (pool != nullptr) {
            (void)hipFree(pool);
        }
    }
};

namespace synapse_kv {
namespace {

// Event pairs created when profiling begins.
constexpr size_t kProfileEvents = 256;

// The launch target of a kernel of `kind` that will be dispatched (`dispatched` false: no kernel follows, so no
// events are taken).
Launch launch_for(SynapseKvCache& cache, int kind, bool dispatched) {
    Launch launch{cache.stream, nullptr, nullptr};
    if (!cache.profiling || !dispatched || cache.profile_seen[kind]++ % cache.profile_every != 0) {
        return launch;
    }
    const size_t index = cache.profiled.size();
    if (index == cache.event_pool.size()) {
        hipEvent_t start = nullptr;
        hipEvent_t stop = nullptr;
        check_hip(hipEventCreate(&start), "profile event");
        if (hipEventCreate(&stop) != hipSuccess) {
            (void)hipEventDestroy(start);
            check_hip(hipErrorOutOfMemory, "profile event");
        }
        cache.event_pool.emplace_back(start, stop);
    }
    cache.profiled.emplace_back(kind, index);
    launch.start = cache.event_pool[index].first;
    launch.stop = cache.event_pool[index].second;
    return launch;
}

// Rejects host memory for a device operand. The runtime query is slow next to a kernel launch, so addresses that
// passed are remembered (a layer's qkv and output buffers are reused every step).
void check_device_pointer(SynapseKvCache& cache, const void* pointer, const char* name) {
    if (pointer == nullptr) {
        fail(SYNAPSE_KV_NULL_POINTER, std::string("null pointer: ") + name);
    }
    auto& seen = cache.checked_pointers;
    const auto found = std::find(seen.begin(), seen.end(), pointer);
    if (found != seen.end()) {
        return;
    }
    hipPointerAttribute_t attributes{};
    if (hipPointerGetAttributes(&attributes, pointer) != hipSuccess || attributes.type != hipMemoryTypeDevice) {
        (void)hipGetLastError();
        invalid(std::string(name) + " must be device memory");
    }
    if (seen.size() >= 256) {
        seen.pop_back();
    }
    seen.insert(seen.begin(), pointer);
}

uint32_t pages_for(const Dims& dims, uint32_t positions) { return (positions + dims.page_tokens - 1) / dims.page_tokens; }

int32_t& slot_page(SynapseKvCache& cache, uint32_t slot, uint32_t logical) {
    return cache.table[static_cast<size_t>(slot) * cache.dims.pages_per_slot + logical];
}

// Shadow resize (same order rules as table_kernel) and its table op.
void shadow_resize(SynapseKvCache& cache, uint32_t slot, uint32_t positions) {
    const uint32_t have = pages_for(cache.dims, cache.capacity[slot]);
    const uint32_t want = pages_for(cache.dims, positions);
    if (want != have) {
        cache.ops.push_back(TableOp{kOpResize, static_cast<int32_t>(slot), static_cast<int32_t>(have),
                                    static_cast<int32_t>(want), cache.fresh_count, {0, 0, 0}});
    }
    for (uint32_t page = have; page < want; ++page) {
        const int32_t id = cache.free_stack.back();
        cache.free_stack.pop_back();
        cache.refcount[id] = 1;
        slot_page(cache, slot, page) = id;
        ++cache.fresh_count;
    }
    for (uint32_t page = have; page-- > want;) {
        const int32_t id = slot_page(cache, slot, page);
        if (--cache.refcount[id] == 0) {
            cache.free_stack.push_back(id);
        }
        slot_page(cache, slot, page) = -1;
    }
    cache.capacity[slot] = positions;
    if (positions < cache.length[slot]) {
        cache.length[slot] = positions;
        cache.fold_next[slot] = -1;
    }
}

void check_slot(const SynapseKvCache& cache, uint32_t slot) {
    if (slot >= cache.dims.slots) {
        invalid("slot " + std::to_string(slot) + " is outside 0.." + std::to_string(cache.dims.slots - 1));
    }
}

void set_device(const SynapseKvCache& cache) { check_hip(hipSetDevice(cache.device), "set device"); }

// Sends the pending table ops and runs the table, zero-fill and copy kernels. The ops go to `fixed` (the static
// scratch, through pageable memory) when given, else to the cache's operation buffer.
void flush_ops(SynapseKvCache& cache, uint8_t* fixed = nullptr) {
    if (cache.ops.empty()) {
        return;
    }
    const size_t bytes = cache.ops.size() * sizeof(TableOp);
    uint8_t* destination = fixed;
    if (fixed != nullptr) {
        std::memcpy(cache.pageable.acquire(bytes), cache.ops.data(), bytes);
        cache.pageable.copy(fixed, bytes, cache.stream);
    } else {
        cache.op_blob.ensure(bytes, "operation buffer");
        void* staging = cache.uploader.acquire(bytes);
        std::memcpy(staging, cache.ops.data(), bytes);
        cache.uploader.copy(cache.op_blob.pointer, bytes, cache.stream);
        destination = cache.op_blob.pointer;
    }
    TableArgs args{};
    args.ops = reinterpret_cast<const TableOp*>(destination);
    args.op_count = static_cast<int32_t>(cache.ops.size());
    args.pages_per_slot = static_cast<int32_t>(cache.dims.pages_per_slot);
    args.max_pages = static_cast<int32_t>(cache.dims.max_pages);
    args.block_table = cache.block_table.pointer;
    args.refcount = cache.device_refcount.pointer;
    args.free_stack = cache.device_free.pointer;
    args.state = cache.device_state.pointer;
    args.fresh = cache.fresh.pointer;
    args.copies = cache.copies.pointer;
    check_hip(launch_table(launch_for(cache, SYNAPSE_KV_KERNEL_TABLE, args.op_count > 0), args), "table kernel");
    PageArgs zero{cache.pool, cache.dims.page_bytes, cache.fresh.pointer, cache.fresh_count};
    check_hip(launch_zero_pages(launch_for(cache, SYNAPSE_KV_KERNEL_PAGES, zero.count > 0), zero), "zero pages");
    PageArgs copy{cache.pool, cache.dims.page_bytes, cache.copies.pointer, cache.copy_count};
    check_hip(launch_copy_pages(launch_for(cache, SYNAPSE_KV_KERNEL_PAGES, copy.count > 0), copy), "copy pages");
    if (cache.activation.enabled != 0) {
        // A copied page keeps its blocks' summaries (the step's writes into it recompute theirs afterwards).
        PageArgs summary_copy{cache.summaries.pointer, cache.summary_page_bytes, cache.copies.pointer,
                              cache.copy_count};
        check_hip(launch_copy_pages(launch_for(cache, SYNAPSE_KV_KERNEL_PAGES, summary_copy.count > 0), summary_copy),
                  "copy summaries");
    }
    cache.ops.clear();
    cache.fresh_count = 0;
    cache.copy_count = 0;
}

// The device address of `scratch` on `device` (the current device), looked up once per device.
uint8_t* scratch_address(int device) {
    static std::mutex mutex;
    static std::array<uint8_t*, 64> addresses{};
    if (device < 0 || device >= static_cast<int>(addresses.size())) {
        invalid("device " + std::to_string(device) + " is past the static scratch table");
    }
    std::lock_guard<std::mutex> lock(mutex);
    if (addresses[device] == nullptr) {
        void* address = nullptr;
        check_hip(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)), "static scratch address");
        if (address == nullptr) {
            fail(SYNAPSE_KV_DEVICE_ERROR, "static scratch has no device address");
        }
        addresses[device] = static_cast<uint8_t*>(address);
    }
    return addresses[device];
}

Geometry geometry(const SynapseKvCache& cache, uint32_t layer) {
    Geometry g{};
    g.pool = cache.pool;
    g.page_bytes = cache.dims.page_bytes;
    g.block_table = cache.block_table.pointer;
    g.pages_per_slot = static_cast<int32_t>(cache.dims.pages_per_slot);
    g.page_tokens = static_cast<int32_t>(cache.dims.page_tokens);
    g.heads = static_cast<int32_t>(cache.dims.heads);
    g.kv_heads = static_cast<int32_t>(cache.dims.kv_heads);
    g.group = static_cast<int32_t>(cache.dims.heads / cache.dims.kv_heads);
    g.head_dim = static_cast<int32_t>(cache.dims.head_dim);
    g.layer = static_cast<int32_t>(layer);
    g.summary_keys = cache.summary_keys;
    return g;
}

size_t align_up(size_t value, size_t alignment) { return (value + alignment - 1) / alignment * alignment; }



// Automatic prefill split: the piece length (in 64-key steps) with the shortest estimated makespan when the
// pieces are spread over the device's resident workgroup slots. Candidates cut the longest block into 1..32
// pieces; a candidate's estimate is the smaller of (rounds of slots) x piece and (average load per slot + one
// piece), the second bounding greedy scheduling of uneven pieces. Splitting further must gain 5%, since every
// split adds partial rows and a merge.
int64_t choose_prefill_chunk(const SynapseKvCache& cache, const SynapseKvBatchToken* tokens,
                             const std::vector<std::pair<int32_t, int32_t>>& runs) {
    std::vector<int64_t> blocks;
    for (const auto& [run_start, run_end] : runs) {
        for (int32_t first = run_start; first < run_end; first += kPrefillTokens) {
            const int32_t size = std::min<int32_t>(kPrefillTokens, run_end - first);
            blocks.push_back((tokens[first + size - 1].position + kStepKeys) / kStepKeys);
        }
    }
    const int64_t heads = cache.dims.kv_heads;
    const int64_t slots = std::max<int32_t>(1, cache.prefill_slots);
    const int64_t longest = *std::max_element(blocks.begin(), blocks.end());
    int64_t total = 0;
    for (int64_t steps : blocks) {
        total += steps * heads;
    }
    const int64_t fewest = kMinPrefillChunk / kStepKeys;
    int64_t best_chunk = longest;
    double best_estimate = 0.0;
    for (int64_t pieces = 1; pieces <= 32; ++pieces) {
        const int64_t chunk = (longest + pieces - 1) / pieces;
        if (pieces > 1 && chunk < fewest) {
            break;
        }
        int64_t items = 0;
        for (int64_t steps : blocks) {
            items += (steps + chunk - 1) / chunk * heads;
        }
        const double rounds = static_cast<double>((items + slots - 1) / slots) * chunk;
        const double greedy = static_cast<double>(total) / slots + chunk;
        const double estimate = std::min(rounds, greedy);
        if (pieces == 1 || estimate < 0.95 * best_estimate) {
            best_estimate = estimate;
            best_chunk = chunk;
        }
    }
    return best_chunk;
}

// Rank keys one key-bound selection job keeps between its tiles and its merge.
size_t select_key_stride(const SynapseKvCache& cache, int32_t most_candidates) {
    const size_t tiles = (static_cast<size_t>(most_candidates) + 63) / 64;
    return tiles * std::min<size_t>(cache.activation.budget_pages, 64);
}

// Builds and uploads the attention plan of a prepared step.
//
// Lone tokens (and prompt runs of FP32 caches) go to the decode kernel: every (token, KV head) row is cut into
// 64-key steps, the steps of all rows are laid end to end and split evenly over the resident decode waves, so each
// wave streams the same number of K/V bytes whatever the ragged lengths. Rows cut by a worker boundary get partial
// rows and a merge entry. FP16 prompt runs (plan_attention, schedule.rs:34-86: consecutive tokens of one slot at
// consecutive positions) go to the MFMA prefill kernel in blocks of kPrefillTokens tokens per KV head, their keys
// split into work items of at most `chunk` keys whose partial rows the merge kernel combines. The chunk is the
// prefill_split_keys option when set, otherwise chosen by choose_prefill_chunk: runs that already fill the device
// are not split (and need no merge), short chunks over long caches are.
// With `fixed`, the plan and the partial rows go to that device memory (the static scratch) instead of the cache's
// buffers, and a plan that does not fit fails before any device work.
struct FixedMemory {
    uint8_t* base;
    size_t bytes;
};

// The XCD of decode worker w's workgroup (the dispatcher places workgroup b on XCD b % kXcds).
int worker_xcd(int w) { return (w / kDecodeBlockWaves) % kXcds; }

// Adaptive split: folds the worker durations of finished timed launches into the XCD speeds. An XCD's speed is the
// cost its workers were planned per tick, relative to the mean over the XCDs; half of each measurement enters the
// running estimate, which stays within 0.5-2. (Per-workgroup speeds, which would follow each CU, measured no
// better: the CUs' order changes from launch to launch, the XCDs' holds.)
void update_xcd_speeds(SynapseKvCache& cache) {
    for (SplitTiming& timing : cache.timing) {
        if (!timing.pending) {
            continue;
        }
        const hipError_t state = hipEventQuery(timing.done);
        if (state == hipErrorNotReady) {
            (void)hipGetLastError();
            continue;
        }
        check_hip(state, "split timing");
        timing.pending = false;
        double cost[kXcds] = {};
        double ticks[kXcds] = {};
        for (int launch = 0; launch < timing.launches; ++launch) {
            const uint32_t* durations = timing.host + static_cast<size_t>(launch) * SplitTiming::kWorkers;
            for (size_t w = 0; w < timing.costs.size(); ++w) {
                cost[worker_xcd(static_cast<int>(w))] += static_cast<double>(timing.costs[w]);
                ticks[worker_xcd(static_cast<int>(w))] += static_cast<double>(durations[w]);
            }
        }
        double mean = 0.0;
        int measured = 0;
        for (int x = 0; x < kXcds; ++x) {
            if (cost[x] > 0.0 && ticks[x] > 0.0) {
                mean += cost[x] / ticks[x];
                ++measured;
            }
        }
        if (measured == 0) {
            continue;
        }
        mean /= measured;
        for (int x = 0; x < kXcds; ++x) {
            if (cost[x] > 0.0 && ticks[x] > 0.0) {
                const double relative = cost[x] / ticks[x] / mean;
                cache.xcd_speed[x] = std::min(2.0, std::max(0.5, 0.5 * cache.xcd_speed[x] + 0.5 * relative));
            }
        }
    }
}

void plan_step(SynapseKvCache& cache, const SynapseKvBatchToken* tokens, int32_t count,
               const std::vector<uint32_t>& old_lengths, const FixedMemory* fixed = nullptr) {
    const Dims& dims = cache.dims;
    const int32_t group = static_cast<int32_t>(dims.heads / dims.kv_heads);
    // A row: keys [key_begin, keys) of one (token, KV head); for a member of a shared set (set >= 0) the keys past
    // the shared prefix, which the set's listed prefill items read once for all members.
    struct Row {
        int32_t token;
        int32_t kv_head;
        int32_t key_begin;
        int32_t keys;
        int32_t set;
        int64_t first_step;
        int64_t steps;
        size_t first_segment;
        int32_t pieces;
        int32_t list;  // >= 0: the row's block list (KV page activation); keys counts list entries times 64
    };
    std::vector<PrefillItem> prefill;
    std::vector<MergeItem> prefill_merges;
    int32_t partial_rows = 0;
    std::vector<int32_t> lone;  // step tokens that go to the decode kernels
    int32_t start = 0;
    std::vector<std::pair<int32_t, int32_t>> runs;
    while (start < count) {
        int32_t end = start + 1;
        while (end < count && tokens[end].slot == tokens[start].slot &&
               tokens[end].position == tokens[end - 1].position + 1) {
            ++end;
        }
        if (end - start == 1 || cache.prefill_runs == 0 || dims.precision != SYNAPSE_KV_F16) {
            for (int32_t index = start; index < end; ++index) {
                lone.push_back(index);
            }
        } else {
            runs.emplace_back(start, end);
        }
        start = end;
    }

    // KV page activation (Qwen2KvPageMasks.cs:21-54): a decode unit is a token before the prompt boundary that is
    // alone in its slot. KvPageSelector.Select (KvPageSelector.cs:17-54) with pages of P = 16, 32 or 64 positions
    // gives its row, per KV head, the sink page 0, `budget` pages of 1 .. candidates (ranked by key bound on the
    // device, or drawn here) and the window pages window_page .. position / P; when the budget covers every candidate
    // the row is dense. Each page is one decode step (its 64-key block read, the keys outside the page masked). Listed rows read their blocks through the decode kernel and take no part in shared-prefix sets.
    struct Unit {
        int32_t window_page;  // -1: dense
        int32_t candidates;
        int32_t entries;
    };
    const SynapseKvPageActivation& activation = cache.activation;
    std::vector<Unit> units(count, Unit{-1, 0, 0});
    if (activation.enabled != 0) {
        std::vector<int32_t> in_slot(dims.slots, 0);
        for (int32_t index = 0; index < count; ++index) {
            ++in_slot[tokens[index].slot];
        }
        for (int32_t index = 0; index < std::min(count, cache.prompt_start); ++index) {
            if (in_slot[tokens[index].slot] != 1) {
                continue;
            }
            const int64_t keys = static_cast<int64_t>(tokens[index].position) + 1;
            const int32_t window_page =
                static_cast<int32_t>(std::max<int64_t>(0, keys - activation.window_tokens) / cache.summary_keys);
            const int32_t candidates = std::max(0, window_page - 1);
            if (static_cast<uint32_t>(candidates) <= activation.budget_pages) {
                continue;
            }
            if (activation.selection == SYNAPSE_KV_SELECT_KEY_BOUND && candidates > kMaxSelectCandidates) {
                fail(SYNAPSE_KV_UNAVAILABLE, "key-bound page selection ranks at most " +
                                                 std::to_string(kMaxSelectCandidates) + " pages; token " +
                                                 std::to_string(index) + " has " + std::to_string(candidates));
            }
            const int32_t own_page = tokens[index].position / cache.summary_keys;
            units[index] = Unit{window_page, candidates,
                                1 + static_cast<int32_t>(activation.budget_pages) + own_page - window_page + 1};
        }
    }

    // Shared prefixes (FP16): lone tokens whose block tables map their leading pages to the same physical pages
    // (copy-on-write forks) form sets of up to kPrefillTokens members. A set's shared pages are those all members
    // map alike, below every member's own position (whose page the step has already made private); listed prefill
    // items read them once for the whole set, and each member's own keys go through the decode kernel.
    struct SharedSet {
        std::vector<int32_t> members;
        int32_t shared_keys;
    };
    std::vector<SharedSet> sets;
    std::vector<int32_t> set_of(count, -1);
    if (cache.shared_prefix != 0 && dims.precision == SYNAPSE_KV_F16 && lone.size() > 1) {
        auto first_page = [&](int32_t index) {
            return cache.table[static_cast<size_t>(tokens[index].slot) * dims.pages_per_slot];
        };
        std::vector<int32_t> order;
        for (int32_t index : lone) {
            if (units[index].window_page < 0) {
                order.push_back(index);
            }
        }
        std::stable_sort(order.begin(), order.end(),
                         [&](int32_t x, int32_t y) { return first_page(x) < first_page(y); });
        const size_t most = static_cast<size_t>(kPrefillTokens);
        for (size_t begin = 0; begin < order.size();) {
            size_t end = begin + 1;
            while (end < order.size() && first_page(order[end]) == first_page(order[begin])) {
                ++end;
            }
            if (end - begin > 1 && first_page(order[begin]) >= 0) {
                const int32_t* reference = &cache.table[static_cast<size_t>(tokens[order[begin]].slot) * dims.pages_per_slot];
                uint32_t pages = dims.pages_per_slot;
                for (size_t k = begin; k < end; ++k) {
                    const int32_t* table = &cache.table[static_cast<size_t>(tokens[order[k]].slot) * dims.pages_per_slot];
                    uint32_t same = 0;
                    const uint32_t below = static_cast<uint32_t>(tokens[order[k]].position) / dims.page_tokens;
                    while (same < std::min(pages, below) && table[same] == reference[same]) {
                        ++same;
                    }
                    pages = same;
                }
                for (size_t first = begin; pages > 0 && first < end; first += most) {
                    const size_t last = std::min(end, first + most);
                    if (last - first < 2) {
                        continue;
                    }
                    SharedSet set{std::vector<int32_t>(order.begin() + first, order.begin() + last),
                                  static_cast<int32_t>(pages * dims.page_tokens)};
                    std::sort(set.members.begin(), set.members.end());
                    for (int32_t member : set.members) {
                        set_of[member] = static_cast<int32_t>(sets.size());
                    }
                    sets.push_back(std::move(set));
                }
            }
            begin = end;
        }
    }

    // Rows: every lone token's (token, KV head) rows, from the token's shared keys on; a listed row's steps are its
    // list entries.
    std::vector<Row> rows;
    int32_t list_entries = 0;
    for (int32_t index : lone) {
        const Unit& unit = units[index];
        const int32_t keys = unit.window_page >= 0 ? unit.entries * kStepKeys : tokens[index].position + 1;
        const int32_t key_begin = set_of[index] >= 0 ? sets[set_of[index]].shared_keys : 0;
        for (uint32_t kv_head = 0; kv_head < dims.kv_heads; ++kv_head) {
            int32_t list = -1;
            if (unit.window_page >= 0) {
                list = list_entries;
                list_entries += unit.entries;
            }
            rows.push_back(Row{index, static_cast<int32_t>(kv_head), key_begin, keys, set_of[index], 0,
                               (keys - key_begin + kStepKeys - 1) / kStepKeys, 0, 0, list});
        }
    }

    // Lists of pages' first keys: [sink page 0][budget pages, ascending][window pages]. Key-bound budget entries are
    // written by
    // the selection kernel of each layer (one list region serves every layer); random draws depend on the layer
    // (seed = Seed * 1000003 + layer * 7919 + kv_head * 104729 + position, Qwen2KvPageMasks.cs:37, in 32-bit
    // wrap-around), so each layer gets its own region.
    const bool random = activation.selection == SYNAPSE_KV_SELECT_RANDOM;
    const uint32_t list_layers = random ? dims.layers : 1;
    std::vector<int32_t> lists(static_cast<size_t>(list_entries) * (list_entries > 0 ? list_layers : 0), -1);
    std::vector<SelectJob> select_jobs;
    int32_t most_candidates = 0;
    std::vector<int32_t> drawn;
    for (const Row& row : rows) {
        if (row.list < 0) {
            continue;
        }
        const Unit& unit = units[row.token];
        const int32_t budget = static_cast<int32_t>(activation.budget_pages);
        const int32_t position = tokens[row.token].position;
        for (uint32_t layer = 0; layer < list_layers; ++layer) {
            int32_t* list = &lists[static_cast<size_t>(layer) * list_entries + row.list];
            const int32_t size = cache.summary_keys;
            list[0] = 0;
            for (int32_t page = unit.window_page; page <= position / size; ++page) {
                list[1 + budget + page - unit.window_page] = page * size;
            }
            if (random) {
                // RandomPages (KvPageSelector.cs:118-129): a partial Fisher-Yates draw over pages 1..candidates.
                const uint32_t seed = static_cast<uint32_t>(activation.seed) * 1000003u + layer * 7919u +
                                      static_cast<uint32_t>(row.kv_head) * 104729u + static_cast<uint32_t>(position);
                SeededRandom generator(static_cast<int32_t>(seed));
                drawn.resize(unit.candidates);
                for (int32_t page = 0; page < unit.candidates; ++page) {
                    drawn[page] = page + 1;
                }
                for (int32_t index = 0; index < budget; ++index) {
                    std::swap(drawn[index], drawn[generator.next(index, unit.candidates)]);
                }
                std::sort(drawn.begin(), drawn.begin() + budget);
                for (int32_t index = 0; index < budget; ++index) {
                    list[1 + index] = drawn[index] * size;
                }
            }
        }
        if (!random) {
            select_jobs.push_back(SelectJob{row.token, row.kv_head, row.list, unit.candidates});
            most_candidates = std::max(most_candidates, unit.candidates);
        }
    }

    // Summary upkeep of the blocks the step writes (after copy-on-write). A token alone in its block that appends
    // at its slot's exact length (fold_next) is folded into the summary by the append kernel; every other written
    // block is recomputed after the appends from its keys below the slot's new length, which leaves it exact for
    // the next append when the slot's positions this step were exactly [old length, new length). A decode unit's
    // candidates end below its window, so a block the step writes is a candidate only with no window at a block's
    // last position; otherwise a recomputation can ride along in the selection launch.
    std::vector<int32_t> touched;
    std::vector<int32_t> extend;
    bool select_reads_touched = false;
    if (activation.enabled != 0) {
        auto block_key = [&](int32_t index) {
            const uint32_t position = static_cast<uint32_t>(tokens[index].position);
            const int32_t page = cache.table[static_cast<size_t>(tokens[index].slot) * dims.pages_per_slot +
                                             position / dims.page_tokens];
            return static_cast<int64_t>(page) * 65536 + (position % dims.page_tokens) / cache.summary_keys;
        };
        std::vector<int64_t> keys(count);
        for (int32_t index = 0; index < count; ++index) {
            keys[index] = block_key(index);
        }
        std::vector<int64_t> sorted = keys;
        std::sort(sorted.begin(), sorted.end());
        std::vector<int32_t> in_slot(dims.slots, 0);
        for (int32_t index = 0; index < count; ++index) {
            ++in_slot[tokens[index].slot];
        }
        extend.assign(count, 0);
        std::vector<std::pair<int64_t, int32_t>> recompute;  // (block key, keys below the slot's new length)
        std::vector<int64_t> lowest(dims.slots, INT64_MAX);
        std::vector<int32_t> written(dims.slots, 0);
        for (int32_t index = 0; index < count; ++index) {
            lowest[tokens[index].slot] = std::min<int64_t>(lowest[tokens[index].slot], tokens[index].position);
            ++written[tokens[index].slot];
        }
        for (int32_t index = 0; index < count; ++index) {
            const int32_t slot = tokens[index].slot;
            const int64_t position = tokens[index].position;
            const auto range = std::equal_range(sorted.begin(), sorted.end(), keys[index]);
            const bool solo = range.second - range.first == 1 && in_slot[slot] == 1;
            const int64_t size = cache.summary_keys;
            if (solo && (position % size == 0 || position == cache.fold_next[slot])) {
                extend[index] = 1;
            } else {
                const int64_t start = position / size * size;
                recompute.emplace_back(keys[index],
                                       static_cast<int32_t>(std::min<int64_t>(size, cache.length[slot] - start)));
                const Unit& unit = units[index];
                if (unit.window_page >= 0 && unit.window_page - 1 >= static_cast<int32_t>(position / size)) {
                    select_reads_touched = true;
                }
            }
        }
        // A slot whose positions this step are exactly [old length, new length) stays exact at its new length.
        for (int32_t index = 0; index < count; ++index) {
            const int32_t slot = tokens[index].slot;
            const bool contiguous = lowest[slot] == old_lengths[slot] &&
                                    cache.length[slot] - old_lengths[slot] == static_cast<uint32_t>(written[slot]);
            cache.fold_next[slot] = contiguous ? static_cast<int64_t>(cache.length[slot]) : -1;
        }
        std::sort(recompute.begin(), recompute.end());
        recompute.erase(std::unique(recompute.begin(), recompute.end()), recompute.end());
        for (const auto& [key, valid] : recompute) {
            touched.push_back(static_cast<int32_t>(key / 65536));
            touched.push_back(static_cast<int32_t>(key % 65536));
            touched.push_back(valid);
        }
    }

    // Even split: the steps of all rows laid end to end, cut into equal shares for the resident wave workers (at
    // least split_keys keys each). A row cut by worker boundaries becomes several segments.
    std::vector<DecodeSegment> segments;
    std::vector<int64_t> planned_costs;  // adaptive split: each worker's share of the cost
    auto split = [&](std::vector<Row>& list, int32_t resident, std::vector<int32_t>& worker_segments) -> int32_t {
        int64_t total_steps = 0;
        for (Row& row : list) {
            row.first_step = total_steps;
            total_steps += row.steps;
        }
        if (total_steps == 0) {
            return 0;
        }
        // Each worker takes at least split_keys keys. When a row would still be cut into more than kWideMergeRows
        // pieces (a second merge launch), workers take enough steps to avoid that if it costs at most kMergeSteps
        // more steps each (about one merge launch of latency).
        int64_t longest = 0;
        for (const Row& row : list) {
            longest = std::max(longest, row.steps);
        }
        int64_t per_worker_min = std::max<int64_t>(1, cache.split_keys / kStepKeys);
        const int64_t filled = std::max(per_worker_min, (total_steps + resident - 1) / resident);
        // A piece holds at least one step, so rows of up to kWideMergeRows steps never need a second level; longer
        // rows are cut into at most ceil(steps / per) + 1 pieces when workers take `per` steps each.
        const int64_t single_level =
            longest <= kWideMergeRows ? 1 : (longest + kWideMergeRows - 2) / (kWideMergeRows - 1);
        if (single_level > filled && single_level - filled <= kMergeSteps) {
            per_worker_min = single_level;
        }
        const int64_t wanted = std::max<int64_t>(1, total_steps / per_worker_min);
        const int32_t workers =
            static_cast<int32_t>(std::min<int64_t>(std::min<int64_t>(wanted, resident), total_steps));
        // Shares are equal in cost, counted in quarter steps: a key step costs 4, and the start of a row in a
        // worker's range costs segment_cost more (its query, RoPE and first block are not overlapped with the
        // previous segment's steps: on C3 a worker with two segments ends about one step later than one with a
        // single segment of the same length).
        // With fewer than four steps per worker the row-start cost only misplaces whole steps: a share of a little
        // more than one step leaves the workers at row starts empty and gives a few others two steps, which then
        // set the launch's length (C1: four of 130 workers). Such splits are even in steps, unless their rows are
        // longer than the 512 pieces a wide merge takes in one round of loads per wave (C2's 513-step rows: the
        // uneven split happens to keep them at 511 pieces, and one more measured slower in the merge).
        const int64_t cost =
            total_steps < 4 * static_cast<int64_t>(workers) && longest <= 64 * kWideWaves ? 0 : cache.segment_cost;
        const int64_t total_cost = 4 * total_steps + cost * static_cast<int64_t>(list.size());
        // With the adaptive split, worker w's share is proportional to its XCD's measured speed.
        std::vector<int64_t> weights;
        if (cache.adaptive_split != 0) {
            weights.resize(static_cast<size_t>(workers) + 1, 0);
            for (int32_t w = 0; w < workers; ++w) {
                const double speed = cache.xcd_speed[worker_xcd(w)];
                weights[w + 1] = weights[w] + static_cast<int64_t>(std::llround(speed * 65536.0));
            }
        }
        auto boundary = [&](int64_t worker) {
            return weights.empty() ? worker * total_cost / workers : total_cost * weights[worker] / weights[workers];
        };
        if (cache.adaptive_split != 0) {
            planned_costs.resize(static_cast<size_t>(workers));
            for (int32_t w = 0; w < workers; ++w) {
                planned_costs[w] = boundary(w + 1) - boundary(w);
            }
        }
        int64_t worker = 0;
        int64_t row_cost = 0;  // cost position of the current row's start
        worker_segments.push_back(static_cast<int32_t>(segments.size()));
        for (Row& row : list) {
            row.first_segment = segments.size();
            const int64_t first = row_cost + cost;  // cost position of the row's first key step
            int64_t step = 0;
            while (step < row.steps) {
                // Key step s occupies [first + 4 s, first + 4 s + 4); a worker takes the steps that start in its
                // share, so every segment holds at least one step.
                while (boundary(worker + 1) <= first + 4 * step) {
                    ++worker;
                    worker_segments.push_back(static_cast<int32_t>(segments.size()));
                }
                const int64_t stop = std::min<int64_t>(row.steps, (boundary(worker + 1) - first + 3) / 4);
                const int32_t key_begin = row.key_begin + static_cast<int32_t>(step * kStepKeys);
                const int32_t key_end = std::min<int32_t>(row.keys, row.key_begin + static_cast<int32_t>(stop * kStepKeys));
                const SynapseKvBatchToken& token = tokens[row.token];
                segments.push_back(DecodeSegment{row.token, row.kv_head, key_begin, key_end, -1, row.list,
                                                 stop == row.steps ? 1 : 0, token.slot, token.position, -1, -1, -1});
                step = stop;
            }
            row.pieces = static_cast<int32_t>(segments.size() - row.first_segment);
            row_cost = first + 4 * row.steps;
        }
        while (static_cast<int32_t>(worker_segments.size()) < workers + 1) {
            worker_segments.push_back(static_cast<int32_t>(segments.size()));
        }
        return workers;
    };
    std::vector<int32_t> worker_segments;
    update_xcd_speeds(cache);
    const int32_t workers = split(rows, cache.decode_waves, worker_segments);
    cache.timing_armed = -1;
    if (cache.adaptive_split != 0 && workers > 0 && workers <= SplitTiming::kWorkers &&
        !cache.timing[cache.timing_next].pending) {
        cache.timing_armed = cache.timing_next;
        cache.timing[cache.timing_next].costs = std::move(planned_costs);
        cache.timing[cache.timing_next].launches = 0;
        cache.timing_next ^= 1;
    }

    // Partial rows and merge entries. A row of its own that was cut gets consecutive partial rows. A shared set's
    // keys are cut, per KV head, into P listed prefill items of about equal length (enough items over all sets to
    // fill the device's prefill workgroup slots, at least kMinSharedSteps steps each). With Q_m own pieces of
    // member m, member m owns the rows base + m * stride .. + P + Q_m - 1 (stride = P + max Q_m): its shared
    // pieces first, then its own.
    std::vector<MergeItem> merges;
    std::vector<int32_t> members;
    for (const Row& row : rows) {
        if (row.set >= 0 || row.pieces < 2) {
            continue;
        }
        merges.push_back(MergeItem{row.token, row.kv_head, partial_rows, row.pieces, -1, {0, 0, 0}});
        for (int32_t piece = 0; piece < row.pieces; ++piece) {
            segments[row.first_segment + piece].row = partial_rows + piece;
        }
        partial_rows += row.pieces;
    }
    std::vector<PrefillItem> listed;
    int32_t listed_tiles = 1;
    if (!sets.empty()) {
        // own_rows[token * kv_heads + kv_head]: the row of a set member's own keys.
        std::vector<const Row*> own_rows(static_cast<size_t>(count) * dims.kv_heads, nullptr);
        for (const Row& row : rows) {
            if (row.set >= 0) {
                own_rows[static_cast<size_t>(row.token) * dims.kv_heads + row.kv_head] = &row;
            }
        }
        int64_t shared_steps = 0;
        for (const SharedSet& set : sets) {
            shared_steps += static_cast<int64_t>(dims.kv_heads) * (set.shared_keys / kStepKeys);
        }
        const int64_t item_steps =
            std::max<int64_t>(kMinSharedSteps, (shared_steps + cache.prefill_slots - 1) / cache.prefill_slots);
        for (const SharedSet& set : sets) {
            const int32_t offset = static_cast<int32_t>(members.size());
            members.insert(members.end(), set.members.begin(), set.members.end());
            const int32_t size = static_cast<int32_t>(set.members.size());
            listed_tiles = std::max(listed_tiles, (size + 15) / 16);
            const int64_t steps = set.shared_keys / kStepKeys;
            const int32_t pieces = static_cast<int32_t>((steps + item_steps - 1) / item_steps);
            for (uint32_t kv_head = 0; kv_head < dims.kv_heads; ++kv_head) {
                int32_t most_own = 0;
                for (int32_t member : set.members) {
                    most_own = std::max(most_own, own_rows[static_cast<size_t>(member) * dims.kv_heads + kv_head]->pieces);
                }
                const int32_t stride = pieces + most_own;
                const int32_t base = partial_rows;
                partial_rows += size * stride;
                for (int32_t piece = 0; piece < pieces; ++piece) {
                    const int32_t begin = static_cast<int32_t>(piece * steps / pieces * kStepKeys);
                    const int32_t finish = static_cast<int32_t>((piece + 1) * steps / pieces * kStepKeys);
                    listed.push_back(PrefillItem{offset, size, static_cast<int32_t>(kv_head), begin, finish, base + piece,
                                                 stride, 1});
                }
                for (int32_t m = 0; m < size; ++m) {
                    const Row& own = *own_rows[static_cast<size_t>(set.members[m]) * dims.kv_heads + kv_head];
                    merges.push_back(MergeItem{own.token, own.kv_head, base + m * stride, pieces + own.pieces, -1,
                                               {0, 0, 0}});
                    for (int32_t piece = 0; piece < own.pieces; ++piece) {
                        segments[own.first_segment + piece].row = base + m * stride + pieces + piece;
                    }
                }
            }
        }
    }

    // Prefill blocks. A block's keys are cut into the fewest pieces of at most `chunk_steps` 64-key steps, of
    // (nearly) equal length.
    int64_t chunk_steps = cache.prefill_split_keys / kStepKeys;
    if (chunk_steps == 0 && !runs.empty()) {
        chunk_steps = choose_prefill_chunk(cache, tokens, runs);
    }
    for (const auto& [run_start, run_end] : runs) {
        for (int32_t first = run_start; first < run_end; first += kPrefillTokens) {
            const int32_t size = std::min<int32_t>(kPrefillTokens, run_end - first);
            const int32_t keys = tokens[first + size - 1].position + 1;
            const int64_t steps = (keys + kStepKeys - 1) / kStepKeys;
            const int32_t splits = static_cast<int32_t>((steps + chunk_steps - 1) / chunk_steps);
            const int32_t stride = static_cast<int32_t>(dims.kv_heads) * splits;
            if (splits > 1) {
                for (int32_t j = 0; j < size; ++j) {
                    for (uint32_t kv_head = 0; kv_head < dims.kv_heads; ++kv_head) {
                        prefill_merges.push_back(MergeItem{first + j, static_cast<int32_t>(kv_head),
                                                           partial_rows + j * stride +
                                                               static_cast<int32_t>(kv_head) * splits,
                                                           splits, -1, {0, 0, 0}});
                    }
                }
            }
            for (uint32_t kv_head = 0; kv_head < dims.kv_heads; ++kv_head) {
                for (int32_t part = 0; part < splits; ++part) {
                    const int32_t begin = static_cast<int32_t>(part * steps / splits * kStepKeys);
                    const int32_t finish =
                        std::min<int32_t>(keys, static_cast<int32_t>((part + 1) * steps / splits * kStepKeys));
                    const int32_t row = splits > 1 ? partial_rows + static_cast<int32_t>(kv_head) * splits + part : -1;
                    prefill.push_back(PrefillItem{first, size, static_cast<int32_t>(kv_head), begin, finish, row,
                                                  stride, 0});
                }
            }
            if (splits > 1) {
                partial_rows += size * stride;
            }
        }
    }
    // Prompt-run items first, then the listed items (a launch of their own when one column tile holds every set).
    const int32_t prompt_items = static_cast<int32_t>(prefill.size());
    prefill.insert(prefill.end(), listed.begin(), listed.end());
    merges.insert(merges.end(), prefill_merges.begin(), prefill_merges.end());
    // Merges of up to kMergeRows partial rows take one wave each, up to kWideMergeRows a workgroup each (the wide
    // launch, after the narrow one); longer ones first combine blocks of 64 rows into intermediate partial rows (a
    // first launch), then merge those.
    std::vector<MergeItem> first_level;
    std::vector<MergeItem> final_level;
    std::vector<MergeItem> wide_level;
    for (MergeItem merge : merges) {
        if (merge.count <= kMergeRows) {
            final_level.push_back(merge);
            continue;
        }
        if (merge.count <= kWideMergeRows) {
            wide_level.push_back(merge);
            continue;
        }
        const int32_t blocks = (merge.count + 63) / 64;
        for (int32_t block = 0; block < blocks; ++block) {
            first_level.push_back(MergeItem{merge.token, merge.kv_head, merge.first_row + 64 * block,
                                            std::min<int32_t>(64, merge.count - 64 * block), partial_rows + block,
                                            {0, 0, 0}});
        }
        const MergeItem combined{merge.token, merge.kv_head, partial_rows, blocks, -1, {0, 0, 0}};
        (blocks <= kMergeRows ? final_level : wide_level).push_back(combined);
        partial_rows += blocks;
    }
    const int32_t first_level_merges = static_cast<int32_t>(first_level.size());
    const int32_t wide_merges = static_cast<int32_t>(wide_level.size());
    merges = std::move(first_level);
    merges.insert(merges.end(), final_level.begin(), final_level.end());
    merges.insert(merges.end(), wide_level.begin(), wide_level.end());

    // Segments as the decode kernel walks them: worker w's first segment at index w (no lookup before the wave's
    // first descriptor read), its later ones after all workers' first ones, chained by `next`; each with the pool
    // page of its first block from the host table (the same pages the step's table operations leave on the device),
    // so the wave's first K/V requests need no table read either.
    {
        std::vector<DecodeSegment> chained(static_cast<size_t>(workers));
        for (int32_t w = 0; w < workers; ++w) {
            const int32_t begin = worker_segments[w];
            const int32_t end = worker_segments[w + 1];
            if (begin == end) {  // a worker without steps (not planned: workers never exceed the steps)
                chained[w] = DecodeSegment{-1, 0, 0, 0, -1, -1, 0, 0, 0, -1, -1, -1};
                continue;
            }
            int32_t previous = w;
            chained[w] = segments[begin];
            for (int32_t i = begin + 1; i < end; ++i) {
                chained[previous].next = static_cast<int32_t>(chained.size());
                previous = static_cast<int32_t>(chained.size());
                chained.push_back(segments[i]);
            }
            chained[previous].next = -1;
        }
        for (DecodeSegment& seg : chained) {
            if (seg.token >= 0 && seg.list < 0) {
                seg.first_page = slot_page(cache, static_cast<uint32_t>(seg.slot),
                                           static_cast<uint32_t>((seg.key_begin & ~(kStepKeys - 1)) / dims.page_tokens));
            }
            if (seg.token >= 0 && seg.last != 0) {
                seg.append_page = slot_page(cache, static_cast<uint32_t>(seg.slot),
                                            static_cast<uint32_t>(seg.position) / dims.page_tokens);
            }
        }
        segments = std::move(chained);
    }
    const size_t tokens_bytes = static_cast<size_t>(count) * sizeof(SynapseKvBatchToken);
    cache.tokens_offset = 0;
    cache.workers_offset = align_up(tokens_bytes, 256);
    cache.members_offset = cache.workers_offset;
    cache.segments_offset = align_up(cache.members_offset + members.size() * sizeof(int32_t), 256);
    cache.merges_offset = align_up(cache.segments_offset + segments.size() * sizeof(DecodeSegment), 256);
    cache.prefill_offset = align_up(cache.merges_offset + merges.size() * sizeof(MergeItem), 256);
    cache.lists_offset = align_up(cache.prefill_offset + prefill.size() * sizeof(PrefillItem), 256);
    cache.select_offset = align_up(cache.lists_offset + lists.size() * sizeof(int32_t), 256);
    cache.touched_offset = align_up(cache.select_offset + select_jobs.size() * sizeof(SelectJob), 256);
    cache.extend_offset = align_up(cache.touched_offset + touched.size() * sizeof(int32_t), 256);
    const size_t total = cache.extend_offset + extend.size() * sizeof(int32_t);
    const size_t partial_out_floats = static_cast<size_t>(partial_rows) * group * dims.head_dim;
    const size_t partial_ml_floats = static_cast<size_t>(partial_rows) * group * 2;
    uint8_t* staging = nullptr;
    if (fixed != nullptr) {
        const size_t ml_offset = align_up(total, 256);
        const size_t out_offset = align_up(ml_offset + partial_ml_floats * sizeof(float), 256);
        const size_t needed = out_offset + partial_out_floats * sizeof(float);
        if (needed > fixed->bytes) {
            invalid("the step needs " + std::to_string(needed) + " bytes of static scratch for its plan and " +
                    std::to_string(partial_rows) + " partial rows; " + std::to_string(fixed->bytes) +
                    " are left of SYNAPSE_KV_STATIC_SCRATCH_BYTES");
        }
        cache.step_blob = fixed->base;
        cache.step_partial_ml = reinterpret_cast<float*>(fixed->base + ml_offset);
        cache.step_partial_out = reinterpret_cast<float*>(fixed->base + out_offset);
        staging = cache.pageable.acquire(total);
    } else {
        cache.select_keys.ensure(select_jobs.size() * select_key_stride(cache, most_candidates), "page selection keys");
        cache.blob.ensure(total, "step buffer");
        cache.partial_out.ensure(partial_out_floats, "attention partials");
        cache.partial_ml.ensure(partial_ml_floats, "attention partial statistics");
        cache.step_blob = cache.blob.pointer;
        cache.step_partial_out = cache.partial_out.pointer;
        cache.step_partial_ml = cache.partial_ml.pointer;
        staging = static_cast<uint8_t*>(cache.uploader.acquire(total));
    }
    std::memcpy(staging + cache.tokens_offset, tokens, tokens_bytes);
    std::memcpy(staging + cache.members_offset, members.data(), members.size() * sizeof(int32_t));
    std::memcpy(staging + cache.segments_offset, segments.data(), segments.size() * sizeof(DecodeSegment));
    std::memcpy(staging + cache.merges_offset, merges.data(), merges.size() * sizeof(MergeItem));
    std::memcpy(staging + cache.prefill_offset, prefill.data(), prefill.size() * sizeof(PrefillItem));
    std::memcpy(staging + cache.lists_offset, lists.data(), lists.size() * sizeof(int32_t));
    std::memcpy(staging + cache.select_offset, select_jobs.data(), select_jobs.size() * sizeof(SelectJob));
    std::memcpy(staging + cache.touched_offset, touched.data(), touched.size() * sizeof(int32_t));
    std::memcpy(staging + cache.extend_offset, extend.data(), extend.size() * sizeof(int32_t));
    if (fixed != nullptr) {
        cache.pageable.copy(cache.step_blob, total, cache.stream);
    } else {
        cache.uploader.copy(cache.step_blob, total, cache.stream);
    }
    cache.step_count = count;
    cache.decode_workers = workers;
    cache.first_level_merges = first_level_merges;
    cache.wide_merges = wide_merges;
    cache.merges = static_cast<int32_t>(merges.size());
    cache.prefill_items = prompt_items;
    cache.listed_items = static_cast<int32_t>(listed.size());
    cache.listed_tiles = listed_tiles;
    cache.list_layer_entries = random ? static_cast<size_t>(list_entries) : 0;
    cache.select_jobs = static_cast<int32_t>(select_jobs.size());
    cache.most_candidates = most_candidates;
    cache.touched_blocks = static_cast<int32_t>(touched.size() / 3);
    cache.select_reads_touched = select_reads_touched;
    // The fused append + decode launch needs every token to own its slot (no token may read another token's
    // position of the same step, and each (token, KV head) row appends its own position only) and no prompt run
    // (whose K/V must be in the pages before its attention); listed items read only pages below every member's
    // position. Under KV page activation every append goes first (its blocks' summaries are recomputed before the
    // selection reads them).
    std::vector<int32_t> slots(count);
    for (int32_t index = 0; index < count; ++index) {
        slots[index] = tokens[index].slot;
    }
    std::sort(slots.begin(), slots.end());
    cache.fusable = prompt_items == 0 && std::adjacent_find(slots.begin(), slots.end()) == slots.end() &&
                    activation.enabled == 0;
    cache.step_ready = true;
}

void validate_desc(const SynapseKvDesc& desc) {
    if (desc.rope_cosines == nullptr || desc.rope_sines == nullptr) {
        fail(SYNAPSE_KV_NULL_POINTER, "null pointer: RoPE tables");
    }
    if (desc.layer_count == 0 || desc.heads == 0 || desc.kv_heads == 0 || desc.heads % desc.kv_heads != 0) {
        invalid("layer, head and KV head counts must be positive, heads a multiple of KV heads");
    }
    if (desc.heads / desc.kv_heads > 8) {
        invalid("at most 8 query heads per KV head (MAX_GROUP)");
    }
    if (desc.head_dim != 64 && desc.head_dim != 128) {
        fail(SYNAPSE_KV_UNAVAILABLE, "unavailable: head dimension " + std::to_string(desc.head_dim) +
                                         " (kernels exist for 64 and 128)");
    }
    if (desc.kv_precision != SYNAPSE_KV_F32 && desc.kv_precision != SYNAPSE_KV_F16) {
        invalid("unknown KV precision " + std::to_string(desc.kv_precision));
    }
    if (desc.page_tokens < 64 || desc.page_tokens > 1024 || desc.page_tokens % 64 != 0) {
        invalid("page_tokens must be a multiple of 64 in 64..1024");
    }
    if (desc.kv_growth_positions == 0 || desc.kv_growth_positions % desc.page_tokens != 0) {
        invalid("kv_growth_positions must be a positive multiple of page_tokens");
    }
    if (desc.max_positions == 0 || desc.session_slots == 0 || desc.step_tokens == 0 || desc.max_pages == 0) {
        invalid("max_positions, session_slots, step_tokens and max_pages must be positive");
    }
    if (desc.max_positions > (1u << 30) || desc.max_pages > (1u << 30) || desc.session_slots > (1u << 16)) {
        invalid("max_positions, max_pages or session_slots is too large");
    }
}

void create_cache(const SynapseKvDesc& desc, SynapseKvCache** output) {
    validate_desc(desc);
    int devices = 0;
    if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0) {
        (void)hipGetLastError();
        fail(SYNAPSE_KV_UNAVAILABLE, "unavailable: no HIP device");
    }
    if (desc.device < 0 || desc.device >= devices) {
        invalid("device " + std::to_string(desc.device) + " does not exist");
    }
    auto* cache = new SynapseKvCache();
    try {
        Dims& dims = cache->dims;
        dims.layers = desc.layer_count;
        dims.heads = desc.heads;
        dims.kv_heads = desc.kv_heads;
        dims.head_dim = desc.head_dim;
        dims.max_positions = desc.max_positions;
        dims.growth = desc.kv_growth_positions;
        dims.page_tokens = desc.page_tokens;
        dims.precision = desc.kv_precision;
        dims.slots = desc.session_slots;
        dims.step_tokens = desc.step_tokens;
        dims.max_pages = desc.max_pages;
        dims.pages_per_slot = pages_for(dims, dims.max_positions);
        dims.page_bytes = static_cast<uint64_t>(dims.layers) * 2 * dims.kv_heads * dims.page_tokens * dims.head_dim *
                          (dims.precision == SYNAPSE_KV_F16 ? 2 : 4);
        cache->device = desc.device;
        set_device(*cache);
        cache->capacity.assign(dims.slots, 0);
        cache->length.assign(dims.slots, 0);
        cache->fold_next.assign(dims.slots, -1);
        cache->table.assign(static_cast<size_t>(dims.slots) * dims.pages_per_slot, -1);
        cache->refcount.assign(dims.max_pages, 0);
        cache->free_stack.resize(dims.max_pages);
        for (uint32_t index = 0; index < dims.max_pages; ++index) {
            cache->free_stack[index] = static_cast<int32_t>(dims.max_pages - 1 - index);
        }
        check_hip(hipMalloc(reinterpret_cast<void**>(&cache->pool), dims.page_bytes * dims.max_pages), "page pool");
        cache->block_table.ensure(cache->table.size(), "block table");
        cache->device_refcount.ensure(dims.max_pages, "reference counts");
        cache->device_free.ensure(dims.max_pages, "free stack");
        cache->device_state.ensure(4, "allocator state");
        cache->fresh.ensure(dims.max_pages, "fresh page list");
        cache->copies.ensure(2ull * dims.max_pages, "copy list");
        const size_t rope = static_cast<size_t>(dims.max_positions) * (dims.head_dim / 2);
        cache->cosines.ensure(rope, "RoPE cosines");
        cache->sines.ensure(rope, "RoPE sines");
        check_hip(hipMemcpy(cache->block_table.pointer, cache->table.data(), cache->table.size() * 4,
                            hipMemcpyHostToDevice), "block table upload");
        check_hip(hipMemcpy(cache->device_refcount.pointer, cache->refcount.data(), dims.max_pages * 4ull,
                            hipMemcpyHostToDevice), "reference count upload");
        check_hip(hipMemcpy(cache->device_free.pointer, cache->free_stack.data(), dims.max_pages * 4ull,
                            hipMemcpyHostToDevice), "free stack upload");
        const int32_t state[4] = {static_cast<int32_t>(dims.max_pages), 0, 0, 0};
        check_hip(hipMemcpy(cache->device_state.pointer, state, sizeof(state), hipMemcpyHostToDevice), "state upload");
        check_hip(hipMemcpy(cache->cosines.pointer, desc.rope_cosines, rope * 4, hipMemcpyHostToDevice), "RoPE upload");
        check_hip(hipMemcpy(cache->sines.pointer, desc.rope_sines, rope * 4, hipMemcpyHostToDevice), "RoPE upload");
        cache->decode_waves =
            decode_resident_waves(cache->device, dims.precision == SYNAPSE_KV_F16, dims.head_dim, cache->prefetch != 0);
        cache->prefill_slots =
            prefill_resident_blocks(cache->device, static_cast<int>(dims.head_dim), static_cast<int>(dims.heads / dims.kv_heads));
    } catch (...) {
        delete cache;
        throw;
    }
    *output = cache;
}

// Growth and copy-on-write of a step in the restatement's order; throws before mutating on any failure.
void prepare_step(SynapseKvCache& cache, const SynapseKvBatchToken* tokens, int32_t count) {
    const Dims& dims = cache.dims;
    std::vector<uint32_t> needed(dims.slots, 0);
    for (int32_t index = 0; index < count; ++index) {
        const SynapseKvBatchToken& token = tokens[index];
        if (token.slot < 0 || static_cast<uint32_t>(token.slot) >= dims.slots || token.position < 0 ||
            static_cast<uint32_t>(token.position) >= dims.max_positions) {
            invalid("batch token " + std::to_string(index) + " (slot " + std::to_string(token.slot) + ", position " +
                    std::to_string(token.position) + ") is out of range");
        }
        needed[token.slot] = std::max<uint32_t>(needed[token.slot], static_cast<uint32_t>(token.position) + 1);
    }
    // Contiguity (PagedKvCache::append, kv_pages.rs:98-100, rejects a position past the length): the positions at
    // or past a slot's length must fill [length, new length) without a gap, so attention never reads a row no
    // token wrote. Positions below the length overwrite (speculation rollback: truncate, then rewrite).
    {
        std::vector<std::vector<uint32_t>> beyond(dims.slots);
        for (int32_t index = 0; index < count; ++index) {
            const SynapseKvBatchToken& token = tokens[index];
            if (static_cast<uint32_t>(token.position) >= cache.length[token.slot]) {
                beyond[token.slot].push_back(static_cast<uint32_t>(token.position));
            }
        }
        for (uint32_t slot = 0; slot < dims.slots; ++slot) {
            auto& positions = beyond[slot];
            std::sort(positions.begin(), positions.end());
            positions.erase(std::unique(positions.begin(), positions.end()), positions.end());
            if (!positions.empty() && positions.size() != needed[slot] - cache.length[slot]) {
                invalid("slot " + std::to_string(slot) + " has length " + std::to_string(cache.length[slot]) +
                        ": the step's positions from there must be contiguous (position " +
                        std::to_string(needed[slot] - 1) + " leaves a gap)");
            }
        }
    }
    std::vector<uint32_t> grown(dims.slots);
    size_t pops = 0;
    for (uint32_t slot = 0; slot < dims.slots; ++slot) {
        grown[slot] = cache.capacity[slot];
        if (needed[slot] > cache.capacity[slot]) {
            grown[slot] = next_capacity(needed[slot], cache.capacity[slot], dims.growth, dims.max_positions);
            pops += pages_for(dims, grown[slot]) - pages_for(dims, cache.capacity[slot]);
        }
    }
    {
        std::vector<int32_t> references;
        std::vector<std::pair<uint32_t, uint32_t>> owned;
        for (int32_t index = 0; index < count; ++index) {
            const uint32_t slot = static_cast<uint32_t>(tokens[index].slot);
            const uint32_t page = static_cast<uint32_t>(tokens[index].position) / dims.page_tokens;
            if (page >= pages_for(dims, cache.capacity[slot])) {
                continue;
            }
            const int32_t id = slot_page(cache, slot, page);
            if (cache.refcount[id] <= 1) {
                continue;
            }
            if (references.empty()) {
                references = cache.refcount;
            }
            const auto key = std::make_pair(slot, page);
            if (std::find(owned.begin(), owned.end(), key) == owned.end() && references[id] > 1) {
                --references[id];
                ++pops;
                owned.push_back(key);
            }
        }
    }
    if (pops > cache.free_stack.size()) {
        fail(SYNAPSE_KV_OUT_OF_MEMORY, "out of device memory: the step needs " + std::to_string(pops) +
                                           " pages and " + std::to_string(cache.free_stack.size()) + " are free");
    }
    for (uint32_t slot = 0; slot < dims.slots; ++slot) {
        if (grown[slot] != cache.capacity[slot]) {
            shadow_resize(cache, slot, grown[slot]);
        }
    }
    for (int32_t index = 0; index < count; ++index) {
        const uint32_t slot = static_cast<uint32_t>(tokens[index].slot);
        const uint32_t page = static_cast<uint32_t>(tokens[index].position) / dims.page_tokens;
        int32_t& entry = slot_page(cache, slot, page);
        if (cache.refcount[entry] > 1) {
            const int32_t fresh = cache.free_stack.back();
            cache.free_stack.pop_back();
            cache.refcount[fresh] = 1;
            --cache.refcount[entry];
            entry = fresh;
            cache.ops.push_back(TableOp{kOpCow, static_cast<int32_t>(slot), static_cast<int32_t>(page),
                                        cache.copy_count, 0, {0, 0, 0}});
            ++cache.copy_count;
        }
    }
    for (uint32_t slot = 0; slot < dims.slots; ++slot) {
        cache.length[slot] = std::max(cache.length[slot], needed[slot]);
    }
}

void require_step(const SynapseKvCache& cache, uint32_t layer) {
    if (!cache.step_ready) {
        invalid("no prepared step: call synapse_kv_step first");
    }
    if (layer >= cache.dims.layers) {
        invalid("layer " + std::to_string(layer) + " is outside 0.." + std::to_string(cache.dims.layers - 1));
    }
}

// The step's appends for one layer; under KV page activation the written blocks' summaries follow (a summary
// launch) unless `defer_summaries` (the caller's selection launch carries them).
void launch_append_layer(SynapseKvCache& cache, uint32_t layer, float* qkv, uint32_t qkv_stride, bool write_back,
                         bool defer_summaries = false) {
    const Dims& dims = cache.dims;
    AppendArgs args{};
    args.geo = geometry(cache, layer);
    args.pool = cache.pool;
    args.tokens = reinterpret_cast<const SynapseKvBatchToken*>(cache.step_blob + cache.tokens_offset);
    args.qkv = qkv;
    args.qkv_stride = static_cast<int32_t>(qkv_stride);
    args.half_dim = static_cast<int32_t>(dims.head_dim / 2);
    args.cosines = cache.cosines.pointer;
    args.sines = cache.sines.pointer;
    args.write_back = write_back ? 1 : 0;
    if (cache.activation.enabled != 0) {
        args.summaries = cache.summaries.pointer;
        args.summary_page_bytes = cache.summary_page_bytes;
        args.extend = reinterpret_cast<const int32_t*>(cache.step_blob + cache.extend_offset);
    }
    check_hip(launch_append(launch_for(cache, SYNAPSE_KV_KERNEL_APPEND, cache.step_count > 0), args, cache.step_count,
                            dims.precision == SYNAPSE_KV_F16),
              "append");
    if (cache.activation.enabled != 0 && cache.touched_blocks > 0 && !defer_summaries) {
        SummaryArgs summary{};
        summary.geo = args.geo;
        summary.summaries = cache.summaries.pointer;
        summary.summary_page_bytes = cache.summary_page_bytes;
        summary.blocks = reinterpret_cast<const int32_t*>(cache.step_blob + cache.touched_offset);
        summary.count = cache.touched_blocks;
        summary.first_layer = static_cast<int32_t>(layer);
        summary.layers = 1;
        check_hip(launch_summaries(launch_for(cache, SYNAPSE_KV_KERNEL_APPEND, summary.count > 0), summary,
                                   dims.precision == SYNAPSE_KV_F16),
                  "key summaries");
    }
}

// Attention of the prepared step for one layer; with `append`, the step's K/V are appended first (fused into the
// decode launch when the step allows it).
void run_attention(SynapseKvCache& cache, uint32_t layer, const float* qkv, uint32_t qkv_stride, float* output,
                   uint32_t out_stride, bool append) {
    require_step(cache, layer);
    const Dims& dims = cache.dims;
    const uint32_t needed = (append ? dims.heads + 2 * dims.kv_heads : dims.heads) * dims.head_dim;
    if (qkv_stride < needed || qkv_stride % 4 != 0) {
        invalid("qkv_stride must be a multiple of 4 and hold the row's " + std::to_string(needed) + " values");
    }
    if (out_stride < dims.heads * dims.head_dim) {
        invalid("out_stride is shorter than heads * head_dim");
    }
    if (reinterpret_cast<uintptr_t>(qkv) % 16 != 0) {
        invalid("qkv must be 16-byte aligned");
    }
    set_device(cache);
    check_device_pointer(cache, qkv, "qkv");
    check_device_pointer(cache, output, "output");
    // With `append`, qkv stays as the caller wrote it: K is rotated on its way into the pages and Q in registers.
    const bool fused = append && cache.fusable;
    // Under KV page activation the appended blocks' summaries ride along in the selection launch when no selection
    // reads them.
    const bool carry_summaries = append && cache.activation.enabled != 0 && cache.select_jobs > 0 &&
                                 !cache.select_reads_touched;
    if (append && !fused) {
        launch_append_layer(cache, layer, const_cast<float*>(qkv), qkv_stride, false, carry_summaries);
    }
    AttentionArgs args{};
    args.geo = geometry(cache, layer);
    args.tokens = reinterpret_cast<const SynapseKvBatchToken*>(cache.step_blob + cache.tokens_offset);
    args.qkv = qkv;
    args.qkv_stride = static_cast<int32_t>(qkv_stride);
    args.output = output;
    args.out_stride = static_cast<int32_t>(out_stride);
    args.scale_log2 = 1.4426950408889634f / std::sqrt(static_cast<float>(dims.head_dim));
    args.rotate = append ? 1 : 0;
    args.append = fused ? 1 : 0;
    args.cosines = cache.cosines.pointer;
    args.sines = cache.sines.pointer;
    args.workers = cache.decode_workers;
    args.members = reinterpret_cast<const int32_t*>(cache.step_blob + cache.members_offset);
    args.segments = reinterpret_cast<const DecodeSegment*>(cache.step_blob + cache.segments_offset);
    args.merges = reinterpret_cast<const MergeItem*>(cache.step_blob + cache.merges_offset);
    args.prefill = reinterpret_cast<const PrefillItem*>(cache.step_blob + cache.prefill_offset);
    args.partial_out = cache.step_partial_out;
    args.partial_ml = cache.step_partial_ml;
    int32_t* lists = reinterpret_cast<int32_t*>(cache.step_blob + cache.lists_offset) +
                     static_cast<size_t>(layer) * cache.list_layer_entries;
    args.lists = lists;
    const bool fp16 = dims.precision == SYNAPSE_KV_F16;
    if (cache.select_jobs > 0) {
        SelectArgs select{};
        select.geo = args.geo;
        select.tokens = args.tokens;
        select.qkv = qkv;
        select.qkv_stride = static_cast<int32_t>(qkv_stride);
        select.rotate = args.rotate;
        select.cosines = cache.cosines.pointer;
        select.sines = cache.sines.pointer;
        select.summaries = cache.summaries.pointer;
        select.summary_page_bytes = cache.summary_page_bytes;
        select.jobs = reinterpret_cast<const SelectJob*>(cache.step_blob + cache.select_offset);
        select.lists = lists;
        select.keys = cache.select_keys.pointer;
        select.key_stride = static_cast<int32_t>(select_key_stride(cache, cache.most_candidates));
        select.budget = static_cast<int32_t>(cache.activation.budget_pages);
        select.job_count = cache.select_jobs;
        if (carry_summaries) {
            select.summary_out = cache.summaries.pointer;
            select.summary_blocks = reinterpret_cast<const int32_t*>(cache.step_blob + cache.touched_offset);
            select.summary_count = cache.touched_blocks;
        }
        check_hip(launch_select(launch_for(cache, SYNAPSE_KV_KERNEL_PAGE_SELECT, true), select, cache.most_candidates,
                                fp16),
                  "page selection");
    }
    const int prompt_items = cache.prefill_items;
    const int listed_items = cache.listed_items;
    if (cache.listed_tiles == 1) {
        check_hip(launch_prefill(launch_for(cache, SYNAPSE_KV_KERNEL_PREFILL, prompt_items > 0), args, 0, prompt_items,
                                 kPrefillTiles, fp16),
                  "prefill attention");
        check_hip(launch_prefill(launch_for(cache, SYNAPSE_KV_KERNEL_PREFILL, listed_items > 0), args, prompt_items,
                                 listed_items, 1, fp16),
                  "shared-prefix attention");
    } else {
        check_hip(launch_prefill(launch_for(cache, SYNAPSE_KV_KERNEL_PREFILL, prompt_items + listed_items > 0), args, 0,
                                 prompt_items + listed_items, kPrefillTiles, fp16),
                  "prefill attention");
    }
    const int timed = args.workers > 0 ? cache.timing_armed : -1;
    if (timed >= 0) {
        args.timing = cache.timing[timed].device + static_cast<size_t>(cache.timing[timed].launches) * SplitTiming::kWorkers;
    }
    check_hip(launch_decode(launch_for(cache, SYNAPSE_KV_KERNEL_DECODE, args.workers > 0), args, fp16, cache.prefetch != 0),
              "decode attention");
    if (timed >= 0) {
        SplitTiming& timing = cache.timing[timed];
        check_hip(hipEventRecord(timing.done, cache.stream), "split timing event");
        timing.pending = true;
        if (++timing.launches == SplitTiming::kLaunches) {
            cache.timing_armed = -1;
        }
    }
    const int first_level = cache.first_level_merges;
    if (first_level > 0) {
        check_hip(launch_merge(launch_for(cache, SYNAPSE_KV_KERNEL_MERGE, true), args, 0, first_level, false),
                  "split merge");
    }
    const int wide = cache.wide_merges;
    const int final_level = cache.merges - first_level - wide;
    check_hip(launch_merge(launch_for(cache, SYNAPSE_KV_KERNEL_MERGE, final_level > 0), args, first_level, final_level,
                           false),
              "split merge");
    if (wide > 0) {
        check_hip(launch_merge(launch_for(cache, SYNAPSE_KV_KERNEL_MERGE, true), args, first_level + final_level, wide,
                               true),
                  "split merge");
    }
}

}  // namespace
}  // namespace synapse_kv

using namespace synapse_kv;

namespace synapse_kv {
bool cache_fused_sums(const SynapseKvCache& cache) { return cache.fused_sums != 0; }
}  // namespace synapse_kv

extern "C" {

uint32_t synapse_kv_abi_version(void) { return SYNAPSE_KV_ABI_VERSION; }

int32_t synapse_kv_probe(SynapseKvDeviceInfo* info) {
    if (info == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: device info");
    }
    return guarded([&] {
        int devices = 0;
        if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0) {
            (void)hipGetLastError();
            fail(SYNAPSE_KV_UNAVAILABLE, "unavailable: no HIP device");
        }
        int device = 0;
        check_hip(hipGetDevice(&device), "current device");
        hipDeviceProp_t properties{};
        check_hip(hipGetDeviceProperties(&properties, device), "device properties");
        SynapseKvDeviceInfo described{};
        std::string name = properties.name;
        if (std::strlen(properties.gcnArchName) != 0) {
            name += std::string(" (") + properties.gcnArchName + ")";
        }
        std::memcpy(described.name, name.data(), std::min<size_t>(name.size(), sizeof(described.name) - 1));
        described.recommended_working_set_bytes = properties.totalGlobalMem;
        described.max_buffer_bytes = properties.totalGlobalMem;
        described.unified_memory = properties.integrated ? 1 : 0;
        described.apple_family = 0;
        *info = described;
    });
}

size_t synapse_kv_last_error(uint8_t* buffer, size_t capacity) {
    const std::string& message = g_last_error;
    if (buffer != nullptr) {
        std::memcpy(buffer, message.data(), std::min(capacity, message.size()));
    }
    return message.size();
}

int32_t synapse_kv_cache_create(const SynapseKvDesc* desc, SynapseKvCache** cache) {
    if (desc == nullptr || cache == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache description or output");
    }
    return guarded([&] { create_cache(*desc, cache); });
}

void synapse_kv_cache_destroy(SynapseKvCache* cache) { delete cache; }

int32_t synapse_kv_set_stream(SynapseKvCache* cache, void* stream) {
    if (cache == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache");
    }
    return guarded([&] {
        set_device(*cache);
        check_hip(hipStreamSynchronize(cache->stream), "stream switch");
        cache->stream = static_cast<hipStream_t>(stream);
    });
}

int32_t synapse_kv_set_option(SynapseKvCache* cache, uint32_t option, uint32_t value) {
    if (cache == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache");
    }
    return guarded([&] {
        if (option == SYNAPSE_KV_OPTION_SPLIT_KEYS) {
            if (value == 0 || value % kStepKeys != 0) {
                invalid("decode split keys must be a positive multiple of 64");
            }
            cache->split_keys = value;
        } else if (option == SYNAPSE_KV_OPTION_PREFILL_RUNS) {
            cache->prefill_runs = value != 0 ? 1 : 0;
        } else if (option == SYNAPSE_KV_OPTION_PROFILE_EVERY) {
            if (value == 0) {
                invalid("profile sampling must be at least 1");
            }
            cache->profile_every = value;
        } else if (option == SYNAPSE_KV_OPTION_DECODE_PREFETCH) {
            cache->prefetch = value != 0 ? 1 : 0;
            cache->decode_waves = decode_resident_waves(cache->device, cache->dims.precision == SYNAPSE_KV_F16,
                                                        cache->dims.head_dim, cache->prefetch != 0);
        } else if (option == SYNAPSE_KV_OPTION_SHARED_PREFIX) {
            cache->shared_prefix = value != 0 ? 1 : 0;
        } else if (option == SYNAPSE_KV_OPTION_FUSED_SUMS) {
            cache->fused_sums = value != 0 ? 1 : 0;
        } else if (option == SYNAPSE_KV_OPTION_SEGMENT_COST) {
            if (value > 64) {
                invalid("the segment cost is 0..64 quarter steps");
            }
            cache->segment_cost = value;
        } else if (option == SYNAPSE_KV_OPTION_ADAPTIVE_SPLIT) {
            if (value != 0) {
                cache->timing[0].allocate();
                cache->timing[1].allocate();
            } else {
                std::fill(std::begin(cache->xcd_speed), std::end(cache->xcd_speed), 1.0);
            }
            cache->adaptive_split = value != 0 ? 1 : 0;
        } else if (option == SYNAPSE_KV_OPTION_PREFILL_SPLIT_KEYS) {
            if (value % kStepKeys != 0) {
                invalid("prefill split keys must be 0 (automatic) or a multiple of 64");
            }
            cache->prefill_split_keys = value;
        } else {
            invalid("unknown option " + std::to_string(option));
        }
        cache->step_ready = false;
    });
}

uint64_t synapse_kv_bytes(const SynapseKvCache* cache) {
    if (cache == nullptr) {
        return 0;
    }
    const uint64_t used = cache->dims.max_pages - cache->free_stack.size();
    return used * cache->dims.page_bytes;
}

int32_t synapse_kv_reserve(SynapseKvCache* cache, uint32_t slot, uint32_t positions) {
    if (cache == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache");
    }
    return guarded([&] {
        check_slot(*cache, slot);
        const Dims& dims = cache->dims;
        if (positions > dims.max_positions) {
            invalid("reserve needs at most the context positions (" + std::to_string(dims.max_positions) + ")");
        }
        const uint32_t current = cache->capacity[slot];
        const uint32_t rounded = reserve_rounded(positions, dims.growth, dims.max_positions);
        if (positions > current || (rounded < current && rounded <= current / 4)) {
            const uint32_t need = pages_for(dims, rounded) > pages_for(dims, current)
                                      ? pages_for(dims, rounded) - pages_for(dims, current)
                                      : 0;
            if (need > cache->free_stack.size()) {
                fail(SYNAPSE_KV_OUT_OF_MEMORY, "out of device memory: reserve needs " + std::to_string(need) +
                                                   " pages and " + std::to_string(cache->free_stack.size()) +
                                                   " are free");
            }
            set_device(*cache);
            shadow_resize(*cache, slot, rounded);
            flush_ops(*cache);
        }
    });
}

int32_t synapse_kv_release(SynapseKvCache* cache, uint32_t slot) {
    if (cache == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache");
    }
    return guarded([&] {
        check_slot(*cache, slot);
        set_device(*cache);
        shadow_resize(*cache, slot, 0);
        cache->length[slot] = 0;
        cache->fold_next[slot] = -1;
        flush_ops(*cache);
    });
}

int32_t synapse_kv_truncate(SynapseKvCache* cache, uint32_t slot, uint32_t length) {
    if (cache == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache");
    }
    return guarded([&] {
        check_slot(*cache, slot);
        if (length > cache->length[slot]) {
            invalid("truncate target " + std::to_string(length) + " is beyond the written length " +
                    std::to_string(cache->length[slot]));
        }
        cache->length[slot] = length;
        cache->fold_next[slot] = -1;  // the block summary covers keys past the new length: recompute on the next write
    });
}

int32_t synapse_kv_fork(SynapseKvCache* cache, uint32_t source, uint32_t target) {
    if (cache == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache");
    }
    return guarded([&] {
        check_slot(*cache, source);
        check_slot(*cache, target);
        if (source == target || cache->capacity[target] != 0) {
            invalid("fork needs a different, empty target slot");
        }
        const Dims& dims = cache->dims;
        const uint32_t shared = pages_for(dims, cache->length[source]);
        for (uint32_t page = 0; page < shared; ++page) {
            const int32_t id = slot_page(*cache, source, page);
            slot_page(*cache, target, page) = id;
            ++cache->refcount[id];
        }
        cache->capacity[target] = std::min(dims.max_positions, shared * dims.page_tokens);
        cache->length[target] = cache->length[source];
        cache->fold_next[target] = -1;
        if (shared != 0) {
            set_device(*cache);
            cache->ops.push_back(TableOp{kOpFork, static_cast<int32_t>(source), static_cast<int32_t>(target),
                                         static_cast<int32_t>(shared), 0, {0, 0, 0}});
            flush_ops(*cache);
        }
    });
}

int32_t synapse_kv_step_prompt(SynapseKvCache* cache, const SynapseKvBatchToken* tokens, size_t count,
                               size_t prompt_start) {
    if (cache == nullptr || tokens == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache or tokens");
    }
    return guarded([&] {
        if (count == 0 || count > cache->dims.step_tokens) {
            invalid("a step holds 1.." + std::to_string(cache->dims.step_tokens) + " tokens");
        }
        if (prompt_start > count) {
            invalid("prompt_start is past the step's last token");
        }
        set_device(*cache);
        cache->step_ready = false;
        const std::vector<uint32_t> old_lengths = cache->length;
        prepare_step(*cache, tokens, static_cast<int32_t>(count));
        flush_ops(*cache);
        cache->prompt_start = static_cast<int32_t>(prompt_start);
        plan_step(*cache, tokens, static_cast<int32_t>(count), old_lengths);
    });
}

int32_t synapse_kv_step(SynapseKvCache* cache, const SynapseKvBatchToken* tokens, size_t count) {
    return synapse_kv_step_prompt(cache, tokens, count, count);
}

int32_t synapse_kv_step_static(SynapseKvCache* cache, const SynapseKvBatchToken* tokens, size_t count,
                               size_t prompt_start) {
    if (cache == nullptr || tokens == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache or tokens");
    }
    return guarded([&] {
        if (count == 0 || count > cache->dims.step_tokens) {
            invalid("a step holds 1.." + std::to_string(cache->dims.step_tokens) + " tokens");
        }
        if (prompt_start > count) {
            invalid("prompt_start is past the step's last token");
        }
        if (cache->activation.enabled != 0) {
            fail(SYNAPSE_KV_UNAVAILABLE, "synapse_kv_step_static does not run KV page activation");
        }
        set_device(*cache);
        uint8_t* base = scratch_address(cache->device);
        cache->step_ready = false;
        // Everything the step changes on the host before its first device work, restored when the step fails
        // (out of pages, or more scratch than there is), so a rejected step changes nothing.
        const std::vector<uint32_t> old_lengths = cache->length;
        const std::vector<uint32_t> old_capacity = cache->capacity;
        const std::vector<int32_t> old_table = cache->table;
        const std::vector<int32_t> old_refcount = cache->refcount;
        const std::vector<int32_t> old_free = cache->free_stack;
        const std::vector<TableOp> old_ops = cache->ops;
        const int32_t old_fresh = cache->fresh_count;
        const int32_t old_copies = cache->copy_count;
        const int32_t old_prompt_start = cache->prompt_start;
        size_t ops_bytes = 0;
        try {
            prepare_step(*cache, tokens, static_cast<int32_t>(count));
            ops_bytes = align_up(cache->ops.size() * sizeof(TableOp), 256);
            if (ops_bytes >= SYNAPSE_KV_STATIC_SCRATCH_BYTES) {
                invalid("the step's table operations do not fit SYNAPSE_KV_STATIC_SCRATCH_BYTES");
            }
            cache->prompt_start = static_cast<int32_t>(prompt_start);
            const FixedMemory fixed{base + ops_bytes, SYNAPSE_KV_STATIC_SCRATCH_BYTES - ops_bytes};
            plan_step(*cache, tokens, static_cast<int32_t>(count), old_lengths, &fixed);
        } catch (...) {
            cache->length = old_lengths;
            cache->capacity = old_capacity;
            cache->table = old_table;
            cache->refcount = old_refcount;
            cache->free_stack = old_free;
            cache->ops = old_ops;
            cache->fresh_count = old_fresh;
            cache->copy_count = old_copies;
            cache->prompt_start = old_prompt_start;
            cache->step_ready = false;
            throw;
        }
        flush_ops(*cache, base);
    });
}

int32_t synapse_kv_set_page_activation(SynapseKvCache* cache, const SynapseKvPageActivation* activation) {
    if (cache == nullptr || activation == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache or activation");
    }
    return guarded([&] {
        const SynapseKvPageActivation wanted = *activation;
        if (wanted.enabled != 0) {
            // KvPageActivation.Validate (KvPageActivation.cs:23-37).
            if (wanted.page_tokens != 16 && wanted.page_tokens != 32 && wanted.page_tokens != 64) {
                invalid("KV pages hold 16, 32, or 64 positions");
            }
            if (wanted.selection != SYNAPSE_KV_SELECT_KEY_BOUND && wanted.selection != SYNAPSE_KV_SELECT_RANDOM) {
                invalid("unknown KV page selection " + std::to_string(wanted.selection));
            }
            if (wanted.budget_pages > INT32_MAX || wanted.window_tokens > INT32_MAX) {
                invalid("budget_pages and window_tokens must be non-negative 32-bit integers");
            }
        }
        set_device(*cache);
        cache->step_ready = false;
        // Summaries are rebuilt when activation is switched on or its page size changes.
        const bool rebuild = wanted.enabled != 0 && (cache->activation.enabled == 0 ||
                                                     static_cast<int32_t>(wanted.page_tokens) != cache->summary_keys);
        if (rebuild) {
            const Dims& dims = cache->dims;
            cache->summary_keys = static_cast<int32_t>(wanted.page_tokens);
            cache->summary_page_bytes =
                summary_page_elements(dims.layers, dims.kv_heads, dims.page_tokens, dims.head_dim, cache->summary_keys) *
                (dims.precision == SYNAPSE_KV_F16 ? 2 : 4);
            cache->summaries.ensure(cache->summary_page_bytes * dims.max_pages, "key summaries");
        }
        if (rebuild) {
            // Summaries of every block of every mapped page, all layers; fold chains start again at block starts.
            std::fill(cache->fold_next.begin(), cache->fold_next.end(), -1);
            const Dims& dims = cache->dims;
            std::vector<int32_t> blocks;
            for (uint32_t page = 0; page < dims.max_pages; ++page) {
                if (cache->refcount[page] > 0) {
                    for (int32_t block = 0; block < static_cast<int32_t>(dims.page_tokens) / cache->summary_keys; ++block) {
                        blocks.push_back(static_cast<int32_t>(page));
                        blocks.push_back(block);
                        blocks.push_back(cache->summary_keys);
                    }
                }
            }
            if (!blocks.empty()) {
                const size_t bytes = blocks.size() * sizeof(int32_t);
                cache->op_blob.ensure(bytes, "operation buffer");
                void* staging = cache->uploader.acquire(bytes);
                std::memcpy(staging, blocks.data(), bytes);
                cache->uploader.copy(cache->op_blob.pointer, bytes, cache->stream);
                SummaryArgs summary{};
                summary.geo = geometry(*cache, 0);
                summary.summaries = cache->summaries.pointer;
                summary.summary_page_bytes = cache->summary_page_bytes;
                summary.blocks = reinterpret_cast<const int32_t*>(cache->op_blob.pointer);
                summary.count = static_cast<int32_t>(blocks.size() / 3);
                summary.first_layer = 0;
                summary.layers = static_cast<int32_t>(dims.layers);
                check_hip(launch_summaries(launch_for(*cache, SYNAPSE_KV_KERNEL_APPEND, true), summary,
                                           dims.precision == SYNAPSE_KV_F16),
                          "key summaries");
            }
        }
        cache->activation = wanted;
    });
}

int32_t synapse_kv_append_rope(SynapseKvCache* cache, uint32_t layer, float* qkv, uint32_t qkv_stride) {
    if (cache == nullptr || qkv == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache or qkv");
    }
    return guarded([&] {
        require_step(*cache, layer);
        const Dims& dims = cache->dims;
        if (qkv_stride < (dims.heads + 2 * dims.kv_heads) * dims.head_dim) {
            invalid("qkv_stride is shorter than (heads + 2 * kv_heads) * head_dim");
        }
        set_device(*cache);
        check_device_pointer(*cache, qkv, "qkv");
        launch_append_layer(*cache, layer, qkv, qkv_stride, true);
    });
}

int32_t synapse_kv_attention(SynapseKvCache* cache, uint32_t layer, const float* qkv, uint32_t qkv_stride,
                             float* output, uint32_t out_stride) {
    if (cache == nullptr || qkv == nullptr || output == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache, qkv or output");
    }
    return guarded([&] { run_attention(*cache, layer, qkv, qkv_stride, output, out_stride, false); });
}

int32_t synapse_kv_append_attention(SynapseKvCache* cache, uint32_t layer, const float* qkv, uint32_t qkv_stride,
                                    float* output, uint32_t out_stride) {
    if (cache == nullptr || qkv == nullptr || output == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache, qkv or output");
    }
    return guarded([&] { run_attention(*cache, layer, qkv, qkv_stride, output, out_stride, true); });
}

int32_t synapse_kv_profile_begin(SynapseKvCache* cache) {
    if (cache == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache");
    }
    return guarded([&] {
        cache->profiled.clear();
        std::fill(std::begin(cache->profile_seen), std::end(cache->profile_seen), 0);
        // Event pairs are created here rather than at a sampled launch, which would put event creation inside the
        // timed work; launch_for adds more only when a profile outgrows the pool.
        while (cache->event_pool.size() < kProfileEvents) {
            hipEvent_t start = nullptr;
            hipEvent_t stop = nullptr;
            check_hip(hipEventCreate(&start), "profile event");
            if (hipEventCreate(&stop) != hipSuccess) {
                (void)hipEventDestroy(start);
                check_hip(hipErrorOutOfMemory, "profile event");
            }
            cache->event_pool.emplace_back(start, stop);
        }
        cache->profiling = true;
    });
}

int32_t synapse_kv_profile_end(SynapseKvCache* cache, SynapseKvProfile* profile) {
    if (cache == nullptr || profile == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache or profile");
    }
    return guarded([&] {
        set_device(*cache);
        cache->profiling = false;
        check_hip(hipStreamSynchronize(cache->stream), "synchronize");
        SynapseKvProfile out{};
        for (const auto& [kind, index] : cache->profiled) {
            float milliseconds = 0.0f;
            const auto& pair = cache->event_pool[index];
            check_hip(hipEventElapsedTime(&milliseconds, pair.first, pair.second), "profile read");
            out.launches[kind] += 1;
            out.milliseconds[kind] += milliseconds;
        }
        cache->profiled.clear();
        *profile = out;
    });
}

int32_t synapse_kv_synchronize(SynapseKvCache* cache) {
    if (cache == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache");
    }
    return guarded([&] {
        set_device(*cache);
        check_hip(hipStreamSynchronize(cache->stream), "synchronize");
    });
}

int32_t synapse_kv_slot_info(const SynapseKvCache* cache, uint32_t slot, uint32_t* capacity, uint32_t* length,
                             uint32_t* pages) {
    if (cache == nullptr || capacity == nullptr || length == nullptr || pages == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache or output");
    }
    return guarded([&] {
        check_slot(*cache, slot);
        *capacity = cache->capacity[slot];
        *length = cache->length[slot];
        *pages = pages_for(cache->dims, cache->capacity[slot]);
    });
}

int32_t synapse_kv_read_block_table(SynapseKvCache* cache, uint32_t slot, int32_t* pages, size_t capacity,
                                    size_t* count) {
    if (cache == nullptr || pages == nullptr || count == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache or output");
    }
    return guarded([&] {
        check_slot(*cache, slot);
        const size_t entries = cache->dims.pages_per_slot;
        if (capacity < entries) {
            invalid("the output holds fewer entries than pages_per_slot (" + std::to_string(entries) + ")");
        }
        set_device(*cache);
        check_hip(hipStreamSynchronize(cache->stream), "synchronize");
        check_hip(hipMemcpy(pages, cache->block_table.pointer + static_cast<size_t>(slot) * entries, entries * 4,
                            hipMemcpyDeviceToHost), "block table read");
        *count = entries;
    });
}

int32_t synapse_kv_read_refcounts(SynapseKvCache* cache, int32_t* counts, size_t capacity) {
    if (cache == nullptr || counts == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache or output");
    }
    return guarded([&] {
        if (capacity < cache->dims.max_pages) {
            invalid("the output holds fewer entries than max_pages");
        }
        set_device(*cache);
        check_hip(hipStreamSynchronize(cache->stream), "synchronize");
        check_hip(hipMemcpy(counts, cache->device_refcount.pointer, cache->dims.max_pages * 4ull, hipMemcpyDeviceToHost),
                  "reference count read");
    });
}

int32_t synapse_kv_read_free_list(SynapseKvCache* cache, int32_t* pages, size_t capacity, size_t* count) {
    if (cache == nullptr || pages == nullptr || count == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache or output");
    }
    return guarded([&] {
        set_device(*cache);
        check_hip(hipStreamSynchronize(cache->stream), "synchronize");
        int32_t state[4] = {0, 0, 0, 0};
        check_hip(hipMemcpy(state, cache->device_state.pointer, sizeof(state), hipMemcpyDeviceToHost), "state read");
        const size_t entries = static_cast<size_t>(std::max(0, state[0]));
        if (capacity < entries) {
            invalid("the output holds fewer entries than the free stack");
        }
        check_hip(hipMemcpy(pages, cache->device_free.pointer, entries * 4, hipMemcpyDeviceToHost), "free stack read");
        *count = entries;
    });
}

int32_t synapse_kv_page_stats(SynapseKvCache* cache, SynapseKvPageStats* stats) {
    if (cache == nullptr || stats == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache or output");
    }
    return guarded([&] {
        set_device(*cache);
        check_hip(hipStreamSynchronize(cache->stream), "synchronize");
        int32_t state[4] = {0, 0, 0, 0};
        check_hip(hipMemcpy(state, cache->device_state.pointer, sizeof(state), hipMemcpyDeviceToHost), "state read");
        SynapseKvPageStats out{};
        out.max_pages = cache->dims.max_pages;
        out.free_pages = static_cast<uint32_t>(cache->free_stack.size());
        out.used_pages = out.max_pages - out.free_pages;
        for (int32_t count : cache->refcount) {
            out.shared_pages += count > 1 ? 1 : 0;
        }
        out.page_bytes = cache->dims.page_bytes;
        out.kv_bytes = static_cast<uint64_t>(out.used_pages) * out.page_bytes;
        out.device_status = static_cast<uint32_t>(state[1]);
        if (state[0] != static_cast<int32_t>(out.free_pages) && out.device_status == 0) {
            out.device_status = 3;  // device free count differs from the host shadow
        }
        *stats = out;
    });
}

int32_t synapse_kv_read_kv(SynapseKvCache* cache, uint32_t slot, uint32_t layer, uint32_t first, uint32_t count,
                           void* keys, void* values) {
    if (cache == nullptr || keys == nullptr || values == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache or output");
    }
    return guarded([&] {
        check_slot(*cache, slot);
        const Dims& dims = cache->dims;
        if (layer >= dims.layers) {
            invalid("layer out of range");
        }
        if (static_cast<uint64_t>(first) + count > cache->capacity[slot]) {
            invalid("positions beyond the slot capacity");
        }
        if (count == 0) {
            return;
        }
        set_device(*cache);
        const size_t element = dims.precision == SYNAPSE_KV_F16 ? 2 : 4;
        const size_t bytes = static_cast<size_t>(count) * dims.kv_heads * dims.head_dim * element;
        DeviceBuffer<uint8_t> staging;
        staging.ensure(2 * bytes, "read staging");
        GatherArgs args{};
        args.geo = geometry(*cache, layer);
        args.slot = static_cast<int32_t>(slot);
        args.first = static_cast<int32_t>(first);
        args.count = static_cast<int32_t>(count);
        args.keys = staging.pointer;
        args.values = staging.pointer + bytes;
        hipError_t error = launch_gather(launch_for(*cache, SYNAPSE_KV_KERNEL_GATHER, true), args, dims.precision == SYNAPSE_KV_F16);
        if (error == hipSuccess) {
            error = hipStreamSynchronize(cache->stream);
        }
        if (error == hipSuccess) {
            error = hipMemcpy(keys, staging.pointer, bytes, hipMemcpyDeviceToHost);
        }
        if (error == hipSuccess) {
            error = hipMemcpy(values, staging.pointer + bytes, bytes, hipMemcpyDeviceToHost);
        }
        staging.reset();
        check_hip(error, "KV read");
    });
}

// ---- Persistent prefix payloads ----

uint64_t synapse_kv_prefix_hash(const uint8_t* bytes, size_t count) {
    uint64_t hash = 0xcbf29ce484222325ull;
    for (size_t i = 0; bytes != nullptr && i < count; ++i) {
        hash ^= bytes[i];
        hash *= 0x100000001b3ull;
    }
    return hash;
}

namespace synapse_kv {
namespace {

// Bytes of one layer's K (or V) rows of `length` positions.
uint64_t prefix_rows_bytes(const Dims& dims, uint32_t length) {
    return static_cast<uint64_t>(length) * dims.kv_heads * dims.head_dim * (dims.precision == SYNAPSE_KV_F16 ? 2 : 4);
}

// The payload checksum: the header (checksum field zero) then the rows as little-endian 64-bit words, the tail
// zero-padded; h = 0xcbf29ce484222325, per word h = rotl64(h ^ mix(w), 23) * 0x100000001b3, finally
// mix(h ^ byte count), mix being the splitmix64 finalizer. Eight bytes per step (a 7B prefix of 32k positions is
// about 1.8 GB).
uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

uint64_t payload_checksum(const SynapseKvPrefixHeader& header, const uint8_t* rows, uint64_t count) {
    static_assert(sizeof(SynapseKvPrefixHeader) % 8 == 0, "the header is whole words");
    SynapseKvPrefixHeader zeroed = header;
    zeroed.checksum = 0;
    uint64_t h = 0xcbf29ce484222325ull;
    auto word = [&](uint64_t w) {
        const uint64_t x = h ^ mix64(w);
        h = ((x << 23) | (x >> 41)) * 0x100000001b3ull;
    };
    const auto* head = reinterpret_cast<const uint8_t*>(&zeroed);
    for (size_t at = 0; at < sizeof(zeroed); at += 8) {
        uint64_t w;
        std::memcpy(&w, head + at, 8);  // little-endian host
        word(w);
    }
    uint64_t at = 0;
    for (; at + 8 <= count; at += 8) {
        uint64_t w;
        std::memcpy(&w, rows + at, 8);
        word(w);
    }
    if (at < count) {
        uint64_t w = 0;
        std::memcpy(&w, rows + at, count - at);
        word(w);
    }
    return mix64(h ^ (sizeof(zeroed) + count));
}

bool same_key(const SynapseKvPrefixKey& a, const SynapseKvPrefixKey& b) {
    return a.model == b.model && a.tokenizer == b.tokenizer && a.rope == b.rope && a.prefix == b.prefix;
}

// The rows of an imported payload written into `slot`'s reserved pages, per layer, and the slot's length set.
void import_rows(SynapseKvCache& cache, uint32_t slot, const SynapseKvPrefixHeader& header, const uint8_t* rows_in,
                 uint64_t rows) {
    const Dims& dims = cache.dims;
    set_device(cache);
    flush_ops(cache);
    DeviceBuffer<uint8_t> staging;
    staging.ensure(2 * rows, "prefix staging");
    for (uint32_t layer = 0; layer < dims.layers; ++layer) {
        hipError_t error = hipStreamSynchronize(cache.stream);  // the staging's previous layer is written
        if (error == hipSuccess) {
            error = hipMemcpy(staging.pointer, rows_in + 2 * rows * layer, 2 * rows, hipMemcpyHostToDevice);
        }
        GatherArgs args{};
        args.geo = geometry(cache, layer);
        args.slot = static_cast<int32_t>(slot);
        args.first = 0;
        args.count = static_cast<int32_t>(header.length);
        args.keys = staging.pointer;
        args.values = staging.pointer + rows;
        if (error == hipSuccess) {
            error = launch_scatter(launch_for(cache, SYNAPSE_KV_KERNEL_GATHER, true), args,
                                   dims.precision == SYNAPSE_KV_F16);
        }
        if (error != hipSuccess) {
            staging.reset();
            check_hip(error, "prefix import");
        }
    }
    check_hip(hipStreamSynchronize(cache.stream), "prefix import");
    staging.reset();
    cache.length[slot] = header.length;
    cache.fold_next[slot] = -1;
    if (cache.activation.enabled != 0) {
        // Key summaries of the imported blocks (the keys below the length).
        std::vector<int32_t> blocks;
        const uint32_t size = static_cast<uint32_t>(cache.summary_keys);
        for (uint32_t position = 0; position < header.length; position += size) {
            blocks.push_back(slot_page(cache, slot, position / dims.page_tokens));
            blocks.push_back(static_cast<int32_t>((position % dims.page_tokens) / size));
            blocks.push_back(static_cast<int32_t>(std::min<uint32_t>(size, header.length - position)));
        }
        const size_t blob = blocks.size() * sizeof(int32_t);
        cache.op_blob.ensure(blob, "operation buffer");
        void* upload = cache.uploader.acquire(blob);
        std::memcpy(upload, blocks.data(), blob);
        cache.uploader.copy(cache.op_blob.pointer, blob, cache.stream);
        SummaryArgs summary{};
        summary.geo = geometry(cache, 0);
        summary.summaries = cache.summaries.pointer;
        summary.summary_page_bytes = cache.summary_page_bytes;
        summary.blocks = reinterpret_cast<const int32_t*>(cache.op_blob.pointer);
        summary.count = static_cast<int32_t>(blocks.size() / 3);
        summary.first_layer = 0;
        summary.layers = static_cast<int32_t>(dims.layers);
        check_hip(launch_summaries(launch_for(cache, SYNAPSE_KV_KERNEL_APPEND, true), summary,
                                   dims.precision == SYNAPSE_KV_F16),
                  "key summaries");
    }
}

void raise_status(int32_t status) {
    if (status != SYNAPSE_KV_OK) {
        throw Failure{status, g_last_error};
    }
}

}  // namespace
}  // namespace synapse_kv

int32_t synapse_kv_export_prefix(SynapseKvCache* cache, uint32_t slot, uint32_t length, const SynapseKvPrefixKey* key,
                                 uint8_t* payload, uint64_t capacity, uint64_t* bytes) {
    if (cache == nullptr || key == nullptr || bytes == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache, key or size output");
    }
    return guarded([&] {
        check_slot(*cache, slot);
        const Dims& dims = cache->dims;
        if (length > cache->length[slot]) {
            invalid("export of " + std::to_string(length) + " positions from a slot holding " +
                    std::to_string(cache->length[slot]));
        }
        const uint64_t rows = prefix_rows_bytes(dims, length);
        const uint64_t total = sizeof(SynapseKvPrefixHeader) + 2 * rows * dims.layers;
        *bytes = total;
        if (payload == nullptr) {
            return;
        }
        if (capacity < total) {
            invalid("the payload needs " + std::to_string(total) + " bytes");
        }
        SynapseKvPrefixHeader header{};
        std::memcpy(header.magic, SYNAPSE_KV_PREFIX_MAGIC, 8);
        header.version = SYNAPSE_KV_PREFIX_VERSION;
        header.header_bytes = sizeof(SynapseKvPrefixHeader);
        header.key = *key;
        header.kv_precision = dims.precision;
        header.layer_count = dims.layers;
        header.kv_heads = dims.kv_heads;
        header.head_dim = dims.head_dim;
        header.length = length;
        header.payload_bytes = 2 * rows * dims.layers;
        uint8_t* out = payload + sizeof(SynapseKvPrefixHeader);
        if (length > 0) {
            set_device(*cache);
            flush_ops(*cache);
            DeviceBuffer<uint8_t> staging;
            staging.ensure(2 * rows, "prefix staging");
            for (uint32_t layer = 0; layer < dims.layers; ++layer) {
                GatherArgs args{};
                args.geo = geometry(*cache, layer);
                args.slot = static_cast<int32_t>(slot);
                args.first = 0;
                args.count = static_cast<int32_t>(length);
                args.keys = staging.pointer;
                args.values = staging.pointer + rows;
                hipError_t error = launch_gather(launch_for(*cache, SYNAPSE_KV_KERNEL_GATHER, true), args,
                                                 dims.precision == SYNAPSE_KV_F16);
                if (error == hipSuccess) {
                    error = hipStreamSynchronize(cache->stream);
                }
                if (error == hipSuccess) {
                    error = hipMemcpy(out + 2 * rows * layer, staging.pointer, 2 * rows, hipMemcpyDeviceToHost);
                }
                if (error != hipSuccess) {
                    staging.reset();
                    check_hip(error, "prefix export");
                }
            }
            staging.reset();
        }
        header.checksum = payload_checksum(header, out, header.payload_bytes);
        std::memcpy(payload, &header, sizeof(header));
    });
}

int32_t synapse_kv_import_prefix(SynapseKvCache* cache, uint32_t slot, const SynapseKvPrefixKey* key,
                                 const uint8_t* payload, uint64_t bytes, uint32_t* length) {
    if (cache == nullptr || key == nullptr || payload == nullptr || length == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: cache, key, payload or length output");
    }
    return guarded([&] {
        check_slot(*cache, slot);
        const Dims& dims = cache->dims;
        if (bytes < sizeof(SynapseKvPrefixHeader)) {
            invalid("a prefix payload starts with a 128-byte header");
        }
        SynapseKvPrefixHeader header;
        std::memcpy(&header, payload, sizeof(header));
        if (std::memcmp(header.magic, SYNAPSE_KV_PREFIX_MAGIC, 8) != 0 || header.version != SYNAPSE_KV_PREFIX_VERSION ||
            header.header_bytes != sizeof(SynapseKvPrefixHeader)) {
            invalid("not a version " + std::to_string(SYNAPSE_KV_PREFIX_VERSION) + " prefix payload");
        }
        if (!same_key(header.key, *key)) {
            invalid("the payload's prefix key differs from the requested one");
        }
        if (header.kv_precision != dims.precision || header.layer_count != dims.layers ||
            header.kv_heads != dims.kv_heads || header.head_dim != dims.head_dim) {
            invalid("the payload's KV type or shape differs from the cache's");
        }
        if (header.length > dims.max_positions) {
            invalid("the payload holds more positions than the context");
        }
        const uint64_t rows = prefix_rows_bytes(dims, header.length);
        if (header.payload_bytes != 2 * rows * dims.layers || bytes < sizeof(header) + header.payload_bytes) {
            invalid("the payload's size does not match its header");
        }
        const uint8_t* rows_in = payload + sizeof(header);
        if (payload_checksum(header, rows_in, header.payload_bytes) != header.checksum) {
            invalid("the payload's checksum does not match its rows");
        }
        if (cache->length[slot] != 0 || cache->capacity[slot] != 0) {
            invalid("import needs an empty slot (release it first)");
        }
        if (header.length > 0) {
            raise_status(synapse_kv_reserve(cache, slot, header.length));
            try {
                import_rows(*cache, slot, header, rows_in, rows);
            } catch (...) {
                // A failed import leaves the slot empty: its pages go back before the error is reported.
                (void)synapse_kv_release(cache, slot);
                throw;
            }
        }
        *length = header.length;
    });
}

int32_t synapse_kv_rope_table(uint32_t head_dim, float theta, float yarn_factor, uint32_t yarn_original,
                              uint32_t positions, float* cosines, float* sines) {
    if (cosines == nullptr || sines == nullptr) {
        return record(SYNAPSE_KV_NULL_POINTER, "null pointer: RoPE tables");
    }
    return guarded([&] {
        if (head_dim == 0 || (head_dim & 1u) != 0 || !std::isfinite(theta) || theta <= 1.0f) {
            invalid("RoPE needs an even head dimension and theta above one");
        }
        // RopeFrequencies (RopeFrequencies.cs:20-81), FP32 expression order as written there.
        const uint32_t half = head_dim / 2;
        const float pi = 3.14159265358979323846f;
        std::vector<float> mix;
        float magnitude = 1.0f;
        if (yarn_factor > 0.0f) {
            if (yarn_original == 0) {
                invalid("YaRN needs the original context length");
            }
            magnitude = 1.0f + (0.1f * std::log(yarn_factor));
            auto correction = [&](float rotations) {
                return static_cast<float>(head_dim) *
                       std::log(static_cast<float>(yarn_original) / (rotations * 2 * pi)) / (2 * std::log(theta));
            };
            const float low = std::max(0.0f, std::floor(correction(32.0f)));
            const float high = std::min(static_cast<float>(head_dim - 1), std::ceil(correction(1.0f)));
            mix.resize(half);
            for (uint32_t index = 0; index < half; ++index) {
                const float ramp = (static_cast<float>(index) - low) / std::max(0.001f, high - low);
                mix[index] = 1 - std::min(1.0f, std::max(0.0f, ramp));
            }
        }
        for (uint32_t position = 0; position < positions; ++position) {
            for (uint32_t index = 0; index < half; ++index) {
                const float exponent = 2.0f * static_cast<float>(index) / static_cast<float>(head_dim);
                const float angle = static_cast<float>(position) / std::pow(theta, exponent);
                const size_t at = static_cast<size_t>(position) * half + index;
                if (mix.empty()) {
                    cosines[at] = std::cos(angle);
                    sines[at] = std::sin(angle);
                } else {
                    const float scaled = (angle / yarn_factor * (1 - mix[index])) + (angle * mix[index]);
                    cosines[at] = std::cos(scaled) * magnitude;
                    sines[at] = std::sin(scaled) * magnitude;
                }
            }
        }
    });
}

}  // extern "C"
