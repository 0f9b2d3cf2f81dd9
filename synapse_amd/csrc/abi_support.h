// ABI support shared by the host files of libsynapse_kv: status codes raised as C++ exceptions inside an entry
// point and turned into the status and thread-local last error at its boundary.
//
// Conventions of native/synapse-gpu/src/Features/GpuKernels/ffi.rs: status codes (error.rs:4-16), a thread-local
// last error copied out by length (ffi.rs:19, 86-104), every entry point guarded (ffi.rs:34-45; C++ exceptions
// here instead of Rust panics).
#pragma once

#include <hip/hip_runtime.h>

#include <new>
#include <stdexcept>
#include <string>

#include "../../include/synapse_kv.h"

namespace synapse_kv {

// The calling thread's last error message (one instance for the whole library).
inline thread_local std::string g_last_error;

struct Failure {
    int32_t status;
    std::string message;
};

[[noreturn]] inline void fail(int32_t status, const std::string& message) { throw Failure{status, message}; }

[[noreturn]] inline void invalid(const std::string& message) {
    fail(SYNAPSE_KV_INVALID_ARGUMENT, "invalid argument: " + message);
}

inline void check_hip(hipError_t error, const char* what) {
    if (error == hipSuccess) {
        return;
    }
    const int32_t status = error == hipErrorOutOfMemory ? SYNAPSE_KV_OUT_OF_MEMORY : SYNAPSE_KV_DEVICE_ERROR;
    fail(status, std::string(status == SYNAPSE_KV_OUT_OF_MEMORY ? "out of device memory: " : "device error: ") + what +
                     ": " + hipGetErrorString(error));
}

inline int32_t record(int32_t status, const std::string& message) {
    g_last_error = message;
    return status;
}

template <typename Body>
int32_t guarded(Body body) {
    try {
        body();
        return SYNAPSE_KV_OK;
    } catch (const Failure& failure) {
        return record(failure.status, failure.message);
    } catch (const std::bad_alloc&) {
        return record(SYNAPSE_KV_OUT_OF_MEMORY, "out of host memory");
    } catch (const std::exception& error) {
        return record(SYNAPSE_KV_PANIC, std::string("a C++ exception was caught at the KV ABI: ") + error.what());
    } catch (...) {
        return record(SYNAPSE_KV_PANIC, "a C++ exception was caught at the KV ABI");
    }
}

}  // namespace synapse_kv
