/* libsynapse_gpu's C ABI version 3, as exported by libsynapse_kv.so for a HIP backend.
 *
 * The reference's managed loader (src/Synapse.Runtime/Features/GpuKernels/NativeGpuLibrary.cs:14-75) binds these
 * eight functions by name from `libsynapse_gpu` and checks ABI version 3 (native/synapse-gpu/src/Features/
 * GpuKernels/ffi.rs:12). libsynapse_kv.so exports them beside its own synapse_kv_* functions, so installing it
 * under that name (or loading it by this path) gives GpuDecoderExecutor a third backend, SYNAPSE_GPU_BACKEND_HIP,
 * with the model API unchanged: the same structs (DecoderDesc 136 bytes, DecoderLayerOffsets 120, BatchToken 16,
 * GpuDeviceInfo 152; the SynapseKv* types of synapse_kv.h are those layouts), status codes, thread-local last
 * error and validation order. Every call forwards to the synapse_kv_decoder_* implementation. */
#ifndef SYNAPSE_GPU_H
#define SYNAPSE_GPU_H

#include "synapse_kv.h"

#ifdef __cplusplus
extern "C" {
#endif

#define SYNAPSE_GPU_ABI_VERSION 3u /* ffi.rs:12 */
#define SYNAPSE_GPU_BACKEND_METAL 1u /* ffi.rs:14: status 3 here, as on a machine that is not macOS */
#define SYNAPSE_GPU_BACKEND_CUDA 2u  /* ffi.rs:16: status 3, this build has no CUDA */
#define SYNAPSE_GPU_BACKEND_HIP 3u   /* the MI355X (gfx950) kernels of this library; other ids are status 2 */

typedef SynapseKvDeviceInfo GpuDeviceInfo;
typedef SynapseKvDecoderDesc DecoderDesc;
typedef SynapseKvLayerOffsets DecoderLayerOffsets;
typedef SynapseKvBatchToken BatchToken;
typedef struct SynapseKvDecoder GpuModel;

/* synapse_gpu_abi_version (ffi.rs:53-57): 3. */
uint32_t synapse_gpu_abi_version(void);

/* synapse_gpu_probe (ffi.rs:59-84): the backend's default device; for SYNAPSE_GPU_BACKEND_HIP the current HIP
 * device, as synapse_kv_probe describes it. Null `info` is status 1. */
int32_t synapse_gpu_probe(uint32_t backend, GpuDeviceInfo* info);

/* synapse_gpu_last_error (ffi.rs:86-104): the calling thread's last message, shared with synapse_kv_last_error. */
size_t synapse_gpu_last_error(uint8_t* buffer, size_t capacity);

/* synapse_gpu_decoder_create (ffi.rs:106-170): null checks, then DecoderPlan::new's validation, then the backend:
 * SYNAPSE_GPU_BACKEND_HIP creates the model on the current HIP device (synapse_kv_decoder_create). */
int32_t synapse_gpu_decoder_create(uint32_t backend, const DecoderDesc* desc, GpuModel** model);

/* synapse_gpu_decoder_forward (ffi.rs:172-211): synapse_kv_decoder_forward. */
int32_t synapse_gpu_decoder_forward(GpuModel* model, const BatchToken* tokens, size_t count, float* logits,
                                    size_t logits_capacity);

/* synapse_gpu_decoder_destroy (ffi.rs:213-227); null is ignored. */
void synapse_gpu_decoder_destroy(GpuModel* model);

/* synapse_gpu_decoder_kv_bytes (ffi.rs:229-248); 0 for null. */
uint64_t synapse_gpu_decoder_kv_bytes(const GpuModel* model);

/* synapse_gpu_decoder_reserve (ffi.rs:250-271). */
int32_t synapse_gpu_decoder_reserve(GpuModel* model, uint32_t slot, uint32_t positions);

#ifdef __cplusplus
}
#endif

#endif /* SYNAPSE_GPU_H */
