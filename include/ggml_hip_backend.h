/*
 * ggml_hip_backend.h -- the ggml backend plugin exports of the MI355X
 * quantized-matmul backend (libggml_hip_qmm.so).
 *
 * They mirror the ten ggml-cuda.h symbols the reference's CUDA backend
 * exports (src/ggml/cuda/backend.zig:1225-1236) with `cuda` replaced by
 * `hip`, plus the pair a dynamically loaded backend library answers
 * (ggml_backend_score / ggml_backend_init, src/ggml/backend_reg.zig:298-340).
 * The registry, devices, buffer types and backends they hand out fill the
 * vtables of ggml_hip_ggml_abi.h.
 *
 * Scope: the device runs MUL_MAT and MUL_MAT_ID with Q4_K / Q6_K / Q8_0
 * weights (and Q5_K / Q4_0 / IQ4_XS), f32 activations and f32 results.  By
 * default supports_op answers false for every other op, so
 * ggml_backend_sched keeps those on the CPU.  With GGML_HIP_FUSION=1 in the
 * environment (read once) it also takes f32 GLU (REGLU, GEGLU, SWIGLU,
 * SWIGLU_OAI, SWIGLU_CLAMP), same-shape f32 ADD and ADD_ID, so that the
 * FFN's gate / up / GLU (and bias) run stays in one split and
 * graph_compute fuses it as the reference's CUDA backend does
 * (cuda/fusion.zig, cuda/mulmat.zig:355-410); GGML_HIP_DISABLE_FUSION=1
 * turns that off again.
 */
#ifndef GGML_HIP_BACKEND_H
#define GGML_HIP_BACKEND_H

#include "ggml_hip_ggml_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_HIP_NAME "HIP"
#define GGML_HIP_MAX_DEVICES 16

/* Registry: name "HIP", one device per visible GPU (ggml_backend_cuda_reg,
 * cuda/backend.zig:1158-1202).  Thread-safe, process-lifetime. */
ggml_backend_reg_t ggml_backend_hip_reg(void);

/* A backend (stream + workspace pool) on `device`, or NULL for an invalid
 * device (ggml_backend_cuda_init, cuda/backend.zig:1205-1222). */
ggml_backend_t ggml_backend_hip_init(int device);

/* True for a backend made by ggml_backend_hip_init (guid match,
 * cuda/backend.zig:737-739). */
bool ggml_backend_is_hip(ggml_backend_t backend);

/* Device memory buffer type of `device`, NULL past the device count
 * (cuda/backend.zig:362-383).  Alignment 128; get_alloc_size pads
 * quantized rows to 512 elements (cuda/backend.zig:315-338). */
ggml_backend_buffer_type_t ggml_backend_hip_buffer_type(int device);

/* Pinned host memory buffer type (cuda/backend.zig:586-590). */
ggml_backend_buffer_type_t ggml_backend_hip_host_buffer_type(void);

int ggml_backend_hip_get_device_count(void);
void ggml_backend_hip_get_device_description(int device, char *description, size_t description_size);
void ggml_backend_hip_get_device_memory(int device, size_t *free, size_t *total);

/* Registering existing host memory as pinned is not offered (always false,
 * the answer the reference gives when registration is disabled,
 * cuda/backend.zig:787-810): allocate from the host buffer type instead. */
bool ggml_backend_hip_register_host_buffer(void *buffer, size_t size);
void ggml_backend_hip_unregister_host_buffer(void *buffer);

/* Dynamic-loading entry points. */
int ggml_backend_score(void);
ggml_backend_reg_t ggml_backend_init(void);

/*
 * Device-independent answers of the device vtable, callable without a GPU
 * (used by the vtable functions and by tests):
 *  - ggml_backend_hip_op_supported: the supports_op predicate
 *    (cuda/supports.zig:111-160 narrowed to this backend's types);
 *  - ggml_backend_hip_tensor_alloc_size: the buffer type's get_alloc_size.
 */
bool ggml_backend_hip_op_supported(const struct ggml_tensor *op);
size_t ggml_backend_hip_tensor_alloc_size(const struct ggml_tensor *tensor);

#ifdef __cplusplus
}
#endif
#endif
