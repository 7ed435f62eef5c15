/*
 * ggml_hip_ggml_abi.h -- the slice of the ggml C ABI the HIP backend layer
 * touches: tensor and graph layouts, the backend vtables and the enums they
 * use.
 *
 * The reference builds against upstream llama.cpp's ggml.h,
 * ggml-backend.h and ggml-backend-impl.h (v1.0.0, b1b770d90), reached
 * through translate-c (src/ggml/c_import.h:1-40); those headers live in its
 * llama.cpp submodule.  This file restates the members the HIP backend reads
 * or fills, in the order the reference's own code relies on:
 *   - ggml_tensor: fields as the reference reads them (type, buffer, ne, nb,
 *     op, op_params, flags, src, view_src, view_offs, data, name, extra) with
 *     the trailing 8-byte `padding` member src/ggml/backend_meta.zig:3221-3222
 *     checks;
 *   - ggml_cgraph and ggml_hash_set: src/ggml/impl.zig:422-435, 469-485
 *     (the reference's own extern declarations);
 *   - vtable members: in the order the CUDA backend initialises them
 *     (src/ggml/cuda/backend.zig:250-265 buffer, :343-352 buffer type,
 *     :714-731 backend, :1032-1048 device, :1141-1146 registry);
 *   - enum ggml_op values: the position of each name in op_name
 *     (src/ggml/types.zig:25-51); ggml_glu_op values likewise from
 *     glu_op_name (types.zig:103-106), read from op_params[0].
 * Numeric ggml_type ids follow ggml.h (GGML_TYPE_Q8_0 = 8, Q4_K = 12, Q6_K =
 * 14, I32 = 26); the kernel-level ABI (ggml_hip_qmm.h) uses the same ids.
 *
 * Define GGML_HIP_USE_UPSTREAM_HEADERS (and include ggml-backend-impl.h
 * first) to compile the backend against the real headers instead; that build
 * is the layout check this restatement gets when the library is linked into
 * the Zig tree.
 */
#ifndef GGML_HIP_GGML_ABI_H
#define GGML_HIP_GGML_ABI_H

#ifndef GGML_HIP_USE_UPSTREAM_HEADERS

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_MAX_DIMS 4
#define GGML_MAX_SRC 10
#define GGML_MAX_OP_PARAMS 64
#define GGML_MAX_NAME 64
#ifndef GGML_BACKEND_API_VERSION
#define GGML_BACKEND_API_VERSION 2
#endif

enum ggml_type {
    GGML_TYPE_F32 = 0,
    GGML_TYPE_F16 = 1,
    GGML_TYPE_Q4_0 = 2,
    GGML_TYPE_Q8_0 = 8,
    GGML_TYPE_Q8_1 = 9,
    GGML_TYPE_Q4_K = 12,
    GGML_TYPE_Q5_K = 13,
    GGML_TYPE_Q6_K = 14,
    GGML_TYPE_Q8_K = 15,
    GGML_TYPE_IQ4_XS = 23,
    GGML_TYPE_I32 = 26,
};

enum ggml_op {
    GGML_OP_NONE = 0,
    GGML_OP_ADD = 2,
    GGML_OP_ADD_ID = 3,
    GGML_OP_MUL_MAT = 28,
    GGML_OP_MUL_MAT_ID = 29,
    GGML_OP_RESHAPE = 35,
    GGML_OP_VIEW = 36,
    GGML_OP_PERMUTE = 37,
    GGML_OP_TRANSPOSE = 38,
    GGML_OP_GLU = 98,
};

/* ggml_tensor.flags bit a graph output carries (the scheduler and the
 * allocator keep such a tensor alive: src/ggml/alloc.zig:635-637, 684) */
#define GGML_TENSOR_FLAG_OUTPUT 2

enum ggml_status {
    GGML_STATUS_ALLOC_FAILED = -2,
    GGML_STATUS_FAILED = -1,
    GGML_STATUS_SUCCESS = 0,
    GGML_STATUS_ABORTED = 1,
};

enum ggml_backend_buffer_usage {
    GGML_BACKEND_BUFFER_USAGE_ANY = 0,
    GGML_BACKEND_BUFFER_USAGE_WEIGHTS = 1,
    GGML_BACKEND_BUFFER_USAGE_COMPUTE = 2,
};

enum ggml_backend_dev_type {
    GGML_BACKEND_DEVICE_TYPE_CPU = 0,
    GGML_BACKEND_DEVICE_TYPE_GPU = 1,
    GGML_BACKEND_DEVICE_TYPE_IGPU = 2,
    GGML_BACKEND_DEVICE_TYPE_ACCEL = 3,
};

struct ggml_backend_buffer;
struct ggml_backend_buffer_type;
struct ggml_backend;
struct ggml_backend_device;
struct ggml_backend_reg;
struct ggml_backend_event;

typedef struct ggml_backend_buffer *ggml_backend_buffer_t;
typedef struct ggml_backend_buffer_type *ggml_backend_buffer_type_t;
typedef struct ggml_backend *ggml_backend_t;
typedef struct ggml_backend_device *ggml_backend_dev_t;
typedef struct ggml_backend_reg *ggml_backend_reg_t;
typedef struct ggml_backend_event *ggml_backend_event_t;
typedef uint8_t ggml_guid[16];
typedef ggml_guid *ggml_guid_t;

struct ggml_tensor {
    enum ggml_type type;
    struct ggml_backend_buffer *buffer;
    int64_t ne[GGML_MAX_DIMS];
    size_t nb[GGML_MAX_DIMS];
    enum ggml_op op;
    int32_t op_params[GGML_MAX_OP_PARAMS / sizeof(int32_t)];
    int32_t flags;
    struct ggml_tensor *src[GGML_MAX_SRC];
    struct ggml_tensor *view_src;
    size_t view_offs;
    void *data;
    char name[GGML_MAX_NAME];
    void *extra;
    char padding[8];
};

/* ggml_hash_set (src/ggml/impl.zig:422-435): open addressing over tensor
 * pointers, slot of p = (p >> 4) % size with linear probing
 * (impl.zig:509-557), occupancy in a bitset of 32-bit words. */
struct ggml_hash_set {
    size_t size;
    uint32_t *used;
    struct ggml_tensor **keys;
};

/* Members up to visited_hash_set are read: use_counts[slot] is the number of
 * times the tensor in that slot is a source of a graph node
 * (src/ggml/graph.zig:1262-1268).  A graph view shares both with its parent
 * graph (graph.zig:252-266), so the counts include uses outside the view. */
struct ggml_cgraph {
    int size;
    int n_nodes;
    int n_leafs;
    struct ggml_tensor **nodes;
    struct ggml_tensor **grads;
    struct ggml_tensor **grad_accs;
    struct ggml_tensor **leafs;
    int32_t *use_counts;
    struct ggml_hash_set visited_hash_set;
    int order;
};

struct ggml_backend_buffer_type_i {
    const char *(*get_name)(ggml_backend_buffer_type_t buft);
    ggml_backend_buffer_t (*alloc_buffer)(ggml_backend_buffer_type_t buft, size_t size);
    void *alloc_buffer_n; /* left NULL: the generic planner serves it */
    size_t (*get_alignment)(ggml_backend_buffer_type_t buft);
    size_t (*get_max_size)(ggml_backend_buffer_type_t buft);
    size_t (*get_alloc_size)(ggml_backend_buffer_type_t buft, const struct ggml_tensor *tensor);
    void *get_alloc_size_n; /* left NULL */
    bool (*is_host)(ggml_backend_buffer_type_t buft);
};

struct ggml_backend_buffer_type {
    struct ggml_backend_buffer_type_i iface;
    ggml_backend_dev_t device;
    void *context;
};

struct ggml_backend_buffer_i {
    void (*free_buffer)(ggml_backend_buffer_t buffer);
    void *(*get_base)(ggml_backend_buffer_t buffer);
    enum ggml_status (*init_tensor)(ggml_backend_buffer_t buffer, struct ggml_tensor *tensor);
    void (*memset_tensor)(ggml_backend_buffer_t buffer, struct ggml_tensor *tensor, uint8_t value, size_t offset,
                          size_t size);
    void (*set_tensor)(ggml_backend_buffer_t buffer, struct ggml_tensor *tensor, const void *data, size_t offset,
                       size_t size);
    void (*get_tensor)(ggml_backend_buffer_t buffer, const struct ggml_tensor *tensor, void *data, size_t offset,
                       size_t size);
    void (*set_tensor_2d)(ggml_backend_buffer_t buffer, struct ggml_tensor *tensor, const void *data, size_t offset,
                          size_t size, size_t n_copies, size_t stride_tensor, size_t stride_data);
    void (*get_tensor_2d)(ggml_backend_buffer_t buffer, const struct ggml_tensor *tensor, void *data, size_t offset,
                          size_t size, size_t n_copies, size_t stride_tensor, size_t stride_data);
    bool (*cpy_tensor)(ggml_backend_buffer_t buffer, const struct ggml_tensor *src, struct ggml_tensor *dst);
    void (*clear)(ggml_backend_buffer_t buffer, uint8_t value);
    void (*reset)(ggml_backend_buffer_t buffer);
    void (*set_tensor_n)(ggml_backend_buffer_t buffer, struct ggml_tensor *const *tensors, const void *const *data,
                         const size_t *offsets, const size_t *sizes, size_t n_tensors);
    void (*get_tensor_n)(ggml_backend_buffer_t buffer, const struct ggml_tensor *const *tensors, void *const *data,
                         const size_t *offsets, const size_t *sizes, size_t n_tensors);
    bool (*cpy_tensor_n)(ggml_backend_buffer_t buffer, const struct ggml_tensor *const *srcs,
                         struct ggml_tensor *const *dsts, size_t n_tensors);
};

struct ggml_backend_buffer {
    struct ggml_backend_buffer_i iface;
    ggml_backend_buffer_type_t buft;
    void *context;
    size_t size;
    enum ggml_backend_buffer_usage usage;
};

/* What the scheduler hands graph_optimize (src/ggml/backend_sched.zig:997-1000,
 * backend.zig:1236): add_alloc_dep(user_data, tensor, until) keeps `tensor`
 * allocated until `until` has run. */
struct ggml_backend_graph_optimize_params {
    void (*add_alloc_dep)(void *user_data, struct ggml_tensor *tensor, struct ggml_tensor *until);
    void *user_data;
};

struct ggml_backend_i {
    const char *(*get_name)(ggml_backend_t backend);
    void (*free)(ggml_backend_t backend);
    void (*set_tensor_async)(ggml_backend_t backend, struct ggml_tensor *tensor, const void *data, size_t offset,
                             size_t size);
    void (*get_tensor_async)(ggml_backend_t backend, const struct ggml_tensor *tensor, void *data, size_t offset,
                             size_t size);
    void (*set_tensor_2d_async)(ggml_backend_t backend, struct ggml_tensor *tensor, const void *data, size_t offset,
                                size_t size, size_t n_copies, size_t stride_tensor, size_t stride_data);
    void (*get_tensor_2d_async)(ggml_backend_t backend, const struct ggml_tensor *tensor, void *data, size_t offset,
                                size_t size, size_t n_copies, size_t stride_tensor, size_t stride_data);
    bool (*cpy_tensor_async)(ggml_backend_t backend_src, ggml_backend_t backend_dst, const struct ggml_tensor *src,
                             struct ggml_tensor *dst);
    void (*synchronize)(ggml_backend_t backend);
    void *graph_plan_create;
    void *graph_plan_free;
    void *graph_plan_update;
    void *graph_plan_compute;
    enum ggml_status (*graph_compute)(ggml_backend_t backend, struct ggml_cgraph *cgraph);
    void (*event_record)(ggml_backend_t backend, ggml_backend_event_t event);
    void (*event_wait)(ggml_backend_t backend, ggml_backend_event_t event);
    void (*graph_optimize)(ggml_backend_t backend, struct ggml_cgraph *cgraph,
                           struct ggml_backend_graph_optimize_params *params);
};

struct ggml_backend {
    ggml_guid_t guid;
    struct ggml_backend_i iface;
    ggml_backend_dev_t device;
    void *context;
};

struct ggml_backend_event {
    struct ggml_backend_device *device;
    void *context;
};

struct ggml_backend_dev_caps {
    bool async;
    bool host_buffer;
    bool buffer_from_host_ptr;
    bool events;
    bool mmap_support;
};

struct ggml_backend_dev_props {
    const char *name;
    const char *description;
    size_t memory_free;
    size_t memory_total;
    enum ggml_backend_dev_type type;
    const char *device_id;
    struct ggml_backend_dev_caps caps;
};

struct ggml_backend_device_i {
    const char *(*get_name)(ggml_backend_dev_t dev);
    const char *(*get_description)(ggml_backend_dev_t dev);
    void (*get_memory)(ggml_backend_dev_t dev, size_t *free, size_t *total);
    enum ggml_backend_dev_type (*get_type)(ggml_backend_dev_t dev);
    void (*get_props)(ggml_backend_dev_t dev, struct ggml_backend_dev_props *props);
    ggml_backend_t (*init_backend)(ggml_backend_dev_t dev, const char *params);
    ggml_backend_buffer_type_t (*get_buffer_type)(ggml_backend_dev_t dev);
    ggml_backend_buffer_type_t (*get_host_buffer_type)(ggml_backend_dev_t dev);
    void *buffer_from_host_ptr; /* left NULL */
    bool (*supports_op)(ggml_backend_dev_t dev, const struct ggml_tensor *op);
    bool (*supports_buft)(ggml_backend_dev_t dev, ggml_backend_buffer_type_t buft);
    bool (*offload_op)(ggml_backend_dev_t dev, const struct ggml_tensor *op);
    ggml_backend_event_t (*event_new)(ggml_backend_dev_t dev);
    void (*event_free)(ggml_backend_dev_t dev, ggml_backend_event_t event);
    void (*event_synchronize)(ggml_backend_dev_t dev, ggml_backend_event_t event);
};

struct ggml_backend_device {
    struct ggml_backend_device_i iface;
    ggml_backend_reg_t reg;
    void *context;
};

struct ggml_backend_reg_i {
    const char *(*get_name)(ggml_backend_reg_t reg);
    size_t (*get_device_count)(ggml_backend_reg_t reg);
    ggml_backend_dev_t (*get_device)(ggml_backend_reg_t reg, size_t index);
    void *(*get_proc_address)(ggml_backend_reg_t reg, const char *name);
};

struct ggml_backend_reg {
    int api_version;
    struct ggml_backend_reg_i iface;
    void *context;
};

#ifdef __cplusplus
}
#endif

#endif /* GGML_HIP_USE_UPSTREAM_HEADERS */
#endif /* GGML_HIP_GGML_ABI_H */
