// backend.hip -- the ggml backend plugin layer: registry, devices, device and
// pinned-host buffer types, buffers and backends, behind the vtables of
// ggml_hip_ggml_abi.h, with graph_compute running MUL_MAT / MUL_MAT_ID on
// the kernels of this library.
//
// It fills the same interfaces the reference's CUDA backend fills
// (src/ggml/cuda/backend.zig: buffer 56-265, buffer type 277-383, pinned host
// 511-590, backend 594-739, device 742-1048, registry 1060-1236) so that
// ggml_backend_sched routes a MUL_MAT whose weight lives in a HIP buffer to
// this device (src/ggml/backend_sched.zig:288-396).  Host code only: plain
// HIP runtime calls; every device call is checked and a failing one aborts
// with the call named, as the reference's cudaCheck does.
#include <hip/hip_runtime.h>

#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <cstring>
#include <mutex>
#include <new>

#include "../../include/ggml_hip_backend.h"
#include "../../include/ggml_hip_qmm.h"

// Present when the library is loaded into a ggml host (the core owns buffer
// structs and frees them with its own allocator); absent in standalone use.
extern "C" __attribute__((weak)) ggml_backend_buffer_t ggml_backend_buffer_init(ggml_backend_buffer_type_t buft,
                                                                                struct ggml_backend_buffer_i iface,
                                                                                void *context, size_t size);

namespace {

[[noreturn]] void hip_fail(hipError_t e, const char *what, const char *file, int line) {
    std::fprintf(stderr, "ggml-hip: %s failed: %s (%s:%d)\n", what, hipGetErrorString(e), file, line);
    std::abort();
}
#define HIP_CHECK(call)                                                          \
    do {                                                                         \
        hipError_t e_ = (call);                                                  \
        if (e_ != hipSuccess) hip_fail(e_, #call, __FILE__, __LINE__);           \
    } while (0)

constexpr int64_t ROW_PADDING = 512;  // MATRIX_ROW_PADDING (cuda/common.zig:50-53)
constexpr size_t ALIGNMENT = 128;     // cuda/backend.zig:315-318

// ---------------------------------------------------------------- type table

struct TypeInfo {
    int64_t blck;
    size_t size;
    bool quantized;
};

TypeInfo type_info(int t) {
    switch (t) {
    case GGML_TYPE_F32: return {1, 4, false};
    case GGML_TYPE_F16: return {1, 2, false};
    case GGML_TYPE_I32: return {1, 4, false};
    case GGML_TYPE_Q8_0: return {32, 34, true};
    case GGML_TYPE_Q4_0: return {32, 18, true};
    case GGML_TYPE_IQ4_XS: return {256, 136, true};
    case GGML_TYPE_Q8_1: return {32, 36, true};
    case GGML_TYPE_Q4_K: return {256, 144, true};
    case GGML_TYPE_Q5_K: return {256, 176, true};
    case GGML_TYPE_Q6_K: return {256, 210, true};
    case GGML_TYPE_Q8_K: return {256, 292, true};
    default: return {0, 0, false};
    }
}

bool weight_type(int t) {
    return t == GGML_TYPE_Q4_0 || t == GGML_TYPE_Q4_K || t == GGML_TYPE_Q5_K || t == GGML_TYPE_Q6_K ||
           t == GGML_TYPE_Q8_0 || t == GGML_TYPE_IQ4_XS;
}

// Alignment the kernels read a weight type's blocks at (16 for the K-quants
// with 144- / 176-byte blocks, 2 otherwise).
size_t weight_align(int t) { return t == GGML_TYPE_Q4_K || t == GGML_TYPE_Q5_K ? 16 : 2; }

size_t row_size(int t, int64_t ne) {
    const TypeInfo ti = type_info(t);
    return ti.blck ? ti.size * (size_t)(ne / ti.blck) : 0;
}

// Bytes spanned by a tensor's elements (ggml_nbytes).
size_t nbytes(const ggml_tensor *t) {
    for (int i = 0; i < GGML_MAX_DIMS; ++i)
        if (t->ne[i] <= 0) return 0;
    const TypeInfo ti = type_info(t->type);
    if (!ti.blck) return 0;
    size_t n;
    if (ti.blck == 1) {
        n = ti.size;
        for (int i = 0; i < GGML_MAX_DIMS; ++i) n += (size_t)(t->ne[i] - 1) * t->nb[i];
    } else {
        n = (size_t)t->ne[0] * t->nb[0] / (size_t)ti.blck;
        for (int i = 1; i < GGML_MAX_DIMS; ++i) n += (size_t)(t->ne[i] - 1) * t->nb[i];
    }
    return n;
}

// Rows dense and in order, dims of extent 1 ignored (ggml_is_contiguous).
bool contiguous(const ggml_tensor *t) {
    const TypeInfo ti = type_info(t->type);
    if (!ti.blck) return false;
    size_t next = ti.size;
    if (t->ne[0] != ti.blck && t->nb[0] != next) return false;
    next *= (size_t)(t->ne[0] / ti.blck);
    for (int i = 1; i < GGML_MAX_DIMS; ++i) {
        if (t->ne[i] != 1) {
            if (t->nb[i] != next) return false;
            next *= (size_t)t->ne[i];
        }
    }
    return true;
}

const ggml_tensor *backing(const ggml_tensor *t) { return t->view_src ? t->view_src : t; }

// ---------------------------------------------------------------- devices

struct DeviceCtx {
    int device;
    char name[16];
    char description[256];
    char pci_bus_id[64];
};

struct BufferTypeCtx {
    int device;
    char name[16];
};

struct BufferCtx {
    int device;
    void *dev_ptr;
    bool own_struct;  // allocated here because no ggml core is linked
};

struct HostBufferCtx {
    void *ptr;
    bool own_struct;
};

struct BackendCtx {
    int device;
    char name[16];
    hipStream_t stream;
    void *ws;
    size_t ws_size;
};

int device_count_probe() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n < GGML_HIP_MAX_DEVICES ? n : GGML_HIP_MAX_DEVICES;
}

int device_count() {
    static int n = device_count_probe();
    return n;
}

// One guid per backend kind (a random 16-byte tag).
ggml_guid hip_guid = {0x5e, 0x1a, 0x7c, 0x93, 0x0b, 0xd4, 0x46, 0x2f, 0x9a, 0x31, 0xe2, 0x58, 0x77, 0x0c, 0xa6, 0x1d};

ggml_backend_buffer_t make_buffer(ggml_backend_buffer_type_t buft, const ggml_backend_buffer_i &iface, void *ctx,
                                  size_t size, bool *own_struct) {
    if (ggml_backend_buffer_init) {
        *own_struct = false;
        return ggml_backend_buffer_init(buft, iface, ctx, size);
    }
    auto *b = new ggml_backend_buffer{};
    b->iface = iface;
    b->buft = buft;
    b->context = ctx;
    b->size = size;
    b->usage = GGML_BACKEND_BUFFER_USAGE_ANY;
    *own_struct = true;
    return b;
}

char *at(void *p, size_t off) { return static_cast<char *>(p) + off; }
const char *at(const void *p, size_t off) { return static_cast<const char *>(p) + off; }

// ---------------------------------------------------------------- device buffer

BufferCtx *buf_ctx(ggml_backend_buffer_t b) { return static_cast<BufferCtx *>(b->context); }

void buf_free(ggml_backend_buffer_t b) {
    BufferCtx *ctx = buf_ctx(b);
    HIP_CHECK(hipSetDevice(ctx->device));
    HIP_CHECK(hipFree(ctx->dev_ptr));
    const bool own = ctx->own_struct;
    delete ctx;
    if (own) delete b;
}

void *buf_base(ggml_backend_buffer_t b) { return buf_ctx(b)->dev_ptr; }

ggml_status buf_init_tensor(ggml_backend_buffer_t b, ggml_tensor *t) {
    if (t->view_src) return GGML_STATUS_SUCCESS;
    // zero the row padding of quantized weights so the kernels read no NaNs
    if (type_info(t->type).quantized && b->usage != GGML_BACKEND_BUFFER_USAGE_COMPUTE) {
        const size_t orig = nbytes(t);
        const size_t padded = ggml_backend_hip_tensor_alloc_size(t);
        if (padded > orig) {
            HIP_CHECK(hipSetDevice(buf_ctx(b)->device));
            HIP_CHECK(hipMemsetAsync(at(t->data, orig), 0, padded - orig, hipStreamPerThread));
            HIP_CHECK(hipStreamSynchronize(hipStreamPerThread));
        }
    }
    return GGML_STATUS_SUCCESS;
}

void buf_memset_tensor(ggml_backend_buffer_t b, ggml_tensor *t, uint8_t value, size_t offset, size_t size) {
    HIP_CHECK(hipSetDevice(buf_ctx(b)->device));
    HIP_CHECK(hipMemsetAsync(at(t->data, offset), value, size, hipStreamPerThread));
    HIP_CHECK(hipStreamSynchronize(hipStreamPerThread));
}

void buf_set_tensor(ggml_backend_buffer_t b, ggml_tensor *t, const void *data, size_t offset, size_t size) {
    HIP_CHECK(hipSetDevice(buf_ctx(b)->device));
    HIP_CHECK(hipMemcpyAsync(at(t->data, offset), data, size, hipMemcpyHostToDevice, hipStreamPerThread));
    HIP_CHECK(hipStreamSynchronize(hipStreamPerThread));
}

void buf_get_tensor(ggml_backend_buffer_t b, const ggml_tensor *t, void *data, size_t offset, size_t size) {
    HIP_CHECK(hipSetDevice(buf_ctx(b)->device));
    HIP_CHECK(hipMemcpyAsync(data, at(t->data, offset), size, hipMemcpyDeviceToHost, hipStreamPerThread));
    HIP_CHECK(hipStreamSynchronize(hipStreamPerThread));
}

void buf_set_tensor_2d(ggml_backend_buffer_t b, ggml_tensor *t, const void *data, size_t offset, size_t size,
                       size_t n_copies, size_t stride_tensor, size_t stride_data) {
    HIP_CHECK(hipSetDevice(buf_ctx(b)->device));
    HIP_CHECK(hipMemcpy2DAsync(at(t->data, offset), stride_tensor, data, stride_data, size, n_copies,
                               hipMemcpyHostToDevice, hipStreamPerThread));
    HIP_CHECK(hipStreamSynchronize(hipStreamPerThread));
}

void buf_get_tensor_2d(ggml_backend_buffer_t b, const ggml_tensor *t, void *data, size_t offset, size_t size,
                       size_t n_copies, size_t stride_tensor, size_t stride_data) {
    HIP_CHECK(hipSetDevice(buf_ctx(b)->device));
    HIP_CHECK(hipMemcpy2DAsync(data, stride_data, at(t->data, offset), stride_tensor, size, n_copies,
                               hipMemcpyDeviceToHost, hipStreamPerThread));
    HIP_CHECK(hipStreamSynchronize(hipStreamPerThread));
}

bool buffer_is_hip(ggml_backend_buffer_t b);

void copy_device(const ggml_tensor *src, ggml_tensor *dst, hipStream_t s) {
    const int sd = buf_ctx(backing(src)->buffer)->device, dd = buf_ctx(backing(dst)->buffer)->device;
    if (sd == dd)
        HIP_CHECK(hipMemcpyAsync(dst->data, src->data, nbytes(src), hipMemcpyDeviceToDevice, s));
    else
        HIP_CHECK(hipMemcpyPeerAsync(dst->data, dd, src->data, sd, nbytes(src), s));
}

bool buf_cpy_tensor(ggml_backend_buffer_t b, const ggml_tensor *src, ggml_tensor *dst) {
    if (!src->buffer || !buffer_is_hip(backing(src)->buffer)) return false;
    HIP_CHECK(hipSetDevice(buf_ctx(b)->device));
    copy_device(src, dst, hipStreamPerThread);
    HIP_CHECK(hipStreamSynchronize(hipStreamPerThread));
    return true;
}

void buf_clear(ggml_backend_buffer_t b, uint8_t value) {
    HIP_CHECK(hipSetDevice(buf_ctx(b)->device));
    HIP_CHECK(hipMemsetAsync(buf_ctx(b)->dev_ptr, value, b->size, hipStreamPerThread));
    HIP_CHECK(hipStreamSynchronize(hipStreamPerThread));
}

void buf_set_tensor_n(ggml_backend_buffer_t b, ggml_tensor *const *ts, const void *const *data, const size_t *offs,
                      const size_t *sizes, size_t n) {
    HIP_CHECK(hipSetDevice(buf_ctx(b)->device));
    for (size_t i = 0; i < n; ++i)
        if (sizes[i])
            HIP_CHECK(hipMemcpyAsync(at(ts[i]->data, offs[i]), data[i], sizes[i], hipMemcpyHostToDevice,
                                     hipStreamPerThread));
    HIP_CHECK(hipStreamSynchronize(hipStreamPerThread));
}

void buf_get_tensor_n(ggml_backend_buffer_t b, const ggml_tensor *const *ts, void *const *data, const size_t *offs,
                      const size_t *sizes, size_t n) {
    HIP_CHECK(hipSetDevice(buf_ctx(b)->device));
    for (size_t i = 0; i < n; ++i)
        if (sizes[i])
            HIP_CHECK(hipMemcpyAsync(data[i], at(ts[i]->data, offs[i]), sizes[i], hipMemcpyDeviceToHost,
                                     hipStreamPerThread));
    HIP_CHECK(hipStreamSynchronize(hipStreamPerThread));
}

bool buf_cpy_tensor_n(ggml_backend_buffer_t b, const ggml_tensor *const *srcs, ggml_tensor *const *dsts, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (!backing(srcs[i])->buffer || !buffer_is_hip(backing(srcs[i])->buffer)) return false;
    HIP_CHECK(hipSetDevice(buf_ctx(b)->device));
    for (size_t i = 0; i < n; ++i) copy_device(srcs[i], dsts[i], hipStreamPerThread);
    HIP_CHECK(hipStreamSynchronize(hipStreamPerThread));
    return true;
}

const ggml_backend_buffer_i buffer_iface = {
    buf_free,          buf_base,          buf_init_tensor, buf_memset_tensor, buf_set_tensor,
    buf_get_tensor,    buf_set_tensor_2d, buf_get_tensor_2d, buf_cpy_tensor,  buf_clear,
    nullptr,           buf_set_tensor_n,  buf_get_tensor_n,  buf_cpy_tensor_n,
};

bool buffer_is_hip(ggml_backend_buffer_t b) { return b && b->iface.free_buffer == buf_free; }

// ---------------------------------------------------------------- device buffer type

const char *buft_name(ggml_backend_buffer_type_t buft) {
    return static_cast<BufferTypeCtx *>(buft->context)->name;
}

ggml_backend_buffer_t buft_alloc(ggml_backend_buffer_type_t buft, size_t size) {
    const int device = static_cast<BufferTypeCtx *>(buft->context)->device;
    HIP_CHECK(hipSetDevice(device));
    void *p = nullptr;
    const hipError_t e = hipMalloc(&p, size ? size : 1);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        std::fprintf(stderr, "ggml-hip: allocating %.2f MiB on device %d: hipMalloc failed: %s\n",
                     (double)size / 1048576.0, device, hipGetErrorString(e));
        return nullptr;
    }
    auto *ctx = new BufferCtx{device, p, false};
    return make_buffer(buft, buffer_iface, ctx, size, &ctx->own_struct);
}

size_t buft_alignment(ggml_backend_buffer_type_t) { return ALIGNMENT; }

size_t buft_alloc_size(ggml_backend_buffer_type_t, const ggml_tensor *t) {
    return ggml_backend_hip_tensor_alloc_size(t);
}

const ggml_backend_buffer_type_i buffer_type_iface = {
    buft_name, buft_alloc, nullptr, buft_alignment, nullptr, buft_alloc_size, nullptr, nullptr,
};

bool buft_is_hip(ggml_backend_buffer_type_t buft) { return buft && buft->iface.get_name == buft_name; }

// ---------------------------------------------------------------- pinned host buffer type

HostBufferCtx *hbuf_ctx(ggml_backend_buffer_t b) { return static_cast<HostBufferCtx *>(b->context); }

void hbuf_free(ggml_backend_buffer_t b) {
    HostBufferCtx *ctx = hbuf_ctx(b);
    HIP_CHECK(hipHostFree(ctx->ptr));
    const bool own = ctx->own_struct;
    delete ctx;
    if (own) delete b;
}
void *hbuf_base(ggml_backend_buffer_t b) { return hbuf_ctx(b)->ptr; }
void hbuf_memset_tensor(ggml_backend_buffer_t, ggml_tensor *t, uint8_t v, size_t off, size_t size) {
    std::memset(at(t->data, off), v, size);
}
void hbuf_set_tensor(ggml_backend_buffer_t, ggml_tensor *t, const void *d, size_t off, size_t size) {
    std::memcpy(at(t->data, off), d, size);
}
void hbuf_get_tensor(ggml_backend_buffer_t, const ggml_tensor *t, void *d, size_t off, size_t size) {
    std::memcpy(d, at(t->data, off), size);
}
void hbuf_clear(ggml_backend_buffer_t b, uint8_t v) { std::memset(hbuf_ctx(b)->ptr, v, b->size); }

const ggml_backend_buffer_i host_buffer_iface = {
    hbuf_free, hbuf_base, nullptr, hbuf_memset_tensor, hbuf_set_tensor, hbuf_get_tensor, nullptr,
    nullptr,   nullptr,   hbuf_clear, nullptr,          nullptr,         nullptr,         nullptr,
};

const char *hbuft_name(ggml_backend_buffer_type_t) { return GGML_HIP_NAME "_Host"; }

ggml_backend_buffer_t hbuft_alloc(ggml_backend_buffer_type_t buft, size_t size) {
    void *p = nullptr;
    const hipError_t e = hipHostMalloc(&p, size ? size : 1, hipHostMallocDefault);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        std::fprintf(stderr, "ggml-hip: failed to allocate %.2f MiB of pinned memory: %s\n",
                     (double)size / 1048576.0, hipGetErrorString(e));
        return nullptr;
    }
    auto *ctx = new HostBufferCtx{p, false};
    return make_buffer(buft, host_buffer_iface, ctx, size, &ctx->own_struct);
}

size_t hbuft_alignment(ggml_backend_buffer_type_t) { return 64; }
size_t hbuft_max_size(ggml_backend_buffer_type_t) { return (size_t)4 << 30; }
size_t hbuft_alloc_size(ggml_backend_buffer_type_t, const ggml_tensor *t) { return nbytes(t); }
bool hbuft_is_host(ggml_backend_buffer_type_t) { return true; }

// ---------------------------------------------------------------- backend

BackendCtx *be_ctx(ggml_backend_t be) { return static_cast<BackendCtx *>(be->context); }

const char *be_name(ggml_backend_t be) { return be_ctx(be)->name; }

void be_free(ggml_backend_t be) {
    BackendCtx *ctx = be_ctx(be);
    HIP_CHECK(hipSetDevice(ctx->device));
    HIP_CHECK(hipStreamSynchronize(ctx->stream));
    if (ctx->ws) HIP_CHECK(hipFree(ctx->ws));
    HIP_CHECK(hipStreamDestroy(ctx->stream));
    delete ctx;
    delete be;
}

void check_own_buffer(BackendCtx *ctx, const ggml_tensor *t) {
    const ggml_backend_buffer_t b = backing(t)->buffer;
    if (!buffer_is_hip(b) || buf_ctx(b)->device != ctx->device) {
        std::fprintf(stderr, "ggml-hip: tensor '%s' is not in a buffer of device %d\n", t->name, ctx->device);
        std::abort();
    }
}

void be_set_tensor_async(ggml_backend_t be, ggml_tensor *t, const void *data, size_t off, size_t size) {
    BackendCtx *ctx = be_ctx(be);
    check_own_buffer(ctx, t);
    HIP_CHECK(hipMemcpyAsync(at(t->data, off), data, size, hipMemcpyHostToDevice, ctx->stream));
}

void be_get_tensor_async(ggml_backend_t be, const ggml_tensor *t, void *data, size_t off, size_t size) {
    BackendCtx *ctx = be_ctx(be);
    check_own_buffer(ctx, t);
    HIP_CHECK(hipMemcpyAsync(data, at(t->data, off), size, hipMemcpyDeviceToHost, ctx->stream));
}

void be_set_tensor_2d_async(ggml_backend_t be, ggml_tensor *t, const void *data, size_t off, size_t size,
                            size_t n_copies, size_t stride_tensor, size_t stride_data) {
    BackendCtx *ctx = be_ctx(be);
    check_own_buffer(ctx, t);
    HIP_CHECK(hipMemcpy2DAsync(at(t->data, off), stride_tensor, data, stride_data, size, n_copies,
                               hipMemcpyHostToDevice, ctx->stream));
}

void be_get_tensor_2d_async(ggml_backend_t be, const ggml_tensor *t, void *data, size_t off, size_t size,
                            size_t n_copies, size_t stride_tensor, size_t stride_data) {
    BackendCtx *ctx = be_ctx(be);
    check_own_buffer(ctx, t);
    HIP_CHECK(hipMemcpy2DAsync(data, stride_data, at(t->data, off), stride_tensor, size, n_copies,
                               hipMemcpyDeviceToHost, ctx->stream));
}

bool be_cpy_tensor_async(ggml_backend_t src_be, ggml_backend_t dst_be, const ggml_tensor *src, ggml_tensor *dst) {
    if (!ggml_backend_is_hip(src_be) || !ggml_backend_is_hip(dst_be)) return false;
    const ggml_backend_buffer_t bs = backing(src)->buffer, bd = backing(dst)->buffer;
    if (!buffer_is_hip(bs) || !buffer_is_hip(bd)) return false;
    BackendCtx *cs = be_ctx(src_be), *cd = be_ctx(dst_be);
    if (cs->device != buf_ctx(bs)->device || cd->device != buf_ctx(bd)->device) return false;
    copy_device(src, dst, cs->stream);
    if (src_be != dst_be) {
        // the destination stream waits for the copy
        hipEvent_t ev;
        HIP_CHECK(hipSetDevice(cs->device));
        HIP_CHECK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
        HIP_CHECK(hipEventRecord(ev, cs->stream));
        HIP_CHECK(hipStreamWaitEvent(cd->stream, ev, 0));
        HIP_CHECK(hipEventDestroy(ev));
    }
    return true;
}

void be_synchronize(ggml_backend_t be) { HIP_CHECK(hipStreamSynchronize(be_ctx(be)->stream)); }

// Grow-only workspace of the backend (the reference's per-device pool,
// mmvq.zig:633-643).  Growing waits for the stream, so no queued kernel
// still uses the old block when it is freed.
void *workspace(BackendCtx *ctx, size_t need) {
    if (need <= ctx->ws_size) return ctx->ws;
    HIP_CHECK(hipStreamSynchronize(ctx->stream));
    if (ctx->ws) HIP_CHECK(hipFree(ctx->ws));
    ctx->ws = nullptr;
    ctx->ws_size = 0;
    size_t sz = need + need / 4;
    sz = (sz + 255) & ~(size_t)255;
    HIP_CHECK(hipMalloc(&ctx->ws, sz));
    ctx->ws_size = sz;
    return ctx->ws;
}

bool report(int rc, const char *what, const ggml_tensor *node) {
    if (rc == 0) return true;
    std::fprintf(stderr, "ggml-hip: %s for node '%s' failed: %s\n", what, node->name,
                 hipGetErrorString((hipError_t)rc));
    return false;
}

// dst[M, N, ne2, ne3] = src0[K, M, ne02, ne03] x src1[K, N, ne2, ne3], src0
// broadcast over dims 2 and 3 (ggml_mul_mat, src/ggml/ops.zig:1072-1083).
bool run_mul_mat(BackendCtx *ctx, const ggml_tensor *node) {
    const ggml_tensor *a = node->src[0], *b = node->src[1];
    const int64_t K = a->ne[0], M = a->ne[1], N = b->ne[1];
    const int64_t r2 = b->ne[2] / a->ne[2], r3 = b->ne[3] / a->ne[3];
    const TypeInfo ta = type_info(a->type);
    const int64_t nbatch = b->ne[2] * b->ne[3];
    if (nbatch > 1 && N <= 8 && b->ne[2] <= 65535 && b->ne[3] <= 65535 && a->nb[1] % ta.size == 0 &&
        a->nb[2] % ta.size == 0 && a->nb[3] % ta.size == 0 && b->nb[1] % 4 == 0 && b->nb[2] % 4 == 0 &&
        b->nb[3] % 4 == 0 && node->nb[2] % 4 == 0 && node->nb[3] % 4 == 0) {
        // Batched decode, as the reference's mulMatVecQ runs it
        // (src/ggml/cuda/mmvq.zig:531-696): every column of every batch to AoS
        // Q8_1 in one launch, then one GEMV launch over channels and samples.
        const int64_t Kp = (K + ROW_PADDING - 1) / ROW_PADDING * ROW_PADDING, cb = Kp / 32;
        void *ws = workspace(ctx, (size_t)(N * nbatch * cb) * 36);
        int rc = hip_qmm_quantize_q8_1(static_cast<const float *>(b->data), ws, K, (int64_t)(b->nb[1] / 4),
                                       (int64_t)(b->nb[2] / 4), (int64_t)(b->nb[3] / 4), Kp, N, b->ne[2], b->ne[3],
                                       ctx->stream);
        if (!report(rc, "hip_qmm_quantize_q8_1", node)) return false;
        rc = hip_qmm_mul_mat_vec_q(a->type, a->data, ws, nullptr, static_cast<float *>(node->data), K, M, N,
                                   (int64_t)(a->nb[1] / ta.size), cb, (int64_t)(node->nb[1] / 4), a->ne[2], b->ne[2],
                                   node->ne[2], (int64_t)(a->nb[2] / ta.size), N * cb, (int64_t)(node->nb[2] / 4),
                                   a->ne[3], node->ne[3], (int64_t)(a->nb[3] / ta.size), N * b->ne[2] * cb,
                                   (int64_t)(node->nb[3] / 4), 0, ctx->stream);
        return report(rc, "hip_qmm_mul_mat_vec_q", node);
    }
    // One batch, or more than 8 columns: the op per (i2, i3) slice (its
    // MMQ takes one weight matrix per launch).
    const size_t need = hip_qmm_mul_mat_workspace_size(a->type, K, M, N);
    void *ws = workspace(ctx, need);
    for (int64_t i3 = 0; i3 < b->ne[3]; ++i3)
        for (int64_t i2 = 0; i2 < b->ne[2]; ++i2) {
            const char *w = at(a->data, (size_t)(i2 / r2) * a->nb[2] + (size_t)(i3 / r3) * a->nb[3]);
            const float *x = reinterpret_cast<const float *>(at(b->data, (size_t)i2 * b->nb[2] + (size_t)i3 * b->nb[3]));
            float *d = reinterpret_cast<float *>(at(node->data, (size_t)i2 * node->nb[2] + (size_t)i3 * node->nb[3]));
            const int rc = hip_qmm_mul_mat(a->type, w, K, M, (int64_t)a->nb[1], x, N, (int64_t)(b->nb[1] / 4), d,
                                           (int64_t)(node->nb[1] / 4), ws, ctx->ws_size, ctx->stream);
            if (!report(rc, "hip_qmm_mul_mat", node)) return false;
        }
    return true;
}

// dst[M, n_used, n_tokens]: row (s, t) = src0[:, :, ids[s, t]] x src1[:, s % ne11, t]
// (ggml_mul_mat_id, src/ggml/ops.zig:1104-1125).
bool run_mul_mat_id(BackendCtx *ctx, const ggml_tensor *node) {
    const ggml_tensor *as = node->src[0], *b = node->src[1], *ids = node->src[2];
    const int64_t K = as->ne[0], M = as->ne[1], n_as = as->ne[2];
    const int64_t ne11 = b->ne[1], n_tokens = b->ne[2], n_ids = ids->ne[0];
    const size_t need = hip_qmm_mul_mat_id_workspace_size(as->type, K, n_as, ne11, n_tokens, n_ids);
    void *ws = workspace(ctx, need);
    const int rc = hip_qmm_mul_mat_id(as->type, as->data, K, M, (int64_t)as->nb[1], (int64_t)as->nb[2], n_as,
                                      static_cast<const float *>(b->data), ne11, n_tokens, (int64_t)(b->nb[1] / 4),
                                      static_cast<const int32_t *>(ids->data), n_ids, (int64_t)(ids->nb[1] / 4),
                                      static_cast<float *>(node->data), (int64_t)(node->nb[1] / 4), ws, ctx->ws_size,
                                      ctx->stream);
    return report(rc, "hip_qmm_mul_mat_id", node);
}

bool is_noop(int op) {
    return op == GGML_OP_NONE || op == GGML_OP_RESHAPE || op == GGML_OP_VIEW || op == GGML_OP_PERMUTE ||
           op == GGML_OP_TRANSPOSE;
}

// ---------------------------------------------------------------- GLU and ADD nodes

float op_param_f32(const ggml_tensor *t, int i) {
    float f;
    std::memcpy(&f, &t->op_params[i], sizeof f);
    return f;
}

// GLU ops with a device implementation (glu_apply): REGLU, GEGLU, SWIGLU,
// SWIGLU_OAI, SWIGLU_CLAMP.  GEGLU_ERF and GEGLU_QUICK stay on the CPU.
bool glu_op_supported(int op) {
    return op == HIP_QMM_GLU_REGLU || op == HIP_QMM_GLU_GEGLU || op == HIP_QMM_GLU_SWIGLU ||
           op == HIP_QMM_GLU_SWIGLU_OAI || op == HIP_QMM_GLU_SWIGLU_CLAMP;
}

bool same_shape(const ggml_tensor *a, const ggml_tensor *b) {
    for (int i = 0; i < GGML_MAX_DIMS; ++i)
        if (a->ne[i] != b->ne[i]) return false;
    return true;
}

bool f32_rows(const ggml_tensor *t) {
    return t->type == GGML_TYPE_F32 && t->nb[0] == 4 && t->nb[1] % 4 == 0 && t->nb[2] % 4 == 0 && t->nb[3] % 4 == 0;
}

// dst = glu(gate, value) row by row (ggml_compute_forward_glu,
// src/ggml/cpu/ops/activation.zig:594-608).  Split form: src0 gates, src1 is
// the value.  One tensor: the halves of each src0 row, the first gating
// unless op_params[1] (swapped) is set (GluRows.halves, activation.zig:365-376).
bool run_glu(BackendCtx *ctx, const ggml_tensor *node) {
    const ggml_tensor *a = node->src[0], *b = node->src[1];
    const int64_t nc = node->ne[0];
    const ggml_tensor *gt = a, *ut = b ? b : a;
    size_t goff = 0, uoff = 0;
    if (!b) (node->op_params[1] ? goff : uoff) = (size_t)nc * 4;
    for (int64_t i3 = 0; i3 < node->ne[3]; ++i3)
        for (int64_t i2 = 0; i2 < node->ne[2]; ++i2) {
            const float *g = reinterpret_cast<const float *>(at(gt->data, i2 * gt->nb[2] + i3 * gt->nb[3] + goff));
            const float *u = reinterpret_cast<const float *>(at(ut->data, i2 * ut->nb[2] + i3 * ut->nb[3] + uoff));
            float *d = reinterpret_cast<float *>(at(node->data, i2 * node->nb[2] + i3 * node->nb[3]));
            const int rc = hip_qmm_glu_f32(node->op_params[0], op_param_f32(node, 2), op_param_f32(node, 3), nc,
                                           node->ne[1], g, (int64_t)(gt->nb[1] / 4), u, (int64_t)(ut->nb[1] / 4), d,
                                           (int64_t)(node->nb[1] / 4), ctx->stream);
            if (!report(rc, "hip_qmm_glu_f32", node)) return false;
        }
    return true;
}

// dst = src0 + src1, all of one shape (ggml_add without broadcasting).
bool run_add(BackendCtx *ctx, const ggml_tensor *node) {
    const ggml_tensor *a = node->src[0], *b = node->src[1];
    for (int64_t i3 = 0; i3 < node->ne[3]; ++i3)
        for (int64_t i2 = 0; i2 < node->ne[2]; ++i2) {
            const float *pa = reinterpret_cast<const float *>(at(a->data, i2 * a->nb[2] + i3 * a->nb[3]));
            const float *pb = reinterpret_cast<const float *>(at(b->data, i2 * b->nb[2] + i3 * b->nb[3]));
            float *d = reinterpret_cast<float *>(at(node->data, i2 * node->nb[2] + i3 * node->nb[3]));
            const int rc = hip_qmm_add_f32(node->ne[0], node->ne[1], pa, (int64_t)(a->nb[1] / 4), pb,
                                           (int64_t)(b->nb[1] / 4), d, (int64_t)(node->nb[1] / 4), ctx->stream);
            if (!report(rc, "hip_qmm_add_f32", node)) return false;
        }
    return true;
}

// dst row (s, t) = src0 row + src1 row ids[t][s] (ggml_add_id; -1: src0 alone).
bool run_add_id(BackendCtx *ctx, const ggml_tensor *node) {
    const ggml_tensor *a = node->src[0], *b = node->src[1], *ids = node->src[2];
    const int rc = hip_qmm_add_id_f32(node->ne[0], node->ne[1], node->ne[2], static_cast<const float *>(a->data),
                                      (int64_t)(a->nb[1] / 4), (int64_t)(a->nb[2] / 4),
                                      static_cast<const float *>(b->data), (int64_t)(b->nb[1] / 4), b->ne[1],
                                      static_cast<const int32_t *>(ids->data), (int64_t)(ids->nb[1] / 4),
                                      static_cast<float *>(node->data), (int64_t)(node->nb[1] / 4),
                                      (int64_t)(node->nb[2] / 4), ctx->stream);
    return report(rc, "hip_qmm_add_id_f32", node);
}

// ---------------------------------------------------------------- fusion
//
// The mul_mat_vec fusions of the reference's CUDA backend
// (ggml_cuda_try_fuse, src/ggml/cuda/fusion.zig:1153-1390, 1482-1520), for
// one activation column:
//   {MUL_MAT, MUL_MAT, GLU}            gate and up GEMVs + GLU, one kernel
//   {MUL_MAT, ADD, MUL_MAT, ADD, GLU}  the same with a bias on each lane
//   {MUL_MAT, ADD}                     GEMV + bias
// A run fuses only when every node in it but the last is read only inside
// the run and is not a graph output (ggml_can_fuse_subgraph_ext,
// src/ggml/graph.zig:1207-1250), with use counts from the graph's hash set.
// Graphs without use counts run unfused.
//
// The fusion is opt-in: by default the device takes MUL_MAT / MUL_MAT_ID
// and the no-op views only, and every other op (GLU, ADD, ADD_ID included)
// stays on the CPU backend.  GGML_HIP_FUSION=1 lets the device take the GLU
// and bias-add nodes as well, so the FFN's gate / up / GLU run stays in one
// split and fuses; GGML_HIP_DISABLE_FUSION=1 (the reference's
// GGML_CUDA_DISABLE_FUSION) turns it off again.  Both are read once.

bool env_flag(const char *name) {
    const char *e = std::getenv(name);
    return e && *e && std::strcmp(e, "0") != 0;
}

bool fusion_disabled() {
    static const bool off = !env_flag("GGML_HIP_FUSION") || env_flag("GGML_HIP_DISABLE_FUSION");
    return off;
}

// ggml_node_get_use_count (src/ggml/graph.zig:1262-1268) through the hash
// lookup of impl.zig:549-557; -1 when the graph carries no use counts.
int use_count(const ggml_cgraph *g, const ggml_tensor *t) {
    const ggml_hash_set &h = g->visited_hash_set;
    if (!g->use_counts || !h.size || !h.used || !h.keys) return -1;
    auto used = [&](size_t i) { return (h.used[i >> 5] >> (i & 31)) & 1u; };
    const size_t start = ((uintptr_t)t >> 4) % h.size;
    size_t i = start;
    while (used(i) && h.keys[i] != t) {
        i = (i + 1) % h.size;
        if (i == start) return -1;
    }
    return used(i) ? g->use_counts[i] : 0;
}

// Nodes i0 .. i0+n-1 but `out` are read only inside the run, are not graph
// outputs and are not views.
bool run_is_closed(const ggml_cgraph *g, int i0, int n, const ggml_tensor *out) {
    for (int i = i0; i < i0 + n; ++i) {
        const ggml_tensor *t = g->nodes[i];
        if (t == out) continue;
        if ((t->flags & GGML_TENSOR_FLAG_OUTPUT) || t->view_src) return false;
        int uses = 0;
        for (int j = i + 1; j < i0 + n; ++j)
            for (int s = 0; s < GGML_MAX_SRC; ++s) uses += g->nodes[j]->src[s] == t;
        if (use_count(g, t) != uses) return false;
    }
    return true;
}

bool overlaps(const void *a, size_t na, const void *b, size_t nb) {
    const uintptr_t pa = (uintptr_t)a, pb = (uintptr_t)b;
    return pa < pb + nb && pb < pa + na;
}

// A fused launch writes its result while other workgroups still read the
// weights, so the result must not land on the weights of either lane.  Under
// op offload the weights are compute-buffer copies that the allocator may
// hand to a later node once their own MUL_MAT is past; unfused, that reuse is
// harmless, fused it is not, so the run then goes unfused.
bool lands_on_weights(const void *out, size_t ob, const ggml_tensor *mm_a, const ggml_tensor *mm_b) {
    for (const ggml_tensor *mm : {mm_a, mm_b}) {
        if (!mm) continue;
        const ggml_tensor *w = mm->src[0];
        if (overlaps(out, ob, w->data, nbytes(w))) return true;
    }
    return false;
}

// A supported MUL_MAT the fused one-column entry point takes
// (ggml_cuda_should_fuse_mul_mat_vec_q, src/ggml/cuda/mulmat.zig:443-462:
// one destination column, f32 in and out; plus the entry point's limits).
bool vec_fusable(const ggml_tensor *mm) {
    const ggml_tensor *w = mm->src[0], *x = mm->src[1];
    for (int i = 1; i < GGML_MAX_DIMS; ++i)
        if (x->ne[i] != 1 || mm->ne[i] != 1 || (i > 1 && w->ne[i] != 1)) return false;
    const int64_t K = w->ne[0];
    if (K % 32 != 0 || K > 32768 || (uintptr_t)x->data % 16 != 0) return false;
    const size_t walign = weight_align(w->type);
    return (uintptr_t)w->data % walign == 0 && w->nb[1] % walign == 0 && mm->nb[0] == 4;
}

// A bias of a MUL_MAT output: f32, the output's shape, dense.
bool bias_ok(const ggml_tensor *b, const ggml_tensor *mm) {
    return b && b->type == GGML_TYPE_F32 && same_shape(b, mm) && b->nb[0] == 4;
}

// The other operand of an ADD that reads mm (getBiasTensor, fusion.zig:910-919).
const ggml_tensor *bias_of(const ggml_tensor *add, const ggml_tensor *mm) {
    if (add->op != GGML_OP_ADD || !same_shape(add->src[0], add->src[1])) return nullptr;
    if (add->src[0] == mm) return add->src[1];
    if (add->src[1] == mm) return add->src[0];
    return nullptr;
}

// Whether t is one of the nodes g->nodes[i0 .. i0+n): a fused launch
// computes none of them before it reads its operands, so such a tensor
// cannot serve as a bias (ADD(mm, mm), or one lane's ADD as the other's bias).
bool in_run(const ggml_cgraph *g, int i0, int n, const ggml_tensor *t) {
    for (int j = i0; j < i0 + n && j < g->n_nodes; ++j)
        if (g->nodes[j] == t) return true;
    return false;
}

// ggml_cuda_should_fuse_mul_mat (src/ggml/cuda/mulmat.zig:355-410) for the
// one-column kernel: same weight type, shape and strides, the same
// activation tensor, a split non-swapped GLU of a fused op.
bool gate_up_fusable(const ggml_tensor *up, const ggml_tensor *gate, const ggml_tensor *glu) {
    const ggml_tensor *wu = up->src[0], *wg = gate->src[0];
    const int op = glu->op_params[0];
    if (op != HIP_QMM_GLU_GEGLU && op != HIP_QMM_GLU_SWIGLU && op != HIP_QMM_GLU_SWIGLU_OAI &&
        op != HIP_QMM_GLU_SWIGLU_CLAMP)
        return false;
    if (glu->op_params[1] != 0 || !glu->src[1] || glu->type != GGML_TYPE_F32 || glu->nb[0] != 4) return false;
    if (wu->type != wg->type || !same_shape(wu, wg)) return false;
    for (int i = 0; i < GGML_MAX_DIMS; ++i)
        if (wu->nb[i] != wg->nb[i]) return false;
    if (up->src[1] != gate->src[1]) return false;
    return vec_fusable(up) && vec_fusable(gate) && same_shape(glu, up);
}

bool launch_fused(BackendCtx *ctx, const ggml_tensor *up, const ggml_tensor *gate, const ggml_tensor *ubias,
                  const ggml_tensor *gbias, const ggml_tensor *out, bool *ok) {
    const ggml_tensor *w = up->src[0], *x = up->src[1];
    const int64_t K = w->ne[0], M = w->ne[1];
    // the result must not land on an input (checkFusionMemoryRanges, fusion.zig)
    const size_t ob = (size_t)M * 4;
    if (overlaps(out->data, ob, x->data, (size_t)K * 4)) return false;
    if (ubias && overlaps(out->data, ob, ubias->data, ob)) return false;
    if (gbias && overlaps(out->data, ob, gbias->data, ob)) return false;
    if (lands_on_weights(out->data, ob, up, gate)) return false;
    const int op = gate ? out->op_params[0] : 0;
    const float alpha = gate ? op_param_f32(out, 2) : 0.0f, limit = gate ? op_param_f32(out, 3) : 0.0f;
    const int rc = hip_qmm_mul_mat_vec_fused(w->type, w->data, gate ? gate->src[0]->data : nullptr, K, M,
                                             (int64_t)w->nb[1], static_cast<const float *>(x->data),
                                             ubias ? static_cast<const float *>(ubias->data) : nullptr,
                                             gbias ? static_cast<const float *>(gbias->data) : nullptr, op, alpha,
                                             limit, static_cast<float *>(out->data), ctx->stream);
    *ok = report(rc, "hip_qmm_mul_mat_vec_fused", out);
    return true;
}

// The MUL_MAT_ID pair of an MoE FFN over at most 8 tokens (the reference's
// MMVQ-with-ids limit, mmvq.zig:116-125): same expert weights' type, shape
// and strides, the same activations and ids, a split non-swapped GLU of a
// fused op, dense rows the ids entry point addresses.
bool gate_up_id_fusable(const ggml_tensor *up, const ggml_tensor *gate, const ggml_tensor *glu) {
    const ggml_tensor *wu = up->src[0], *wg = gate->src[0], *x = up->src[1];
    const int op = glu->op_params[0];
    if (op != HIP_QMM_GLU_GEGLU && op != HIP_QMM_GLU_SWIGLU && op != HIP_QMM_GLU_SWIGLU_OAI &&
        op != HIP_QMM_GLU_SWIGLU_CLAMP)
        return false;
    if (glu->op_params[1] != 0 || !glu->src[1] || glu->type != GGML_TYPE_F32 || glu->nb[0] != 4) return false;
    if (wu->type != wg->type || !same_shape(wu, wg)) return false;
    for (int i = 0; i < GGML_MAX_DIMS; ++i)
        if (wu->nb[i] != wg->nb[i]) return false;
    if (up->src[1] != gate->src[1] || up->src[2] != gate->src[2] || !same_shape(glu, up)) return false;
    if (glu->nb[2] != (size_t)glu->ne[1] * glu->nb[1] || glu->nb[1] % 4) return false;
    if (x->nb[2] != (size_t)x->ne[1] * x->nb[1]) return false;  // row (t, i11) at (t * ne11 + i11) * nb1
    const int64_t K = wu->ne[0], n_tokens = x->ne[2];
    const size_t walign = weight_align(wu->type);
    return n_tokens <= 8 && n_tokens * glu->ne[1] <= 65535 && K % 32 == 0 && K <= 32768 &&
           (uintptr_t)x->data % 16 == 0 && x->nb[1] % 16 == 0 && (uintptr_t)wu->data % walign == 0 &&
           (uintptr_t)wg->data % walign == 0 && wu->nb[1] % walign == 0 && wu->nb[2] % walign == 0;
}

bool launch_fused_id(BackendCtx *ctx, const ggml_tensor *up, const ggml_tensor *gate, const ggml_tensor *out,
                     bool *ok) {
    const ggml_tensor *w = up->src[0], *x = up->src[1], *ids = up->src[2];
    const int64_t K = w->ne[0], M = w->ne[1];
    const size_t ob = nbytes(out);
    if (overlaps(out->data, ob, x->data, nbytes(x)) || overlaps(out->data, ob, ids->data, nbytes(ids)) ||
        lands_on_weights(out->data, ob, up, gate))
        return false;
    const int rc = hip_qmm_mul_mat_id_vec_fused(
        w->type, w->data, gate->src[0]->data, K, M, (int64_t)w->nb[1], (int64_t)w->nb[2], w->ne[2],
        static_cast<const float *>(x->data), x->ne[1], x->ne[2], (int64_t)(x->nb[1] / 4),
        static_cast<const int32_t *>(ids->data), ids->ne[0], (int64_t)(ids->nb[1] / 4), out->op_params[0],
        op_param_f32(out, 2), op_param_f32(out, 3), static_cast<float *>(out->data), (int64_t)(out->nb[1] / 4),
        ctx->stream);
    *ok = report(rc, "hip_qmm_mul_mat_id_vec_fused", out);
    return true;
}

// ---- prefill: {MUL_MAT gate, MUL_MAT up, GLU} and its MUL_MAT_ID form into
// the fused MMQ (the reference's shouldFuseMulMatQ, src/ggml/cuda/mulmat.zig:
// 548-571, then mul_mat_q with the gate, fusion.zig:1226-1298, 1391).

// The gate/up weights and GLU checks the fused kernels share: a split
// non-swapped f32 GLU of an op they apply, weights of one type, shape and
// strides, the same activations.
bool gate_up_pair_ok(const ggml_tensor *up, const ggml_tensor *gate, const ggml_tensor *glu) {
    const ggml_tensor *wu = up->src[0], *wg = gate->src[0];
    const int op = glu->op_params[0];
    if (op != HIP_QMM_GLU_GEGLU && op != HIP_QMM_GLU_SWIGLU && op != HIP_QMM_GLU_SWIGLU_OAI &&
        op != HIP_QMM_GLU_SWIGLU_CLAMP)
        return false;
    if (glu->op_params[1] != 0 || !glu->src[1] || glu->type != GGML_TYPE_F32 || glu->nb[0] != 4) return false;
    if (wu->type != wg->type || !same_shape(wu, wg)) return false;
    for (int i = 0; i < GGML_MAX_DIMS; ++i)
        if (wu->nb[i] != wg->nb[i]) return false;
    return up->src[1] == gate->src[1] && up->src[2] == gate->src[2] && same_shape(glu, up);
}

// Dense: one 2-D product of 2+ f32 columns that each product alone would run
// on the MMQ tile kernel (hip_qmm_mul_mat_glu_fused), dense columns.
bool gate_up_mmq_fusable(const ggml_tensor *up, const ggml_tensor *gate, const ggml_tensor *glu) {
    if (!gate_up_pair_ok(up, gate, glu)) return false;
    const ggml_tensor *w = up->src[0], *x = up->src[1];
    for (int i = 2; i < GGML_MAX_DIMS; ++i)
        if (w->ne[i] != 1 || x->ne[i] != 1) return false;
    if (x->type != GGML_TYPE_F32 || x->nb[0] != 4 || x->nb[1] % 4 != 0 || glu->nb[1] % 4 != 0) return false;
    return hip_qmm_mul_mat_glu_fused(w->type, w->ne[0], w->ne[1], x->ne[1]) == 1;
}

bool launch_fused_mmq(BackendCtx *ctx, const ggml_tensor *up, const ggml_tensor *gate, const ggml_tensor *out,
                      bool *ok) {
    const ggml_tensor *w = up->src[0], *x = up->src[1];
    const int64_t K = w->ne[0], M = w->ne[1], N = x->ne[1];
    if (overlaps(out->data, nbytes(out), x->data, nbytes(x)) || lands_on_weights(out->data, nbytes(out), up, gate))
        return false;
    void *ws = workspace(ctx, hip_qmm_mul_mat_glu_workspace_size(w->type, K, M, N));
    const int rc = hip_qmm_mul_mat_glu(w->type, w->data, gate->src[0]->data, K, M, (int64_t)w->nb[1],
                                       static_cast<const float *>(x->data), N, (int64_t)(x->nb[1] / 4),
                                       out->op_params[0], op_param_f32(out, 2), op_param_f32(out, 3),
                                       static_cast<float *>(out->data), (int64_t)(out->nb[1] / 4), ws, ctx->ws_size,
                                       ctx->stream);
    *ok = report(rc, "hip_qmm_mul_mat_glu", out);
    return true;
}

// MUL_MAT_ID over more than 8 tokens: the grouped fused MMQ, with the layout
// hip_qmm_mul_mat_id addresses (rows (t, i11) of x and (t, s) of dst dense).
bool gate_up_id_mmq_fusable(const ggml_tensor *up, const ggml_tensor *gate, const ggml_tensor *glu) {
    if (!gate_up_pair_ok(up, gate, glu)) return false;
    const ggml_tensor *w = up->src[0], *x = up->src[1];
    if (glu->nb[2] != (size_t)glu->ne[1] * glu->nb[1] || glu->nb[1] % 4) return false;
    if (x->nb[2] != (size_t)x->ne[1] * x->nb[1] || x->nb[1] % 4 || x->nb[0] != 4) return false;
    return x->ne[2] > 8 && w->ne[0] % 256 == 0;
}

bool launch_fused_id_mmq(BackendCtx *ctx, const ggml_tensor *up, const ggml_tensor *gate, const ggml_tensor *out,
                         bool *ok) {
    const ggml_tensor *w = up->src[0], *x = up->src[1], *ids = up->src[2];
    const int64_t K = w->ne[0], M = w->ne[1], n_as = w->ne[2];
    const int64_t ne11 = x->ne[1], n_tokens = x->ne[2], n_ids = ids->ne[0];
    const size_t ob = nbytes(out);
    if (overlaps(out->data, ob, x->data, nbytes(x)) || overlaps(out->data, ob, ids->data, nbytes(ids)) ||
        lands_on_weights(out->data, ob, up, gate))
        return false;
    void *ws = workspace(ctx, hip_qmm_mul_mat_id_workspace_size(w->type, K, n_as, ne11, n_tokens, n_ids));
    const int rc = hip_qmm_mul_mat_id_glu(
        w->type, w->data, gate->src[0]->data, K, M, (int64_t)w->nb[1], (int64_t)w->nb[2], n_as,
        static_cast<const float *>(x->data), ne11, n_tokens, (int64_t)(x->nb[1] / 4),
        static_cast<const int32_t *>(ids->data), n_ids, (int64_t)(ids->nb[1] / 4), out->op_params[0],
        op_param_f32(out, 2), op_param_f32(out, 3), static_cast<float *>(out->data), (int64_t)(out->nb[1] / 4), ws,
        ctx->ws_size, ctx->stream);
    *ok = report(rc, "hip_qmm_mul_mat_id_glu", out);
    return true;
}

// ---- shared expert: a routed {MUL_MAT_ID, MUL_MAT_ID, GLU} and a shared
// expert's {MUL_MAT, MUL_MAT, GLU} on the same tokens in one launch (the
// reference's shared_up / shared_gate / shared_dst fusion,
// src/ggml/cuda/fusion.zig:930-955, mmvq.zig:300-320, 574-590).

// Nodes idx[0..n) but the outputs are read only inside the set, are not graph
// outputs and are not views (ggml_can_fuse_subgraph_ext, src/ggml/graph.zig:1207-1250).
bool set_is_closed(const ggml_cgraph *g, const int *idx, int n, const ggml_tensor *out_a, const ggml_tensor *out_b) {
    for (int a = 0; a < n; ++a) {
        const ggml_tensor *t = g->nodes[idx[a]];
        if (t == out_a || t == out_b) continue;
        if ((t->flags & GGML_TENSOR_FLAG_OUTPUT) || t->view_src) return false;
        int uses = 0;
        for (int b = 0; b < n; ++b)
            for (int k = 0; k < GGML_MAX_SRC; ++k) uses += g->nodes[idx[b]]->src[k] == t;
        if (use_count(g, t) != uses) return false;
    }
    return true;
}

// Whether {a, b} are the nodes k and k + 1 in either order.
bool node_pair(const ggml_cgraph *g, int k, const ggml_tensor *a, const ggml_tensor *b) {
    return (a == g->nodes[k] && b == g->nodes[k + 1]) || (b == g->nodes[k] && a == g->nodes[k + 1]);
}

// A split, non-swapped f32 GLU of an op the fused kernels apply.
bool fusable_glu(const ggml_tensor *glu) {
    const int op = glu->op_params[0];
    return (op == HIP_QMM_GLU_GEGLU || op == HIP_QMM_GLU_SWIGLU || op == HIP_QMM_GLU_SWIGLU_OAI ||
            op == HIP_QMM_GLU_SWIGLU_CLAMP) &&
           glu->op_params[1] == 0 && glu->src[1] && glu->type == GGML_TYPE_F32 && glu->nb[0] == 4;
}

bool same_weights(const ggml_tensor *a, const ggml_tensor *b) {
    if (a->type != b->type || !same_shape(a, b)) return false;
    for (int i = 0; i < GGML_MAX_DIMS; ++i)
        if (a->nb[i] != b->nb[i]) return false;
    return true;
}

// ggml_cuda_match_shared_expert (src/ggml/cuda/fusion.zig:853-905): the
// routed experts' gate / up / GLU at r and a shared expert's at s, checks
// that do not depend on the batch size (graph_optimize gives every batch the
// same order; try_fuse checks the batch).
bool match_shared_expert(const ggml_cgraph *g, int r, int s) {
    if (r + 2 >= g->n_nodes || s + 2 >= g->n_nodes || s < r + 3) return false;
    const int idx[6] = {r, r + 1, r + 2, s, s + 1, s + 2};
    const int ops[6] = {GGML_OP_MUL_MAT_ID, GGML_OP_MUL_MAT_ID, GGML_OP_GLU, GGML_OP_MUL_MAT, GGML_OP_MUL_MAT, GGML_OP_GLU};
    for (int k = 0; k < 6; ++k)
        if (g->nodes[idx[k]]->op != ops[k] || !ggml_backend_hip_op_supported(g->nodes[idx[k]])) return false;
    const ggml_tensor *routed = g->nodes[r + 2], *shared = g->nodes[s + 2];
    if (!set_is_closed(g, idx, 6, routed, shared)) return false;
    const ggml_tensor *gate = routed->src[0], *up = routed->src[1];
    const ggml_tensor *sgate = shared->src[0], *sup = shared->src[1];
    if (!node_pair(g, r, gate, up) || !node_pair(g, s, sgate, sup) || !fusable_glu(routed) || !fusable_glu(shared))
        return false;
    if (routed->op_params[0] != shared->op_params[0] || routed->op_params[2] != shared->op_params[2] ||
        routed->op_params[3] != shared->op_params[3])
        return false;
    if (!same_weights(up->src[0], gate->src[0]) || up->src[1] != gate->src[1] || up->src[2] != gate->src[2] ||
        !same_weights(sup->src[0], sgate->src[0]) || sup->src[1] != sgate->src[1])
        return false;
    const ggml_tensor *input = up->src[1], *w = up->src[0], *sw = sup->src[0], *sx = sup->src[1];
    if (input->op != GGML_OP_RESHAPE || input->src[0] != sx || input->ne[1] != 1 || input->ne[3] != 1 ||
        !contiguous(input) || !contiguous(sx) || sx->ne[2] != 1 || sx->ne[3] != 1)
        return false;
    if (w->type != sw->type || w->ne[0] != sw->ne[0] || w->ne[1] != sw->ne[1] || w->nb[1] != sw->nb[1] ||
        w->ne[3] != 1 || sw->ne[2] != 1 || sw->ne[3] != 1 || !contiguous(sw) || !contiguous(sgate->src[0]))
        return false;
    if (!contiguous(routed) || !contiguous(shared) || sw->op != GGML_OP_NONE || sgate->src[0]->op != GGML_OP_NONE)
        return false;
    return true;
}

// The routed and shared lanes at i .. i+5 in one launch, when the batch fits
// the fused ids kernel; false leaves them to run unfused.
bool launch_shared_expert(BackendCtx *ctx, const ggml_cgraph *g, int i, bool *ok) {
    const ggml_tensor *routed = g->nodes[i + 2], *shared = g->nodes[i + 5];
    const ggml_tensor *gate = routed->src[0], *up = routed->src[1], *sgate = shared->src[0], *sup = shared->src[1];
    if (!gate_up_id_fusable(up, gate, routed)) return false;
    const ggml_tensor *w = up->src[0], *x = up->src[1], *ids = up->src[2];
    const size_t walign = weight_align(w->type);
    const int64_t K = w->ne[0], M = w->ne[1], n_tokens = x->ne[2];
    if ((uintptr_t)sup->src[0]->data % walign || (uintptr_t)sgate->src[0]->data % walign) return false;
    if (shared->ne[0] != M || shared->ne[1] != n_tokens || shared->nb[1] % 4 ||
        n_tokens * (ids->ne[0] + 1) > 65535)
        return false;
    const size_t ob = nbytes(routed), sb = nbytes(shared);
    if (overlaps(routed->data, ob, x->data, nbytes(x)) || overlaps(routed->data, ob, ids->data, nbytes(ids)) ||
        overlaps(shared->data, sb, x->data, nbytes(x)) || overlaps(shared->data, sb, ids->data, nbytes(ids)) ||
        overlaps(routed->data, ob, shared->data, sb) || lands_on_weights(routed->data, ob, up, gate) ||
        lands_on_weights(routed->data, ob, sup, sgate) || lands_on_weights(shared->data, sb, up, gate) ||
        lands_on_weights(shared->data, sb, sup, sgate))
        return false;
    const int rc = hip_qmm_mul_mat_id_vec_fused_shared(
        w->type, w->data, gate->src[0]->data, K, M, (int64_t)w->nb[1], (int64_t)w->nb[2], w->ne[2],
        static_cast<const float *>(x->data), n_tokens, (int64_t)(x->nb[2] / 4), static_cast<const int32_t *>(ids->data),
        ids->ne[0], (int64_t)(ids->nb[1] / 4), routed->op_params[0], op_param_f32(routed, 2),
        op_param_f32(routed, 3), static_cast<float *>(routed->data), (int64_t)(routed->nb[1] / 4),
        sup->src[0]->data, sgate->src[0]->data, static_cast<float *>(shared->data), (int64_t)(shared->nb[1] / 4),
        ctx->stream);
    *ok = report(rc, "hip_qmm_mul_mat_id_vec_fused_shared", routed);
    return true;
}

// ---- MUL_MAT_ID bias lanes (ADD_ID; fusion.zig:1308-1360 gated,
// :1482-1520 one lane): the ADD_ID reads the MUL_MAT_ID as src0, with the same
// ids, and its src1 is the per-expert bias [nrows, n_as].
const ggml_tensor *id_bias_of(const ggml_tensor *add_id, const ggml_tensor *mm) {
    if (add_id->op != GGML_OP_ADD_ID || add_id->src[0] != mm || add_id->src[2] != mm->src[2]) return nullptr;
    const ggml_tensor *b = add_id->src[1], *w = mm->src[0];
    if (!b || b->type != GGML_TYPE_F32 || b->nb[0] != 4 || b->nb[1] % 4 || b->ne[0] != w->ne[1] ||
        b->ne[1] != w->ne[2] || !same_shape(add_id, mm))
        return nullptr;
    return b;
}

// A lone MUL_MAT_ID the fused ids kernel takes (the gated check without a gate).
bool id_lane_fusable(const ggml_tensor *mm, const ggml_tensor *out) {
    const ggml_tensor *w = mm->src[0], *x = mm->src[1];
    if (out->type != GGML_TYPE_F32 || out->nb[0] != 4 || out->nb[1] % 4 ||
        out->nb[2] != (size_t)out->ne[1] * out->nb[1])
        return false;
    const int64_t K = w->ne[0], n_tokens = x->ne[2];
    const size_t walign = weight_align(w->type);
    return n_tokens <= 8 && n_tokens * out->ne[1] <= 65535 && K % 32 == 0 && K <= 32768 &&
           (uintptr_t)x->data % 16 == 0 && x->nb[1] % 16 == 0 && x->nb[2] == (size_t)x->ne[1] * x->nb[1] &&
           (uintptr_t)w->data % walign == 0 && w->nb[1] % walign == 0 && w->nb[2] % walign == 0;
}

bool launch_fused_id_bias(BackendCtx *ctx, const ggml_tensor *up, const ggml_tensor *gate, const ggml_tensor *ub,
                          const ggml_tensor *gb, const ggml_tensor *out, bool *ok) {
    const ggml_tensor *w = up->src[0], *x = up->src[1], *ids = up->src[2];
    const int64_t K = w->ne[0], M = w->ne[1];
    if (gb && gb->nb[1] != ub->nb[1]) return false;  // one expert stride for both biases
    const size_t ob = nbytes(out);
    if (overlaps(out->data, ob, x->data, nbytes(x)) || overlaps(out->data, ob, ids->data, nbytes(ids)) ||
        overlaps(out->data, ob, ub->data, nbytes(ub)) || (gb && overlaps(out->data, ob, gb->data, nbytes(gb))) ||
        lands_on_weights(out->data, ob, up, gate))
        return false;
    const int rc = hip_qmm_mul_mat_id_vec_fused_bias(
        w->type, w->data, gate ? gate->src[0]->data : nullptr, K, M, (int64_t)w->nb[1], (int64_t)w->nb[2], w->ne[2],
        static_cast<const float *>(x->data), x->ne[1], x->ne[2], (int64_t)(x->nb[1] / 4),
        static_cast<const int32_t *>(ids->data), ids->ne[0], (int64_t)(ids->nb[1] / 4),
        static_cast<const float *>(ub->data), gb ? static_cast<const float *>(gb->data) : nullptr,
        (int64_t)(ub->nb[1] / 4), gate ? out->op_params[0] : 0, gate ? op_param_f32(out, 2) : 0.0f,
        gate ? op_param_f32(out, 3) : 0.0f, static_cast<float *>(out->data), (int64_t)(out->nb[1] / 4), ctx->stream);
    *ok = report(rc, "hip_qmm_mul_mat_id_vec_fused_bias", out);
    return true;
}

// Nodes consumed by a fused launch at node i (0: none); *ok false on a failed launch.
int try_fuse(BackendCtx *ctx, const ggml_cgraph *g, int i, bool *ok) {
    if (fusion_disabled()) return 0;
    auto node = [&](int k) { return k < g->n_nodes ? g->nodes[k] : nullptr; };
    auto is = [&](int k, int op) { return node(k) && node(k)->op == op && ggml_backend_hip_op_supported(node(k)); };
    if (g->nodes[i]->op == GGML_OP_MUL_MAT_ID) {
        if (match_shared_expert(g, i, i + 3) && launch_shared_expert(ctx, g, i, ok)) return 6;
        if (is(i + 1, GGML_OP_ADD_ID) && is(i + 2, GGML_OP_MUL_MAT_ID) && is(i + 3, GGML_OP_ADD_ID) &&
            is(i + 4, GGML_OP_GLU)) {
            // which lane gates follows from the GLU's sources (fusion.zig:1313-1325)
            const ggml_tensor *glu = node(i + 4), *ma = node(i), *mb = node(i + 2);
            const ggml_tensor *gbn = glu->src[0], *ubn = glu->src[1];
            const bool a_gates = gbn == node(i + 1) && ubn == node(i + 3);
            const bool b_gates = gbn == node(i + 3) && ubn == node(i + 1);
            if (a_gates || b_gates) {
                const ggml_tensor *gate = a_gates ? ma : mb, *up = a_gates ? mb : ma;
                const ggml_tensor *gb = id_bias_of(gbn, gate), *ub = id_bias_of(ubn, up);
                if (gb && ub && !in_run(g, i, 5, gb) && !in_run(g, i, 5, ub) && gate_up_id_fusable(up, gate, glu) &&
                    run_is_closed(g, i, 5, glu) && launch_fused_id_bias(ctx, up, gate, ub, gb, glu, ok))
                    return 5;
            }
        }
        if (is(i + 1, GGML_OP_MUL_MAT_ID) && is(i + 2, GGML_OP_GLU)) {
            const ggml_tensor *glu = node(i + 2);
            const ggml_tensor *gate = glu->src[0], *up = glu->src[1];
            const bool pair = (gate == node(i) && up == node(i + 1)) || (gate == node(i + 1) && up == node(i));
            if (pair && gate_up_id_fusable(up, gate, glu) && run_is_closed(g, i, 3, glu) &&
                launch_fused_id(ctx, up, gate, glu, ok))
                return 3;
            if (pair && gate_up_id_mmq_fusable(up, gate, glu) && run_is_closed(g, i, 3, glu) &&
                launch_fused_id_mmq(ctx, up, gate, glu, ok))
                return 3;
        }
        if (is(i + 1, GGML_OP_ADD_ID)) {
            const ggml_tensor *mm = node(i), *add = node(i + 1);
            const ggml_tensor *b = id_bias_of(add, mm);
            if (b && !in_run(g, i, 2, b) && id_lane_fusable(mm, add) && run_is_closed(g, i, 2, add) &&
                launch_fused_id_bias(ctx, mm, nullptr, b, nullptr, add, ok))
                return 2;
        }
        return 0;
    }
    if (g->nodes[i]->op != GGML_OP_MUL_MAT) return 0;
    if (is(i + 1, GGML_OP_ADD) && is(i + 2, GGML_OP_MUL_MAT) && is(i + 3, GGML_OP_ADD) && is(i + 4, GGML_OP_GLU)) {
        const ggml_tensor *glu = node(i + 4);
        const ggml_tensor *ma = node(i), *aa = node(i + 1), *mb = node(i + 2), *ab = node(i + 3);
        const ggml_tensor *ba = bias_of(aa, ma), *bb = bias_of(ab, mb);
        // which lane gates follows from the GLU's sources (fusion.zig:1313-1325)
        const bool a_gates = glu->src[0] == aa && glu->src[1] == ab;
        const bool b_gates = glu->src[0] == ab && glu->src[1] == aa;
        if (bias_ok(ba, ma) && bias_ok(bb, mb) && !in_run(g, i, 5, ba) && !in_run(g, i, 5, bb) &&
            (a_gates || b_gates)) {
            const ggml_tensor *gate = a_gates ? ma : mb, *up = a_gates ? mb : ma;
            const ggml_tensor *gb = a_gates ? ba : bb, *ub = a_gates ? bb : ba;
            if (gate_up_fusable(up, gate, glu) && run_is_closed(g, i, 5, glu) &&
                launch_fused(ctx, up, gate, ub, gb, glu, ok))
                return 5;
        }
    }
    if (is(i + 1, GGML_OP_MUL_MAT) && is(i + 2, GGML_OP_GLU)) {
        const ggml_tensor *glu = node(i + 2);
        const ggml_tensor *gate = glu->src[0], *up = glu->src[1];
        const bool pair = (gate == node(i) && up == node(i + 1)) || (gate == node(i + 1) && up == node(i));
        if (pair && gate_up_fusable(up, gate, glu) && run_is_closed(g, i, 3, glu) &&
            launch_fused(ctx, up, gate, nullptr, nullptr, glu, ok))
            return 3;
        if (pair && gate_up_mmq_fusable(up, gate, glu) && run_is_closed(g, i, 3, glu) &&
            launch_fused_mmq(ctx, up, gate, glu, ok))
            return 3;
    }
    if (is(i + 1, GGML_OP_ADD)) {
        const ggml_tensor *mm = node(i), *add = node(i + 1);
        const ggml_tensor *b = bias_of(add, mm);
        if (bias_ok(b, mm) && !in_run(g, i, 2, b) && vec_fusable(mm) && same_shape(add, mm) &&
            run_is_closed(g, i, 2, add) &&
            launch_fused(ctx, mm, nullptr, b, nullptr, add, ok))
            return 2;
    }
    return 0;
}

ggml_status be_graph_compute(ggml_backend_t be, ggml_cgraph *g) {
    BackendCtx *ctx = be_ctx(be);
    HIP_CHECK(hipSetDevice(ctx->device));
    for (int i = 0; i < g->n_nodes; ++i) {
        const ggml_tensor *node = g->nodes[i];
        if (is_noop(node->op) || nbytes(node) == 0) continue;
        if (!ggml_backend_hip_op_supported(node)) {
            std::fprintf(stderr, "ggml-hip: node '%s' (op %d) is not supported by this backend\n", node->name,
                         (int)node->op);
            return GGML_STATUS_FAILED;
        }
        bool ok = true;
        if (const int n = try_fuse(ctx, g, i, &ok)) {
            if (!ok) return GGML_STATUS_FAILED;
            i += n - 1;
            continue;
        }
        switch (node->op) {
        case GGML_OP_MUL_MAT: ok = run_mul_mat(ctx, node); break;
        case GGML_OP_MUL_MAT_ID: ok = run_mul_mat_id(ctx, node); break;
        case GGML_OP_GLU: ok = run_glu(ctx, node); break;
        case GGML_OP_ADD_ID: ok = run_add_id(ctx, node); break;
        default: ok = run_add(ctx, node); break;
        }
        if (!ok) return GGML_STATUS_FAILED;
    }
    return GGML_STATUS_SUCCESS;
}

// The reference's graph_optimize grouping for the shared expert
// (src/ggml/cuda/graph.zig:826-848): after each routed gate / up / GLU, the
// first matching shared-expert triple before the next routed pair is moved
// up to follow it (it reads only the layer input and its weights, so the
// order stays topological), and the routed input and ids are kept allocated
// until the shared GLU has run, so the fused launch's operands cannot alias
// its second output.  Then, as graph.zig:849-862 does, every gate / up / GLU
// run the fused MMQ takes keeps its nodes and their sources (weights,
// activations, ids) allocated until the GLU (addAllocDeps, graph.zig:753-770),
// so the GLU's result cannot be placed on memory the fused kernel still
// reads.  Nothing moves with fusion disabled.
void add_alloc_deps(ggml_cgraph *g, ggml_backend_graph_optimize_params *params, int start, int last) {
    for (int i = start; i < last; ++i) {
        ggml_tensor *n = g->nodes[i];
        params->add_alloc_dep(params->user_data, n, g->nodes[last]);
        for (ggml_tensor *s : n->src)
            if (s) params->add_alloc_dep(params->user_data, s, g->nodes[last]);
    }
}

void be_graph_optimize(ggml_backend_t, ggml_cgraph *g, ggml_backend_graph_optimize_params *params) {
    if (fusion_disabled() || !g) return;
    for (int r = 0; r + 5 < g->n_nodes; ++r) {
        if (g->nodes[r]->op != GGML_OP_MUL_MAT_ID) continue;
        for (int j = r + 3; j + 2 < g->n_nodes; ++j) {
            if (g->nodes[j]->op == GGML_OP_MUL_MAT_ID && g->nodes[j + 1]->op == GGML_OP_MUL_MAT_ID) break;
            if (g->nodes[j]->op != GGML_OP_MUL_MAT || !match_shared_expert(g, r, j)) continue;
            std::rotate(g->nodes + r + 3, g->nodes + j, g->nodes + j + 3);
            const ggml_tensor *up = g->nodes[r + 2]->src[1];
            if (params && params->add_alloc_dep) {
                params->add_alloc_dep(params->user_data, up->src[1], g->nodes[r + 5]);
                params->add_alloc_dep(params->user_data, up->src[2], g->nodes[r + 5]);
            }
            r += 5;
            break;
        }
    }
    if (!params || !params->add_alloc_dep) return;
    for (int i = 0; i + 2 < g->n_nodes; ++i) {
        const ggml_tensor *glu = g->nodes[i + 2], *n0 = g->nodes[i], *n1 = g->nodes[i + 1];
        if (glu->op != GGML_OP_GLU || n0->op != n1->op) continue;
        const ggml_tensor *gate = glu->src[0], *up = glu->src[1];
        if (!((gate == n0 && up == n1) || (gate == n1 && up == n0))) continue;
        const bool mmq = n0->op == GGML_OP_MUL_MAT     ? gate_up_mmq_fusable(up, gate, glu)
                         : n0->op == GGML_OP_MUL_MAT_ID ? gate_up_id_mmq_fusable(up, gate, glu)
                                                        : false;
        if (!mmq) continue;
        add_alloc_deps(g, params, i, i + 2);
        i += 2;
    }
}

void be_event_record(ggml_backend_t be, ggml_backend_event_t ev) {
    HIP_CHECK(hipEventRecord(static_cast<hipEvent_t>(ev->context), be_ctx(be)->stream));
}

void be_event_wait(ggml_backend_t be, ggml_backend_event_t ev) {
    if (!ggml_backend_is_hip(be)) {
        std::fprintf(stderr, "ggml-hip: event_wait on a foreign backend\n");
        std::abort();
    }
    HIP_CHECK(hipStreamWaitEvent(be_ctx(be)->stream, static_cast<hipEvent_t>(ev->context), 0));
}

const ggml_backend_i backend_iface = {
    be_name,
    be_free,
    be_set_tensor_async,
    be_get_tensor_async,
    be_set_tensor_2d_async,
    be_get_tensor_2d_async,
    be_cpy_tensor_async,
    be_synchronize,
    nullptr,
    nullptr,
    nullptr,
    nullptr,
    be_graph_compute,
    be_event_record,
    be_event_wait,
    be_graph_optimize,
};

// ---------------------------------------------------------------- device vtable

DeviceCtx *dev_ctx(ggml_backend_dev_t dev) { return static_cast<DeviceCtx *>(dev->context); }

const char *dev_name(ggml_backend_dev_t dev) { return dev_ctx(dev)->name; }
const char *dev_description(ggml_backend_dev_t dev) { return dev_ctx(dev)->description; }
void dev_memory(ggml_backend_dev_t dev, size_t *free, size_t *total) {
    ggml_backend_hip_get_device_memory(dev_ctx(dev)->device, free, total);
}
ggml_backend_dev_type dev_type(ggml_backend_dev_t) { return GGML_BACKEND_DEVICE_TYPE_GPU; }

void dev_props(ggml_backend_dev_t dev, ggml_backend_dev_props *p) {
    p->name = dev_name(dev);
    p->description = dev_description(dev);
    p->type = dev_type(dev);
    p->device_id = dev_ctx(dev)->pci_bus_id[0] ? dev_ctx(dev)->pci_bus_id : nullptr;
    dev_memory(dev, &p->memory_free, &p->memory_total);
    p->caps.async = true;
    p->caps.host_buffer = true;
    p->caps.buffer_from_host_ptr = false;
    p->caps.events = true;
    p->caps.mmap_support = true;
}

ggml_backend_t dev_init_backend(ggml_backend_dev_t dev, const char *) {
    return ggml_backend_hip_init(dev_ctx(dev)->device);
}
ggml_backend_buffer_type_t dev_buffer_type(ggml_backend_dev_t dev) {
    return ggml_backend_hip_buffer_type(dev_ctx(dev)->device);
}
ggml_backend_buffer_type_t dev_host_buffer_type(ggml_backend_dev_t) { return ggml_backend_hip_host_buffer_type(); }
bool dev_supports_op(ggml_backend_dev_t, const ggml_tensor *op) { return ggml_backend_hip_op_supported(op); }
bool dev_supports_buft(ggml_backend_dev_t dev, ggml_backend_buffer_type_t buft) {
    return buft_is_hip(buft) && buft->device == dev;
}

// Ops whose weights sit in host memory are worth shipping to the GPU from a
// batch of 32 columns on (get_op_batch_size / offload_op,
// cuda/backend.zig:992-1006, the default GGML_OP_OFFLOAD_MIN_BATCH).
bool dev_offload_op(ggml_backend_dev_t, const ggml_tensor *op) {
    const int64_t batch = op->op == GGML_OP_MUL_MAT ? op->ne[1] : op->op == GGML_OP_MUL_MAT_ID ? op->ne[2] : 0;
    return batch >= 32 && ggml_backend_hip_op_supported(op);
}

ggml_backend_event_t dev_event_new(ggml_backend_dev_t dev) {
    HIP_CHECK(hipSetDevice(dev_ctx(dev)->device));
    hipEvent_t e;
    HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    return new ggml_backend_event{dev, e};
}
void dev_event_free(ggml_backend_dev_t, ggml_backend_event_t ev) {
    HIP_CHECK(hipEventDestroy(static_cast<hipEvent_t>(ev->context)));
    delete ev;
}
void dev_event_synchronize(ggml_backend_dev_t, ggml_backend_event_t ev) {
    HIP_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(ev->context)));
}

const ggml_backend_device_i device_iface = {
    dev_name,      dev_description,      dev_memory,       dev_type,       dev_props,
    dev_init_backend, dev_buffer_type,   dev_host_buffer_type, nullptr,    dev_supports_op,
    dev_supports_buft, dev_offload_op,   dev_event_new,    dev_event_free, dev_event_synchronize,
};

// ---------------------------------------------------------------- registry

struct Registry {
    std::mutex mu;
    bool ready = false;
    ggml_backend_reg reg{};
    ggml_backend_device devices[GGML_HIP_MAX_DEVICES]{};
    DeviceCtx dev_ctx[GGML_HIP_MAX_DEVICES]{};
    int count = 0;
    bool buft_ready = false;
    ggml_backend_buffer_type bufts[GGML_HIP_MAX_DEVICES]{};
    BufferTypeCtx buft_ctx[GGML_HIP_MAX_DEVICES]{};
    bool host_ready = false;
    ggml_backend_buffer_type host_buft{};
};

Registry &registry() {
    static Registry r;
    return r;
}

const char *reg_name(ggml_backend_reg_t) { return GGML_HIP_NAME; }
size_t reg_device_count(ggml_backend_reg_t) { return (size_t)registry().count; }
ggml_backend_dev_t reg_device(ggml_backend_reg_t, size_t i) {
    Registry &r = registry();
    if (i >= (size_t)r.count) {
        std::fprintf(stderr, "ggml-hip: device index %zu out of range\n", i);
        std::abort();
    }
    return &r.devices[i];
}
void *reg_proc_address(ggml_backend_reg_t, const char *name) {
    if (!name) return nullptr;
    if (!std::strcmp(name, "ggml_backend_register_host_buffer"))
        return reinterpret_cast<void *>(&ggml_backend_hip_register_host_buffer);
    if (!std::strcmp(name, "ggml_backend_unregister_host_buffer"))
        return reinterpret_cast<void *>(&ggml_backend_hip_unregister_host_buffer);
    return nullptr;
}

const ggml_backend_reg_i reg_iface = {reg_name, reg_device_count, reg_device, reg_proc_address};

void describe(int device, char *out, size_t n) {
    hipDeviceProp_t prop;
    HIP_CHECK(hipGetDeviceProperties(&prop, device));
    std::snprintf(out, n, "%s", prop.name);
}

}  // namespace

// ================================================================ C ABI

extern "C" {

bool ggml_backend_hip_op_supported(const ggml_tensor *op) {
    if (!op) return false;
    if (is_noop(op->op)) return true;
    // Unless the fusion is on (GGML_HIP_FUSION=1) the GLU and bias-add nodes
    // have no reason to be on the device: the answer is MUL_MAT / MUL_MAT_ID
    // and the no-op views, and everything else stays on the CPU.
    if ((op->op == GGML_OP_GLU || op->op == GGML_OP_ADD || op->op == GGML_OP_ADD_ID) && fusion_disabled())
        return false;
    if (op->op == GGML_OP_GLU) {
        // f32 GLU of a device op (glu_op_supported), split or one-tensor form
        const ggml_tensor *a = op->src[0], *b = op->src[1];
        if (!a || !f32_rows(a) || !f32_rows(op) || !glu_op_supported(op->op_params[0])) return false;
        if (b) return f32_rows(b) && same_shape(a, b) && same_shape(op, a);
        if (a->ne[0] != 2 * op->ne[0]) return false;
        for (int i = 1; i < GGML_MAX_DIMS; ++i)
            if (a->ne[i] != op->ne[i]) return false;
        return true;
    }
    if (op->op == GGML_OP_ADD) {
        // same-shape f32 add (the bias add of the GEMV fusion); no broadcasting
        const ggml_tensor *a = op->src[0], *b = op->src[1];
        return a && b && f32_rows(a) && f32_rows(b) && f32_rows(op) && same_shape(a, b) && same_shape(a, op);
    }
    if (op->op == GGML_OP_ADD_ID) {
        // f32 rows plus a row of b chosen per (slot, token) by int32 ids (the
        // per-expert bias of an MoE projection, ggml_add_id, ops.zig:113-130)
        const ggml_tensor *a = op->src[0], *b = op->src[1], *ids = op->src[2];
        if (!a || !b || !ids || !f32_rows(a) || !f32_rows(b) || !f32_rows(op) || !same_shape(a, op)) return false;
        if (ids->type != GGML_TYPE_I32 || ids->nb[0] != 4 || ids->nb[1] % 4 != 0) return false;
        return b->ne[0] == a->ne[0] && ids->ne[0] == a->ne[1] && ids->ne[1] == a->ne[2] && a->ne[3] == 1 &&
               b->ne[2] == 1 && b->ne[3] == 1;
    }
    if (op->op != GGML_OP_MUL_MAT && op->op != GGML_OP_MUL_MAT_ID) return false;
    const ggml_tensor *a = op->src[0], *b = op->src[1];
    if (!a || !b || !weight_type(a->type) || b->type != GGML_TYPE_F32 || op->type != GGML_TYPE_F32) return false;
    const TypeInfo ta = type_info(a->type);
    // rows of elements, each row read with its own stride (cuda/supports.zig:111-114)
    if (a->nb[0] != ta.size || b->nb[0] != 4 || op->nb[0] != 4) return false;
    if (a->ne[0] % ta.blck != 0 || a->ne[0] > ((int64_t)1 << 30) || b->ne[0] != a->ne[0]) return false;
    if (b->nb[1] % 4 != 0 || op->nb[1] % 4 != 0) return false;
    if (op->op == GGML_OP_MUL_MAT) {
        if (a->ne[2] <= 0 || a->ne[3] <= 0 || b->ne[2] % a->ne[2] != 0 || b->ne[3] % a->ne[3] != 0) return false;
        return op->ne[0] == a->ne[1] && op->ne[1] == b->ne[1];
    }
    // MUL_MAT_ID: src2 = ids [n_used, n_tokens] I32
    const ggml_tensor *ids = op->src[2];
    if (!ids || ids->type != GGML_TYPE_I32 || ids->nb[0] != 4 || ids->nb[1] % 4 != 0) return false;
    if (a->ne[0] % 256 != 0 || a->ne[2] > 1024 || a->ne[3] != 1) return false;
    const int64_t n_ids = ids->ne[0], n_tokens = ids->ne[1];
    if (b->ne[1] != 1 && b->ne[1] != n_ids) return false;
    if (b->ne[2] != n_tokens || b->ne[3] != 1 || op->ne[1] != n_ids || op->ne[2] != n_tokens) return false;
    // activations and results as dense rows: (token, slot) at (t*rows + s) * row stride
    if (b->nb[2] != (size_t)b->ne[1] * b->nb[1] || op->nb[2] != (size_t)op->ne[1] * op->nb[1]) return false;
    return n_tokens * n_ids <= 0x7FFFFFFF;
}

size_t ggml_backend_hip_tensor_alloc_size(const ggml_tensor *t) {
    size_t size = nbytes(t);
    const int64_t ne0 = t->ne[0];
    // pad quantized rows to 512 elements (cuda/backend.zig:321-338)
    if (type_info(t->type).quantized && ne0 % ROW_PADDING != 0) size += row_size(t->type, ROW_PADDING - ne0 % ROW_PADDING);
    return size;
}

int ggml_backend_hip_get_device_count(void) { return device_count(); }

void ggml_backend_hip_get_device_description(int device, char *description, size_t description_size) {
    if (!description || !description_size) return;
    if (device < 0 || device >= device_count()) {
        description[0] = 0;
        return;
    }
    describe(device, description, description_size);
}

void ggml_backend_hip_get_device_memory(int device, size_t *free, size_t *total) {
    HIP_CHECK(hipSetDevice(device));
    HIP_CHECK(hipMemGetInfo(free, total));
}

bool ggml_backend_hip_register_host_buffer(void *, size_t) { return false; }
void ggml_backend_hip_unregister_host_buffer(void *) {}

ggml_backend_reg_t ggml_backend_hip_reg(void) {
    Registry &r = registry();
    std::lock_guard<std::mutex> lock(r.mu);
    if (!r.ready) {
        r.count = device_count();
        for (int i = 0; i < r.count; ++i) {
            DeviceCtx &c = r.dev_ctx[i];
            c.device = i;
            std::snprintf(c.name, sizeof c.name, GGML_HIP_NAME "%d", i);
            describe(i, c.description, sizeof c.description);
            char bus[64] = {0};
            if (hipDeviceGetPCIBusId(bus, sizeof bus, i) == hipSuccess) {
                for (char *p = bus; *p; ++p) *p = (char)std::tolower((unsigned char)*p);
                std::snprintf(c.pci_bus_id, sizeof c.pci_bus_id, "%s", bus);
            } else {
                (void)hipGetLastError();
            }
            r.devices[i].iface = device_iface;
            r.devices[i].reg = &r.reg;
            r.devices[i].context = &c;
        }
        r.reg.api_version = GGML_BACKEND_API_VERSION;
        r.reg.iface = reg_iface;
        r.reg.context = nullptr;
        r.ready = true;
    }
    return &r.reg;
}

ggml_backend_buffer_type_t ggml_backend_hip_buffer_type(int device) {
    ggml_backend_reg_t reg = ggml_backend_hip_reg();
    Registry &r = registry();
    std::lock_guard<std::mutex> lock(r.mu);
    if (device < 0 || device >= r.count) return nullptr;
    if (!r.buft_ready) {
        for (int i = 0; i < r.count; ++i) {
            r.buft_ctx[i].device = i;
            std::snprintf(r.buft_ctx[i].name, sizeof r.buft_ctx[i].name, GGML_HIP_NAME "%d", i);
            r.bufts[i].iface = buffer_type_iface;
            r.bufts[i].device = reg_device(reg, (size_t)i);
            r.bufts[i].context = &r.buft_ctx[i];
        }
        r.buft_ready = true;
    }
    return &r.bufts[device];
}

ggml_backend_buffer_type_t ggml_backend_hip_host_buffer_type(void) {
    ggml_backend_reg_t reg = ggml_backend_hip_reg();
    Registry &r = registry();
    std::lock_guard<std::mutex> lock(r.mu);
    if (!r.host_ready) {
        r.host_buft.iface = {hbuft_name, hbuft_alloc, nullptr, hbuft_alignment, hbuft_max_size,
                             hbuft_alloc_size, nullptr, hbuft_is_host};
        r.host_buft.device = r.count > 0 ? reg_device(reg, 0) : nullptr;
        r.host_buft.context = nullptr;
        r.host_ready = true;
    }
    return &r.host_buft;
}

ggml_backend_t ggml_backend_hip_init(int device) {
    if (device < 0 || device >= device_count()) {
        std::fprintf(stderr, "ggml-hip: invalid device %d\n", device);
        return nullptr;
    }
    ggml_backend_reg_t reg = ggml_backend_hip_reg();
    HIP_CHECK(hipSetDevice(device));
    auto *ctx = new BackendCtx{};
    ctx->device = device;
    std::snprintf(ctx->name, sizeof ctx->name, GGML_HIP_NAME "%d", device);
    HIP_CHECK(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
    auto *be = new ggml_backend{};
    be->guid = &hip_guid;
    be->iface = backend_iface;
    be->device = reg_device(reg, (size_t)device);
    be->context = ctx;
    return be;
}

bool ggml_backend_is_hip(ggml_backend_t backend) {
    return backend && backend->guid && std::memcmp(*backend->guid, hip_guid, sizeof(ggml_guid)) == 0;
}

int ggml_backend_score(void) { return device_count() > 0 ? 100 : 0; }

ggml_backend_reg_t ggml_backend_init(void) { return ggml_backend_hip_reg(); }

}  // extern "C"
