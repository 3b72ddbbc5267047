// llg_runtime.hip -- device handle, object registry, weight upload (GGUF bytes
// -> HBM row format), dequant, and the two Metal-parity entry points
// (metal/metal_bridge.h:7-20).
#include "llg_common.hpp"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <unordered_map>

struct LlgDevice {
    int device = 0;
    int cus = 0;
    hipStream_t stream = nullptr;
    // device address of this GPU's `scratch` array (null if the lookup failed;
    // scratch_err then holds its error)
    uint8_t *scratch = nullptr;
    hipError_t scratch_err = hipSuccess;
    std::unordered_map<int64_t, LlgObject *> objects;
    int64_t next_id = 1;
    void *ws = nullptr;
    size_t ws_bytes = 0;
    uint8_t *sync = nullptr;  // LLG_SYNC_BYTES, zeroed at allocation
    uint64_t *mvslots = nullptr;  // chunked matvecs' hand-off slots, zero between calls
    size_t mvslots_bytes = 0;
    int check_handoff = 0;  // LLG_CHECK_HANDOFF at creation (llg_dev_check)
    std::string last_error;
    bool tearing_down = false;  // llg_hip_free: every object is freed in one sweep
};

// Scratch of the allocation-free entry points: a fixed array in each GPU's
// memory, held until the process ends.  Host code never passes `scratch`
// itself to a kernel or copy (in host code the name is only a stand-in): it
// uses the address hipGetSymbolAddress returns for the current device, kept
// per device handle (LlgDevice::scratch).  Every call on one GPU shares the
// array, so calls that overlap on one GPU (several handles or streams) race.
static __device__ __align__(256) uint8_t scratch[LLG_SCRATCH_BYTES];

LlgDevice *llg_dev(LlgHipDevice h) { return reinterpret_cast<LlgDevice *>(h); }

uint8_t *llg_dev_scratch(LlgDevice *d, size_t bytes, int *rc) {
    *rc = 0;
    if (!d->scratch) {
        *rc = llg_hip_error(d, d->scratch_err, "scratch address lookup at init");
        return nullptr;
    }
    if (bytes > (size_t)LLG_SCRATCH_BYTES) {
        *rc = llg_set_error(d, LLG_E_SCRATCH,
                            "needs %zu bytes of scratch, above the fixed %zu of the "
                            "allocation-free entry points",
                            bytes, (size_t)LLG_SCRATCH_BYTES);
        return nullptr;
    }
    return d->scratch;
}
uint8_t *llg_dev_sync(LlgDevice *d, int *rc) {
    *rc = 0;
    if (d->sync) return d->sync;
    if (hipMalloc(&d->sync, LLG_SYNC_BYTES) != hipSuccess) {
        d->sync = nullptr;
        *rc = llg_set_error(d, LLG_E_NOMEM, "sync area allocation failed");
        return nullptr;
    }
    if (hipError_t e = hipMemsetAsync(d->sync, 0, LLG_SYNC_BYTES, d->stream); e != hipSuccess) {
        hipFree(d->sync);
        d->sync = nullptr;
        *rc = llg_hip_error(d, e, "sync area clear");
        return nullptr;
    }
    return d->sync;
}
uint64_t *llg_dev_mvslots(LlgDevice *d, size_t bytes, int *rc) {
    *rc = 0;
    if (bytes <= d->mvslots_bytes) return d->mvslots;
    size_t want = bytes < ((size_t)256 << 10) ? ((size_t)256 << 10) : bytes;
    want = (want + 4095) & ~(size_t)4095;
    if (d->mvslots) {  // every slot of the old area is zero again once the stream is idle
        hipStreamSynchronize(d->stream);
        hipFree(d->mvslots);
        d->mvslots = nullptr;
        d->mvslots_bytes = 0;
    }
    if (hipMalloc(&d->mvslots, want) != hipSuccess) {
        d->mvslots = nullptr;
        *rc = llg_set_error(d, LLG_E_NOMEM, "matvec slot area of %zu bytes failed", want);
        return nullptr;
    }
    if (hipError_t e = hipMemsetAsync(d->mvslots, 0, want, d->stream); e != hipSuccess) {
        hipFree(d->mvslots);
        d->mvslots = nullptr;
        *rc = llg_hip_error(d, e, "matvec slot area clear");
        return nullptr;
    }
    d->mvslots_bytes = want;
    return d->mvslots;
}
hipStream_t llg_dev_stream(LlgDevice *d) { return d->stream; }
int llg_dev_check(LlgDevice *d) { return d->check_handoff; }
int llg_device_id(LlgDevice *d) { return d->device; }
int llg_cu_count(LlgDevice *d) { return d->cus; }

int llg_set_error(LlgDevice *d, int code, const char *fmt, ...) {
    if (d) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        d->last_error = buf;
    }
    return code;
}

int llg_hip_error(LlgDevice *d, hipError_t e, const char *what) {
    return llg_set_error(d, (int)e, "%s: %s (hip error %d)", what, hipGetErrorString(e), (int)e);
}

LlgObject *llg_get(LlgDevice *d, int64_t h, int kind) {
    auto it = d->objects.find(h);
    if (it == d->objects.end() || it->second->released) return nullptr;
    if (kind && it->second->kind != kind) return nullptr;
    return it->second;
}

int64_t llg_register(LlgDevice *d, LlgObject *o) {
    int64_t id = d->next_id++;
    o->id_self = id;
    d->objects[id] = o;
    return id;
}

extern void llg_window_destroy(LlgDevice *d, LlgObject *o);
extern void llg_model_destroy(LlgDevice *d, LlgObject *o);

// Frees an object's state and memory (the caller has taken it out of the
// registry, or is sweeping the registry).
static void destroy_object(LlgDevice *d, LlgObject *o) {
    if (o->kind == LLG_KIND_WINDOW) llg_window_destroy(d, o);
    if (o->kind == LLG_KIND_MODEL) llg_model_destroy(d, o);
    if (o->d) hipFree(o->d);
    if (o->tiled) hipFree(o->tiled);
    delete o;
}

void llg_ref(LlgObject *o) {
    if (o) o->refs++;
}

void llg_unref(LlgDevice *d, LlgObject *o) {
    // during llg_hip_free the sweep frees every object (o may already be gone)
    if (!o || d->tearing_down) return;
    if (--o->refs == 0 && o->released) {
        d->objects.erase(o->id_self);
        destroy_object(d, o);
    }
}

void *llg_ws(LlgDevice *d, size_t bytes, int *rc) {
    *rc = 0;
    if (bytes <= d->ws_bytes) return d->ws;
    size_t want = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
    want = (want + 4095) & ~(size_t)4095;
    if (d->ws) {
        hipStreamSynchronize(d->stream);
        hipFree(d->ws);
        d->ws = nullptr;
        d->ws_bytes = 0;
    }
    hipError_t e = hipMalloc(&d->ws, want);
    if (e != hipSuccess) {
        d->ws = nullptr;
        *rc = llg_set_error(d, LLG_E_NOMEM, "workspace allocation of %zu bytes failed", want);
        return nullptr;
    }
    d->ws_bytes = want;
    return d->ws;
}

int llg_h2d(LlgDevice *d, void *dst, const void *src, size_t bytes) {
    if (!bytes) return 0;
    LLG_HIP_TRY(d, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, d->stream));
    return 0;
}

int llg_d2h(LlgDevice *d, void *dst, const void *src, size_t bytes) {
    if (!bytes) return 0;
    LLG_HIP_TRY(d, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, d->stream));
    return 0;
}

int llg_sync_dev(LlgDevice *d) {
    LLG_HIP_TRY(d, hipStreamSynchronize(d->stream));
    return 0;
}

// ---------------------------------------------------------------------------
// Repack: GGUF row bytes -> HBM row format (see llg_common.hpp).
// One thread per 32-element block (Q4_0/Q8_0) or per element (F16/F32).
// ---------------------------------------------------------------------------
__global__ void k_repack(const uint8_t *__restrict__ src, long long src_row_bytes,
                         uint8_t *__restrict__ dst, long long dst_stride, long long dst_off,
                         RowFmt f, long long total) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    if (f.type == LLG_TYPE_Q4_0 || f.type == LLG_TYPE_Q8_0) {
        const int qbytes = f.type == LLG_TYPE_Q4_0 ? 16 : 32;
        const long long r = i / f.nb;
        const int b = (int)(i % f.nb);
        const uint8_t *s = src + r * src_row_bytes + (long long)b * (2 + qbytes);
        uint8_t *row = dst + r * dst_stride + dst_off;
        row[f.d_off + 2 * b] = s[0];
        row[f.d_off + 2 * b + 1] = s[1];
        for (int k = 0; k < qbytes; k++) row[(long long)b * qbytes + k] = s[2 + k];
    } else {
        const int es = f.type == LLG_TYPE_F16 ? 2 : 4;
        const long long r = i / f.cols;
        const int c = (int)(i % f.cols);
        const uint8_t *s = src + r * src_row_bytes + (long long)c * es;
        uint8_t *o = dst + r * dst_stride + dst_off + (long long)c * es;
        for (int k = 0; k < es; k++) o[k] = s[k];
    }
}

static int repack_launch(LlgDevice *d, const uint8_t *src, uint8_t *dst, long long dst_stride,
                         long long dst_off, const RowFmt &f, int rows) {
    long long per_row = (f.type == LLG_TYPE_Q4_0 || f.type == LLG_TYPE_Q8_0) ? f.nb : f.cols;
    long long total = per_row * rows;
    if (total == 0) return 0;
    long long grid = (total + 255) / 256;
    hipLaunchKernelGGL(k_repack, dim3((unsigned)grid), dim3(256), 0, d->stream, src,
                       llg_gguf_row_bytes(f.type, f.cols), dst, dst_stride, dst_off, f, total);
    LLG_LAUNCH_CHECK(d, "repack");
    return 0;
}

// Upload helper: `src` is host (from_device == 0) or device memory holding
// `nsrc` GGUF tensors of `rows` rows each.
static int upload_rows(LlgDevice *d, const void *const *srcs, int nsrc, int from_device, int type,
                       int rows, int cols, int kind, int64_t *out) {
    if (!out || rows <= 0) return llg_set_error(d, LLG_E_ARG, "upload: bad rows/out");
    for (int i = 0; i < nsrc; i++)
        if (!srcs[i]) return llg_set_error(d, LLG_E_ARG, "upload: null source");
    RowFmt f;
    int rc = llg_row_fmt(type, cols, &f);
    if (rc == LLG_E_TYPE) return llg_set_error(d, rc, "upload: unsupported ggml type %d", type);
    if (rc == LLG_E_ALIGN)
        return llg_set_error(d, rc, "upload: %d elements not divisible by block size 32", cols);
    if (rc) return llg_set_error(d, rc, "upload: bad cols %d", cols);
    if (kind == LLG_KIND_BUNDLE && cols % 32)
        return llg_set_error(d, LLG_E_ALIGN, "bundle: hidden size %d not a multiple of 32", cols);
    const long long row_bytes = llg_gguf_row_bytes(type, cols);
    const long long stride = f.stride * nsrc;
    const size_t bytes = (size_t)stride * rows;
    uint8_t *dmem = nullptr;
    if (hipMalloc(&dmem, bytes) != hipSuccess)
        return llg_set_error(d, LLG_E_NOMEM, "upload: hipMalloc(%zu) failed", bytes);
    if (hipError_t e = hipMemsetAsync(dmem, 0, bytes, d->stream); e != hipSuccess) {
        hipFree(dmem);
        return llg_hip_error(d, e, "upload memset");
    }
    uint8_t *tmp = nullptr;
    const size_t src_bytes = (size_t)row_bytes * rows;
    if (!from_device) {
        if (hipMalloc(&tmp, src_bytes) != hipSuccess) {
            hipFree(dmem);
            return llg_set_error(d, LLG_E_NOMEM, "upload: staging hipMalloc(%zu) failed", src_bytes);
        }
    }
    for (int i = 0; i < nsrc && rc == 0; i++) {
        const uint8_t *s = reinterpret_cast<const uint8_t *>(srcs[i]);
        if (!from_device) {
            hipError_t e = hipMemcpyAsync(tmp, s, src_bytes, hipMemcpyHostToDevice, d->stream);
            if (e != hipSuccess) rc = llg_hip_error(d, e, "upload copy");
            s = tmp;
        }
        if (rc == 0) rc = repack_launch(d, s, dmem, stride, f.stride * i, f, rows);
        if (rc == 0 && !from_device) {
            hipError_t e = hipStreamSynchronize(d->stream);
            if (e != hipSuccess) rc = llg_hip_error(d, e, "upload sync");
        }
    }
    if (rc == 0) {
        hipError_t e = hipStreamSynchronize(d->stream);
        if (e != hipSuccess) rc = llg_hip_error(d, e, "upload sync");
    }
    if (tmp) hipFree(tmp);
    if (rc) {
        hipFree(dmem);
        return rc;
    }
    LlgObject *o = new LlgObject();
    o->kind = kind;
    o->d = dmem;
    o->bytes = bytes;
    o->fmt = f;
    o->rows = rows;
    o->stride = stride;
    o->ext = nullptr;
    *out = llg_register(d, o);
    return 0;
}

extern "C" {

int llg_hip_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n > 0 ? 1 : 0;
}

LlgHipDevice llg_hip_init(void) {
    if (!llg_hip_available()) return nullptr;
    LlgDevice *d = new LlgDevice();
    if (const char *e = getenv("LLG_CHECK_HANDOFF")) d->check_handoff = e[0] && e[0] != '0';
    if (hipGetDevice(&d->device) != hipSuccess) d->device = 0;
    if (hipSetDevice(d->device) != hipSuccess || hipStreamCreate(&d->stream) != hipSuccess) {
        delete d;
        return nullptr;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, d->device) == hipSuccess)
        d->cus = prop.multiProcessorCount;
    if (d->cus <= 0) d->cus = 256;
    // this device's copy of the scratch array (the device is current here)
    d->scratch_err = hipGetSymbolAddress(reinterpret_cast<void **>(&d->scratch), HIP_SYMBOL(scratch));
    if (d->scratch_err != hipSuccess) d->scratch = nullptr;
    return reinterpret_cast<LlgHipDevice>(d);
}

void llg_hip_free(LlgHipDevice h) {
    LlgDevice *d = llg_dev(h);
    if (!d) return;
    hipStreamSynchronize(d->stream);
    d->tearing_down = true;  // holders' unrefs free nothing: the sweep frees all
    for (auto &kv : d->objects) destroy_object(d, kv.second);
    d->objects.clear();
    if (d->ws) hipFree(d->ws);
    if (d->sync) hipFree(d->sync);
    if (d->mvslots) hipFree(d->mvslots);
    hipStreamDestroy(d->stream);
    delete d;
}

const char *llg_hip_last_error(LlgHipDevice h) {
    LlgDevice *d = llg_dev(h);
    if (!d) return "null device handle";
    return d->last_error.c_str();
}

void *llg_hip_stream(LlgHipDevice h) {
    LlgDevice *d = llg_dev(h);
    return d ? reinterpret_cast<void *>(d->stream) : nullptr;
}

int llg_hip_workspace_bytes(LlgHipDevice h, size_t *bytes) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    if (!bytes) return llg_set_error(d, LLG_E_ARG, "workspace_bytes: null output");
    *bytes = d->ws_bytes;
    return 0;
}

int llg_hip_sync(LlgHipDevice h) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    return llg_sync_dev(d);
}

int llg_hip_upload_matrix(LlgHipDevice h, const void *raw, int type, int rows, int cols,
                          int64_t *mat) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    const void *srcs[1] = {raw};
    return upload_rows(d, srcs, 1, 0, type, rows, cols, LLG_KIND_MATRIX, mat);
}

int llg_hipd_upload_matrix(LlgHipDevice h, const void *raw, int type, int rows, int cols,
                           int64_t *mat) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    const void *srcs[1] = {raw};
    return upload_rows(d, srcs, 1, 1, type, rows, cols, LLG_KIND_MATRIX, mat);
}

int llg_hip_upload_bundle(LlgHipDevice h, const void *up, const void *down_t, int type, int hd,
                          int ff, int64_t *bundle) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    const void *srcs[2] = {up, down_t};
    return upload_rows(d, srcs, 2, 0, type, ff, hd, LLG_KIND_BUNDLE, bundle);
}

int llg_hipd_upload_bundle(LlgHipDevice h, const void *up, const void *down_t, int type, int hd,
                           int ff, int64_t *bundle) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    const void *srcs[2] = {up, down_t};
    return upload_rows(d, srcs, 2, 1, type, ff, hd, LLG_KIND_BUNDLE, bundle);
}

int llg_hip_release(LlgHipDevice h, int64_t handle) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *o = llg_get(d, handle, 0);
    if (!o) return llg_set_error(d, LLG_E_HANDLE, "release: unknown handle %lld", (long long)handle);
    hipStreamSynchronize(d->stream);
    if (o->refs > 0) {  // a window or model still reads it: retire the handle only
        o->released = true;
        return 0;
    }
    d->objects.erase(handle);
    destroy_object(d, o);
    return 0;
}

int llg_hip_object_info(LlgHipDevice h, int64_t handle, int *type, int *rows, int *cols,
                        int64_t *row_stride) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *o = llg_get(d, handle, 0);
    if (!o) return llg_set_error(d, LLG_E_HANDLE, "object_info: unknown handle");
    if (type) *type = o->fmt.type;
    if (rows) *rows = o->rows;
    if (cols) *cols = o->fmt.cols;
    if (row_stride) *row_stride = o->stride;
    return 0;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Dequant (tensor/dtype.go:12-82), bit-exact: q * d with the reference's
// f16 conversion.  One thread per output element.
// ---------------------------------------------------------------------------
__global__ void k_dequant(const uint8_t *__restrict__ base, long long stride, long long sub_off,
                          int sub_count, long long sub_stride, RowFmt f, long long total,
                          float *__restrict__ out) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const long long per_row = (long long)f.cols * sub_count;
    const long long r = i / per_row;
    const long long rem = i % per_row;
    const int sub = (int)(rem / f.cols);
    const int c = (int)(rem % f.cols);
    const uint8_t *row = base + r * stride + sub_off + sub * sub_stride;
    const float v = llg_dequant_elem(row, f, c);
    out[i] = v;
}

extern "C" int llg_hip_dequant(LlgHipDevice h, int64_t handle, int row0, int nrows, float *out) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *o = llg_get(d, handle, 0);
    if (!o || o->kind == LLG_KIND_WINDOW || o->kind == LLG_KIND_MODEL)
        return llg_set_error(d, LLG_E_HANDLE, "dequant: unknown handle");
    if (!out || nrows < 0 || row0 < 0 || row0 + nrows > o->rows)
        return llg_set_error(d, LLG_E_RANGE, "dequant: rows [%d,%d) outside [0,%d)", row0,
                             row0 + nrows, o->rows);
    if (nrows == 0) return 0;
    const int sub_count = o->kind == LLG_KIND_BUNDLE ? 2 : 1;
    const long long total = (long long)nrows * o->fmt.cols * sub_count;
    int rc;
    float *dout = (float *)llg_ws(d, (size_t)total * 4, &rc);
    if (rc) return rc;
    hipLaunchKernelGGL(k_dequant, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, d->stream,
                       o->d + (long long)row0 * o->stride, o->stride, 0LL, sub_count,
                       o->fmt.stride, o->fmt, total, dout);
    LLG_LAUNCH_CHECK(d, "dequant");
    if ((rc = llg_d2h(d, out, dout, (size_t)total * 4))) return rc;
    return llg_sync_dev(d);
}

// ---------------------------------------------------------------------------
// Metal-parity matvec (metal_bridge.m:19-30) and rmsnorm (metal_bridge.m:34-59).
// ---------------------------------------------------------------------------
__global__ void k_matvec_f32(const float *__restrict__ w, int rows, int cols,
                             const float *__restrict__ x, float *__restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *wr = w + (size_t)row * cols;
    float s = 0.0f;
    for (int j = lane; j < cols; j += 64) s += wr[j] * x[j];
    s = llg_wave_sum(s);
    if (lane == 0) y[row] = s;
}

__global__ void k_rmsnorm(const float *__restrict__ x, const float *__restrict__ w,
                          float *__restrict__ out, int n, float eps) {
    __shared__ float part[16];
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) s += x[i] * x[i];
    s = llg_wave_sum(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    float tot = 0.0f;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) tot += part[i];
    // tensor/ops.go:128-129: rms in double, scale = 1/rms in float
    const float rms = (float)sqrt((double)(tot / (float)n) + (double)eps);
    const float scale = 1.0f / rms;
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = x[i] * scale * w[i];
}

extern "C" int llg_hip_matvec(LlgHipDevice h, const float *w, int rows, int cols, const float *x,
                              float *y) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    if (!w || !x || !y || rows <= 0 || cols <= 0)
        return llg_set_error(d, LLG_E_ARG, "matvec: bad arguments");
    const size_t wb = (size_t)rows * cols * 4;
    const size_t off_x = (wb + 255) & ~(size_t)255;
    const size_t off_y = off_x + (((size_t)cols * 4 + 255) & ~(size_t)255);
    int rc;
    uint8_t *ws = (uint8_t *)llg_ws(d, off_y + (size_t)rows * 4, &rc);
    if (rc) return rc;
    if ((rc = llg_h2d(d, ws, w, wb))) return rc;
    if ((rc = llg_h2d(d, ws + off_x, x, (size_t)cols * 4))) return rc;
    hipLaunchKernelGGL(k_matvec_f32, dim3((rows + 3) / 4), dim3(256), 0, d->stream,
                       (const float *)ws, rows, cols, (const float *)(ws + off_x),
                       (float *)(ws + off_y));
    LLG_LAUNCH_CHECK(d, "matvec");
    if ((rc = llg_d2h(d, y, ws + off_y, (size_t)rows * 4))) return rc;
    return llg_sync_dev(d);
}

extern "C" int llg_hip_rmsnorm(LlgHipDevice h, const float *x, const float *weight, float *out,
                               int n, float eps) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    if (!x || !weight || !out || n <= 0)
        return llg_set_error(d, LLG_E_ARG, "rmsnorm: bad arguments");
    const size_t nb = ((size_t)n * 4 + 255) & ~(size_t)255;
    int rc;
    uint8_t *ws = (uint8_t *)llg_ws(d, 3 * nb, &rc);
    if (rc) return rc;
    if ((rc = llg_h2d(d, ws, x, (size_t)n * 4))) return rc;
    if ((rc = llg_h2d(d, ws + nb, weight, (size_t)n * 4))) return rc;
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(1024), 0, d->stream, (const float *)ws,
                       (const float *)(ws + nb), (float *)(ws + 2 * nb), n, eps);
    LLG_LAUNCH_CHECK(d, "rmsnorm");
    if ((rc = llg_d2h(d, out, ws + 2 * nb, (size_t)n * 4))) return rc;
    return llg_sync_dev(d);
}
