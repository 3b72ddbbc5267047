// llg_ffn.hip -- gathered sparse FFN over row-column bundles
// (inference/ffn_flash.go:254-299, window.go:143-180) and the dense
// dequant-matvec FFN (inference/forward.go:318-353, tensor/ops.go:39-60).
//
// Sparse FFN, two passes over the active list:
//   k_sparse_up   one wavefront per active neuron: u_j = act(up_j . x);
//                 lane l reduces blocks l, l+64, ... of the up row (16-byte
//                 nibble loads, f16 scale), then a wavefront sum.  Also
//                 zeroes `out` for the next pass.
//   k_sparse_down workgroup (slice s, group g): the 256 outputs of 8
//                 consecutive blocks of the down rows, over neurons of
//                 group g; u_j == 0 rows are skipped as at ffn_flash.go:290;
//                 one fp32 atomic add per output per workgroup.  The
//                 blockIdx -> (s, g) map keeps all slices of one neuron
//                 group on one XCD so the group's scale lines are fetched
//                 into that XCD's L2 once.
#include "llg_common.hpp"
#include "llg_internal.hpp"

#define UP_WAVES 4
#define DN_SLICE_BLOCKS 8

template <int T>
__global__ __launch_bounds__(256) void k_sparse_up(
    const uint8_t *__restrict__ base, long long bstride, RowFmt f,
    const int32_t *__restrict__ slot_of, const float *__restrict__ x,
    const int32_t *__restrict__ active, const int32_t *__restrict__ n_active_p, int act,
    float *__restrict__ u, float *__restrict__ out) {
    const int n_active = *n_active_p;
    const int gtid = blockIdx.x * blockDim.x + threadIdx.x;
    for (int i = gtid; i < f.cols; i += gridDim.x * blockDim.x) out[i] = 0.0f;
    const int lane = threadIdx.x & 63;
    const int nwaves = gridDim.x * UP_WAVES;
    for (int j = blockIdx.x * UP_WAVES + (threadIdx.x >> 6); j < n_active; j += nwaves) {
        const int n = active[j];
        const long long slot = slot_of ? slot_of[n] : n;
        if (slot < 0) {  // not resident: window.go:150-152 leaves the activation at 0
            if (lane == 0) u[j] = 0.0f;
            continue;
        }
        const uint8_t *row = base + slot * bstride;
        float s = 0.0f;
        for (int b = lane; b < f.nb; b += 64)
            s += llg_block_dot<T>(row, f, b, reinterpret_cast<const float4 *>(x + b * 32));
        s = llg_wave_sum(s);
        if (lane == 0) u[j] = llg_act(act, s);
    }
}

template <int T>
__global__ __launch_bounds__(256) void k_sparse_down(
    const uint8_t *__restrict__ base, long long bstride, RowFmt f,
    const int32_t *__restrict__ slot_of, const int32_t *__restrict__ active,
    const int32_t *__restrict__ n_active_p, const float *__restrict__ u, int n_slices,
    int n_groups, float *__restrict__ out) {
    __shared__ float red[4][DN_SLICE_BLOCKS * 32];
    // XCD-aware tile map: workgroups are dispatched round-robin over 8 XCDs,
    // so id % 8 selects the XCD; group g lives on XCD g % 8.
    const int id = blockIdx.x;
    const int xcd = id & 7;
    const int k = id >> 3;
    const int g = xcd + 8 * (k / n_slices);
    const int s = k % n_slices;
    const int n_active = *n_active_p;
    const int chunk = (n_active + n_groups - 1) / n_groups;
    const int j0 = g * chunk;
    const int j1 = min(n_active, j0 + chunk);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int bl = lane & 7;
    const int sub = lane >> 3;
    const int b = s * DN_SLICE_BLOCKS + bl;
    float acc[32];
#pragma unroll
    for (int e = 0; e < 32; e++) acc[e] = 0.0f;
    if (b < f.nb) {
        for (int j = j0 + wave * 8 + sub; j < j1; j += 32) {
            const float uj = u[j];
            if (uj == 0.0f) continue;  // ffn_flash.go:290 / window.go:167
            const int n = active[j];
            const long long slot = slot_of ? slot_of[n] : n;
            llg_block_axpy<T>(base + slot * bstride + f.stride, f, b, uj, acc);
        }
    }
#pragma unroll
    for (int e = 0; e < 32; e++) {
        float v = acc[e];
        v += __shfl_xor(v, 8, 64);
        v += __shfl_xor(v, 16, 64);
        v += __shfl_xor(v, 32, 64);
        acc[e] = v;
    }
    if (sub == 0) {
#pragma unroll
        for (int e = 0; e < 32; e++) red[wave][bl * 32 + e] = acc[e];
    }
    __syncthreads();
    const int t = threadIdx.x;
    const int o = s * DN_SLICE_BLOCKS * 32 + t;
    if (o < f.cols && j0 < j1) {
        const float v = red[0][t] + red[1][t] + red[2][t] + red[3][t];
        unsafeAtomicAdd(out + o, v);
    }
}

size_t llg_sparse_ws_bytes(int max_active) {
    return (size_t)llg_align((long long)(max_active > 0 ? max_active : 1) * 4, 256);
}

template <int T>
static void sparse_launch(hipStream_t st, const uint8_t *base, long long bstride, const RowFmt &f,
                          const int32_t *slot_of, const float *x, const int32_t *active,
                          const int32_t *n_active, int max_active, int act, float *out,
                          float *u) {
    int up_grid = (max_active + UP_WAVES - 1) / UP_WAVES;
    if (up_grid < 1) up_grid = 1;
    if (up_grid > 1024) up_grid = 1024;
    hipLaunchKernelGGL(k_sparse_up<T>, dim3(up_grid), dim3(256), 0, st, base, bstride, f,
                       slot_of, x, active, n_active, act, u, out);
    const int n_slices = (f.nb + DN_SLICE_BLOCKS - 1) / DN_SLICE_BLOCKS;
    int n_groups = (max_active + 15) / 16;
    n_groups = (n_groups + 7) / 8 * 8;
    if (n_groups < 8) n_groups = 8;
    if (n_groups > 64) n_groups = 64;
    hipLaunchKernelGGL(k_sparse_down<T>, dim3(n_slices * n_groups), dim3(256), 0, st, base,
                       bstride, f, slot_of, active, n_active, u, n_slices, n_groups, out);
}

int llg_sparse_enqueue(LlgDevice *d, const uint8_t *base, long long bstride, const RowFmt &f,
                       const int32_t *slot_of, const float *d_x, const int32_t *d_active,
                       const int32_t *d_n_active, int max_active, int act, float *d_out,
                       uint8_t *ws) {
    hipStream_t st = llg_dev_stream(d);
    float *u = reinterpret_cast<float *>(ws);
    switch (f.type) {
    case LLG_TYPE_Q4_0:
        sparse_launch<LLG_TYPE_Q4_0>(st, base, bstride, f, slot_of, d_x, d_active, d_n_active,
                                     max_active, act, d_out, u);
        break;
    case LLG_TYPE_Q8_0:
        sparse_launch<LLG_TYPE_Q8_0>(st, base, bstride, f, slot_of, d_x, d_active, d_n_active,
                                     max_active, act, d_out, u);
        break;
    case LLG_TYPE_F16:
        sparse_launch<LLG_TYPE_F16>(st, base, bstride, f, slot_of, d_x, d_active, d_n_active,
                                    max_active, act, d_out, u);
        break;
    case LLG_TYPE_F32:
        sparse_launch<LLG_TYPE_F32>(st, base, bstride, f, slot_of, d_x, d_active, d_n_active,
                                    max_active, act, d_out, u);
        break;
    default:
        return llg_set_error(d, LLG_E_TYPE, "sparse ffn: unsupported type %d", f.type);
    }
    LLG_LAUNCH_CHECK(d, "sparse ffn");
    return 0;
}

// ---------------------------------------------------------------------------
// Dense dequant-matvec: y[r] = act(sum_b block_dot(row r, b, x)).
// Each wavefront owns MV_ROWS consecutive rows and reuses every x block it
// loads for all of them.
// ---------------------------------------------------------------------------
#define MV_ROWS 2

template <int T>
__global__ __launch_bounds__(256) void k_matvec_q(const uint8_t *__restrict__ w, long long stride,
                                                  RowFmt f, int rows, const float *__restrict__ x,
                                                  int act, float *__restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int r0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * MV_ROWS;
    if (r0 >= rows) return;
    float s[MV_ROWS];
#pragma unroll
    for (int i = 0; i < MV_ROWS; i++) s[i] = 0.0f;
    for (int b = lane; b < f.nb; b += 64) {
        float4 x4[8];
        const float4 *xp = reinterpret_cast<const float4 *>(x + b * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) x4[i] = xp[i];
#pragma unroll
        for (int i = 0; i < MV_ROWS; i++)
            if (r0 + i < rows) s[i] += llg_block_dot<T>(w + (long long)(r0 + i) * stride, f, b, x4);
    }
#pragma unroll
    for (int i = 0; i < MV_ROWS; i++) {
        const float v = llg_wave_sum(s[i]);
        if (lane == 0 && r0 + i < rows) y[r0 + i] = act >= 0 ? llg_act(act, v) : v;
    }
}

int llg_matvec_enqueue(LlgDevice *d, const LlgObject *w, const float *d_x, int act, float *d_y) {
    hipStream_t st = llg_dev_stream(d);
    const RowFmt &f = w->fmt;
    const int grid = (w->rows + 4 * MV_ROWS - 1) / (4 * MV_ROWS);
    switch (f.type) {
    case LLG_TYPE_Q4_0:
        hipLaunchKernelGGL(k_matvec_q<LLG_TYPE_Q4_0>, dim3(grid), dim3(256), 0, st, w->d,
                           w->stride, f, w->rows, d_x, act, d_y);
        break;
    case LLG_TYPE_Q8_0:
        hipLaunchKernelGGL(k_matvec_q<LLG_TYPE_Q8_0>, dim3(grid), dim3(256), 0, st, w->d,
                           w->stride, f, w->rows, d_x, act, d_y);
        break;
    case LLG_TYPE_F16:
        hipLaunchKernelGGL(k_matvec_q<LLG_TYPE_F16>, dim3(grid), dim3(256), 0, st, w->d,
                           w->stride, f, w->rows, d_x, act, d_y);
        break;
    case LLG_TYPE_F32:
        hipLaunchKernelGGL(k_matvec_q<LLG_TYPE_F32>, dim3(grid), dim3(256), 0, st, w->d,
                           w->stride, f, w->rows, d_x, act, d_y);
        break;
    default:
        return llg_set_error(d, LLG_E_TYPE, "matvec: unsupported type %d", f.type);
    }
    LLG_LAUNCH_CHECK(d, "matvec_q");
    return 0;
}

// ---------------------------------------------------------------------------
// Entry points
// ---------------------------------------------------------------------------
static int check_bundle(LlgDevice *d, int64_t hb, LlgObject **b) {
    *b = llg_get(d, hb, LLG_KIND_BUNDLE);
    if (!*b) return llg_set_error(d, LLG_E_HANDLE, "unknown bundle handle %lld", (long long)hb);
    return 0;
}

static int check_matvec(LlgDevice *d, const LlgObject *w) {
    if (w->fmt.cols % 32)
        return llg_set_error(d, LLG_E_ALIGN, "matvec: cols %d not a multiple of 32", w->fmt.cols);
    return 0;
}

extern "C" {

int llg_hipd_ffn_sparse(LlgHipDevice h, int64_t hb, const float *d_x, const int32_t *d_active,
                        const int32_t *d_n_active, int act, float *d_out) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *b;
    int rc = check_bundle(d, hb, &b);
    if (rc) return rc;
    if (!d_x || !d_active || !d_n_active || !d_out)
        return llg_set_error(d, LLG_E_ARG, "ffn_sparse: null pointer");
    uint8_t *ws = (uint8_t *)llg_ws(d, llg_sparse_ws_bytes(b->rows), &rc);
    if (rc) return rc;
    return llg_sparse_enqueue(d, b->d, b->stride, b->fmt, nullptr, d_x, d_active, d_n_active,
                              b->rows, act, d_out, ws);
}

int llg_hip_ffn_sparse(LlgHipDevice h, int64_t hb, const float *x, const int32_t *active,
                       int n_active, int act, float *out) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *b;
    int rc = check_bundle(d, hb, &b);
    if (rc) return rc;
    if (!x || !out || n_active < 0 || (n_active > 0 && !active))
        return llg_set_error(d, LLG_E_ARG, "ffn_sparse: bad arguments");
    const int hd = b->fmt.cols, ff = b->rows;
    for (int j = 0; j < n_active; j++)  // storage.go:292-294
        if (active[j] < 0 || active[j] >= ff)
            return llg_set_error(d, LLG_E_RANGE, "row %d out of range [0,%d)", active[j], ff);
    if (n_active == 0) {  // ffn_flash.go:255-257
        for (int i = 0; i < hd; i++) out[i] = 0.0f;
        return 0;
    }
    const long long o_x = 0;
    const long long o_act = llg_align((long long)hd * 4, 256);
    const long long o_n = o_act + llg_align((long long)n_active * 4, 256);
    const long long o_out = o_n + 256;
    const long long o_ws = o_out + llg_align((long long)hd * 4, 256);
    uint8_t *ws = (uint8_t *)llg_ws(d, o_ws + llg_sparse_ws_bytes(n_active), &rc);
    if (rc) return rc;
    const int32_t n32 = n_active;
    if ((rc = llg_h2d(d, ws + o_x, x, (size_t)hd * 4))) return rc;
    if ((rc = llg_h2d(d, ws + o_act, active, (size_t)n_active * 4))) return rc;
    if ((rc = llg_h2d(d, ws + o_n, &n32, 4))) return rc;
    rc = llg_sparse_enqueue(d, b->d, b->stride, b->fmt, nullptr, (const float *)(ws + o_x),
                            (const int32_t *)(ws + o_act), (const int32_t *)(ws + o_n), n_active,
                            act, (float *)(ws + o_out), ws + o_ws);
    if (rc) return rc;
    if ((rc = llg_d2h(d, out, ws + o_out, (size_t)hd * 4))) return rc;
    return llg_sync_dev(d);
}

int llg_hipd_ffn_predict_sparse(LlgHipDevice h, int64_t hwup, int64_t hwout, int64_t hbias,
                                int64_t hb, const float *d_a, const float *d_x, float thr,
                                int act, float *d_out, int32_t *d_active, int32_t *d_n_active) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *wup, *wout, *bias, *b;
    int rc = llg_check_predictor(d, hwup, hwout, hbias, &wup, &wout, &bias);
    if (rc) return rc;
    if ((rc = check_bundle(d, hb, &b))) return rc;
    if (wout->rows != b->rows || wup->fmt.cols != b->fmt.cols)
        return llg_set_error(d, LLG_E_ARG, "predict_sparse: predictor/bundle shape mismatch");
    if (!d_a || !d_x || !d_out || !d_active || !d_n_active)
        return llg_set_error(d, LLG_E_ARG, "predict_sparse: null pointer");
    const long long o_sp = llg_align(llg_predict_ws_bytes(wup->rows, wout->rows), 256);
    uint8_t *ws = (uint8_t *)llg_ws(d, o_sp + llg_sparse_ws_bytes(b->rows), &rc);
    if (rc) return rc;
    rc = llg_predict_enqueue(d, wup, wout, bias, d_a, thr, d_active, d_n_active, nullptr, ws);
    if (rc) return rc;
    return llg_sparse_enqueue(d, b->d, b->stride, b->fmt, nullptr, d_x, d_active, d_n_active,
                              b->rows, act, d_out, ws + o_sp);
}

int llg_hip_ffn_predict_sparse(LlgHipDevice h, int64_t hwup, int64_t hwout, int64_t hbias,
                               int64_t hb, const float *a, const float *x, float thr, int act,
                               float *out, int32_t *active, int *n_active) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *wup, *wout, *bias, *b;
    int rc = llg_check_predictor(d, hwup, hwout, hbias, &wup, &wout, &bias);
    if (rc) return rc;
    if ((rc = check_bundle(d, hb, &b))) return rc;
    if (!a || !x || !out) return llg_set_error(d, LLG_E_ARG, "predict_sparse: null pointer");
    const int hd = b->fmt.cols, ff = b->rows;
    const long long o_a = 0;
    const long long o_x = llg_align((long long)hd * 4, 256);
    const long long o_out = o_x + llg_align((long long)hd * 4, 256);
    const long long o_act = o_out + llg_align((long long)hd * 4, 256);
    const long long o_n = o_act + llg_align((long long)ff * 4, 256);
    const long long o_ws = o_n + 256;
    const long long o_sp = o_ws + llg_align(llg_predict_ws_bytes(wup->rows, ff), 256);
    uint8_t *ws = (uint8_t *)llg_ws(d, o_sp + llg_sparse_ws_bytes(ff), &rc);
    if (rc) return rc;
    if ((rc = llg_h2d(d, ws + o_a, a, (size_t)hd * 4))) return rc;
    if ((rc = llg_h2d(d, ws + o_x, x, (size_t)hd * 4))) return rc;
    rc = llg_predict_enqueue(d, wup, wout, bias, (const float *)(ws + o_a), thr,
                             (int32_t *)(ws + o_act), (int32_t *)(ws + o_n), nullptr, ws + o_ws);
    if (rc) return rc;
    rc = llg_sparse_enqueue(d, b->d, b->stride, b->fmt, nullptr, (const float *)(ws + o_x),
                            (const int32_t *)(ws + o_act), (const int32_t *)(ws + o_n), ff, act,
                            (float *)(ws + o_out), ws + o_sp);
    if (rc) return rc;
    int32_t n = 0;
    if ((rc = llg_d2h(d, out, ws + o_out, (size_t)hd * 4))) return rc;
    if ((rc = llg_d2h(d, &n, ws + o_n, 4))) return rc;
    if ((rc = llg_sync_dev(d))) return rc;
    if (active && (rc = llg_d2h(d, active, ws + o_act, (size_t)n * 4))) return rc;
    if (n_active) *n_active = n;
    return llg_sync_dev(d);
}

int llg_hipd_matvec_q(LlgHipDevice h, int64_t hm, const float *d_x, float *d_y) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *w = llg_get(d, hm, LLG_KIND_MATRIX);
    if (!w) return llg_set_error(d, LLG_E_HANDLE, "matvec_q: unknown matrix handle");
    int rc = check_matvec(d, w);
    if (rc) return rc;
    if (!d_x || !d_y) return llg_set_error(d, LLG_E_ARG, "matvec_q: null pointer");
    return llg_matvec_enqueue(d, w, d_x, -1, d_y);
}

int llg_hip_matvec_q(LlgHipDevice h, int64_t hm, const float *x, float *y) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *w = llg_get(d, hm, LLG_KIND_MATRIX);
    if (!w) return llg_set_error(d, LLG_E_HANDLE, "matvec_q: unknown matrix handle");
    int rc = check_matvec(d, w);
    if (rc) return rc;
    if (!x || !y) return llg_set_error(d, LLG_E_ARG, "matvec_q: null pointer");
    const long long o_y = llg_align((long long)w->fmt.cols * 4, 256);
    uint8_t *ws = (uint8_t *)llg_ws(d, o_y + (size_t)w->rows * 4, &rc);
    if (rc) return rc;
    if ((rc = llg_h2d(d, ws, x, (size_t)w->fmt.cols * 4))) return rc;
    if ((rc = llg_matvec_enqueue(d, w, (const float *)ws, -1, (float *)(ws + o_y)))) return rc;
    if ((rc = llg_d2h(d, y, ws + o_y, (size_t)w->rows * 4))) return rc;
    return llg_sync_dev(d);
}

static int check_dense(LlgDevice *d, int64_t hu, int64_t hd_, LlgObject **up, LlgObject **down) {
    *up = llg_get(d, hu, LLG_KIND_MATRIX);
    *down = llg_get(d, hd_, LLG_KIND_MATRIX);
    if (!*up || !*down) return llg_set_error(d, LLG_E_HANDLE, "ffn_dense: unknown matrix handle");
    if ((*down)->fmt.cols != (*up)->rows || (*down)->rows != (*up)->fmt.cols)
        return llg_set_error(d, LLG_E_ARG, "ffn_dense: up [%d x %d] / down [%d x %d] mismatch",
                             (*up)->rows, (*up)->fmt.cols, (*down)->rows, (*down)->fmt.cols);
    int rc = check_matvec(d, *up);
    if (!rc) rc = check_matvec(d, *down);
    return rc;
}

int llg_hipd_ffn_dense(LlgHipDevice h, int64_t hu, int64_t hdn, const float *d_x, int act,
                       float *d_out) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *up, *down;
    int rc = check_dense(d, hu, hdn, &up, &down);
    if (rc) return rc;
    if (!d_x || !d_out) return llg_set_error(d, LLG_E_ARG, "ffn_dense: null pointer");
    float *hid = (float *)llg_ws(d, (size_t)up->rows * 4, &rc);
    if (rc) return rc;
    if ((rc = llg_matvec_enqueue(d, up, d_x, act, hid))) return rc;
    return llg_matvec_enqueue(d, down, hid, -1, d_out);
}

int llg_hip_ffn_dense(LlgHipDevice h, int64_t hu, int64_t hdn, const float *x, int act,
                      float *out) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *up, *down;
    int rc = check_dense(d, hu, hdn, &up, &down);
    if (rc) return rc;
    if (!x || !out) return llg_set_error(d, LLG_E_ARG, "ffn_dense: null pointer");
    const int hd = up->fmt.cols, ff = up->rows;
    const long long o_out = llg_align((long long)hd * 4, 256);
    const long long o_h = o_out + llg_align((long long)hd * 4, 256);
    uint8_t *ws = (uint8_t *)llg_ws(d, o_h + (size_t)ff * 4, &rc);
    if (rc) return rc;
    if ((rc = llg_h2d(d, ws, x, (size_t)hd * 4))) return rc;
    if ((rc = llg_matvec_enqueue(d, up, (const float *)ws, act, (float *)(ws + o_h)))) return rc;
    if ((rc = llg_matvec_enqueue(d, down, (const float *)(ws + o_h), -1, (float *)(ws + o_out))))
        return rc;
    if ((rc = llg_d2h(d, out, ws + o_out, (size_t)hd * 4))) return rc;
    return llg_sync_dev(d);
}

}  // extern "C"
