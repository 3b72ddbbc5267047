// llg_predictor.hip -- low-rank activation predictor and active-neuron
// selection (inference/predictor.go:51-83).
//
//   hidden = ReLU(WUp[rank x h] . a)           k_pred_hidden (split over h)
//   logit  = WOut[ff x rank] . hidden (+bias)   k_pred_logits (64-neuron tiles)
//   active = {i : logit_i > thr}, ascending     wave ballot per tile -> 64-bit
//                                               mask, then k_compact (one
//                                               workgroup: popcount scan + write)
#include "llg_common.hpp"
#include "llg_internal.hpp"

#define PRED_SPLIT 4
#define TILE 64

// partial[s * rank + r] = sum over the s-th quarter of row r of WUp . a
__global__ void k_pred_hidden(const uint8_t *__restrict__ wup, long long stride, int h, int rank,
                              const float *__restrict__ a, float *__restrict__ partial) {
    const int r = blockIdx.x / PRED_SPLIT;
    const int s = blockIdx.x % PRED_SPLIT;
    const int lane = threadIdx.x;
    const float *row = reinterpret_cast<const float *>(wup + (long long)r * stride);
    const int chunk = (h + PRED_SPLIT - 1) / PRED_SPLIT;
    const int c0 = s * chunk;
    const int c1 = min(h, c0 + chunk);
    float acc = 0.0f;
    if ((h & 3) == 0 && (chunk & 3) == 0) {
        const float4 *r4 = reinterpret_cast<const float4 *>(row);
        const float4 *a4 = reinterpret_cast<const float4 *>(a);
        for (int j = (c0 >> 2) + lane; j < (c1 >> 2); j += 64) {
            const float4 w = r4[j], v = a4[j];
            acc += w.x * v.x;
            acc += w.y * v.y;
            acc += w.z * v.z;
            acc += w.w * v.w;
        }
    } else {
        for (int j = c0 + lane; j < c1; j += 64) acc += row[j] * a[j];
    }
    acc = llg_wave_sum(acc);
    if (lane == 0) partial[s * rank + r] = acc;
}

// One workgroup of 256 threads per 64-neuron tile.  Writes the tile's
// 64-bit active mask (bit i <=> logit[tile*64+i] > thr) and, optionally, logits.
__global__ void k_pred_logits(const uint8_t *__restrict__ wout, long long stride, int ff,
                              int rank, const float *__restrict__ partial,
                              const float *__restrict__ bias, float thr,
                              float *__restrict__ logits, unsigned long long *__restrict__ mask) {
    extern __shared__ float sh[];  // [rank] hidden, then [TILE] logits
    float *hid = sh;
    float *lg = sh + rank;
    for (int r = threadIdx.x; r < rank; r += blockDim.x) {
        float v = 0.0f;
        for (int s = 0; s < PRED_SPLIT; s++) v += partial[s * rank + r];
        hid[r] = v < 0.0f ? 0.0f : v;  // predictor.go:61 ReLU
    }
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int tile0 = blockIdx.x * TILE;
    if ((rank & 3) == 0 && rank <= 256 && (64 % (rank >> 2)) == 0) {
        // lanes_per_row float4 lanes per row, rows_per_pass rows per wave pass
        const int lpr = rank >> 2;
        const int rpp = 64 / lpr;
        const int sub = lane / lpr;
        const int c4 = lane % lpr;
        const float4 hv = reinterpret_cast<const float4 *>(hid)[c4];
        for (int base = wave * (TILE / 4); base < (wave + 1) * (TILE / 4); base += rpp) {
            const int i = tile0 + base + sub;
            float acc = 0.0f;
            if (i < ff && base + sub < (wave + 1) * (TILE / 4)) {
                const float4 w =
                    reinterpret_cast<const float4 *>(wout + (long long)i * stride)[c4];
                acc = w.x * hv.x;
                acc += w.y * hv.y;
                acc += w.z * hv.z;
                acc += w.w * hv.w;
            }
            for (int o = lpr >> 1; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
            if (c4 == 0 && base + sub < (wave + 1) * (TILE / 4)) lg[base + sub] = acc;
        }
    } else {
        for (int t = wave * (TILE / 4); t < (wave + 1) * (TILE / 4); t++) {
            const int i = tile0 + t;
            float acc = 0.0f;
            if (i < ff) {
                const float *w = reinterpret_cast<const float *>(wout + (long long)i * stride);
                for (int c = lane; c < rank; c += 64) acc += w[c] * hid[c];
            }
            acc = llg_wave_sum(acc);
            if (lane == 0) lg[t] = acc;
        }
    }
    __syncthreads();
    if (wave == 0) {
        const int i = tile0 + lane;
        bool on = false;
        if (i < ff) {
            float v = lg[lane];
            if (bias) v += bias[i];  // predictor.go:69-73
            if (logits) logits[i] = v;
            on = v > thr;  // predictor.go:78 (strict >)
        }
        const unsigned long long m = __ballot(on);
        if (lane == 0) mask[blockIdx.x] = m;
    }
}

// Masks from given logits (predictor.go:76-82 on its own).
__global__ void k_select_mask(const float *__restrict__ logits, int ff, float thr,
                              unsigned long long *__restrict__ mask) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const bool on = i < ff && logits[i] > thr;
    const unsigned long long m = __ballot(on);
    if ((threadIdx.x & 63) == 0 && (i >> 6) < (ff + 63) / 64) mask[i >> 6] = m;
}

// Ascending compaction of the tile masks into the active list, by one
// workgroup of 1024 threads: exclusive scan of popcounts, then each thread
// writes the set bits of its tile in increasing bit order.
__global__ void k_compact(const unsigned long long *__restrict__ mask, int n_tiles,
                          int32_t *__restrict__ active, int32_t *__restrict__ n_active) {
    __shared__ int wsum[16];
    __shared__ int carry_sh;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    if (threadIdx.x == 0) carry_sh = 0;
    __syncthreads();
    for (int t0 = 0; t0 < n_tiles; t0 += blockDim.x) {
        const int t = t0 + threadIdx.x;
        const unsigned long long m = t < n_tiles ? mask[t] : 0ull;
        const int c = __popcll(m);
        int incl = c;
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o, 64);
            if (lane >= o) incl += v;
        }
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();
        int before = carry_sh;
        for (int w = 0; w < wave; w++) before += wsum[w];
        int total = carry_sh;
        for (int w = 0; w < nw; w++) total += wsum[w];
        int pos = before + incl - c;
        unsigned long long mm = m;
        while (mm) {
            const int bit = __ffsll((long long)mm) - 1;
            active[pos++] = t * 64 + bit;
            mm &= mm - 1;
        }
        __syncthreads();
        if (threadIdx.x == 0) carry_sh = total;
        __syncthreads();
    }
    if (threadIdx.x == 0) *n_active = carry_sh;
}

int llg_predict_ws_bytes(int rank, int ff) {
    return (int)(llg_align((long long)PRED_SPLIT * rank * 4, 256) +
                 llg_align((long long)((ff + 63) / 64) * 8, 256));
}

int llg_predict_enqueue(LlgDevice *d, LlgObject *wup, LlgObject *wout, LlgObject *bias,
                        const float *d_a, float thr, int32_t *d_active, int32_t *d_n_active,
                        float *d_logits, uint8_t *ws) {
    const int h = wup->fmt.cols, rank = wup->rows, ff = wout->rows;
    float *partial = reinterpret_cast<float *>(ws);
    unsigned long long *mask = reinterpret_cast<unsigned long long *>(
        ws + llg_align((long long)PRED_SPLIT * rank * 4, 256));
    hipStream_t st = llg_dev_stream(d);
    hipLaunchKernelGGL(k_pred_hidden, dim3(rank * PRED_SPLIT), dim3(64), 0, st, wup->d,
                       wup->stride, h, rank, d_a, partial);
    LLG_LAUNCH_CHECK(d, "pred_hidden");
    const int n_tiles = (ff + TILE - 1) / TILE;
    const float *d_bias = bias ? reinterpret_cast<const float *>(bias->d) : nullptr;
    hipLaunchKernelGGL(k_pred_logits, dim3(n_tiles), dim3(256), (rank + TILE) * sizeof(float),
                       st, wout->d, wout->stride, ff, rank, partial, d_bias, thr, d_logits, mask);
    LLG_LAUNCH_CHECK(d, "pred_logits");
    hipLaunchKernelGGL(k_compact, dim3(1), dim3(1024), 0, st, mask, n_tiles, d_active,
                       d_n_active);
    LLG_LAUNCH_CHECK(d, "compact");
    return 0;
}

static int check_predictor(LlgDevice *d, int64_t hwup, int64_t hwout, int64_t hbias,
                           LlgObject **wup, LlgObject **wout, LlgObject **bias) {
    *wup = llg_get(d, hwup, LLG_KIND_MATRIX);
    *wout = llg_get(d, hwout, LLG_KIND_MATRIX);
    *bias = hbias ? llg_get(d, hbias, LLG_KIND_MATRIX) : nullptr;
    // predictor.go:52-54: weights must be loaded
    if (!*wup || !*wout || (hbias && !*bias))
        return llg_set_error(d, LLG_E_HANDLE, "predictor: weights not loaded");
    if ((*wup)->fmt.type != LLG_TYPE_F32 || (*wout)->fmt.type != LLG_TYPE_F32 ||
        (*bias && (*bias)->fmt.type != LLG_TYPE_F32))
        return llg_set_error(d, LLG_E_TYPE, "predictor: weights must be F32");
    if ((*wout)->fmt.cols != (*wup)->rows)
        return llg_set_error(d, LLG_E_ARG, "predictor: W_out cols %d != rank %d",
                             (*wout)->fmt.cols, (*wup)->rows);
    if (*bias && (*bias)->fmt.cols * (*bias)->rows != (*wout)->rows)
        return llg_set_error(d, LLG_E_ARG, "predictor: bias length != ff");
    if (*bias && (*bias)->rows != 1)
        return llg_set_error(d, LLG_E_ARG, "predictor: bias must be a [1 x ff] matrix");
    return 0;
}

int llg_check_predictor(LlgDevice *d, int64_t hwup, int64_t hwout, int64_t hbias,
                        LlgObject **wup, LlgObject **wout, LlgObject **bias) {
    return check_predictor(d, hwup, hwout, hbias, wup, wout, bias);
}

extern "C" {

int llg_hipd_predict(LlgHipDevice h, int64_t hwup, int64_t hwout, int64_t hbias, const float *d_a,
                     float thr, int32_t *d_active, int32_t *d_n_active, float *d_logits) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *wup, *wout, *bias;
    int rc = check_predictor(d, hwup, hwout, hbias, &wup, &wout, &bias);
    if (rc) return rc;
    if (!d_a || !d_active || !d_n_active) return llg_set_error(d, LLG_E_ARG, "predict: null");
    uint8_t *ws = (uint8_t *)llg_ws(d, llg_predict_ws_bytes(wup->rows, wout->rows), &rc);
    if (rc) return rc;
    return llg_predict_enqueue(d, wup, wout, bias, d_a, thr, d_active, d_n_active, d_logits, ws);
}

int llg_hip_predict(LlgHipDevice h, int64_t hwup, int64_t hwout, int64_t hbias, const float *a,
                    float thr, int32_t *active, int *n_active, float *logits) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *wup, *wout, *bias;
    int rc = check_predictor(d, hwup, hwout, hbias, &wup, &wout, &bias);
    if (rc) return rc;
    if (!a || !active || !n_active) return llg_set_error(d, LLG_E_ARG, "predict: null");
    const int hd = wup->fmt.cols, rank = wup->rows, ff = wout->rows;
    const long long o_a = 0;
    const long long o_act = o_a + llg_align((long long)hd * 4, 256);
    const long long o_n = o_act + llg_align((long long)ff * 4, 256);
    const long long o_lg = o_n + 256;
    const long long o_ws = o_lg + llg_align((long long)ff * 4, 256);
    uint8_t *ws = (uint8_t *)llg_ws(d, o_ws + llg_predict_ws_bytes(rank, ff), &rc);
    if (rc) return rc;
    if ((rc = llg_h2d(d, ws + o_a, a, (size_t)hd * 4))) return rc;
    rc = llg_predict_enqueue(d, wup, wout, bias, (const float *)(ws + o_a), thr,
                             (int32_t *)(ws + o_act), (int32_t *)(ws + o_n),
                             logits ? (float *)(ws + o_lg) : nullptr, ws + o_ws);
    if (rc) return rc;
    int32_t n = 0;
    if ((rc = llg_d2h(d, &n, ws + o_n, 4))) return rc;
    if ((rc = llg_sync_dev(d))) return rc;
    if ((rc = llg_d2h(d, active, ws + o_act, (size_t)n * 4))) return rc;
    if (logits && (rc = llg_d2h(d, logits, ws + o_lg, (size_t)ff * 4))) return rc;
    *n_active = n;
    return llg_sync_dev(d);
}

int llg_hip_select(LlgHipDevice h, const float *logits, int ff, float thr, int32_t *active,
                   int *n_active) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    if (!logits || !active || !n_active || ff <= 0)
        return llg_set_error(d, LLG_E_ARG, "select: bad arguments");
    const int n_tiles = (ff + 63) / 64;
    const long long o_act = llg_align((long long)ff * 4, 256);
    const long long o_n = o_act + llg_align((long long)ff * 4, 256);
    const long long o_m = o_n + 256;
    int rc;
    uint8_t *ws = (uint8_t *)llg_ws(d, o_m + (size_t)n_tiles * 8, &rc);
    if (rc) return rc;
    if ((rc = llg_h2d(d, ws, logits, (size_t)ff * 4))) return rc;
    hipStream_t st = llg_dev_stream(d);
    unsigned long long *mask = reinterpret_cast<unsigned long long *>(ws + o_m);
    hipLaunchKernelGGL(k_select_mask, dim3((ff + 255) / 256), dim3(256), 0, st,
                       (const float *)ws, ff, thr, mask);
    LLG_LAUNCH_CHECK(d, "select_mask");
    hipLaunchKernelGGL(k_compact, dim3(1), dim3(1024), 0, st, mask, n_tiles,
                       (int32_t *)(ws + o_act), (int32_t *)(ws + o_n));
    LLG_LAUNCH_CHECK(d, "compact");
    int32_t n = 0;
    if ((rc = llg_d2h(d, &n, ws + o_n, 4))) return rc;
    if ((rc = llg_sync_dev(d))) return rc;
    if ((rc = llg_d2h(d, active, ws + o_act, (size_t)n * 4))) return rc;
    *n_active = n;
    return llg_sync_dev(d);
}

}  // extern "C"
