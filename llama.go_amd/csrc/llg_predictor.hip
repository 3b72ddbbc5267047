// llg_predictor.hip -- low-rank activation predictor and active-neuron
// selection (inference/predictor.go:51-83).
//
//   hidden = ReLU(WUp[rank x h] . a)           k_pred_hidden: rank x 8 wavefronts,
//                                               each one eighth of a row; partials
//                                               are summed (and ReLU'd) by the reader
//   logit  = WOut[ff x rank] . hidden (+bias)   k_pred_logits: 64-neuron tiles
//   active = {i : logit_i > thr}, ascending     wavefront ballot per tile -> 64-bit
//                                               mask, then k_compact (one workgroup:
//                                               popcount scan + ordered writes)
#include "llg_common.hpp"
#include "llg_internal.hpp"
#include "llg_pred_tile.hpp"

#define PRED_SPLIT LLG_PRED_SPLIT

// partial[s * rank + r] = WUp[r, chunk s] . a[chunk s].  The grid also zeroes
// `zero_out`, `zero_ctr[0..n_ctr)` and `*zero_extra` (each optional), which
// the kernels that follow accumulate into.
__global__ __launch_bounds__(256) void k_pred_hidden(const uint8_t *__restrict__ wup,
                                                     long long stride, int h, int rank,
                                                     const float *__restrict__ a,
                                                     float *__restrict__ partial,
                                                     float *__restrict__ zero_out, int zero_n,
                                                     int32_t *__restrict__ zero_ctr, int n_ctr,
                                                     int32_t *__restrict__ zero_extra,
                                                     const float *__restrict__ add_to) {
    const int gtid = blockIdx.x * blockDim.x + threadIdx.x;
    if (zero_out) {  // cleared, or (add_to) accumulated: zero_out[i] += add_to[i]
        for (int i = gtid; i < zero_n; i += gridDim.x * blockDim.x)
            zero_out[i] = add_to ? zero_out[i] + add_to[i] : 0.0f;
    }
    if (zero_ctr && gtid < n_ctr) zero_ctr[gtid] = 0;
    if (zero_extra && gtid == 0) *zero_extra = 0;
    const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= rank * PRED_SPLIT) return;
    const int r = wid / PRED_SPLIT;
    const int s = wid % PRED_SPLIT;
    const float *row = reinterpret_cast<const float *>(wup + (long long)r * stride);
    const float acc = llg_pred_split_dot(row, a, h, s);
    if ((threadIdx.x & 63) == 0) partial[s * rank + r] = acc;
}

// One workgroup of 256 threads per 64-neuron tile: logits, optional output,
// and the tile's 64-bit active mask (bit i <=> logit[tile*64+i] > thr).
__global__ __launch_bounds__(256) void k_pred_logits(const uint8_t *__restrict__ wout,
                                                     long long stride, int ff, int rank,
                                                     const float *__restrict__ partial,
                                                     const float *__restrict__ bias, float thr,
                                                     float *__restrict__ logits,
                                                     unsigned long long *__restrict__ mask) {
    extern __shared__ float sh[];  // [rank] hidden (16-byte aligned), then [64] logits
    float *hid = sh;
    float *lg = sh + ((rank + 3) & ~3);
    const int tile0 = blockIdx.x * 64;
    WoutTile t;
    load_wout_tile(t, wout, stride, ff, rank, tile0);
    load_hidden<PRED_SPLIT>(hid, partial, rank);
    __syncthreads();
    finish_logits(t, wout, stride, ff, rank, tile0, hid, lg);
    __syncthreads();
    if ((threadIdx.x >> 6) == 0) {
        const int lane = threadIdx.x & 63;
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
__global__ __launch_bounds__(1024) void k_compact(const unsigned long long *__restrict__ mask,
                                                  int n_tiles, int32_t *__restrict__ active,
                                                  int32_t *__restrict__ n_active) {
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
    if (threadIdx.x == 0 && n_active) *n_active = carry_sh;
}

int llg_predict_ws_bytes(int rank, int ff) {
    return (int)(llg_align((long long)PRED_SPLIT * rank * 4, 256) +
                 llg_align((long long)((ff + 63) / 64) * 8, 256));
}

void llg_pred_ws_layout(uint8_t *ws, int rank, float **partial, unsigned long long **mask) {
    *partial = reinterpret_cast<float *>(ws);
    *mask = reinterpret_cast<unsigned long long *>(
        ws + llg_align((long long)PRED_SPLIT * rank * 4, 256));
}

int llg_pred_split() { return PRED_SPLIT; }

int llg_pred_hidden_enqueue(LlgDevice *d, LlgObject *wup, const float *d_a, uint8_t *ws,
                            float **partial, unsigned long long **mask, int *psplit,
                            float *zero_out, int zero_n, int32_t *zero_ctr, int n_ctr,
                            int32_t *zero_extra, const float *add_to) {
    const int h = wup->fmt.cols, rank = wup->rows;
    llg_pred_ws_layout(ws, rank, partial, mask);
    *psplit = PRED_SPLIT;
    const int grid = (rank * PRED_SPLIT + 3) / 4;
    hipLaunchKernelGGL(k_pred_hidden, dim3(grid), dim3(256), 0, llg_dev_stream(d), wup->d,
                       wup->stride, h, rank, d_a, *partial, zero_out, zero_n, zero_ctr, n_ctr,
                       zero_extra, add_to);
    LLG_LAUNCH_CHECK(d, "pred_hidden");
    return 0;
}

int llg_compact_enqueue(LlgDevice *d, const unsigned long long *mask, int n_tiles,
                        int32_t *d_active, int32_t *d_n_active) {
    hipLaunchKernelGGL(k_compact, dim3(1), dim3(1024), 0, llg_dev_stream(d), mask, n_tiles,
                       d_active, d_n_active);
    LLG_LAUNCH_CHECK(d, "compact");
    return 0;
}

// Hidden partials (also clearing zero_out[0..zero_n) and *zero_extra) and the
// tile masks; *mask_out points into ws.
int llg_pred_masks_enqueue(LlgDevice *d, LlgObject *wup, LlgObject *wout, LlgObject *bias,
                           const float *d_a, float thr, uint8_t *ws,
                           unsigned long long **mask_out, float *zero_out, int zero_n,
                           int32_t *zero_extra) {
    const int ff = wout->rows, rank = wup->rows;
    float *partial;
    int psplit;
    int rc = llg_pred_hidden_enqueue(d, wup, d_a, ws, &partial, mask_out, &psplit, zero_out,
                                     zero_n, nullptr, 0, zero_extra);
    if (rc) return rc;
    const int n_tiles = (ff + 63) / 64;
    const float *d_bias = bias ? reinterpret_cast<const float *>(bias->d) : nullptr;
    const size_t lds = (size_t)(((rank + 3) & ~3) + 64) * sizeof(float);
    hipLaunchKernelGGL(k_pred_logits, dim3(n_tiles), dim3(256), lds, llg_dev_stream(d), wout->d,
                       wout->stride, ff, rank, partial, d_bias, thr, (float *)nullptr, *mask_out);
    LLG_LAUNCH_CHECK(d, "pred_logits");
    return 0;
}

int llg_predict_enqueue(LlgDevice *d, LlgObject *wup, LlgObject *wout, LlgObject *bias,
                        const float *d_a, float thr, int32_t *d_active, int32_t *d_n_active,
                        float *d_logits, uint8_t *ws) {
    float *partial;
    unsigned long long *mask;
    int psplit;
    int rc = llg_pred_hidden_enqueue(d, wup, d_a, ws, &partial, &mask, &psplit, nullptr, 0,
                                     nullptr, 0, nullptr);
    if (rc) return rc;
    return llg_pred_logits_enqueue(d, wout, bias, thr, ws, d_active, d_n_active, d_logits);
}

int llg_pred_logits_enqueue(LlgDevice *d, LlgObject *wout, LlgObject *bias, float thr,
                            uint8_t *ws, int32_t *d_active, int32_t *d_n_active,
                            float *d_logits) {
    const int ff = wout->rows, rank = wout->fmt.cols;
    float *partial;
    unsigned long long *mask;
    llg_pred_ws_layout(ws, rank, &partial, &mask);
    const int n_tiles = (ff + 63) / 64;
    const float *d_bias = bias ? reinterpret_cast<const float *>(bias->d) : nullptr;
    const size_t lds = (size_t)(((rank + 3) & ~3) + 64) * sizeof(float);
    hipLaunchKernelGGL(k_pred_logits, dim3(n_tiles), dim3(256), lds, llg_dev_stream(d), wout->d,
                       wout->stride, ff, rank, partial, d_bias, thr, d_logits, mask);
    LLG_LAUNCH_CHECK(d, "pred_logits");
    return llg_compact_enqueue(d, mask, n_tiles, d_active, d_n_active);
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
    if (*bias && ((*bias)->rows != 1 || (*bias)->fmt.cols != (*wout)->rows))
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
    unsigned long long *mask = reinterpret_cast<unsigned long long *>(ws + o_m);
    hipLaunchKernelGGL(k_select_mask, dim3((ff + 255) / 256), dim3(256), 0, llg_dev_stream(d),
                       (const float *)ws, ff, thr, mask);
    LLG_LAUNCH_CHECK(d, "select_mask");
    if ((rc = llg_compact_enqueue(d, mask, n_tiles, (int32_t *)(ws + o_act),
                                  (int32_t *)(ws + o_n))))
        return rc;
    int32_t n = 0;
    if ((rc = llg_d2h(d, &n, ws + o_n, 4))) return rc;
    if ((rc = llg_sync_dev(d))) return rc;
    if ((rc = llg_d2h(d, active, ws + o_act, (size_t)n * 4))) return rc;
    *n_active = n;
    return llg_sync_dev(d);
}

}  // extern "C"
