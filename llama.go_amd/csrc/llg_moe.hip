// llg_moe.hip -- Mixture-of-Experts FFN (inference/moe_forward.go:32-150).
//
// Per token:
//   k_moe_router   logits = Router[n_exp x hidden] . x, softmax with the
//                  reference's op order (forward.go:463-479: max-subtract,
//                  exp in double rounded to float, sequential fp32 sum,
//                  divide), descending stable sort (ties -> lower index),
//                  top-k, wsum guard and p/wsum (moe_forward.go:42-68)
//   k_moe_gateup   h[s][j] = silu(gate_e[j] . x) * (up_e[j] . x) for the k
//                  chosen experts (moe_forward.go:101-132)
//   k_moe_down     out[d] = sum_s w_s * (down_e[d] . h[s]) accumulated in the
//                  chosen order, starting from 0 (moe_forward.go:71-77, 141-148)
// Expert e's rows are e*eff + j of gate/up and e*hidden + d of down, the
// addressing of ReadContiguousRows (flash/storage.go:72-94).
// Batches of 16 or more tokens over Q4_0 experts go to the grouped MFMA GEMM
// path (llg_moe_gemm.hip); smaller batches and other types use the kernels
// below token by token.
#include "llg_common.hpp"
#include "llg_internal.hpp"

#define MOE_MAX_EXP 64
#define MOE_MAX_K 8

// Softmax + stable descending top-k over `lg` (n_exp values), one thread.
__device__ void moe_route_one(const float *lg, int n_exp, int k, int32_t *ids, float *w) {
    float p[MOE_MAX_EXP];
    int idx[MOE_MAX_EXP];
    float mx = lg[0];
    for (int e = 0; e < n_exp; e++)
        if (lg[e] > mx) mx = lg[e];
    float sum = 0.0f;
    for (int e = 0; e < n_exp; e++) {
        const float v = (float)exp((double)(lg[e] - mx));
        p[e] = v;
        sum += v;
    }
    for (int e = 0; e < n_exp; e++) p[e] /= sum;
    for (int e = 0; e < n_exp; e++) idx[e] = e;
    for (int i = 1; i < n_exp; i++) {  // insertion sort: equal scores keep index order
        const int cur = idx[i];
        int j = i;
        while (j > 0 && p[cur] > p[idx[j - 1]]) {
            idx[j] = idx[j - 1];
            j--;
        }
        idx[j] = cur;
    }
    float wsum = 0.0f;
    for (int s = 0; s < k; s++) wsum += p[idx[s]];
    if (wsum < 1e-9f) wsum = 1.0f;
    for (int s = 0; s < k; s++) {
        ids[s] = idx[s];
        w[s] = p[idx[s]] / wsum;
    }
}

// One workgroup per token; wavefront e computes logit e.
__global__ __launch_bounds__(512) void k_moe_router(const uint8_t *__restrict__ router,
                                                    long long stride, int hidden, int n_exp, int k,
                                                    const float *__restrict__ x,
                                                    const float *__restrict__ given_logits,
                                                    int32_t *__restrict__ ids,
                                                    float *__restrict__ w) {
    __shared__ float lg[MOE_MAX_EXP];
    const int t = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if (given_logits) {
        for (int e = threadIdx.x; e < n_exp; e += blockDim.x) lg[e] = given_logits[(size_t)t * n_exp + e];
    } else {
        const float *xt = x + (size_t)t * hidden;
        for (int e = wave; e < n_exp; e += nw) {
            const float *row = reinterpret_cast<const float *>(router + (long long)e * stride);
            float s = 0.0f;
            for (int dd = lane; dd < hidden; dd += 64) s += row[dd] * xt[dd];
            s = llg_wave_sum(s);
            if (lane == 0) lg[e] = s;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) moe_route_one(lg, n_exp, k, ids + (size_t)t * k, w + (size_t)t * k);
}

// Wavefront per (token, slot, j): gate and up rows share every x block load.
template <int T>
__global__ __launch_bounds__(256) void k_moe_gateup(const uint8_t *__restrict__ gate,
                                                    const uint8_t *__restrict__ up,
                                                    long long stride, RowFmt f, int eff, int k,
                                                    int n_tok, const int32_t *__restrict__ ids,
                                                    const float *__restrict__ x,
                                                    float *__restrict__ hbuf) {
    const int lane = threadIdx.x & 63;
    const long long total = (long long)n_tok * k * eff;
    const long long nwaves = (long long)gridDim.x * 4;
    for (long long i = (long long)blockIdx.x * 4 + (threadIdx.x >> 6); i < total; i += nwaves) {
        const int j = (int)(i % eff);
        const long long ts = i / eff;  // token * k + slot
        const int t = (int)(ts / k);
        const int e = ids[ts];
        const long long r = (long long)e * eff + j;
        const uint8_t *gr = gate + r * stride;
        const uint8_t *ur = up + r * stride;
        const float *xt = x + (size_t)t * f.cols;
        float g = 0.0f, u = 0.0f;
        for (int b = lane; b < f.nb; b += 64) {
            float4 x4[8];
            const float4 *xp = reinterpret_cast<const float4 *>(xt + b * 32);
#pragma unroll
            for (int q = 0; q < 8; q++) x4[q] = xp[q];
            g += llg_block_dot<T>(gr, f, b, x4);
            u += llg_block_dot<T>(ur, f, b, x4);
        }
        g = llg_wave_sum(g);
        u = llg_wave_sum(u);
        if (lane == 0) {
            const float silu = g / (1.0f + (float)exp(-(double)g));  // moe_forward.go:130
            hbuf[i] = silu * u;
        }
    }
}

// Wavefront per (token, MOE_DN_ROWS consecutive outputs d); h blocks are
// loaded once per slot and reused across those rows.
#define MOE_DN_ROWS 4
template <int T>
__global__ __launch_bounds__(256) void k_moe_down(const uint8_t *__restrict__ down,
                                                  long long stride, RowFmt f, int hidden, int k,
                                                  int n_tok, const int32_t *__restrict__ ids,
                                                  const float *__restrict__ wts,
                                                  const float *__restrict__ hbuf,
                                                  float *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int groups = (hidden + MOE_DN_ROWS - 1) / MOE_DN_ROWS;
    const long long total = (long long)n_tok * groups;
    const long long nwaves = (long long)gridDim.x * 4;
    const int eff = f.cols;
    for (long long i = (long long)blockIdx.x * 4 + (threadIdx.x >> 6); i < total; i += nwaves) {
        const int t = (int)(i / groups);
        const int d0 = (int)(i % groups) * MOE_DN_ROWS;
        float res[MOE_DN_ROWS];
#pragma unroll
        for (int q = 0; q < MOE_DN_ROWS; q++) res[q] = 0.0f;
        for (int s = 0; s < k; s++) {
            const int e = ids[(size_t)t * k + s];
            const float ws = wts[(size_t)t * k + s];
            const float *h = hbuf + ((size_t)t * k + s) * eff;
            float acc[MOE_DN_ROWS];
#pragma unroll
            for (int q = 0; q < MOE_DN_ROWS; q++) acc[q] = 0.0f;
            for (int b = lane; b < f.nb; b += 64) {
                float4 h4[8];
                const float4 *hp = reinterpret_cast<const float4 *>(h + b * 32);
#pragma unroll
                for (int q = 0; q < 8; q++) h4[q] = hp[q];
#pragma unroll
                for (int q = 0; q < MOE_DN_ROWS; q++)
                    if (d0 + q < hidden)
                        acc[q] += llg_block_dot<T>(
                            down + ((long long)e * hidden + d0 + q) * stride, f, b, h4);
            }
#pragma unroll
            for (int q = 0; q < MOE_DN_ROWS; q++) res[q] += ws * llg_wave_sum(acc[q]);
        }
        if (lane == 0) {
#pragma unroll
            for (int q = 0; q < MOE_DN_ROWS; q++)
                if (d0 + q < hidden) out[(size_t)t * hidden + d0 + q] = res[q];
        }
    }
}

struct MoeArgs {
    LlgObject *router, *gate, *up, *down;
    int n_exp, k, hidden, eff;
};

static int check_moe(LlgDevice *d, int64_t hr, int64_t hg, int64_t hu, int64_t hd, int n_exp,
                     int k, MoeArgs *a) {
    // moe_forward.go:38-40
    if (k <= 0 || n_exp <= 0 || k > n_exp || n_exp > MOE_MAX_EXP || k > MOE_MAX_K)
        return llg_set_error(d, LLG_E_HPARAM,
                             "moeFFN: invalid hparams nExperts=%d k=%d (max %d experts, k<=%d)",
                             n_exp, k, MOE_MAX_EXP, MOE_MAX_K);
    a->router = llg_get(d, hr, LLG_KIND_MATRIX);
    a->gate = llg_get(d, hg, LLG_KIND_MATRIX);
    a->up = llg_get(d, hu, LLG_KIND_MATRIX);
    a->down = llg_get(d, hd, LLG_KIND_MATRIX);
    if (!a->router || !a->gate || !a->up || !a->down)
        return llg_set_error(d, LLG_E_HANDLE, "moeFFN: unknown matrix handle");
    a->n_exp = n_exp;
    a->k = k;
    a->hidden = a->gate->fmt.cols;
    if (a->router->fmt.type != LLG_TYPE_F32 || a->router->rows != n_exp ||
        a->router->fmt.cols != a->hidden)
        return llg_set_error(d, LLG_E_ARG, "moeFFN: router must be F32 [n_exp x hidden]");
    if (a->gate->rows % n_exp)
        return llg_set_error(d, LLG_E_ARG, "moeFFN: gate rows not a multiple of n_exp");
    a->eff = a->gate->rows / n_exp;
    if (a->eff <= 0) return llg_set_error(d, LLG_E_HPARAM, "moeFFN: expertFF must be > 0");
    if (a->up->rows != a->gate->rows || a->up->fmt.cols != a->hidden ||
        a->up->fmt.type != a->gate->fmt.type)
        return llg_set_error(d, LLG_E_ARG, "moeFFN: up_exps shape/type differs from gate_exps");
    if (a->down->rows != n_exp * a->hidden || a->down->fmt.cols != a->eff ||
        a->down->fmt.type != a->gate->fmt.type)
        return llg_set_error(d, LLG_E_ARG, "moeFFN: down_exps must be [n_exp*hidden x eff]");
    if (a->hidden % 32 || a->eff % 32)
        return llg_set_error(d, LLG_E_ALIGN, "moeFFN: hidden and expertFF must be multiples of 32");
    return 0;
}

static bool use_gemm(const MoeArgs &a, int n_tok) {
    return llg_moe_gemm_supported(a.gate->fmt.type, a.hidden, a.eff, n_tok);
}

static size_t moe_ws_bytes(const MoeArgs &a, int n_tok) {
    const size_t head = (size_t)llg_align((long long)n_tok * a.k * 4, 256) * 2;
    if (use_gemm(a, n_tok))
        return head + llg_moe_gemm_ws_bytes(n_tok, a.k, a.n_exp, a.hidden, a.eff);
    return head + (size_t)n_tok * a.k * a.eff * 4;
}

template <int T>
static void moe_launch_experts(hipStream_t st, const MoeArgs &a, int n_tok, const int32_t *ids,
                               const float *w, const float *x, float *hbuf, float *out) {
    const long long gu_waves = (long long)n_tok * a.k * a.eff;
    long long g1 = (gu_waves + 3) / 4;
    if (g1 > 8192) g1 = 8192;
    hipLaunchKernelGGL(k_moe_gateup<T>, dim3((unsigned)g1), dim3(256), 0, st, a.gate->d, a.up->d,
                       a.gate->stride, a.gate->fmt, a.eff, a.k, n_tok, ids, x, hbuf);
    const long long dn_waves = (long long)n_tok * ((a.hidden + MOE_DN_ROWS - 1) / MOE_DN_ROWS);
    long long g2 = (dn_waves + 3) / 4;
    if (g2 > 8192) g2 = 8192;
    hipLaunchKernelGGL(k_moe_down<T>, dim3((unsigned)g2), dim3(256), 0, st, a.down->d,
                       a.down->stride, a.down->fmt, a.hidden, a.k, n_tok, ids, w, hbuf, out);
}

static int moe_enqueue(LlgDevice *d, const MoeArgs &a, const float *d_x, int n_tok, float *d_out,
                       int32_t *d_ids, float *d_w, uint8_t *ws) {
    hipStream_t st = llg_dev_stream(d);
    const long long kb = llg_align((long long)n_tok * a.k * 4, 256);
    int32_t *ids = d_ids ? d_ids : reinterpret_cast<int32_t *>(ws);
    float *w = d_w ? d_w : reinterpret_cast<float *>(ws + kb);
    float *hbuf = reinterpret_cast<float *>(ws + 2 * kb);
    hipLaunchKernelGGL(k_moe_router, dim3(n_tok), dim3(512), 0, st, a.router->d, a.router->stride,
                       a.hidden, a.n_exp, a.k, d_x, (const float *)nullptr, ids, w);
    LLG_LAUNCH_CHECK(d, "moe_router");
    if (use_gemm(a, n_tok))  // batched tokens: grouped MFMA GEMMs
        return llg_moe_gemm_enqueue(d, a.gate, a.up, a.down, a.n_exp, a.k, a.hidden, a.eff, d_x,
                                    n_tok, ids, w, d_out, ws + 2 * kb);
    switch (a.gate->fmt.type) {
    case LLG_TYPE_Q4_0:
        moe_launch_experts<LLG_TYPE_Q4_0>(st, a, n_tok, ids, w, d_x, hbuf, d_out);
        break;
    case LLG_TYPE_Q8_0:
        moe_launch_experts<LLG_TYPE_Q8_0>(st, a, n_tok, ids, w, d_x, hbuf, d_out);
        break;
    case LLG_TYPE_F16:
        moe_launch_experts<LLG_TYPE_F16>(st, a, n_tok, ids, w, d_x, hbuf, d_out);
        break;
    case LLG_TYPE_F32:
        moe_launch_experts<LLG_TYPE_F32>(st, a, n_tok, ids, w, d_x, hbuf, d_out);
        break;
    default:
        return llg_set_error(d, LLG_E_TYPE, "moe: unsupported type");
    }
    LLG_LAUNCH_CHECK(d, "moe experts");
    return 0;
}

extern "C" {

int llg_hipd_moe_ffn(LlgHipDevice h, int64_t hr, int64_t hg, int64_t hu, int64_t hdn, int n_exp,
                     int k, const float *d_x, int n_tok, float *d_out, int32_t *d_ids,
                     float *d_w) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    MoeArgs a;
    int rc = check_moe(d, hr, hg, hu, hdn, n_exp, k, &a);
    if (rc) return rc;
    if (!d_x || !d_out || n_tok <= 0) return llg_set_error(d, LLG_E_ARG, "moe: bad arguments");
    if (((uintptr_t)d_x | (uintptr_t)d_out) & 15)
        return llg_set_error(d, LLG_E_ALIGN, "moe: x and out must be 16-byte aligned");
    uint8_t *ws = (uint8_t *)llg_ws(d, moe_ws_bytes(a, n_tok), &rc);
    if (rc) return rc;
    return moe_enqueue(d, a, d_x, n_tok, d_out, d_ids, d_w, ws);
}

int llg_hip_moe_ffn(LlgHipDevice h, int64_t hr, int64_t hg, int64_t hu, int64_t hdn, int n_exp,
                    int k, const float *x, int n_tok, float *out, int32_t *ids, float *wts) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    MoeArgs a;
    int rc = check_moe(d, hr, hg, hu, hdn, n_exp, k, &a);
    if (rc) return rc;
    if (!x || !out || n_tok <= 0) return llg_set_error(d, LLG_E_ARG, "moe: bad arguments");
    const size_t xb = (size_t)n_tok * a.hidden * 4;
    const long long o_out = llg_align((long long)xb, 256);
    const long long o_ids = o_out + llg_align((long long)xb, 256);
    const long long o_w = o_ids + llg_align((long long)n_tok * k * 4, 256);
    const long long o_ws = o_w + llg_align((long long)n_tok * k * 4, 256);
    uint8_t *ws = (uint8_t *)llg_ws(d, o_ws + moe_ws_bytes(a, n_tok), &rc);
    if (rc) return rc;
    if ((rc = llg_h2d(d, ws, x, xb))) return rc;
    rc = moe_enqueue(d, a, (const float *)ws, n_tok, (float *)(ws + o_out),
                     (int32_t *)(ws + o_ids), (float *)(ws + o_w), ws + o_ws);
    if (rc) return rc;
    if ((rc = llg_d2h(d, out, ws + o_out, xb))) return rc;
    if (ids && (rc = llg_d2h(d, ids, ws + o_ids, (size_t)n_tok * k * 4))) return rc;
    if (wts && (rc = llg_d2h(d, wts, ws + o_w, (size_t)n_tok * k * 4))) return rc;
    return llg_sync_dev(d);
}

int llg_hip_moe_route(LlgHipDevice h, const float *logits, int n_tok, int n_exp, int k,
                      int32_t *ids, float *wts) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    if (k <= 0 || n_exp <= 0 || k > n_exp || n_exp > MOE_MAX_EXP || k > MOE_MAX_K)
        return llg_set_error(d, LLG_E_HPARAM, "moe_route: invalid nExperts=%d k=%d", n_exp, k);
    if (!logits || !ids || !wts || n_tok <= 0)
        return llg_set_error(d, LLG_E_ARG, "moe_route: bad arguments");
    const long long o_ids = llg_align((long long)n_tok * n_exp * 4, 256);
    const long long o_w = o_ids + llg_align((long long)n_tok * k * 4, 256);
    int rc;
    uint8_t *ws = (uint8_t *)llg_ws(d, o_w + (size_t)n_tok * k * 4, &rc);
    if (rc) return rc;
    if ((rc = llg_h2d(d, ws, logits, (size_t)n_tok * n_exp * 4))) return rc;
    hipLaunchKernelGGL(k_moe_router, dim3(n_tok), dim3(64), 0, llg_dev_stream(d),
                       (const uint8_t *)nullptr, 0LL, 0, n_exp, k, (const float *)nullptr,
                       (const float *)ws, (int32_t *)(ws + o_ids), (float *)(ws + o_w));
    LLG_LAUNCH_CHECK(d, "moe_route");
    if ((rc = llg_d2h(d, ids, ws + o_ids, (size_t)n_tok * k * 4))) return rc;
    if ((rc = llg_d2h(d, wts, ws + o_w, (size_t)n_tok * k * 4))) return rc;
    return llg_sync_dev(d);
}

}  // extern "C"
