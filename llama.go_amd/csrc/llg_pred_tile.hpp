// llg_pred_tile.hpp -- the 64-neuron logit tile shared by the predict-only
// kernel (llg_predictor.hip) and the predictor-fused sparse FFN (llg_sparse.hip).
//
// A workgroup of 4 wavefronts owns neurons [tile0, tile0 + 64); wavefront w
// owns 16 of them.  Quad layout: lane l handles row l/4 of its wavefront and
// the float4 columns 4*i + l%4 (i < V = rank/16), so each load instruction
// reads 64 contiguous bytes from each of 16 rows, and a row's dot product is
// finished with two DPP quad steps.  All V <= 8 loads of a lane are issued
// (load_wout_tile) before the hidden vector is ready; finish_logits then
// reduces them against ReLU(hidden) held in LDS.  Ranks that are not a
// multiple of 16 or exceed 128 take a scalar loop.
#pragma once
#include "llg_common.hpp"

#define PRED_MAXV 8

struct WoutTile {
    float4 w[PRED_MAXV];
    int v;      // float4 per lane (rank / 16), 0 = scalar path
    int r, q;   // row within the wavefront's 16, quarter
};

__device__ __forceinline__ void load_wout_tile(WoutTile &t, const uint8_t *__restrict__ wout,
                                               long long stride, int ff, int rank, int tile0) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    t.v = (rank % 16 == 0 && rank <= 16 * PRED_MAXV) ? rank / 16 : 0;
    t.r = lane >> 2;
    t.q = lane & 3;
    if (!t.v) return;
    const int i = tile0 + wave * 16 + t.r;
    const float4 *row = reinterpret_cast<const float4 *>(wout + (long long)i * stride);
#pragma unroll
    for (int k = 0; k < PRED_MAXV; k++)
        t.w[k] = (k < t.v && i < ff) ? row[4 * k + t.q] : make_float4(0.f, 0.f, 0.f, 0.f);
}

// hid: ReLU(hidden) in LDS (rank floats, 16-byte aligned); lg: 64 floats in LDS.
__device__ __forceinline__ void finish_logits(const WoutTile &t, const uint8_t *__restrict__ wout,
                                              long long stride, int ff, int rank, int tile0,
                                              const float *hid, float *lg) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (t.v) {
        const float4 *h4 = reinterpret_cast<const float4 *>(hid);
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < PRED_MAXV; k++) {
            if (k < t.v) {
                const float4 hv = h4[4 * k + t.q];
                acc += t.w[k].x * hv.x;
                acc += t.w[k].y * hv.y;
                acc += t.w[k].z * hv.z;
                acc += t.w[k].w * hv.w;
            }
        }
        acc = llg_quad_sum(acc);
        if (t.q == 0) lg[wave * 16 + t.r] = acc;
    } else {
        for (int r = 0; r < 16; r++) {
            const int i = tile0 + wave * 16 + r;
            float acc = 0.0f;
            if (i < ff) {
                const float *w = reinterpret_cast<const float *>(wout + (long long)i * stride);
                for (int c = lane; c < rank; c += 64) acc += w[c] * hid[c];
            }
            acc = llg_wave_sum(acc);
            if (lane == 0) lg[wave * 16 + r] = acc;
        }
    }
}

// hid[r] = ReLU(sum of the PS partials) (predictor.go:57-61); the PS loads
// of a thread are issued together.
template <int PS>
__device__ __forceinline__ void load_hidden(float *hid, const float *__restrict__ partial,
                                            int rank) {
    for (int r = threadIdx.x; r < rank; r += blockDim.x) {
        float p[PS];
#pragma unroll
        for (int s = 0; s < PS; s++) p[s] = partial[s * rank + r];
        float v = 0.0f;
#pragma unroll
        for (int s = 0; s < PS; s++) v += p[s];
        hid[r] = v < 0.0f ? 0.0f : v;
    }
}
