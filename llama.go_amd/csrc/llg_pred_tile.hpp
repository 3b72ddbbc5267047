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
#define LLG_PRED_SPLIT 8  // chunks of a WUp row: partial dots per hidden unit
#define LLG_HID_LOADS 4   // float4 loads a lane issues together

// Chunk s (of LLG_PRED_SPLIT) of the dots of R WUp rows with a
// (predictor.go:57), by the whole wavefront; every lane gets each row's sum
// in out[].  The rows share the loads of a; each row's sum is the same as
// with R = 1.
template <int R>
__device__ __forceinline__ void llg_pred_split_dots(const float *const (&rows)[R],
                                                    const float *__restrict__ a, int h, int s,
                                                    float (&out)[R]) {
    const int lane = threadIdx.x & 63;
    float acc[R];
#pragma unroll
    for (int k = 0; k < R; k++) acc[k] = 0.0f;
    if ((h & 3) == 0) {
        const int h4 = h >> 2;
        const int chunk = (h4 + LLG_PRED_SPLIT - 1) / LLG_PRED_SPLIT;
        const int c0 = s * chunk, c1 = min(h4, c0 + chunk);
        const float4 *a4 = reinterpret_cast<const float4 *>(a);
        for (int j0 = c0 + lane; j0 < c1; j0 += 64 * LLG_HID_LOADS) {
            float4 w[R][LLG_HID_LOADS], v[LLG_HID_LOADS];
#pragma unroll
            for (int i = 0; i < LLG_HID_LOADS; i++) {
                const int j = j0 + 64 * i;
#pragma unroll
                for (int k = 0; k < R; k++)
                    w[k][i] = j < c1 ? reinterpret_cast<const float4 *>(rows[k])[j]
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
                v[i] = j < c1 ? a4[j] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int k = 0; k < R; k++) {
#pragma unroll
                for (int i = 0; i < LLG_HID_LOADS; i++) {
                    acc[k] += w[k][i].x * v[i].x;
                    acc[k] += w[k][i].y * v[i].y;
                    acc[k] += w[k][i].z * v[i].z;
                    acc[k] += w[k][i].w * v[i].w;
                }
            }
        }
    } else {
        const int chunk = (h + LLG_PRED_SPLIT - 1) / LLG_PRED_SPLIT;
        const int c0 = s * chunk, c1 = min(h, c0 + chunk);
        for (int j = c0 + lane; j < c1; j += 64) {
            const float av = a[j];
#pragma unroll
            for (int k = 0; k < R; k++) acc[k] += rows[k][j] * av;
        }
    }
#pragma unroll
    for (int k = 0; k < R; k++) out[k] = llg_wave_sum(acc[k]);
}

__device__ __forceinline__ float llg_pred_split_dot(const float *__restrict__ row,
                                                    const float *__restrict__ a, int h, int s) {
    const float *const rows[1] = {row};
    float out[1];
    llg_pred_split_dots<1>(rows, a, h, s, out);
    return out[0];
}

// ReLU of a hidden unit from its LLG_PRED_SPLIT partial dots, added in chunk
// order (predictor.go:57-61).
__device__ __forceinline__ float llg_hidden_from_parts(const float *p) {
    float v = 0.0f;
#pragma unroll
    for (int s = 0; s < LLG_PRED_SPLIT; s++) v += p[s];
    return v < 0.0f ? 0.0f : v;
}

// Hidden units handed from the predictor workgroups of one launch to its tile
// workgroups (the sync area, LLG_SYNC_BYTES, holding LLG_SYNC_COPIES copies
// of the slots so that the readers of one copy are few).  Slot r holds (epoch << 32) |
// the bits of ReLU(hidden[r]), written as one 64-bit relaxed atomic at agent
// scope, so a reader that sees this launch's epoch in a slot has that slot's
// value: no fence and no separate flag.  The epoch is the word at the head of
// the area plus 1; the partial-sum kernel that ends the step advances the
// word, so a slot read during a launch holds either this launch's epoch or an
// older one (the area starts zeroed).
__device__ __forceinline__ void llg_slot_put(uint64_t *slot, uint32_t epoch, float v) {
    __hip_atomic_store(slot, ((uint64_t)epoch << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t llg_slot_get(const uint64_t *slot) {
    return __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The epoch word, read as a vector load (a scalar load's wait would come
// before the loads that follow it); written by the previous kernel.
__device__ __forceinline__ uint32_t llg_epoch_get(const uint32_t *ctr) {
    return __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct WoutTile {
    float4 w[PRED_MAXV];
    int v;      // float4 per lane (rank / 16), 0 = scalar path; wavefront-uniform
    int r, q;   // row within the wavefront's 16, quarter
};

// Every load is unconditional (a row past ff reads row ff - 1, whose logit
// the caller does not use; a slot k >= v repeats group v - 1), so that no
// load sits under a branch and the waits after them stay exact.
__device__ __forceinline__ void load_wout_tile(WoutTile &t, const uint8_t *__restrict__ wout,
                                               long long stride, int ff, int rank, int tile0) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    t.v = __builtin_amdgcn_readfirstlane((rank % 16 == 0 && rank <= 16 * PRED_MAXV) ? rank / 16 : 0);
    t.r = lane >> 2;
    t.q = lane & 3;
    if (!t.v) return;
    const int i = min(tile0 + wave * 16 + t.r, ff - 1);
    const float4 *row = reinterpret_cast<const float4 *>(wout + (long long)i * stride);
#pragma unroll
    for (int k = 0; k < PRED_MAXV; k++) t.w[k] = row[4 * min(k, t.v - 1) + t.q];
}

// The logit of row t.r of the wavefront's 16 in every lane of its quad: the
// loaded WOut groups against ReLU(hidden) in LDS (hid, rank floats, 16-byte
// aligned), every LDS read issued before the products, which run in group
// order k < v.
__device__ __forceinline__ float wout_tile_dot(const WoutTile &t, const float *hid) {
    const float4 *h4 = reinterpret_cast<const float4 *>(hid);
    float4 hv[PRED_MAXV];
#pragma unroll
    for (int k = 0; k < PRED_MAXV; k++) hv[k] = h4[4 * min(k, t.v - 1) + t.q];
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < PRED_MAXV; k++) {
        if (k < t.v) {
            acc += t.w[k].x * hv[k].x;
            acc += t.w[k].y * hv[k].y;
            acc += t.w[k].z * hv[k].z;
            acc += t.w[k].w * hv[k].w;
        }
    }
    return llg_quad_sum(acc);
}

// hid: ReLU(hidden) in LDS (rank floats, 16-byte aligned); lg: 64 floats in LDS.
__device__ __forceinline__ void finish_logits(const WoutTile &t, const uint8_t *__restrict__ wout,
                                              long long stride, int ff, int rank, int tile0,
                                              const float *hid, float *lg) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (t.v) {
        const float acc = wout_tile_dot(t, hid);
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
    static_assert(PS == LLG_PRED_SPLIT, "one split count");
    for (int r = threadIdx.x; r < rank; r += blockDim.x) {
        float p[PS];
#pragma unroll
        for (int s = 0; s < PS; s++) p[s] = partial[s * rank + r];
        hid[r] = llg_hidden_from_parts(p);
    }
}
