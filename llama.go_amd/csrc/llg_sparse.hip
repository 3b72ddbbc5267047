// llg_sparse.hip -- gathered sparse FFN over row-column bundles
// (inference/ffn_flash.go:195-299, window.go:143-180).
//
// Three ways in:
//
//  A. predictor-fused step (ffnFlash path 2, ffn_flash.go:225-231), 2 launches:
//     K1 k_tile_ffn: its first workgroups compute the predictor's hidden units
//        (the sums of k_pred_hidden, llg_predictor.hip) and hand them to the
//        tile workgroups as epoch-tagged slots (a caller without a sync area,
//        or with hidden partials of its own, runs k_pred_hidden first); then
//        one workgroup per two 64-neuron tiles (Q4_0/Q8_0; one
//        tile for F16/F32): logits from WOut rows, strict '>' against the
//        threshold via a wavefront ballot (one mask word per tile), then each
//        active neuron's up row (u = act(up . x)) and, in the same round of
//        loads, its down row (the two rows are one contiguous bundle); the
//        workgroup's partial output, sum of u * down over its active neurons
//        in ascending order, goes to its own row of `part`
//     K2 k_tile_reduce: out = sum of the partial rows in row order
//  B. explicit active list (ffnSparseLoad, NeuronCache.FFNForward), 2 launches:
//     k_list_up: one wavefront per listed neuron, pair j = (row, u_j)
//     k_sparse_down: one workgroup per output block of 32 outputs reads every
//        pair (each thread a stride of the list)
//  C. the window's update + FFN step (NeuronCache.Update then FFNForward,
//     window.go:71-180), 1 launch: k_win_step's up workgroups (B's up rows,
//     a loaded neuron read from the layer's bundle and copied into its row),
//     down workgroups (B's down sums, their rows requested before the
//     activations exist, which arrive as epoch-tagged slots) and one
//     workgroup for the update of the counts and the residency
//
// No output is summed with atomics, and every sum has a fixed order, so the
// results are bit-identical from run to run.  u == 0 rows are skipped as at
// ffn_flash.go:290.
//
// x is staged once per workgroup in LDS with a 36-float stride per 32-float
// block, so the 16-byte reads of 16 consecutive lanes (one block each) hit
// 64 distinct banks.  Every lane issues the loads of all its blocks before it
// uses any of them.
//
// k_sparse_down: each thread adds its pairs in list order, then a fixed
// shuffle/DPP transpose reduction per wavefront and an ordered sum over the
// wavefronts finish the block.  blockIdx -> block keeps neighbouring blocks
// (which share the rows' cache lines) on one XCD (workgroups go round-robin
// over the 8 XCDs).
#include "llg_common.hpp"
#include "llg_internal.hpp"
#include "llg_pred_tile.hpp"
#include "llg_window_upd.hpp"

#include <algorithm>

#define XS_STRIDE 36      // floats per staged 32-float x block (bank-conflict-free)
#define BATCH 4           // blocks whose loads a lane issues together
#define PRED_SPLIT_N 8    // partials per hidden unit written by k_pred_hidden
#define DN_THREADS 512    // k_sparse_down workgroup: one tile (or list stride) per thread

// KN: one-pass rounds of float4 per thread (rows past KN * blockDim float4
// take the looped form); callers pass the fewest that cover 160 blocks.
template <int KN = 8, class Issue = LlgNoIssue>
__device__ __forceinline__ void stage_x(float *xs, const float *__restrict__ x, int nb,
                                        Issue &&issue = Issue()) {
    llg_stage_x_sum<XS_STRIDE, KN>(xs, x, nb, issue);
}
// rounds that cover 160 blocks (1280 float4) with nt threads
constexpr int stage_rounds(int nt) { return (1280 + nt - 1) / nt; }

// Up-row dot products of two rows by one wavefront (row < 0: no row, result
// 0): lane l owns blocks l, l+64, ...; the bytes of up to BATCH blocks of both
// rows are requested before any is used.  The row indices are made
// wavefront-uniform and loads are never under a per-lane condition (either
// makes the compiler wait for each load before issuing the next): a lane past
// the last block reloads it and drops the result.
// issued(): called once the pass's loads are issued, before any is used.
template <int T, typename Issued = LlgNoIssue>
__device__ __forceinline__ void row_dot2_pass(const uint8_t *p0, const uint8_t *p1, bool v0,
                                              bool v1, const RowFmt &f, const float *xs, int b0,
                                              float &a0, float &a1, Issued &&issued = Issued()) {
    const int lane = threadIdx.x & 63;
    BlockRaw<T> r0[BATCH], r1[BATCH];
#pragma unroll
    for (int i = 0; i < BATCH; i++) {  // straight-line loads (p0/p1 point at row 0 if unused)
        const int b = min(b0 + lane + 64 * i, f.nb - 1);
        llg_block_load<T>(r0[i], p0, f, b);
        llg_block_load<T>(r1[i], p1, f, b);
    }
    __builtin_amdgcn_sched_barrier(0);  // issued() stays behind these loads
    issued();
#pragma unroll
    for (int i = 0; i < BATCH; i++) {
        const int b = b0 + lane + 64 * i;
        if (b < f.nb) {
            const float *xb = xs + b * XS_STRIDE;
            const float4 *x4 = reinterpret_cast<const float4 *>(xb);
            const float d0 = llg_raw_dot<T>(r0[i], x4, xb[32]);
            const float d1 = llg_raw_dot<T>(r1[i], x4, xb[32]);
            a0 += v0 ? d0 : 0.0f;
            a1 += v1 ? d1 : 0.0f;
        }
    }
}

// p0/p1: the rows (valid when v0/v1; otherwise any readable row).
// issued(): run once the first pass's loads are issued.
template <int T, typename Issued = LlgNoIssue>
__device__ __forceinline__ void row_dot2p(const uint8_t *p0, const uint8_t *p1, bool v0, bool v1,
                                          const RowFmt &f, const float *xs, float &s0,
                                          float &s1, Issued &&issued = Issued()) {
    float a0 = 0.0f, a1 = 0.0f;
    if (f.nb <= 64 * BATCH) {
        row_dot2_pass<T>(p0, p1, v0, v1, f, xs, 0, a0, a1, issued);
    } else {
        row_dot2_pass<T>(p0, p1, v0, v1, f, xs, 0, a0, a1, issued);
        for (int b0 = 64 * BATCH; b0 < f.nb; b0 += 64 * BATCH)
            row_dot2_pass<T>(p0, p1, v0, v1, f, xs, b0, a0, a1);
    }
    s0 = llg_wave_sum(a0);
    s1 = llg_wave_sum(a1);
}

template <int T>
__device__ __forceinline__ void row_dot2(const uint8_t *__restrict__ base, long long bstride,
                                         int row0, int row1, const RowFmt &f, const float *xs,
                                         float &s0, float &s1) {
    row0 = __builtin_amdgcn_readfirstlane(row0);
    row1 = __builtin_amdgcn_readfirstlane(row1);
    const bool v0 = row0 >= 0, v1 = row1 >= 0;
    row_dot2p<T>(base + (long long)(v0 ? row0 : 0) * bstride,
                 base + (long long)(v1 ? row1 : 0) * bstride, v0, v1, f, xs, s0, s1);
}

// Copy of one bundle (n16 16-byte units) by a wavefront: bc_issue loads the
// first 64 * N units (N <= 5), bc_store stores them (the caller issues other
// loads in between, so that one wait covers both), bc_rest copies the rest.
typedef unsigned int bc_u4 __attribute__((ext_vector_type(4)));
template <int N>
struct BundleCopy {
    bc_u4 v[N];
};
template <int N>
__device__ __forceinline__ void bc_issue(BundleCopy<N> &c, const bc_u4 *__restrict__ sp, int n16) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < N; k++) c.v[k] = sp[min(lane + 64 * k, n16 - 1)];
}
template <int N>
__device__ __forceinline__ void bc_store(const BundleCopy<N> &c, bc_u4 *__restrict__ dp, int n16) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < N; k++)
        if (lane + 64 * k < n16) dp[lane + 64 * k] = c.v[k];
}
template <int N>
__device__ __forceinline__ void bc_rest(const bc_u4 *__restrict__ sp, bc_u4 *__restrict__ dp,
                                        int n16) {
    for (int u = 64 * N + (int)(threadIdx.x & 63); u < n16; u += 64) dp[u] = sp[u];
}
// units held across the dot: a whole Q4_0/Q8_0 bundle of up to 5120 bytes
template <int T>
constexpr int bc_first() {
    return T == LLG_TYPE_Q4_0 || T == LLG_TYPE_Q8_0 ? 5 : 1;
}

// Up-row dot products of NR rows (wavefront-uniform indices, < 0: none, sum
// unspecified) by one wavefront, NBATCH blocks per lane per pass, all loads
// of a pass issued before any is used.  WHOLE: the caller guarantees that the
// first pass reaches past block 64 (NBATCH - 1) (its batches before the last
// are whole).  issued(): called once, when the first pass's loads are issued
// (before any is used).
template <int T, int NR, int NBATCH, bool WHOLE, typename Issued = LlgNoIssue>
__device__ __forceinline__ void row_dotn(const uint8_t *__restrict__ base, long long bstride,
                                         const int (&row)[NR], const RowFmt &f, const float *xs,
                                         float (&s)[NR], Issued &&issued = Issued()) {
    const int lane = threadIdx.x & 63;
    const uint8_t *p[NR];
    bool v[NR];
#pragma unroll
    for (int q = 0; q < NR; q++) {
        const int r = __builtin_amdgcn_readfirstlane(row[q]);
        v[q] = r >= 0;
        p[q] = base + (long long)(v[q] ? r : 0) * bstride;
        s[q] = 0.0f;
    }
    using Pass = BlockRaw<T>[NBATCH][NR];
    auto load = [&](Pass &r, int b0) {
#pragma unroll
        for (int i = 0; i < NBATCH; i++)
#pragma unroll
            for (int q = 0; q < NR; q++)
                llg_block_load<T>(r[i][q], p[q], f, min(b0 + lane + 64 * i, f.nb - 1));
    };
    {
        // The first pass straight-line, issued() right behind its loads, and
        // no dot under a condition: lanes past the row's end (only in the last
        // batch, if WHOLE) dot the clamped copy with its scale zeroed
        // (llg_block_keep).  A fixed number of
        // loads then follows each block, so each dot waits for its own
        // blocks; a conditional dot would let the compiler sink its loads
        // behind issued()'s (or a loop head would wait for all).  The sum of
        // a row < 0 is left unspecified (the caller drops it).
        Pass r;
        load(r, 0);
        __builtin_amdgcn_sched_barrier(0);  // issued() stays behind these loads
        issued();
#pragma unroll
        for (int i = 0; i < NBATCH; i++) {
            const int b = lane + 64 * i;
            const float *xb = xs + min(b, f.nb - 1) * XS_STRIDE;
            const float4 *x4 = reinterpret_cast<const float4 *>(xb);
#pragma unroll
            for (int q = 0; q < NR; q++) {
                BlockRaw<T> rb = r[i][q];
                if (!WHOLE || i == NBATCH - 1) llg_block_keep<T>(rb, b < f.nb);
                s[q] += llg_raw_dot<T>(rb, x4, xb[32]);
            }
        }
    }
    for (int b0 = 64 * NBATCH; b0 < f.nb; b0 += 64 * NBATCH) {  // rows past 64 NBATCH blocks
        Pass r;
        load(r, b0);
#pragma unroll
        for (int i = 0; i < NBATCH; i++) {
            const int b = b0 + lane + 64 * i;
            if (b < f.nb) {
                const float *xb = xs + b * XS_STRIDE;
                const float4 *x4 = reinterpret_cast<const float4 *>(xb);
#pragma unroll
                for (int q = 0; q < NR; q++) s[q] += llg_raw_dot<T>(r[i][q], x4, xb[32]);
            }
        }
    }
#pragma unroll
    for (int q = 0; q < NR; q++) s[q] = llg_wave_sum(s[q]);
}

// B. explicit list: pair j = (row of active[j], act(up . x)).
// The count read on the device is clamped to the pair capacity `cap`, and a
// neuron outside [0, n_rows) counts as absent (activation 0), so no list
// makes the kernel read or write out of bounds.  res (a window's residency,
// optional): a neuron with res[n] == 0 is not resident and keeps activation 0
// (window.go:150-152).
template <int T>
__global__ __launch_bounds__(256) void k_list_up(
    const uint8_t *base, long long bstride, RowFmt f, const int32_t *__restrict__ res,
    const float *__restrict__ x, const int32_t *__restrict__ active,
    const int32_t *__restrict__ n_active_p, int cap, int n_rows, int act,
    int2 *__restrict__ pairs) {
    extern __shared__ float xs[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int first = blockIdx.x * 4;
    const int stride = (int)gridDim.x * 4;
    const int jf = first + wave;
    const int n_active = min(max(*n_active_p, 0), cap);
    if (first >= n_active) return;  // whole workgroup idle: skip the x staging
    auto valid = [&](int n) { return n >= 0 && n < n_rows ? n : -1; };
    // One pair: entries j and j1 = j + stride (j < n_active), neurons m0, m1
    // (-1 past the count or out of range); with res, a neuron not resident
    // has no row.
    struct Rows {
        int row0, row1;
    };
    auto rows = [&](int m0, int m1) {
        Rows r{m0, m1};
        if (res) {
            r.row0 = m0 < 0 || res[m0] == 0 ? -1 : m0;
            r.row1 = m1 < 0 || res[m1] == 0 ? -1 : m1;
        }
        return r;
    };
    auto pair = [&](int j, const Rows &r) {
        const int j1 = j + stride;
        float s0, s1;
        row_dot2<T>(base, bstride, r.row0, r.row1, f, xs, s0, s1);
        if (lane == 0) {  // a row without a neuron keeps activation 0 (window.go:150-152)
            pairs[j] = make_int2(r.row0, __float_as_int(r.row0 >= 0 ? llg_act(act, s0) : 0.0f));
            if (j1 < n_active)
                pairs[j1] = make_int2(r.row1, __float_as_int(r.row1 >= 0 ? llg_act(act, s1) : 0.0f));
        }
    };
    // The first pair's entries (never past the count: the list holds
    // n_active entries) are requested while x is in flight.
    const bool has0 = jf < n_active;
    int a0 = -1, a1 = -1;
    stage_x<stage_rounds(256)>(xs, x, f.nb, [&]() {
        a0 = active[min(jf, n_active - 1)];
        a1 = active[min(jf + stride, n_active - 1)];
    });
    const int m0 = has0 ? valid(a0) : -1;
    const int m1 = jf + stride < n_active ? valid(a1) : -1;
    const Rows r0 = rows(m0, m1);
    __syncthreads();
    if (has0) pair(jf, r0);
    for (int j = jf + 2 * stride; j < n_active; j += 2 * stride) {
        const int j1 = j + stride;
        const int n0 = valid(active[j]);
        const int n1 = j1 < n_active ? valid(active[j1]) : -1;
        pair(j, rows(n0, n1));
    }
}

// Sum of v[0..31] over the wavefront by halving exchanges: at each step a
// lane keeps half of its values and adds the partner's copy of that half.
// The partners are lane ^ 32, ^ 16, ^ 8, ^ 7, ^ 2 and ^ 1: each step's
// partner agrees in the lane bits that already chose the half (so it holds
// the same elements) and covers a disjoint set of lanes.  Lane l returns the
// total of element l >> 1.  The exchange pattern is fixed, so the result is
// the same on every run.
__device__ __forceinline__ float dn_wave_transpose_sum(const float (&v)[32]) {
    const int lane = threadIdx.x & 63;
    float a[16], b[8], c[4], d[2];
    const bool h5 = lane & 32, h4 = lane & 16, h3 = lane & 8, h2 = lane & 4, h1 = lane & 2;
#pragma unroll
    for (int m = 0; m < 16; m++)
        a[m] = (h5 ? v[m + 16] : v[m]) + __shfl_xor(h5 ? v[m] : v[m + 16], 32, 64);
#pragma unroll
    for (int m = 0; m < 8; m++)
        b[m] = (h4 ? a[m + 8] : a[m]) + __shfl_xor(h4 ? a[m] : a[m + 8], 16, 64);
#pragma unroll
    for (int m = 0; m < 4; m++)  // row_ror:8 pairs lanes that differ in bit 3
        c[m] = (h3 ? b[m + 4] : b[m]) + llg_dpp<0x128>(h3 ? b[m] : b[m + 4]);
#pragma unroll
    for (int m = 0; m < 2; m++)  // row_half_mirror pairs lane i with i ^ 7: bit 2 differs,
                                 // bits 3-5 (the element so far) agree
        d[m] = (h2 ? c[m + 2] : c[m]) + llg_dpp<0x141>(h2 ? c[m] : c[m + 2]);
    const float e = (h1 ? d[1] : d[0]) + llg_dpp<0x4E>(h1 ? d[0] : d[1]);  // bit 1
    return e + llg_dpp<0xB1>(e);                                           // bit 0
}

#define TU 64  // neurons per predictor tile (one mask word)

// One round of the tile's up rows with the activations kept in LDS, over the
// first nw wavefronts: active neuron k = k0 + wave + nw*i (i < NR) of the
// tile on this wavefront, ul[k] = act(up . x).  issued(): called once this
// wavefront's loads of the round are issued (at once when it has no row).
// FIRST: the first round (its own copy of the dot per row length).
template <int T, int NR, bool FIRST, typename Issued = LlgNoIssue>
__device__ __forceinline__ void tile_u_round(const uint8_t *__restrict__ base, long long bstride,
                                             const RowFmt &f, const float *xs, const int *tl,
                                             int cnt, int k0, int tile0, int act, float *ul,
                                             int nw, Issued &&issued = Issued()) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int rows[NR];
#pragma unroll
    for (int i = 0; i < NR; i++) {
        const int k = k0 + wave + nw * i;
        rows[i] = __builtin_amdgcn_readfirstlane(k < cnt ? tile0 + tl[k] : -1);
    }
    if (rows[0] < 0) {  // wavefront-uniform: nothing in this round
        issued();
        return;
    }
    float s[NR];
    if constexpr (FIRST) {
        // batches per pass: the fewest whose first pass reaches the row's end
        // (at most 3), so only the last batch has lanes past it
        if (f.nb > 128)
            row_dotn<T, NR, 3, true>(base, bstride, rows, f, xs, s, issued);
        else if (f.nb > 64)
            row_dotn<T, NR, 2, true>(base, bstride, rows, f, xs, s, issued);
        else
            row_dotn<T, NR, 1, true>(base, bstride, rows, f, xs, s, issued);
    } else {  // further rounds (more active neurons than wavefronts): one copy
        row_dotn<T, NR, 3, false>(base, bstride, rows, f, xs, s, issued);
    }
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int i = 0; i < NR; i++)
            if (rows[i] >= 0) ul[k0 + wave + nw * i] = llg_act(act, s[i]);
    }
}

// A quarter of a 32-element block of a row in the row format: the bytes of
// elements [8 q, 8 q + 8) of block b, and the block scale (Q4_0: word q of the
// block's nibbles; Q8_0: bytes 8q..8q+7; F16/F32: 8 values).
template <int T>
struct QuarterRaw;
template <>
struct QuarterRaw<LLG_TYPE_Q4_0> {
    uint32_t q;
    unsigned short d;
};
template <>
struct QuarterRaw<LLG_TYPE_Q8_0> {
    uint2 q;
    unsigned short d;
};
template <>
struct QuarterRaw<LLG_TYPE_F16> {
    uint4 q;
};
template <>
struct QuarterRaw<LLG_TYPE_F32> {
    float4 q[2];
};

template <int T>
__device__ __forceinline__ void quarter_load(QuarterRaw<T> &r, const uint8_t *__restrict__ row,
                                             const RowFmt &f, int b, int q) {
    if constexpr (T == LLG_TYPE_Q4_0) {
        r.q = *reinterpret_cast<const uint32_t *>(row + (size_t)b * 16 + q * 4);
        r.d = *reinterpret_cast<const unsigned short *>(row + f.d_off + b * 2);
    } else if constexpr (T == LLG_TYPE_Q8_0) {
        r.q = *reinterpret_cast<const uint2 *>(row + (size_t)b * 32 + q * 8);
        r.d = *reinterpret_cast<const unsigned short *>(row + f.d_off + b * 2);
    } else if constexpr (T == LLG_TYPE_F16) {
        r.q = *reinterpret_cast<const uint4 *>(row + (size_t)b * 64 + q * 16);
    } else {
        const float4 *p = reinterpret_cast<const float4 *>(row + (size_t)b * 128 + q * 32);
        r.q[0] = p[0];
        r.q[1] = p[1];
    }
}

// acc[0..7] += u * dequant(quarter block), with the quantized types' offset
// folded into *corr (the caller subtracts corr from every element once):
// Q4_0 adds u d (64 + q) (a nibble under the f16 exponent bits 0x5400 is
// exactly 64 + q, multiplied into fp32 by v_fma_mix) and corr 72 u d; Q8_0
// adds u d (q + 128) and corr 128 u d.
template <int T>
__device__ __forceinline__ void quarter_axpy(const QuarterRaw<T> &r, float u, float (&acc)[8],
                                             float &corr) {
    if constexpr (T == LLG_TYPE_Q4_0) {
        const float s = u * llg_f16(r.d);
        corr += 72.0f * s;
        const uint32_t w = r.q, m = 0x00F000F0u, e = 0x54005400u;
        // nibble p of the word is element p
        const half2_llg p0 = __builtin_bit_cast(half2_llg, llg_and_or(w << 4, m, e));
        const half2_llg p1 = __builtin_bit_cast(half2_llg, llg_and_or(w, m, e));
        const half2_llg p2 = __builtin_bit_cast(half2_llg, llg_and_or(w >> 4, m, e));
        const half2_llg p3 = __builtin_bit_cast(half2_llg, llg_and_or(w >> 8, m, e));
        acc[0] = __builtin_fmaf((float)p0[0], s, acc[0]);
        acc[1] = __builtin_fmaf((float)p1[0], s, acc[1]);
        acc[2] = __builtin_fmaf((float)p2[0], s, acc[2]);
        acc[3] = __builtin_fmaf((float)p3[0], s, acc[3]);
        acc[4] = __builtin_fmaf((float)p0[1], s, acc[4]);
        acc[5] = __builtin_fmaf((float)p1[1], s, acc[5]);
        acc[6] = __builtin_fmaf((float)p2[1], s, acc[6]);
        acc[7] = __builtin_fmaf((float)p3[1], s, acc[7]);
    } else if constexpr (T == LLG_TYPE_Q8_0) {
        const float s = u * llg_f16(r.d);
        corr += 128.0f * s;
        const uint32_t w[2] = {r.q.x, r.q.y};
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t v = w[i] ^ 0x80808080u;
#pragma unroll
            for (int k = 0; k < 4; k++) acc[4 * i + k] += s * (float)((v >> (8 * k)) & 0xFF);
        }
    } else if constexpr (T == LLG_TYPE_F16) {
        const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            acc[2 * k] += u * llg_f16(w[k] & 0xFFFF);
            acc[2 * k + 1] += u * llg_f16(w[k] >> 16);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            acc[4 * i + 0] += u * r.q[i].x;
            acc[4 * i + 1] += u * r.q[i].y;
            acc[4 * i + 2] += u * r.q[i].z;
            acc[4 * i + 3] += u * r.q[i].w;
        }
    }
}

// 64-neuron tiles per k_tile_ffn workgroup, and its threads: Q4_0 takes two
// tiles on 1024 threads (one workgroup per CU, 128 registers); the wider
// rows of the other types need more registers and take one tile on 512
// threads.
template <int T>
constexpr int tf_tiles() {
    return T == LLG_TYPE_Q4_0 ? 2 : 1;
}
template <int T>
constexpr int tf_threads() {
    return 512 * tf_tiles<T>();
}
// Down rows a k_tile_ffn thread holds at once (quarter blocks), by type.
template <int T>
constexpr int tf_dk() {
    return T == LLG_TYPE_Q4_0 || T == LLG_TYPE_Q8_0 ? 16 : (T == LLG_TYPE_F16 ? 8 : 4);
}

// The logit of row 16 w + l / 4 of the tile in every lane l of wavefront w
// (the quad layout of load_wout_tile; the scalar layout for other ranks),
// the same sums as finish_logits.
__device__ __forceinline__ float tile_logit(const WoutTile &t, const uint8_t *__restrict__ wout,
                                            long long stride, int ff, int rank, int tile0,
                                            const float *hid) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (t.v) return wout_tile_dot(t, hid);
    float mine = 0.0f;
    for (int r = 0; r < 16; r++) {
        const int i = tile0 + wave * 16 + r;
        float acc = 0.0f;
        if (i < ff) {
            const float *w = reinterpret_cast<const float *>(wout + (long long)i * stride);
            for (int c = lane; c < rank; c += 64) acc += w[c] * hid[c];
        }
        acc = llg_wave_sum(acc);
        if ((lane >> 2) == r) mine = acc;
    }
    return mine;
}

// Bits 0, 4, 8, ..., 60 of m as a 16-bit word (bit r = bit 4 r).
__device__ __forceinline__ uint32_t quad_bits(unsigned long long m) {
    m &= 0x1111111111111111ull;
    m = (m | (m >> 3)) & 0x0303030303030303ull;
    m = (m | (m >> 6)) & 0x000F000F000F000Full;
    m = (m | (m >> 12)) & 0x000000FF000000FFull;
    m = (m | (m >> 24)) & 0xFFFFull;
    return (uint32_t)m;
}

// The predictor inside the tile launch (ffnFlash path 2 with the predictor
// input given): the first n_hid workgroups compute the hidden units and hand
// them to the tile workgroups through the sync slots (llg_pred_tile.hpp).
// They come first in the grid, so they are dispatched before any tile
// workgroup that waits for them.  n_hid = 0: the hidden partials are in
// `partial`, written by an earlier kernel.
struct HidArgs {
    const uint8_t *wup;  // WUp (rank rows of h floats)
    long long wstride;
    int h;
    const float *a;          // predictor input
    uint64_t *slots;         // sync slots, after the epoch word at ctr
    const uint32_t *ctr;
    int n_hid;               // predictor workgroups at the head of the grid
    float *acc_out;          // optional: acc_out[i] += acc_add[i], i < acc_n
    const float *acc_add;
    int acc_n;
    int check;               // llg_dev_check: every unit computed by the tiles after the wait
};

// Wo . attn and the predictor in the tile launch (a Falcon layer,
// llg_model.hip).  The predictor's input is attn_out = Wo . attn (ffnFlash
// path 2 after attention, ffn_flash.go:157-161), and its first product WUp .
// attn_out (predictor.go:57) is linear in attn, so it equals P . attn with P
// = WUp . Wo formed once at load.  The attention kernel leaves, per (split s,
// head h), pd[s][h][j] = P[j][head h's columns] . acc_s (the split's
// unnormalised output) beside its (m, l).  The first n_comb workgroups merge
// them per unit as the attention splits merge (e = exp(m - max m), the sum
// of pd e times 1 / sum of l e, llg_attn_merge4's steps), add the heads and
// hand ReLU of the sum to the tile workgroups through the sync slots.  The
// last n_wo workgroups stage the merged attention output (llg_stage_attn) and
// add their rows of Wo . attn into resid (x += attnOut, ffn_flash.go:161).
struct WoArgs {
    const uint8_t *w;  // Wo rows (Q4_0 or Q8_0), f.cols = the attention width
    long long stride;
    RowFmt f;
    int rows;          // Wo's rows: the residual's length
    float *resid;
    LlgAttnParts ap;
    const float *pd;   // [n_split][n_heads][rank]
    int n_comb, n_wo;  // workgroups at the head and at the tail of the grid
};
#define WO_NB 3   // Wo blocks per lane per row (rows of at most 192 blocks)

// Spin bound of a tile workgroup's wait for its hidden units (about 30 ms);
// past it the workgroup computes the missing units itself.
#define HID_POLLS (1 << 16)

// A predictor workgroup: RPW hidden units; wavefront s < LLG_PRED_SPLIT takes
// chunk s of each unit's WUp row (the sums of k_pred_hidden, the rows sharing
// the loads of a), then every copy of the units' slots is written.
template <int NW>
__device__ __forceinline__ void tile_hid_role(const HidArgs &ha, int rank, float *sh) {
    constexpr int RPW = NW / LLG_PRED_SPLIT;  // hidden units per workgroup
    static_assert(RPW >= 1 && NW % LLG_PRED_SPLIT == 0, "whole units per workgroup");
    // the epoch word as a vector load ahead of the row loads, waited on only
    // at the slot stores
    const uint32_t ctr = llg_epoch_get(ha.ctr);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r0 = blockIdx.x * RPW;
    if (wave < LLG_PRED_SPLIT) {
        const float *rows[RPW];
#pragma unroll
        for (int k = 0; k < RPW; k++)  // a unit past rank rereads the last row
            rows[k] = reinterpret_cast<const float *>(ha.wup + (long long)min(r0 + k, rank - 1) * ha.wstride);
        float p[RPW];
        llg_pred_split_dots<RPW>(rows, ha.a, ha.h, wave, p);
        if ((threadIdx.x & 63) == 0) {
#pragma unroll
            for (int k = 0; k < RPW; k++) sh[k * LLG_PRED_SPLIT + wave] = p[k];
        }
    }
    __syncthreads();
    if ((int)threadIdx.x < RPW * LLG_SYNC_COPIES) {
        const int k = threadIdx.x % RPW, c = threadIdx.x / RPW;
        if (r0 + k < rank)
            llg_slot_put(ha.slots + c * LLG_SYNC_SLOTS + r0 + k, ctr + 1u,
                         llg_hidden_from_parts(sh + k * LLG_PRED_SPLIT));
    }
    if (ha.acc_out)
        for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < ha.acc_n; i += ha.n_hid * blockDim.x)
            ha.acc_out[i] += ha.acc_add[i];
}

// Hidden unit j of the predictor (ReLU'd, predictor.go:61) from the attention
// kernel's per-split fold partials, by the whole wavefront: lane l takes
// heads l, l + 64, ..., each merged over the splits with llg_attn_merge4's
// steps, and the lanes' sums are added by llg_wave_sum.  Every lane gets the
// value.
__device__ __forceinline__ float comb_unit(const WoArgs &wa, int rank, int j) {
    const int lane = threadIdx.x & 63;
    const LlgAttnParts &ap = wa.ap;
    const float2 *ml = reinterpret_cast<const float2 *>(ap.ml);
    float acc = 0.0f;
    for (int h0 = 0; h0 < ap.n_heads; h0 += 128) {  // two heads per lane per round
        // every split slot of both heads requested before any is used (a slot
        // past n_split rereads split 0 and is skipped)
        float2 m[2][LLG_ATTN_SPLIT_MAX];
        float a[2][LLG_ATTN_SPLIT_MAX];
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int h = min(h0 + lane + 64 * k, ap.n_heads - 1);
#pragma unroll
            for (int s = 0; s < LLG_ATTN_SPLIT_MAX; s++) {
                const int sc = s < ap.n_split ? s : 0;
                m[k][s] = ml[sc * ap.n_heads + h];
                a[k][s] = wa.pd[((size_t)sc * ap.n_heads + h) * rank + j];
            }
        }
#pragma unroll
        for (int k = 0; k < 2; k++) {
            if (h0 + lane + 64 * k >= ap.n_heads) continue;
            float M = m[k][0].x;
#pragma unroll
            for (int s = 1; s < LLG_ATTN_SPLIT_MAX; s++)
                if (s < ap.n_split) M = fmaxf(M, m[k][s].x);
            float L = 0.0f, v = 0.0f;
#pragma unroll
            for (int s = 0; s < LLG_ATTN_SPLIT_MAX; s++)
                if (s < ap.n_split) {
                    const float e = m[k][s].x == -INFINITY ? 0.0f : expf(m[k][s].x - M);
                    L += m[k][s].y * e;
                    v += a[k][s] * e;
                }
            const float rl = 1.0f / L;
            acc += v * rl;
        }
    }
    const float hv = llg_wave_sum(acc);
    return hv < 0.0f ? 0.0f : hv;
}

// A combiner workgroup: wavefront w takes hidden unit NW b + w and writes it
// to every copy of its slot.
template <int NW>
__device__ __forceinline__ void tile_comb_role(const WoArgs &wa, const HidArgs &ha, int rank) {
    const uint32_t ctr = llg_epoch_get(ha.ctr);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = blockIdx.x * NW + wave;
    if (j >= rank) return;  // uniform per wavefront
    const float hv = comb_unit(wa, rank, j);
    if (lane < LLG_SYNC_COPIES) llg_slot_put(ha.slots + lane * LLG_SYNC_SLOTS + j, ctr + 1u, hv);
}

// A Wo workgroup b: in pass p, wavefront w takes row (p n_wo + b) NW + w
// (lane l: blocks l, l + 64, l + 128) of the staged merged attention output;
// each pass's row loads are requested before the previous pass's dots (two
// buffers).  The rows are not on the tiles' path (only the partial-sum kernel
// reads resid).
template <int WT, int NW>
__device__ __forceinline__ void tile_wo_role(const WoArgs &wa, int b, float *xs) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const RowFmt &f = wa.f;
    BlockRaw<WT> q[2][WO_NB];
    const int n_pass = (wa.rows + wa.n_wo * NW - 1) / (wa.n_wo * NW);
    auto row_of = [&](int p) { return (p * wa.n_wo + b) * NW + wave; };
    auto issue = [&](int p, int buf) {
#pragma unroll
        for (int i = 0; i < WO_NB; i++)
            llg_block_load<WT>(q[buf][i], wa.w + (long long)min(row_of(p), wa.rows - 1) * wa.stride,
                               f, min(lane + 64 * i, f.nb - 1));
    };
    auto pass = [&](int p, int buf) {
        float sv = 0.0f;
#pragma unroll
        for (int i = 0; i < WO_NB; i++) {
            const int bl = lane + 64 * i;
            if (bl < f.nb) {
                const float *xb = xs + bl * XS_STRIDE;
                sv += llg_raw_dot<WT>(q[buf][i], reinterpret_cast<const float4 *>(xb), xb[32]);
            }
        }
        if (p + 2 < n_pass) issue(p + 2, buf);
        const float v = llg_wave_sum(sv);
        const int r = row_of(p);
        if (lane == 0 && r < wa.rows) wa.resid[r] = wa.resid[r] + v;
    };
    llg_stage_attn<XS_STRIDE, WT == LLG_TYPE_Q8_0 ? 1 : 2>(xs, wa.ap, 0, f.nb, [&]() {
        // every wavefront's staging loads ahead of any row load (a CU returns
        // vector loads in request order)
        __builtin_amdgcn_s_barrier();
        issue(0, 0);
    });
    __syncthreads();
    if (n_pass > 1) issue(1, 1);
    for (int p = 0; p < n_pass; p += 2) {  // uniform
        pass(p, 0);
        if (p + 1 < n_pass) pass(p + 1, 1);
    }
}

// Rows of Wo per workgroup of the tile launch: WO_PASSES passes.
#define WO_PASSES 4
template <int NW>
constexpr int wo_rows_per_wg() {
    return WO_PASSES * NW;
}

// The copy of the slots a tile workgroup reads: one per group of workgroups
// that the round-robin dispatch puts on one XCD.
__device__ __forceinline__ const uint64_t *tile_slot_copy(const HidArgs &ha) {
    return ha.slots + (blockIdx.x % LLG_SYNC_COPIES) * LLG_SYNC_SLOTS;
}

// A tile workgroup's hidden units from the slots: wavefront w takes units w
// * 64 + lane (+ the thread count per further pass); v0 is the first pass's
// slot value, requested with the x staging.  A unit whose slot does not show
// the epoch within HID_POLLS polls is computed here with the predictor
// workgroups' sums (the same value), so the wait always ends.
__device__ __forceinline__ void tile_take_hidden(float *hid, const HidArgs &ha, int rank,
                                                 uint32_t epoch, uint64_t v0) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint64_t *slots = tile_slot_copy(ha);
    for (int r0 = wave * 64; r0 < rank; r0 += blockDim.x) {
        const int r = min(r0 + lane, rank - 1);
        uint64_t v = r0 == wave * 64 ? v0 : llg_slot_get(slots + r);
        for (int polls = 0; !__all((uint32_t)(v >> 32) == epoch) && polls < HID_POLLS; polls++) {
            __builtin_amdgcn_s_sleep(1);
            v = llg_slot_get(slots + r);
        }
        float hv = __uint_as_float((uint32_t)v);
        unsigned long long miss = __ballot(ha.check || (uint32_t)(v >> 32) != epoch);
        while (miss) {  // wavefront-uniform
            const int l = __ffsll((long long)miss) - 1;
            miss &= miss - 1;
            const int u = r0 + l;
            if (u >= rank) continue;
            const float *row = reinterpret_cast<const float *>(ha.wup + (long long)u * ha.wstride);
            float val = 0.0f;  // the chunk sums in order, as llg_hidden_from_parts
#pragma unroll 1
            for (int s = 0; s < LLG_PRED_SPLIT; s++) val += llg_pred_split_dot(row, ha.a, ha.h, s);
            if (lane == l) hv = val < 0.0f ? 0.0f : val;
        }
        if (r0 + lane < rank) hid[r0 + lane] = hv;
    }
}

// A tile workgroup's hidden units from the combiner workgroups' slots, as
// tile_take_hidden: a unit whose slot does not show the epoch within
// HID_POLLS polls is combined by the wavefront itself (comb_unit, the same
// value), so the wait always ends.
__device__ __forceinline__ void tile_take_comb(float *hid, const WoArgs &wa, const HidArgs &ha,
                                               int rank, uint32_t epoch) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint64_t *slots = tile_slot_copy(ha);
    for (int r0 = wave * 64; r0 < rank; r0 += blockDim.x) {
        const int r = min(r0 + lane, rank - 1);
        uint64_t v = llg_slot_get(slots + r);
        for (int polls = 0; !__all((uint32_t)(v >> 32) == epoch) && polls < HID_POLLS; polls++) {
            __builtin_amdgcn_s_sleep(1);
            v = llg_slot_get(slots + r);
        }
        float hv = __uint_as_float((uint32_t)v);
        unsigned long long miss = __ballot(ha.check || (uint32_t)(v >> 32) != epoch);
        while (miss) {  // wavefront-uniform
            const int l = __ffsll((long long)miss) - 1;
            miss &= miss - 1;
            const int u = r0 + l;
            if (u >= rank) continue;
            const float val = comb_unit(wa, rank, u);
            if (lane == l) hv = val;
        }
        if (r0 + lane < rank) hid[r0 + lane] = hv;
    }
}

// A'. The predictor-fused tiles with their down products (the form the step
// uses): a workgroup owns tf_tiles 64-neuron tiles (WOut rows: 16 per
// wavefront; the ballot writes one mask word per tile and the workgroup's
// ascending active list), then
//   - every wavefront takes up rows (active neuron k on wavefront k mod the
//     wavefront count): ul[k] = act(up . x) in LDS;
//   - the top ceil(4 nb / 64) wavefronts also own the output quarter blocks
//     (8 outputs) of the workgroup's partial: right after their up-row loads
//     each of their threads requests its first quarter block of the down row
//     of each active neuron (up to tf_dk at once), so the down bytes arrive
//     in the round of the up rows (a neuron's up and down rows are one
//     contiguous bundle);
//   - part[w][o] = sum over the workgroup's active neurons, ascending, of
//     u * down[o] (a zero u is skipped, ffn_flash.go:290).
// Every workgroup writes its partial (zeros when nothing is active), and
// k_tile_reduce adds the partials in a fixed order, so the result is the
// same on every run.
// WO: the instance with Wo's workgroups at the head of the grid (k_tile_wo_ffn).
template <int T, bool WO>
__device__ __forceinline__ void tile_ffn_body(
    const uint8_t *__restrict__ wout, long long wstride, int ff, int rank,
    const float *__restrict__ partial, const float *__restrict__ bias, float thr,
    const uint8_t *__restrict__ base, long long bstride, RowFmt f, const float *__restrict__ x,
    int act, unsigned long long *__restrict__ mask, float *__restrict__ part, int pstride,
    const HidArgs &ha, const WoArgs &wa) {
    extern __shared__ float sh[];
    constexpr int TW = tf_tiles<T>(), NT = TW * TU, NTH = tf_threads<T>(), NW = NTH / 64;
    if ((int)blockIdx.x < ha.n_hid) {
        tile_hid_role<NW>(ha, rank, sh);
        return;
    }
    if constexpr (WO) {
        if ((int)blockIdx.x < wa.n_comb) {
            tile_comb_role<NW>(wa, ha, rank);
            return;
        }
        const int wb = (int)blockIdx.x - ((int)gridDim.x - wa.n_wo);  // Wo workgroups last
        if (wb >= 0) {
            if (wa.f.type == LLG_TYPE_Q4_0)
                tile_wo_role<LLG_TYPE_Q4_0, NW>(wa, wb, sh);
            else
                tile_wo_role<LLG_TYPE_Q8_0, NW>(wa, wb, sh);
            return;
        }
    }
    const int ti = blockIdx.x - ha.n_hid - (WO ? wa.n_comb : 0);  // this workgroup's tiles
    float *xs = sh;                                     // nb * XS_STRIDE
    float *hid = xs + f.nb * XS_STRIDE;                 // rank (16-byte aligned)
    float *ul = hid + ((rank + 3) & ~3);                // NT activations
    uint32_t *wm = reinterpret_cast<uint32_t *>(ul + NT);  // NW 16-row masks
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int *tl = reinterpret_cast<int *>(wm + NW) + wave * NT;  // this wavefront's active list
    const int n0 = ti * NT, n1 = min(ff, n0 + NT);
    WoutTile t;  // logits: wavefronts with neurons in the tile
    const bool lw = wave * 16 < n1 - n0;
    uint64_t hv0 = 0;
    uint32_t ctr = 0;
    if (ha.n_hid) {
        // WOut, x, then the epoch word and the hidden units' first poll
        if (lw) load_wout_tile(t, wout, wstride, n1, rank, n0);
        stage_x<stage_rounds(NTH)>(xs, x, f.nb, [&]() {
            ctr = llg_epoch_get(ha.ctr);
            if (wave * 64 < rank) hv0 = llg_slot_get(tile_slot_copy(ha) + min(wave * 64 + lane, rank - 1));
        });
    } else if (WO) {
        if (lw) load_wout_tile(t, wout, wstride, n1, rank, n0);  // used after the barrier
        stage_x<stage_rounds(NTH)>(xs, x, f.nb, [&]() { ctr = llg_epoch_get(ha.ctr); });
    } else {
        if (lw) load_wout_tile(t, wout, wstride, n1, rank, n0);  // used after the barrier
        stage_x<stage_rounds(NTH)>(xs, x, f.nb);
    }
    if (ha.n_hid)
        tile_take_hidden(hid, ha, rank, ctr + 1u, hv0);
    else if constexpr (WO)
        tile_take_comb(hid, wa, ha, rank, ctr + 1u);
    else
        load_hidden<PRED_SPLIT_N>(hid, partial, rank);
    __syncthreads();
    if (wave < NT / 16) {
        // the strict '>' of the logits of this wavefront's 16 rows (the four
        // lanes of a row agree), as a 16-bit mask
        bool on = false;
        if (lw) {
            float v = tile_logit(t, wout, wstride, n1, rank, n0, hid);
            const int i = n0 + wave * 16 + (lane >> 2);
            if (i < n1) {
                if (bias) v += bias[i];  // predictor.go:69-73
                on = v > thr;            // predictor.go:78
            }
        }
        const uint32_t m16 = quad_bits(__ballot(on));
        if (lane == 0) wm[wave] = m16;
    }
    __syncthreads();
    // every wavefront forms the tile masks and its own copy of the ascending
    // active list (no further barrier)
    unsigned long long mw[TW];
    int cnt = 0;
#pragma unroll
    for (int w = 0; w < TW; w++) {
        mw[w] = (unsigned long long)wm[4 * w] | ((unsigned long long)wm[4 * w + 1] << 16) |
                ((unsigned long long)wm[4 * w + 2] << 32) |
                ((unsigned long long)wm[4 * w + 3] << 48);
        const unsigned long long lt = (1ull << lane) - 1ull;
        if ((mw[w] >> lane) & 1ull) tl[cnt + __popcll(mw[w] & lt)] = TU * w + lane;
        cnt += __popcll(mw[w]);
        if (wave == 0 && lane == 0 && n0 + TU * w < n1) mask[ti * TW + w] = mw[w];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // The top n_dw wavefronts own the down quarter blocks: thread j of them
    // (j = tid - 64 n_uw) takes quarter blocks i = j, j + 64 n_dw, ... (block
    // i / 4, quarter i % 4).  Every wavefront takes up rows.
    constexpr int DK = tf_dk<T>();
    const int n_qb = 4 * f.nb;  // quarter blocks
    const int n_dw = min((n_qb + 63) / 64, NTH / 64);
    const int n_uw = NTH / 64 - n_dw;
    const int j = (int)threadIdx.x - 64 * n_uw;
    const int dstep = 64 * n_dw;
    const uint8_t *dbase = base + f.stride;  // down row of neuron n: dbase + n * bstride
    QuarterRaw<T> dr[DK];
    // lane q of a down wavefront holds active neuron k0 + q's workgroup-local
    // index (one LDS read per round; each row index is then a readlane); in
    // the first round the lanes past the count repeat the last active neuron
    int trow = cnt > 0 ? tl[min(lane, cnt - 1)] : 0;
    // the first quarter block's down bytes of the first DK active neurons,
    // requested right after this wavefront's up-row loads, so that they
    // arrive in the round of the up rows (address clamped for the lanes past
    // the last quarter block).  All DK slots are requested, a slot past the
    // active count rereading the last active neuron's lines (the tile's first
    // row if none is active): with a fixed number of loads behind the up row,
    // its dot waits for the up row alone, where a count-dependent number made
    // it wait for every down load.
    // Every wavefront passes one workgroup barrier (no memory wait) right
    // after requesting its first up row: a CU returns loads in request order,
    // so this puts every up row ahead of every down load.
    auto issue_down = [&]() {
        __builtin_amdgcn_s_barrier();
        const int ic = min(j, n_qb - 1);
#pragma unroll
        for (int k = 0; k < DK; k++) {
            const int n = n0 + __builtin_amdgcn_readlane(trow, k);
            quarter_load<T>(dr[k], dbase + (long long)n * bstride, f, ic >> 2, ic & 3);
        }
    };
    // up rows: every wavefront takes active neuron k = wave (+ 16 per further
    // round, which a workgroup needs for more than 16 active neurons).  The
    // down and the up-only wavefronts have separate copies of the first
    // round, each with its own fixed count of loads behind the up row.
    if (wave >= n_uw)
        tile_u_round<T, 1, true>(base, bstride, f, xs, tl, cnt, 0, n0, act, ul, NW, issue_down);
    else
        tile_u_round<T, 1, true>(base, bstride, f, xs, tl, cnt, 0, n0, act, ul, NW,
                                 [] { __builtin_amdgcn_s_barrier(); });
    for (int k0 = NW; k0 < cnt; k0 += NW)
        tile_u_round<T, 1, false>(base, bstride, f, xs, tl, cnt, k0, n0, act, ul, NW);
    __syncthreads();
    if (wave < n_uw) return;  // uniform per wavefront (no barrier follows)
    for (int i = j; i - j < n_qb; i += dstep) {  // uniform bound: every lane runs each pass
        const int ic = min(i, n_qb - 1);
        float acc[8];
        float corr = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] = 0.0f;
        for (int k0 = 0; k0 < cnt; k0 += DK) {
            // activations of this round's neurons, one LDS read (lane q: k0 + q)
            const float uq = k0 + lane < cnt ? ul[k0 + lane] : 0.0f;
            if (k0 > 0 || i != j) {  // later rounds (the first is in flight already)
                trow = k0 + lane < cnt ? tl[k0 + lane] : 0;
#pragma unroll
                for (int k = 0; k < DK; k++) {
                    if (k0 + k < cnt) {
                        const int n = n0 + __builtin_amdgcn_readlane(trow, k);
                        quarter_load<T>(dr[k], dbase + (long long)n * bstride, f, ic >> 2, ic & 3);
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < DK; k++) {
                if (k0 + k < cnt) {
                    const float u = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(uq), k));
                    if (u != 0.0f) quarter_axpy<T>(dr[k], u, acc, corr);
                }
            }
        }
        if (i < n_qb) {
            float4 *o4 = reinterpret_cast<float4 *>(part + (long long)ti * pstride + i * 8);
#pragma unroll
            for (int e = 0; e < 2; e++)
                o4[e] = make_float4(acc[4 * e] - corr, acc[4 * e + 1] - corr,
                                    acc[4 * e + 2] - corr, acc[4 * e + 3] - corr);
        }
    }
}

template <int T>
__global__ __launch_bounds__(tf_threads<T>(), tf_threads<T>() / 256) void k_tile_ffn(
    const uint8_t *__restrict__ wout, long long wstride, int ff, int rank,
    const float *__restrict__ partial, const float *__restrict__ bias, float thr,
    const uint8_t *__restrict__ base, long long bstride, RowFmt f, const float *__restrict__ x,
    int act, unsigned long long *__restrict__ mask, float *__restrict__ part, int pstride,
    HidArgs ha) {
    tile_ffn_body<T, false>(wout, wstride, ff, rank, partial, bias, thr, base, bstride, f, x, act,
                            mask, part, pstride, ha, WoArgs{});
}

// The same with Wo's workgroups (WoArgs) at the head of the grid.
template <int T>
__global__ __launch_bounds__(tf_threads<T>(), tf_threads<T>() / 256) void k_tile_wo_ffn(
    const uint8_t *__restrict__ wout, long long wstride, int ff, int rank,
    const float *__restrict__ bias, float thr, const uint8_t *__restrict__ base,
    long long bstride, RowFmt f, const float *__restrict__ x, int act,
    unsigned long long *__restrict__ mask, float *__restrict__ part, int pstride, HidArgs ha,
    WoArgs wa) {
    tile_ffn_body<T, true>(wout, wstride, ff, rank, nullptr, bias, thr, base, bstride, f, x, act,
                           mask, part, pstride, ha, wa);
}

// out[32 b + e] (+)= sum over the partial rows t < n_parts of part[t][32 b +
// e].  Workgroup b (256 threads): thread (g, c) sums the float4 column c of
// the block over rows g, g + 32, g + 64, ... in that order (all loads of a
// batch issued together), then the 32 group sums are added pairwise in a
// fixed tree, so the order is the same on every run.  With ACC the sum is
// added to out (a residual), else stored.  Workgroup 0 also writes the number
// of active neurons (the popcounts of the tile masks).  stats (optional, cols
// a multiple of 32): the block's (sum, M2) of the values written, for the
// LayerNorm prologue of the next matvec over out (LlgLnArgs).  ctr
// (optional): the epoch word of the tile launch's sync area, advanced here.
#define TR_GROUPS 32  // the tree below is written for 32 groups
#define TR_BATCH 5
template <bool ACC>
__global__ __launch_bounds__(256) void k_tile_reduce(const float *__restrict__ part, int pstride,
                                                     int n_parts, int n_tiles, int cols,
                                                     const unsigned long long *__restrict__ mask,
                                                     int32_t *__restrict__ n_active_out,
                                                     float *__restrict__ out,
                                                     float2 *__restrict__ stats,
                                                     uint32_t *__restrict__ ctr) {
    __shared__ float4 red[TR_GROUPS][8];
    __shared__ int cnt[4];
    const int b = blockIdx.x, tid = threadIdx.x;
    const int c = tid & 7, g = tid >> 3;
    const int o = b * 32 + 4 * c;
    const float4 *p = reinterpret_cast<const float4 *>(part + b * 32) + c;
    const int ps4 = pstride / 4;
    // v with every bit cleared unless keep (an exact 0 or v, by an AND the
    // compiler cannot turn into a branch, so no load is sunk into one)
    auto keep4 = [](float4 v, bool keep) {
        const uint32_t m = keep ? 0xFFFFFFFFu : 0u;
        uint32_t r[4];
        const uint32_t x[4] = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z),
                               __float_as_uint(v.w)};
#pragma unroll
        for (int k = 0; k < 4; k++) asm("v_and_b32 %0, %1, %2" : "=v"(r[k]) : "v"(x[k]), "v"(m));
        return make_float4(__uint_as_float(r[0]), __uint_as_float(r[1]), __uint_as_float(r[2]),
                           __uint_as_float(r[3]));
    };
    // The first batch of partial rows, straight-line and first: a loop head
    // would wait for every earlier load, and loads requested before these
    // would return ahead of them.
    float4 v[TR_BATCH];
#pragma unroll
    for (int i = 0; i < TR_BATCH; i++)
        v[i] = p[(long long)min(g + TR_GROUPS * i, n_parts - 1) * ps4];
    // the epoch word, read unconditionally (a word of the first partial row
    // without one) so that no branch waits for it, and advanced at the end
    const uint32_t c0 = llg_epoch_get(ctr ? ctr : reinterpret_cast<const uint32_t *>(part));
    // the tile masks (block 0 counts the active neurons from them), also
    // requested now rather than after the sums
    unsigned long long mk[2];
#pragma unroll
    for (int k = 0; k < 2; k++) mk[k] = mask[min(tid + 256 * k, n_tiles - 1)];
    // the residual (stored by group 0), behind the partial rows; requested by
    // every wavefront, so that each has the same count of loads to wait on
    __builtin_amdgcn_sched_barrier(0);
    float4 prev = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (ACC)
        prev = make_float4(out[min(o + 0, cols - 1)], out[min(o + 1, cols - 1)],
                           out[min(o + 2, cols - 1)], out[min(o + 3, cols - 1)]);
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < TR_BATCH; i++) {  // rows in the order g, g + 32, ...
        const float4 a = keep4(v[i], g + TR_GROUPS * i < n_parts);
        s.x += a.x;
        s.y += a.y;
        s.z += a.z;
        s.w += a.w;
    }
    for (int t0 = g + TR_GROUPS * TR_BATCH; t0 < n_parts; t0 += TR_GROUPS * TR_BATCH) {
#pragma unroll
        for (int i = 0; i < TR_BATCH; i++)
            v[i] = p[(long long)min(t0 + TR_GROUPS * i, n_parts - 1) * ps4];
#pragma unroll
        for (int i = 0; i < TR_BATCH; i++) {
            const float4 a = keep4(v[i], t0 + TR_GROUPS * i < n_parts);
            s.x += a.x;
            s.y += a.y;
            s.z += a.z;
            s.w += a.w;
        }
    }
    int na = 0;
    if (n_active_out && b == 0) {
#pragma unroll
        for (int k = 0; k < 2; k++)
            if (tid + 256 * k < n_tiles) na += __popcll(mk[k]);
        for (int i = tid + 512; i < n_tiles; i += 256) na += __popcll(mask[i]);
    }
    red[g][c] = s;
    if (n_active_out && b == 0) {
        for (int d = 32; d > 0; d >>= 1) na += __shfl_xor(na, d, 64);
        if ((tid & 63) == 0) cnt[tid >> 6] = na;
    }
    __syncthreads();
    // The group sums pairwise in a fixed tree (the same order on every run):
    // level h adds group g + h into g for g < h, h = 16, 8, 4, 2, 1.  Wavefront
    // 0 (groups 0-7) forms levels 16 and 8 from LDS and the rest by shuffles
    // (group g + h sits 8 h lanes up), so one barrier serves the whole tree.
    float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
    if (tid < 64) {
        auto add = [](float4 a, float4 v) {
            return make_float4(a.x + v.x, a.y + v.y, a.z + v.z, a.w + v.w);
        };
        float4 t = add(add(red[g][c], red[g + 16][c]), add(red[g + 8][c], red[g + 24][c]));
#pragma unroll
        for (int h = 4; h > 0; h >>= 1) {
            const float4 v = make_float4(__shfl_down(t.x, 8 * h, 64), __shfl_down(t.y, 8 * h, 64),
                                         __shfl_down(t.z, 8 * h, 64), __shfl_down(t.w, 8 * h, 64));
            t = add(t, v);
        }
        sum = t;  // the tree's result in lanes 0-7 (group 0)
    }
    const float4 val =
        ACC ? make_float4(prev.x + sum.x, prev.y + sum.y, prev.z + sum.z, prev.w + sum.w) : sum;
    if (g == 0) {
        if (o + 0 < cols) out[o + 0] = val.x;
        if (o + 1 < cols) out[o + 1] = val.y;
        if (o + 2 < cols) out[o + 2] = val.z;
        if (o + 3 < cols) out[o + 3] = val.w;
        if (stats) {  // lanes 0-7 of wavefront 0 hold the block
            const float2 bs = llg_block32_stats(val);
            if (c == 0) stats[b] = bs;
        }
    }
    if (n_active_out && b == 0 && tid == 0) *n_active_out = cnt[0] + cnt[1] + cnt[2] + cnt[3];
    if (ctr && b == 0 && tid == 0) *ctr = c0 + 1u;  // the next launch's epoch
}

// Most pairs a k_sparse_down thread loads at once, by type (the row bytes of
// all of them are in flight together).
template <int T>
constexpr int dn_np() {
    return T == LLG_TYPE_F32 ? 2 : (T == LLG_TYPE_F16 ? 4 : (T == LLG_TYPE_Q8_0 ? 8 : 16));
}

// acc[32] += u * dequant(block b of the down row) for the first nvalid of the
// NP entries e[] = (row, u bits) (a pair with u == 0 is skipped,
// ffn_flash.go:290).  Every load is issued before any is used; skipped
// entries read row 0 (in bounds), so no load sits under a per-lane condition.
template <int T, int NP>
__device__ __forceinline__ void dn_batch(const uint8_t *__restrict__ base, long long bstride,
                                         const RowFmt &f, int b, const int2 (&e)[NP], int nvalid,
                                         float (&acc)[32], float &corr) {
    BlockRaw<T> r[NP];
    float u[NP];
#pragma unroll
    for (int k = 0; k < NP; k++) {
        u[k] = __int_as_float(e[k].y);
        const bool v = k < nvalid && u[k] != 0.0f;
        llg_block_load<T>(r[k], base + (long long)(v ? e[k].x : 0) * bstride + f.stride, f, b);
    }
#pragma unroll
    for (int k = 0; k < NP; k++)
        if (k < nvalid && u[k] != 0.0f) llg_raw_axpy<T>(r[k], u[k], acc, corr);
}

// Entries j = tid + bd * (i0 + i), i < K, of a dense list of n (get(j) reads
// entry j) shared by bd threads, through dn_batch.
template <int T, int K, class Get>
__device__ __forceinline__ void dn_run(const uint8_t *__restrict__ base, long long bstride,
                                       const RowFmt &f, int b, int n, int i0, Get &&get,
                                       float (&acc)[32], float &corr, int tid, int bd) {
    int2 e[K];
#pragma unroll
    for (int i = 0; i < K; i++) e[i] = get(min(tid + bd * (i0 + i), n - 1));
    const int mine = (n - tid + bd - 1) / bd;  // entries of this thread in the list
    dn_batch<T, K>(base, bstride, f, b, e, min(max(mine - i0, 0), K), acc, corr);
}

// Every entry of a dense list of n shared by bd threads (this one is tid),
// ceil(n / bd) per thread: the batch size follows that count (uniform over
// the wavefront), so a thread issues no loads for entries it does not have.
template <int T, class Get>
__device__ __forceinline__ void dn_list(const uint8_t *__restrict__ base, long long bstride,
                                        const RowFmt &f, int b, int n, Get &&get,
                                        float (&acc)[32], float &corr, int tid, int bd) {
    constexpr int KM = dn_np<T>();
    const int per = (n + bd - 1) / bd;
    for (int i0 = 0; i0 < per; i0 += KM) {
        const int k = min(per - i0, KM);
        if (k == 1)
            dn_run<T, 1>(base, bstride, f, b, n, i0, get, acc, corr, tid, bd);
        else if (k == 2)
            dn_run<T, 2>(base, bstride, f, b, n, i0, get, acc, corr, tid, bd);
        else if (k <= 4)
            dn_run<T, (KM < 4 ? KM : 4)>(base, bstride, f, b, n, i0, get, acc, corr, tid, bd);
        else if (k <= 8)
            dn_run<T, (KM < 8 ? KM : 8)>(base, bstride, f, b, n, i0, get, acc, corr, tid, bd);
        else
            dn_run<T, KM>(base, bstride, f, b, n, i0, get, acc, corr, tid, bd);
    }
}

// Down products over a plain pair list pairs[0..*count) (the count is
// clamped to `cap`), split evenly over the threads.  Workgroup = output block
// b (32 outputs): out[32 b + e] = sum over the pairs of u * down_row[32 b +
// e], the wavefronts' sums added in order.
template <int T>
__global__ __launch_bounds__(DN_THREADS) void k_sparse_down(
    const uint8_t *__restrict__ base, long long bstride, RowFmt f, const int2 *__restrict__ pairs,
    const int32_t *__restrict__ count_p, int cap, int per_xcd, float *__restrict__ out) {
    __shared__ float red[DN_THREADS / 64][32];
    const int b = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (b >= f.nb) return;  // uniform over the workgroup
    const int tid = threadIdx.x, bd = blockDim.x, lane = tid & 63, wave = tid >> 6;
    const int nw = bd >> 6;
    const int o = b * 32 + (lane >> 1);
    float acc[32];
    float corr = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; e++) acc[e] = 0.0f;
    const int n = min(max(*count_p, 0), cap);
    dn_list<T>(base, bstride, f, b, n, [&](int j) { return pairs[j]; }, acc, corr, tid, bd);
#pragma unroll
    for (int e = 0; e < 32; e++) acc[e] -= corr;
    const float ws = dn_wave_transpose_sum(acc);
    if ((lane & 1) == 0) red[wave][lane >> 1] = ws;
    __syncthreads();
    if (wave == 0 && (lane & 1) == 0) {
        float sum = 0.0f;
        for (int w = 0; w < nw; w++) sum += red[w][lane >> 1];
        if (o < f.cols) out[o] = sum;
    }
}

// ---------------------------------------------------------------------------
// C. The window's update + FFN step in one launch (window.go:71-180).
// Workgroups of ws_threads<T>() threads:
//   [0, n_up)            up rows: wavefront-pair entries (j, j + S), S = the
//                        up wavefronts.  A neuron not resident at the start of
//                        the update (win_resident) is read from the layer's
//                        bundle (u.src) while its whole bundle is copied into
//                        its row of the resident buffer (loadRows,
//                        window.go:207-245), a resident one from its row; the
//                        activation of entry j goes to u.uslot[j], tagged with
//                        the update's number;
//   [n_up, n_up + n_dn)  one output block each: every thread requests block b
//                        of the down rows of its entries (from the source of
//                        the entry's up row) and then waits for their slots;
//                        the sums of k_sparse_down;
//   the last WS_UPD ones the update of the counts and the residency, split
//                        over them (win_update_part), from the state at the
//                        start.
// The up workgroups wait for nothing and come first in the grid, so every
// wait of a down workgroup ends.  A slot still stale after WS_POLLS polls is
// computed by the down workgroup itself with the up workgroups' sums (x staged
// the same way), so the result does not depend on which one computed it.
#define WS_POLLS (1 << 16)
#define WS_UP_MAX 64   // up workgroups (two entries per wavefront and round)
#define WS_UPD 16      // update workgroups

// Threads of a k_win_step workgroup: 512, or 256 for F32 rows (whose up-row
// dots need the registers of two wavefronts per SIMD).
template <int T>
constexpr int ws_threads() {
    return T == LLG_TYPE_F32 ? 256 : 512;
}

// The up row's source of neuron n (< 0: none) in update e: the layer's bundle
// when n was not resident at the start, else its resident row.
__device__ __forceinline__ bool ws_from_src(const LlgWinUpd &u, int n) {
    return n >= 0 && !win_resident(u.res, n, u.epoch);
}

// One batch of K entries j = tid + bd * (i0 + k) of the down role (nvalid of
// them are below the count): block b of each down row requested from the
// entry's source, then the activation slots polled.  missing: entries whose
// slot stayed stale (their activation is then computed by ws_fill_missing).
template <int T, int K>
__device__ __forceinline__ void ws_down_batch(const LlgWinUpd &u, long long bstride,
                                              const RowFmt &f, int b, const int32_t *active,
                                              int n_rows, int n, int i0, int tid, int bd,
                                              float (&acc)[32], float &corr, float *xs, int act,
                                              const float *x) {
    BlockRaw<T> r[K];
    int nn[K];
    bool fs[K];
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int j = min(tid + bd * (i0 + k), n - 1);
        const int a = active[j];
        nn[k] = a >= 0 && a < n_rows ? a : -1;
    }
#pragma unroll
    for (int k = 0; k < K; k++) fs[k] = ws_from_src(u, nn[k]);
#pragma unroll
    for (int k = 0; k < K; k++) {
        const uint8_t *row = (fs[k] ? u.src : u.dst) + (long long)(nn[k] >= 0 ? nn[k] : 0) * bstride;
        llg_block_load<T>(r[k], row + f.stride, f, b);
    }
    const int mine = (n - tid + bd - 1) / bd;  // entries of this thread in the list
    const int nvalid = min(max(mine - i0, 0), K);
    uint64_t v[K];
#pragma unroll
    for (int k = 0; k < K; k++) v[k] = llg_slot_get(u.uslot + min(tid + bd * (i0 + k), n - 1));
    auto ready = [&]() {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < K; k++)
            ok = ok && (k >= nvalid || nn[k] < 0 || (uint32_t)(v[k] >> 32) == (uint32_t)u.epoch);
        return ok;
    };
    // every slot polled again together (a slot already seen holds the same
    // word), so that each poll is one memory round
    for (int polls = 0; !__all(ready()) && polls < WS_POLLS; polls++) {
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int k = 0; k < K; k++) v[k] = llg_slot_get(u.uslot + min(tid + bd * (i0 + k), n - 1));
    }
    // A slot still stale (never seen in a working launch): in rounds, every
    // thread with a stale entry lists one of them, the wavefronts compute the
    // listed up rows with the up workgroups' sums (x staged the same way) and
    // write their slots, and the threads read their slots again.  With
    // u.check every valid entry counts as stale until it has been computed
    // here once (after the wait, so that value is the last one written to
    // its slot).
    if (__syncthreads_or(!ready() || u.check)) {
        __shared__ int ws_n;
        __shared__ int3 ws_list[ws_threads<T>()];
        const int lane = threadIdx.x & 63;
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        bool redo[K];
#pragma unroll
        for (int k = 0; k < K; k++) redo[k] = u.check;
        auto stale = [&](int k) {
            return k < nvalid && nn[k] >= 0 &&
                   (redo[k] || (uint32_t)(v[k] >> 32) != (uint32_t)u.epoch);
        };
        stage_x<stage_rounds(ws_threads<T>())>(xs, x, f.nb);
        for (;;) {  // uniform: ends when no thread has a stale entry
            if (threadIdx.x == 0) ws_n = 0;
            __syncthreads();
            int3 mine = make_int3(-1, 0, 0);
            int mk = -1;
#pragma unroll
            for (int k = K - 1; k >= 0; k--)
                if (stale(k)) {
                    mine = make_int3(tid + bd * (i0 + k), nn[k], fs[k] ? 1 : 0);
                    mk = k;
                }
            if (mine.x >= 0) ws_list[atomicAdd(&ws_n, 1)] = mine;
            __syncthreads();
            const int cnt = ws_n;
            if (cnt == 0) break;
            for (int i = wave; i < cnt; i += ws_threads<T>() / 64) {
                const int3 e = ws_list[i];
                const uint8_t *p = (e.z ? u.src : u.dst) + (long long)e.y * bstride;
                float s0, s1;
                row_dot2p<T>(p, p, true, false, f, xs, s0, s1);
                if (lane == 0) llg_slot_put(u.uslot + e.x, u.epoch, llg_act(act, s0));
            }
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
#pragma unroll
            for (int k = 0; k < K; k++) {
                if (stale(k)) v[k] = llg_slot_get(u.uslot + tid + bd * (i0 + k));
                if (k == mk) redo[k] = false;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < K; k++) {
        const float uk = __uint_as_float((uint32_t)v[k]);
        if (k < nvalid && nn[k] >= 0 && uk != 0.0f) llg_raw_axpy<T>(r[k], uk, acc, corr);
    }
}

template <int T>
__global__ __launch_bounds__(ws_threads<T>()) void k_win_step(
    RowFmt f, long long bstride, const float *__restrict__ x, const int32_t *__restrict__ active,
    const int32_t *__restrict__ n_active_p, int cap, int n_rows, int act, int n_up, int per_xcd,
    float *__restrict__ out, LlgWinUpd u) {
    constexpr int NTH = ws_threads<T>(), NW = NTH / 64;
    extern __shared__ float xs[];
    __shared__ float red[NW][32];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n_dn = 8 * per_xcd;
    if ((int)blockIdx.x >= n_up + n_dn) {  // the update (the bitmap in the x staging's LDS)
        win_update_part(u, active, min(max(*n_active_p, 0), cap), n_rows,
                        (int)blockIdx.x - n_up - n_dn, WS_UPD, reinterpret_cast<uint32_t *>(xs));
        return;
    }
    auto valid = [&](int n) { return n >= 0 && n < n_rows ? n : -1; };
    if ((int)blockIdx.x < n_up) {
        const int S = n_up * NW;  // up wavefronts
        const int jf = blockIdx.x * NW + wave;
        const int n_act = min(max(*n_active_p, 0), cap);
        if ((int)blockIdx.x * NW >= n_act) return;  // whole workgroup idle
        const int n16 = (int)(bstride >> 4);
        constexpr int NC = bc_first<T>();
        auto pair = [&](int j, int m0, int m1, bool f0, bool f1) {
            const int j1 = j + S;
            const int row0 = __builtin_amdgcn_readfirstlane(m0);
            const int row1 = __builtin_amdgcn_readfirstlane(m1);
            const uint8_t *p0 = (f0 ? u.src : u.dst) + (long long)(row0 >= 0 ? row0 : 0) * bstride;
            const uint8_t *p1 = (f1 ? u.src : u.dst) + (long long)(row1 >= 0 ? row1 : 0) * bstride;
            const bc_u4 *sp0 = reinterpret_cast<const bc_u4 *>(p0);
            const bc_u4 *sp1 = reinterpret_cast<const bc_u4 *>(p1);
            bc_u4 *dp0 = reinterpret_cast<bc_u4 *>(u.dst + (long long)(f0 ? row0 : 0) * bstride);
            bc_u4 *dp1 = reinterpret_cast<bc_u4 *>(u.dst + (long long)(f1 ? row1 : 0) * bstride);
            BundleCopy<NC> c0, c1;
            if (f0) bc_issue(c0, sp0, n16);
            if (f1) bc_issue(c1, sp1, n16);
            float s0, s1;
            // the copies are stored once the dot's loads are in flight
            row_dot2p<T>(p0, p1, row0 >= 0, row1 >= 0, f, xs, s0, s1, [&]() {
                if (f0) bc_store(c0, dp0, n16);
                if (f1) bc_store(c1, dp1, n16);
            });
            if (f0) bc_rest<NC>(sp0, dp0, n16);
            if (f1) bc_rest<NC>(sp1, dp1, n16);
            if (lane == 0) {  // an entry without a neuron has activation 0
                llg_slot_put(u.uslot + j, u.epoch, row0 >= 0 ? llg_act(act, s0) : 0.0f);
                if (j1 < n_act)
                    llg_slot_put(u.uslot + j1, u.epoch, row1 >= 0 ? llg_act(act, s1) : 0.0f);
            }
        };
        // the first pair's entries (never past the count: the list holds
        // n_act entries) are requested while x is in flight
        const bool has0 = jf < n_act;
        int a0 = -1, a1 = -1;
        stage_x<stage_rounds(NTH)>(xs, x, f.nb, [&]() {
            a0 = active[min(jf, n_act - 1)];
            a1 = active[min(jf + S, n_act - 1)];
        });
        const int m0 = has0 ? valid(a0) : -1;
        const int m1 = jf + S < n_act ? valid(a1) : -1;
        const bool f0 = __builtin_amdgcn_readfirstlane((int)ws_from_src(u, m0));
        const bool f1 = __builtin_amdgcn_readfirstlane((int)ws_from_src(u, m1));
        __syncthreads();
        if (has0) pair(jf, m0, m1, f0, f1);
        for (int j = jf + 2 * S; j < n_act; j += 2 * S) {
            const int j1 = j + S;
            const int n0 = valid(active[j]);
            const int n1 = j1 < n_act ? valid(active[j1]) : -1;
            pair(j, n0, n1, __builtin_amdgcn_readfirstlane((int)ws_from_src(u, n0)),
                 __builtin_amdgcn_readfirstlane((int)ws_from_src(u, n1)));
        }
        return;
    }
    // the down role: output block b
    const int bi = (int)blockIdx.x - n_up;
    const int b = (bi & 7) * per_xcd + (bi >> 3);
    if (b >= f.nb) return;  // uniform over the workgroup
    const int tid = threadIdx.x, bd = blockDim.x;
    const int o = b * 32 + (lane >> 1);
    float acc[32];
    float corr = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; e++) acc[e] = 0.0f;
    const int n = min(max(*n_active_p, 0), cap);
    // entries per batch: the config's 909 entries are 2 per thread; a longer
    // list takes more batches
    constexpr int KM = T == LLG_TYPE_F32 ? 1 : (T == LLG_TYPE_F16 ? 2 : 4);
    const int per = (n + bd - 1) / bd;
    for (int i0 = 0; i0 < per; i0 += KM)  // uniform over the workgroup
        ws_down_batch<T, KM>(u, bstride, f, b, active, n_rows, n, i0, tid, bd, acc, corr, xs, act,
                             x);
#pragma unroll
    for (int e = 0; e < 32; e++) acc[e] -= corr;
    const float ws = dn_wave_transpose_sum(acc);
    if ((lane & 1) == 0) red[wave][lane >> 1] = ws;
    __syncthreads();
    if (wave == 0 && (lane & 1) == 0) {
        float sum = 0.0f;
        for (int w = 0; w < NW; w++) sum += red[w][lane >> 1];
        if (o < f.cols) out[o] = sum;
    }
}

// ---------------------------------------------------------------------------
// Host-side enqueue helpers
// ---------------------------------------------------------------------------
size_t llg_sparse_ws_bytes(int max_active) {
    return (size_t)llg_align((long long)(max_active > 0 ? max_active : 1) * 8, 256) + 256;
}

static size_t xs_bytes(const RowFmt &f) { return (size_t)f.nb * XS_STRIDE * 4; }

// k_sparse_down's grid: 8 * ceil(nb / 8) workgroups (one per output block,
// the block order spread evenly over the 8 XCDs); a list launch uses one
// thread per entry, 64 to DN_THREADS, a tiled launch DN_THREADS.
static int down_per_xcd(const RowFmt &f) { return (f.nb + 7) / 8; }
static int down_threads(int items) {
    const int t = (items + 63) / 64 * 64;
    return t < 64 ? 64 : (t > DN_THREADS ? DN_THREADS : t);
}

template <int T>
static void launch_list(hipStream_t st, const uint8_t *base, long long bstride, const RowFmt &f,
                        const int32_t *res, const float *x, const int32_t *active,
                        const int32_t *n_active, int max_active, int n_rows, int act,
                        float *out, int2 *pairs) {
    int grid = (max_active + 3) / 4;
    if (grid < 1) grid = 1;
    if (grid > 512) grid = 512;
    hipLaunchKernelGGL((k_list_up<T>), dim3(grid), dim3(256), xs_bytes(f), st, base, bstride, f,
                       res, x, active, n_active, max_active, n_rows, act, pairs);
    const int px = down_per_xcd(f);
    hipLaunchKernelGGL((k_sparse_down<T>), dim3(8 * px), dim3(down_threads(max_active)), 0, st,
                       base, bstride, f, (const int2 *)pairs, n_active, max_active, px, out);
}

int llg_sparse_enqueue(LlgDevice *d, const uint8_t *base, long long bstride, const RowFmt &f,
                       const int32_t *res, const float *d_x, const int32_t *d_active,
                       const int32_t *d_n_active, int max_active, int n_rows, int act,
                       float *d_out, uint8_t *ws) {
    if (int rc = llg_check_act(d, act)) return rc;
    if (xs_bytes(f) > 64 * 1024)
        return llg_set_error(d, LLG_E_ARG, "sparse ffn: hidden size %d too large", f.cols);
    hipStream_t st = llg_dev_stream(d);
    int2 *pairs = reinterpret_cast<int2 *>(ws);
    switch (f.type) {
    case LLG_TYPE_Q4_0:
        launch_list<LLG_TYPE_Q4_0>(st, base, bstride, f, res, d_x, d_active, d_n_active,
                                   max_active, n_rows, act, d_out, pairs);
        break;
    case LLG_TYPE_Q8_0:
        launch_list<LLG_TYPE_Q8_0>(st, base, bstride, f, res, d_x, d_active, d_n_active,
                                   max_active, n_rows, act, d_out, pairs);
        break;
    case LLG_TYPE_F16:
        launch_list<LLG_TYPE_F16>(st, base, bstride, f, res, d_x, d_active, d_n_active,
                                  max_active, n_rows, act, d_out, pairs);
        break;
    case LLG_TYPE_F32:
        launch_list<LLG_TYPE_F32>(st, base, bstride, f, res, d_x, d_active, d_n_active,
                                  max_active, n_rows, act, d_out, pairs);
        break;
    default:
        return llg_set_error(d, LLG_E_TYPE, "sparse ffn: unsupported type %d", f.type);
    }
    LLG_LAUNCH_CHECK(d, "sparse ffn");
    return 0;
}

template <int T>
static void launch_win_step(hipStream_t st, const LlgWinUpd &u, const RowFmt &f,
                            long long bstride, const float *x, const int32_t *active,
                            const int32_t *n_active, int cap, int n_rows, int act, float *out) {
    constexpr int PER_WG = 2 * (ws_threads<T>() / 64);  // entries of an up workgroup per round
    int n_up = (cap + PER_WG - 1) / PER_WG;
    n_up = n_up < 1 ? 1 : (n_up > WS_UP_MAX ? WS_UP_MAX : n_up);
    const int px = down_per_xcd(f);
    // LDS: the staged x, or an update workgroup's bitmap of the listed set
    const size_t lds = std::max(xs_bytes(f), (size_t)win_bitmap_words(n_rows) * 4);
    hipLaunchKernelGGL((k_win_step<T>), dim3(n_up + 8 * px + WS_UPD), dim3(ws_threads<T>()), lds,
                       st, f, bstride, x, active, n_active, cap, n_rows, act, n_up, px, out, u);
}

int llg_win_step_enqueue(LlgDevice *d, const LlgWinUpd &u, const RowFmt &f, long long bstride,
                         const float *d_x, const int32_t *d_active, const int32_t *d_n_active,
                         int cap, int n_rows, int act, float *d_out) {
    if (int rc = llg_check_act(d, act)) return rc;
    if (!u.src || !u.dst || !u.uslot || (bstride & 15) || cap < 1)
        return llg_set_error(d, LLG_E_ARG, "window step: bad window state");
    if (xs_bytes(f) > 64 * 1024)
        return llg_set_error(d, LLG_E_ARG, "window step: hidden size %d too large", f.cols);
    if ((size_t)win_bitmap_words(n_rows) * 4 > 48 * 1024)
        return llg_set_error(d, LLG_E_ARG, "window step: %d neurons too many", n_rows);
    hipStream_t st = llg_dev_stream(d);
    switch (f.type) {
    case LLG_TYPE_Q4_0:
        launch_win_step<LLG_TYPE_Q4_0>(st, u, f, bstride, d_x, d_active, d_n_active, cap, n_rows,
                                       act, d_out);
        break;
    case LLG_TYPE_Q8_0:
        launch_win_step<LLG_TYPE_Q8_0>(st, u, f, bstride, d_x, d_active, d_n_active, cap, n_rows,
                                       act, d_out);
        break;
    case LLG_TYPE_F16:
        launch_win_step<LLG_TYPE_F16>(st, u, f, bstride, d_x, d_active, d_n_active, cap, n_rows,
                                      act, d_out);
        break;
    case LLG_TYPE_F32:
        launch_win_step<LLG_TYPE_F32>(st, u, f, bstride, d_x, d_active, d_n_active, cap, n_rows,
                                      act, d_out);
        break;
    default:
        return llg_set_error(d, LLG_E_TYPE, "window step: unsupported type %d", f.type);
    }
    LLG_LAUNCH_CHECK(d, "window step");
    return 0;
}

// Workspace of the fused path: the predictor's partials and masks, then the
// tiles' partial outputs (one row of nb * 32 floats per tile).
size_t llg_fused_ws_bytes(int rank, int ff, int nb) {
    const long long n_tiles = (ff + 63) / 64;  // an upper bound on the partial rows
    return (size_t)llg_predict_ws_bytes(rank, ff) + (size_t)llg_align(n_tiles * nb * 32 * 4, 256);
}

// LDS of k_tile_ffn: staged x, hidden, activations, the logit masks and a
// per-wavefront active list.
template <int T>
static size_t tile_lds_bytes(const RowFmt &f, int rank) {
    constexpr int NT = tf_tiles<T>() * TU, NW = tf_threads<T>() / 64;
    return xs_bytes(f) + (size_t)(((rank + 3) & ~3) + NT + NW + NW * NT) * 4;
}

template <int T>
static void launch_fused(hipStream_t st, LlgObject *wout, const float *partial,
                         const float *bias, float thr, LlgObject *b, const float *x, int act,
                         unsigned long long *mask, float *part, int32_t *n_active, float *out,
                         bool accumulate, float2 *stats, HidArgs ha, WoArgs wa) {
    const int ff = wout->rows, rank = wout->fmt.cols;
    const int n_tiles = (ff + 63) / 64;
    const RowFmt &f = b->fmt;
    const int pstride = f.nb * 32;
    constexpr int NT = tf_tiles<T>() * TU, NW = tf_threads<T>() / 64;
    const int n_parts = (ff + NT - 1) / NT;  // tile workgroups, one partial row each
    if (ha.slots && ha.wup) ha.n_hid = (rank + NW / LLG_PRED_SPLIT - 1) / (NW / LLG_PRED_SPLIT);
    size_t lds = tile_lds_bytes<T>(f, rank);
    if (wa.w) {
        wa.n_comb = (rank + NW - 1) / NW;
        wa.n_wo = (wa.rows + wo_rows_per_wg<NW>() - 1) / wo_rows_per_wg<NW>();
        lds = std::max(lds, (size_t)wa.f.nb * XS_STRIDE * 4);
    }
    if (wa.w)
        hipLaunchKernelGGL((k_tile_wo_ffn<T>), dim3(wa.n_comb + n_parts + wa.n_wo), dim3(tf_threads<T>()), lds,
                           st, wout->d, wout->stride, ff, rank, bias, thr, b->d, b->stride, f, x,
                           act, mask, part, pstride, ha, wa);
    else
        hipLaunchKernelGGL((k_tile_ffn<T>), dim3(ha.n_hid + n_parts), dim3(tf_threads<T>()), lds,
                           st, wout->d, wout->stride, ff, rank, partial, bias, thr, b->d,
                           b->stride, f, x, act, mask, part, pstride, ha);
    uint32_t *ctr = ha.slots ? const_cast<uint32_t *>(ha.ctr) : nullptr;
    if (accumulate)
        hipLaunchKernelGGL((k_tile_reduce<true>), dim3(f.nb), dim3(256), 0, st,
                           (const float *)part, pstride, n_parts, n_tiles, f.cols,
                           (const unsigned long long *)mask, n_active, out, stats, ctr);
    else
        hipLaunchKernelGGL((k_tile_reduce<false>), dim3(f.nb), dim3(256), 0, st,
                           (const float *)part, pstride, n_parts, n_tiles, f.cols,
                           (const unsigned long long *)mask, n_active, out, stats, ctr);
}

static int fused_tail(LlgDevice *d, LlgObject *wout, LlgObject *bias, LlgObject *b,
                      const float *d_x, float thr, int act, float *d_out, int32_t *d_active,
                      int32_t *d_n_active, uint8_t *ws, bool accum, float2 *d_stats,
                      const HidArgs &ha, const WoArgs &wa = WoArgs{}) {
    if (int rc = llg_check_act(d, act)) return rc;
    const RowFmt &f = b->fmt;
    if (d_stats && f.cols % 32)
        return llg_set_error(d, LLG_E_ARG, "predict_sparse: block statistics need 32 | %d", f.cols);
    const int ff = wout->rows, rank = wout->fmt.cols;
    const int n_tiles = (ff + 63) / 64;
    const size_t lds = f.type == LLG_TYPE_Q4_0 ? tile_lds_bytes<LLG_TYPE_Q4_0>(f, rank)
                                               : tile_lds_bytes<LLG_TYPE_F32>(f, rank);
    if (lds > 64 * 1024)
        return llg_set_error(d, LLG_E_ARG, "predict_sparse: hidden size %d too large", f.cols);
    if (llg_pred_split() != PRED_SPLIT_N)
        return llg_set_error(d, LLG_E_ARG, "predict_sparse: hidden split %d != %d",
                             llg_pred_split(), PRED_SPLIT_N);
    float *part = reinterpret_cast<float *>(ws + llg_predict_ws_bytes(rank, ff));
    float *partial;
    unsigned long long *mask;
    llg_pred_ws_layout(ws, rank, &partial, &mask);
    const float *d_bias = bias ? reinterpret_cast<const float *>(bias->d) : nullptr;
    hipStream_t st = llg_dev_stream(d);
    switch (f.type) {
    case LLG_TYPE_Q4_0:
        launch_fused<LLG_TYPE_Q4_0>(st, wout, partial, d_bias, thr, b, d_x, act, mask, part,
                                    d_n_active, d_out, accum, d_stats, ha, wa);
        break;
    case LLG_TYPE_Q8_0:
        launch_fused<LLG_TYPE_Q8_0>(st, wout, partial, d_bias, thr, b, d_x, act, mask, part,
                                    d_n_active, d_out, accum, d_stats, ha, wa);
        break;
    case LLG_TYPE_F16:
        launch_fused<LLG_TYPE_F16>(st, wout, partial, d_bias, thr, b, d_x, act, mask, part,
                                   d_n_active, d_out, accum, d_stats, ha, wa);
        break;
    case LLG_TYPE_F32:
        launch_fused<LLG_TYPE_F32>(st, wout, partial, d_bias, thr, b, d_x, act, mask, part,
                                   d_n_active, d_out, accum, d_stats, ha, wa);
        break;
    default:
        return llg_set_error(d, LLG_E_TYPE, "predict_sparse: unsupported type %d", f.type);
    }
    LLG_LAUNCH_CHECK(d, "predict_sparse");
    if (d_active) return llg_compact_enqueue(d, mask, n_tiles, d_active, nullptr);
    return 0;
}

// ffnFlash path 2 on the device.  With a sync area (sync, LLG_SYNC_BYTES)
// and rank <= LLG_SYNC_SLOTS: the tile launch computes the predictor's hidden
// units in its first workgroups, then k_tile_reduce; otherwise k_pred_hidden
// first.  Plus the ascending active list through k_compact when d_active is
// given; d_n_active (optional) receives the number of active neurons.
int llg_fused_enqueue(LlgDevice *d, LlgObject *wup, LlgObject *wout, LlgObject *bias,
                      LlgObject *b, const float *d_a, const float *d_x, float thr, int act,
                      float *d_out, int32_t *d_active, int32_t *d_n_active, uint8_t *ws,
                      uint8_t *sync, const float *d_out_add, float2 *d_stats) {
    if (int rc = llg_check_act(d, act)) return rc;
    if (sync && wup->rows <= LLG_SYNC_SLOTS && wup->fmt.type == LLG_TYPE_F32) {
        HidArgs ha{};
        ha.wup = wup->d;
        ha.wstride = wup->stride;
        ha.h = wup->fmt.cols;
        ha.a = d_a;
        ha.ctr = reinterpret_cast<const uint32_t *>(sync);
        ha.slots = reinterpret_cast<uint64_t *>(sync + LLG_SYNC_HEAD);
        ha.check = llg_dev_check(d);
        // with d_out_add, the predictor workgroups first add d_out_add to out
        // and k_tile_reduce adds the FFN output to that (out ends as (out +
        // d_out_add) + the FFN output, the residual order of ffn_flash.go:161-166)
        if (d_out_add) {
            ha.acc_out = d_out;
            ha.acc_add = d_out_add;
            ha.acc_n = b->fmt.cols;
        }
        return fused_tail(d, wout, bias, b, d_x, thr, act, d_out, d_active, d_n_active, ws,
                          d_out_add != nullptr, d_stats, ha);
    }
    float *partial;
    unsigned long long *mask;
    int psplit;
    // k_tile_reduce stores out; with d_out_add, k_pred_hidden first adds
    // d_out_add to out and k_tile_reduce adds the FFN output to that
    int rc = llg_pred_hidden_enqueue(d, wup, d_a, ws, &partial, &mask, &psplit,
                                     d_out_add ? d_out : nullptr, b->fmt.cols, nullptr, 0,
                                     nullptr, d_out_add);
    if (rc) return rc;
    return llg_fused_tail_enqueue(d, wout, bias, b, d_x, thr, act, d_out, d_active, d_n_active,
                                  ws, d_out_add != nullptr, d_stats);
}

int llg_fused_tail_enqueue(LlgDevice *d, LlgObject *wout, LlgObject *bias, LlgObject *b,
                           const float *d_x, float thr, int act, float *d_out,
                           int32_t *d_active, int32_t *d_n_active, uint8_t *ws, bool accum,
                           float2 *d_stats) {
    return fused_tail(d, wout, bias, b, d_x, thr, act, d_out, d_active, d_n_active, ws, accum,
                      d_stats, HidArgs{});
}

bool llg_fused_wo_ok(const LlgObject *wo, int rank, int hidden) {
    const RowFmt &f = wo->fmt;
    return rank <= LLG_SYNC_SLOTS && (f.type == LLG_TYPE_Q4_0 || f.type == LLG_TYPE_Q8_0) &&
           f.nb <= WO_NB * 64 && (size_t)f.nb * XS_STRIDE * 4 <= 64 * 1024 && wo->rows == hidden &&
           f.cols % 32 == 0;
}

int llg_fused_wo_enqueue(LlgDevice *d, const LlgObject *wo, const LlgAttnParts &ap,
                         const float *pd, LlgObject *wout, LlgObject *bias, LlgObject *b,
                         const float *d_x, float thr, int act, float *d_resid,
                         int32_t *d_n_active, uint8_t *ws, uint8_t *sync, float2 *d_stats) {
    const int rank = wout->fmt.cols;
    if (!sync || !llg_fused_wo_ok(wo, rank, b->fmt.cols) || ap.n_split < 1 ||
        ap.n_split > LLG_ATTN_SPLIT_MAX || ap.n_heads * ap.head_dim != wo->fmt.cols)
        return llg_set_error(d, LLG_E_ARG, "Wo in the tile launch: rank %d, width %d", rank,
                             wo->fmt.cols);
    HidArgs ha{};
    ha.ctr = reinterpret_cast<const uint32_t *>(sync);
    ha.slots = reinterpret_cast<uint64_t *>(sync + LLG_SYNC_HEAD);
    ha.check = llg_dev_check(d);
    WoArgs wa{};
    wa.w = wo->d;
    wa.stride = wo->stride;
    wa.f = wo->fmt;
    wa.rows = wo->rows;
    wa.resid = d_resid;
    wa.ap = ap;
    wa.pd = pd;
    return fused_tail(d, wout, bias, b, d_x, thr, act, d_resid, nullptr, d_n_active, ws, true,
                      d_stats, ha, wa);
}
