// llg_sparse.hip -- gathered sparse FFN over row-column bundles
// (inference/ffn_flash.go:195-299, window.go:143-180).
//
// Two ways in:
//
//  A. predictor-fused step (ffnFlash path 2, ffn_flash.go:225-231), 3 launches:
//     K1 k_pred_hidden (llg_predictor.hip): hidden partials; zeroes out/counters
//     K2 k_tile_up: one workgroup per 64-neuron tile: logits from WOut rows,
//        strict '>' against the threshold via a wavefront ballot, then the up
//        dot product of each of the tile's active neurons, u = act(up . x),
//        one neuron per wavefront of 8 (two when more than 8 are active);
//        nonzero u go to the tile's own 64 pair slots (an LDS counter orders
//        them), so no two workgroups touch one address
//     K3 k_sparse_down over the tiles' pairs
//  B. explicit active list (ffnSparseLoad, NeuronCache.FFNForward), 2 launches:
//     k_list_up: one wavefront per listed neuron, pair j = (row, u_j)
//     K3 k_sparse_down
//
// x is staged once per workgroup in LDS with a 36-float stride per 32-float
// block, so the 16-byte reads of 16 consecutive lanes (one block each) hit
// 64 distinct banks.  Every lane issues the loads of all its blocks before it
// uses any of them.
//
// k_sparse_down: workgroup (slice s of 8 blocks = 256 outputs, pair group g);
// the four wavefronts split the group's pairs, 8 pairs per wavefront pass
// (lane = pair sub-index * 8 + block); u == 0 rows are skipped as at
// ffn_flash.go:290; the per-slice sums are reduced across lanes (one DPP step)
// and through LDS, and added to out with one fp32 atomic per output.  blockIdx -> (s, g) keeps all
// slices of a group on one XCD (workgroups go round-robin over the 8 XCDs).
#include "llg_common.hpp"
#include "llg_internal.hpp"
#include "llg_pred_tile.hpp"

#define XS_STRIDE 36      // floats per staged 32-float x block (bank-conflict-free)
#define DN_SLICE 8        // blocks per down slice
#define BATCH 4           // blocks whose loads a lane issues together
#define PRED_SPLIT_N 8    // partials per hidden unit written by k_pred_hidden
#define DN_HEAD 8         // pair slots per tile that k_sparse_down reads with the counts
#define DN_RED_ST 36      // LDS floats per (row, block) partial in the down reduction
#define TILE_THREADS 512  // k_tile_up workgroup: 8 wavefronts for the up rows

__device__ __forceinline__ void stage_x(float *xs, const float *__restrict__ x, int nb) {
    llg_stage_x_sum<XS_STRIDE>(xs, x, nb);
}

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

// Up-row dot products of NR rows (wavefront-uniform indices, < 0: none) by
// one wavefront, NBATCH blocks per lane per pass, all loads of a pass issued
// before any is used; same conventions as row_dot2.
template <int T, int NR, int NBATCH>
__device__ __forceinline__ void row_dotn(const uint8_t *__restrict__ base, long long bstride,
                                         const int (&row)[NR], const RowFmt &f, const float *xs,
                                         float (&s)[NR]) {
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
    for (int b0 = 0; b0 < f.nb; b0 += 64 * NBATCH) {
        BlockRaw<T> r[NBATCH][NR];
#pragma unroll
        for (int i = 0; i < NBATCH; i++)
#pragma unroll
            for (int q = 0; q < NR; q++)
                llg_block_load<T>(r[i][q], p[q], f, min(b0 + lane + 64 * i, f.nb - 1));
#pragma unroll
        for (int i = 0; i < NBATCH; i++) {
            const int b = b0 + lane + 64 * i;
            if (b < f.nb) {
                const float *xb = xs + b * XS_STRIDE;
                const float4 *x4 = reinterpret_cast<const float4 *>(xb);
#pragma unroll
                for (int q = 0; q < NR; q++) {
                    const float d = llg_raw_dot<T>(r[i][q], x4, xb[32]);
                    s[q] += v[q] ? d : 0.0f;
                }
            }
        }
    }
#pragma unroll
    for (int q = 0; q < NR; q++) s[q] = llg_wave_sum(s[q]);
}

// One round of the tile's up rows: neuron k0 + wave + nw*i (i < NR) on this
// wavefront; nonzero u go to the tile's pair slots through the LDS counter.
template <int T, int NR>
__device__ __forceinline__ void tile_up_round(const uint8_t *__restrict__ base, long long bstride,
                                              const RowFmt &f, const float *xs, const int *tl,
                                              int *ctr, int cnt, int k0, int tile0, int act,
                                              int2 *__restrict__ tpairs) {
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    int rows[NR];
#pragma unroll
    for (int i = 0; i < NR; i++) {
        const int k = k0 + wave + nw * i;
        rows[i] = k < cnt ? tile0 + tl[k] : -1;
    }
    if (rows[0] < 0) return;  // wavefront-uniform: nothing in this round
    float s[NR];
    row_dotn<T, NR, NR == 1 ? 4 : 3>(base, bstride, rows, f, xs, s);
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int i = 0; i < NR; i++) {
            if (rows[i] < 0) break;
            const float u = llg_act(act, s[i]);
            if (u != 0.0f) {  // ffn_flash.go:290 skips zero activations
                const int pos = atomicAdd(ctr, 1);  // LDS atomic, tile-local slot
                tpairs[pos] = make_int2(rows[i], __float_as_int(u));
            }
        }
    }
}

// B. explicit list: pair j = (row of active[j], act(up . x)); also zeroes out.
// With src (windowed rows): a neuron n with fresh[n] == epoch (loaded by this
// token's update) is read from row n of src, and its whole bundle is copied
// to its resident row on the way (the gather of loadRows, window.go:207-245,
// done by the first reader).
// (base and dst are the same buffer then: base is not __restrict__.)  FR
// selects that form (fr.src set), which holds the copies in registers.
// The count read on the device is clamped to the pair capacity `cap`, and a
// neuron outside [0, n_rows) counts as absent (activation 0), so no list
// makes the kernel read or write out of bounds.
template <int T, bool FR>
__global__ __launch_bounds__(256) void k_list_up(
    const uint8_t *base, long long bstride, RowFmt f, const int32_t *__restrict__ slot_of,
    const float *__restrict__ x, const int32_t *__restrict__ active,
    const int32_t *__restrict__ n_active_p, int cap, int n_rows, int act,
    int2 *__restrict__ pairs, float *__restrict__ out, LlgFreshRows fr) {
    extern __shared__ float xs[];
    const int n_active = min(max(*n_active_p, 0), cap);
    const int gtid = blockIdx.x * blockDim.x + threadIdx.x;
    for (int i = gtid; i < f.cols; i += gridDim.x * blockDim.x) out[i] = 0.0f;
    const int first = blockIdx.x * 4;
    if (first >= n_active) return;  // whole workgroup idle: skip the x staging
    stage_x(xs, x, f.nb);
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int stride = gridDim.x * 4;
    for (int j = first + (threadIdx.x >> 6); j < n_active; j += 2 * stride) {
        const int j1 = j + stride;
        auto neuron = [&](int jj) {
            const int n = active[jj];
            return n >= 0 && n < n_rows ? n : -1;
        };
        const int n0 = neuron(j);
        const int n1 = j1 < n_active ? neuron(j1) : -1;
        const int row0 = n0 < 0 ? -1 : (slot_of ? slot_of[n0] : n0);
        const int row1 = n1 < 0 ? -1 : (slot_of ? slot_of[n1] : n1);
        float s0, s1;
        if constexpr (FR) {
            const int r0 = __builtin_amdgcn_readfirstlane(row0);
            const int r1 = __builtin_amdgcn_readfirstlane(row1);
            const bool f0 = __builtin_amdgcn_readfirstlane(r0 >= 0 && fr.fresh[n0] == fr.epoch);
            const bool f1 = __builtin_amdgcn_readfirstlane(r1 >= 0 && fr.fresh[n1] == fr.epoch);
            const uint8_t *p0 = f0 ? fr.src + (long long)n0 * bstride
                                   : base + (long long)(r0 >= 0 ? r0 : 0) * bstride;
            const uint8_t *p1 = f1 ? fr.src + (long long)n1 * bstride
                                   : base + (long long)(r1 >= 0 ? r1 : 0) * bstride;
            const int n16 = (int)(bstride >> 4);
            constexpr int NC = bc_first<T>();
            const bc_u4 *sp0 = reinterpret_cast<const bc_u4 *>(p0);
            const bc_u4 *sp1 = reinterpret_cast<const bc_u4 *>(p1);
            bc_u4 *dp0 = reinterpret_cast<bc_u4 *>(fr.dst + (long long)(f0 ? r0 : 0) * bstride);
            bc_u4 *dp1 = reinterpret_cast<bc_u4 *>(fr.dst + (long long)(f1 ? r1 : 0) * bstride);
            BundleCopy<NC> c0, c1;
            if (f0) bc_issue(c0, sp0, n16);
            if (f1) bc_issue(c1, sp1, n16);
            // the copies are stored once the dot's loads are in flight
            row_dot2p<T>(p0, p1, r0 >= 0, r1 >= 0, f, xs, s0, s1, [&]() {
                if (f0) bc_store(c0, dp0, n16);
                if (f1) bc_store(c1, dp1, n16);
            });
            if (f0) bc_rest<NC>(sp0, dp0, n16);
            if (f1) bc_rest<NC>(sp1, dp1, n16);
        } else {
            row_dot2<T>(base, bstride, row0, row1, f, xs, s0, s1);
        }
        if (lane == 0) {  // a non-resident row keeps activation 0 (window.go:150-152)
            pairs[j] = make_int2(row0, __float_as_int(row0 >= 0 ? llg_act(act, s0) : 0.0f));
            if (j1 < n_active)
                pairs[j1] = make_int2(row1, __float_as_int(row1 >= 0 ? llg_act(act, s1) : 0.0f));
        }
    }
}

// A. predictor-fused tile kernel.  Tile t writes its nonzero (row, u) pairs
// to pairs[t*64 + k], k < tile_cnt[t]: fixed slots, so no global counter.
template <int T>
__global__ __launch_bounds__(TILE_THREADS, 2) void k_tile_up(
    const uint8_t *__restrict__ wout, long long wstride, int ff, int rank,
    const float *__restrict__ partial, const float *__restrict__ bias, float thr,
    const uint8_t *__restrict__ base, long long bstride, RowFmt f, const float *__restrict__ x,
    int act, unsigned long long *__restrict__ mask, int2 *__restrict__ pairs,
    int32_t *__restrict__ tile_cnt) {
    extern __shared__ float sh[];
    float *xs = sh;                                     // nb * XS_STRIDE
    float *hid = xs + f.nb * XS_STRIDE;                 // rank (16-byte aligned)
    float *lg = hid + ((rank + 3) & ~3);                // 64
    int *tl = reinterpret_cast<int *>(lg + 64);         // 64 tile-local indices, count, nnz
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tile0 = blockIdx.x * 64;
    WoutTile t;  // logits: wavefronts 0-3 (16 neurons each)
    if (wave < 4) load_wout_tile(t, wout, wstride, ff, rank, tile0);  // used after the barrier
    stage_x(xs, x, f.nb);
    load_hidden<PRED_SPLIT_N>(hid, partial, rank);
    __syncthreads();
    if (wave < 4) finish_logits(t, wout, wstride, ff, rank, tile0, hid, lg);
    __syncthreads();
    if (wave == 0) {
        const int i = tile0 + lane;
        bool on = false;
        if (i < ff) {
            float v = lg[lane];
            if (bias) v += bias[i];  // predictor.go:69-73
            on = v > thr;            // predictor.go:78
        }
        const unsigned long long m = __ballot(on);
        const int before = __popcll(m & ((1ull << lane) - 1ull));
        if (on) tl[before] = lane;
        if (lane == 0) {
            tl[64] = __popcll(m);
            tl[65] = 0;
            if (mask) mask[blockIdx.x] = m;
        }
    }
    __syncthreads();
    const int cnt = tl[64];
    // up rows of the active neurons on all TILE_THREADS/64 wavefronts, one
    // round of loads for up to 16 (1 or 2 rows per wavefront by count)
    constexpr int UPMAX = T == LLG_TYPE_F32 ? 1 : 2;
    const int nw = TILE_THREADS / 64;
    int2 *tpairs = pairs + (size_t)blockIdx.x * 64;
    if (cnt <= nw || UPMAX == 1) {
        for (int k0 = 0; k0 < cnt; k0 += nw)
            tile_up_round<T, 1>(base, bstride, f, xs, tl, &tl[65], cnt, k0, tile0, act, tpairs);
    } else {
        if constexpr (UPMAX == 2)
            for (int k0 = 0; k0 < cnt; k0 += 2 * nw)
                tile_up_round<T, 2>(base, bstride, f, xs, tl, &tl[65], cnt, k0, tile0, act, tpairs);
    }
    __syncthreads();
    if (threadIdx.x == 0) tile_cnt[blockIdx.x] = tl[65];
}

// Pairs come either as a plain list pairs[0..*count) (TILED = false; the
// count is clamped to the capacity n_tiles) or in
// per-tile slots pairs[t*64 + k], k < tile_cnt[t] (TILED = true); for the
// latter, group g owns tiles [g*tg, (g+1)*tg) and its workgroups enumerate
// them through a prefix sum of the counts.  With TILED, workgroup 0 also
// writes the number of active neurons (popcounts of the tile masks).
template <int T, bool TILED>
__global__ __launch_bounds__(256) void k_sparse_down(
    const uint8_t *__restrict__ base, long long bstride, RowFmt f, const int2 *__restrict__ pairs,
    const int32_t *__restrict__ count_p, const int32_t *__restrict__ tile_cnt, int n_tiles,
    const unsigned long long *__restrict__ mask, int32_t *__restrict__ n_active_out,
    int n_slices, int n_groups, float *__restrict__ out) {
    __shared__ __attribute__((aligned(16))) float red[16 * DN_SLICE * DN_RED_ST];
    __shared__ int pref[65];
    __shared__ int2 head[64 * DN_HEAD];  // the first DN_HEAD pair slots of each tile
    const int id = blockIdx.x;
    const int xcd = id & 7;
    const int k = id >> 3;
    const int g = xcd + 8 * (k / n_slices);
    const int s = k % n_slices;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int j0, j1, tg = 0, t0 = 0;
    if (TILED) {
        tg = (n_tiles + n_groups - 1) / n_groups;  // <= 64 (checked on the host)
        t0 = g * tg;
        // the counts and the first DN_HEAD slots of every tile, in one round
        for (int i = threadIdx.x; i < tg * DN_HEAD; i += blockDim.x) {
            const int tt = min(t0 + i / DN_HEAD, n_tiles - 1);
            head[i] = pairs[tt * 64 + i % DN_HEAD];
        }
        if (wave == 0) {
            const int c = (lane < tg && t0 + lane < n_tiles) ? tile_cnt[t0 + lane] : 0;
            int incl = c;
            for (int o = 1; o < 64; o <<= 1) {
                const int v = __shfl_up(incl, o, 64);
                if (lane >= o) incl += v;
            }
            pref[lane + 1] = incl;
            if (lane == 0) pref[0] = 0;
        }
        if (id == 0 && wave == 1 && n_active_out) {
            int c = 0;
            for (int i = lane; i < n_tiles; i += 64) c += __popcll(mask[i]);
            for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
            if (lane == 0) *n_active_out = c;
        }
        __syncthreads();
        j0 = 0;
        j1 = pref[64];
    } else {
        const int count = min(max(*count_p, 0), n_tiles);
        const int chunk = (count + n_groups - 1) / n_groups;
        j0 = g * chunk;
        j1 = min(count, j0 + chunk);
    }
    if (j0 >= j1) return;  // uniform over the workgroup: nothing to add
    const int bl = lane & 7;
    const int sub = lane >> 3;
    const int b = s * DN_SLICE + bl;
    const int bc = min(b, f.nb - 1);  // lanes past the last block load it and drop it
    float acc[32];
    float corr = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; e++) acc[e] = 0.0f;
    {
        for (int j = j0 + wave * 8 + sub; j < j1; j += 64) {
            // two pairs per pass: both rows' bytes are requested before either is used
            int2 p0, p1 = make_int2(0, 0);
            if (TILED) {
                int t = 0;
                while (pref[t + 1] <= j) t++;
                int k = j - pref[t];
                p0 = k < DN_HEAD ? head[t * DN_HEAD + k] : pairs[(t0 + t) * 64 + k];
                if (j + 32 < j1) {
                    const int jj = j + 32;
                    while (pref[t + 1] <= jj) t++;
                    k = jj - pref[t];
                    p1 = k < DN_HEAD ? head[t * DN_HEAD + k] : pairs[(t0 + t) * 64 + k];
                }
            } else {
                p0 = pairs[j];
                if (j + 32 < j1) p1 = pairs[j + 32];
            }
            float u0 = __int_as_float(p0.y), u1 = __int_as_float(p1.y);
            if (b >= f.nb) u0 = u1 = 0.0f;
            // Unconditional loads (a row index of a zero activation may be -1 or
            // stale: such lanes read row 0); only the use is skipped, as
            // ffn_flash.go:290 skips u == 0.
            BlockRaw<T> r0, r1;
            llg_block_load<T>(r0, base + (long long)(u0 != 0.0f ? p0.x : 0) * bstride + f.stride, f, bc);
            llg_block_load<T>(r1, base + (long long)(u1 != 0.0f ? p1.x : 0) * bstride + f.stride, f, bc);
            if (u0 != 0.0f) llg_raw_axpy<T>(r0, u0, acc, corr);
            if (u1 != 0.0f) llg_raw_axpy<T>(r1, u1, acc, corr);
        }
    }
    // Sum over the 8 pair sub-lanes and 4 wavefronts sharing block bl: one DPP
    // step folds sub-lanes 2r+1 into 2r (row_ror:8 within each 16-lane row),
    // then the 16 partial sums per output meet in LDS (row stride 36 floats).
#pragma unroll
    for (int e = 0; e < 32; e++) {
        const float v = acc[e] - corr;
        acc[e] = v + llg_dpp<0x128>(v);
    }
    if ((lane & 8) == 0) {
        float *dst = &red[((wave * 4 + (lane >> 4)) * DN_SLICE + bl) * DN_RED_ST];
#pragma unroll
        for (int q = 0; q < 8; q++)
            *reinterpret_cast<float4 *>(dst + 4 * q) =
                make_float4(acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]);
    }
    __syncthreads();
    const int t = threadIdx.x;
    const int o = s * DN_SLICE * 32 + t;
    float sum = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; r++) sum += red[(r * DN_SLICE + (t >> 5)) * DN_RED_ST + (t & 31)];
    if (o < f.cols) unsafeAtomicAdd(out + o, sum);
}

// ---------------------------------------------------------------------------
// Host-side enqueue helpers
// ---------------------------------------------------------------------------
size_t llg_sparse_ws_bytes(int max_active) {
    return (size_t)llg_align((long long)(max_active > 0 ? max_active : 1) * 8, 256) + 256;
}

static size_t xs_bytes(const RowFmt &f) { return (size_t)f.nb * XS_STRIDE * 4; }

// 8 or 16 pair groups (a multiple of the 8 XCDs): enough workgroups to spread
// the rows, few enough that the atomics per output stay small.
static int down_groups(int max_pairs) { return max_pairs > 256 ? 16 : 8; }

template <int T>
static void launch_down(hipStream_t st, const uint8_t *base, long long bstride, const RowFmt &f,
                        const int2 *pairs, const int32_t *count, int max_pairs, float *out) {
    const int n_slices = (f.nb + DN_SLICE - 1) / DN_SLICE;
    const int n_groups = down_groups(max_pairs);
    hipLaunchKernelGGL((k_sparse_down<T, false>), dim3(n_slices * n_groups), dim3(256), 0, st,
                       base, bstride, f, pairs, count, (const int32_t *)nullptr, max_pairs,
                       (const unsigned long long *)nullptr, (int32_t *)nullptr, n_slices,
                       n_groups, out);
}

template <int T>
static void launch_list(hipStream_t st, const uint8_t *base, long long bstride, const RowFmt &f,
                        const int32_t *slot_of, const float *x, const int32_t *active,
                        const int32_t *n_active, int max_active, int n_rows, int act,
                        float *out, int2 *pairs, const LlgFreshRows &fr) {
    int grid = (max_active + 3) / 4;
    if (grid < 1) grid = 1;
    if (grid > 2048) grid = 2048;
    if (fr.src)
        hipLaunchKernelGGL((k_list_up<T, true>), dim3(grid), dim3(256), xs_bytes(f), st, base,
                           bstride, f, slot_of, x, active, n_active, max_active, n_rows, act,
                           pairs, out, fr);
    else
        hipLaunchKernelGGL((k_list_up<T, false>), dim3(grid), dim3(256), xs_bytes(f), st, base,
                           bstride, f, slot_of, x, active, n_active, max_active, n_rows, act,
                           pairs, out, fr);
    launch_down<T>(st, base, bstride, f, pairs, n_active, max_active, out);
}

int llg_sparse_enqueue(LlgDevice *d, const uint8_t *base, long long bstride, const RowFmt &f,
                       const int32_t *slot_of, const float *d_x, const int32_t *d_active,
                       const int32_t *d_n_active, int max_active, int n_rows, int act,
                       float *d_out, uint8_t *ws, const LlgFreshRows *fresh) {
    if (int rc = llg_check_act(d, act)) return rc;
    const LlgFreshRows fr = fresh ? *fresh : LlgFreshRows{nullptr, nullptr, 0, nullptr};
    if (fr.src && (!slot_of || !fr.fresh || !fr.dst || (bstride & 15)))
        return llg_set_error(d, LLG_E_ARG, "sparse ffn: windowed rows need slots and tags");
    if (xs_bytes(f) > 64 * 1024)
        return llg_set_error(d, LLG_E_ARG, "sparse ffn: hidden size %d too large", f.cols);
    hipStream_t st = llg_dev_stream(d);
    int2 *pairs = reinterpret_cast<int2 *>(ws);
    switch (f.type) {
    case LLG_TYPE_Q4_0:
        launch_list<LLG_TYPE_Q4_0>(st, base, bstride, f, slot_of, d_x, d_active, d_n_active,
                                   max_active, n_rows, act, d_out, pairs, fr);
        break;
    case LLG_TYPE_Q8_0:
        launch_list<LLG_TYPE_Q8_0>(st, base, bstride, f, slot_of, d_x, d_active, d_n_active,
                                   max_active, n_rows, act, d_out, pairs, fr);
        break;
    case LLG_TYPE_F16:
        launch_list<LLG_TYPE_F16>(st, base, bstride, f, slot_of, d_x, d_active, d_n_active,
                                  max_active, n_rows, act, d_out, pairs, fr);
        break;
    case LLG_TYPE_F32:
        launch_list<LLG_TYPE_F32>(st, base, bstride, f, slot_of, d_x, d_active, d_n_active,
                                  max_active, n_rows, act, d_out, pairs, fr);
        break;
    default:
        return llg_set_error(d, LLG_E_TYPE, "sparse ffn: unsupported type %d", f.type);
    }
    LLG_LAUNCH_CHECK(d, "sparse ffn");
    return 0;
}

size_t llg_fused_ws_bytes(int rank, int ff) {
    const long long n_tiles = (ff + 63) / 64;
    return (size_t)llg_predict_ws_bytes(rank, ff) + (size_t)llg_align(n_tiles * 64 * 8, 256) +
           (size_t)llg_align(n_tiles * 4, 256);
}

template <int T>
static void launch_fused(hipStream_t st, LlgObject *wout, const float *partial, const float *bias,
                         float thr, LlgObject *b, const float *x, int act,
                         unsigned long long *mask, int2 *pairs, int32_t *tile_cnt,
                         int32_t *n_active, float *out) {
    const int ff = wout->rows, rank = wout->fmt.cols;
    const int n_tiles = (ff + 63) / 64;
    const RowFmt &f = b->fmt;
    const size_t lds = xs_bytes(f) + (size_t)(((rank + 3) & ~3) + 64 + 66) * 4;
    hipLaunchKernelGGL(k_tile_up<T>, dim3(n_tiles), dim3(TILE_THREADS), lds, st, wout->d, wout->stride, ff,
                       rank, partial, bias, thr, b->d, b->stride, f, x, act, mask, pairs,
                       tile_cnt);
    const int n_slices = (f.nb + DN_SLICE - 1) / DN_SLICE;
    const int n_groups = down_groups(ff);
    hipLaunchKernelGGL((k_sparse_down<T, true>), dim3(n_slices * n_groups), dim3(256), 0, st,
                       b->d, b->stride, f, pairs, (const int32_t *)nullptr, tile_cnt, n_tiles,
                       mask, n_active, n_slices, n_groups, out);
}

// ffnFlash path 2 on the device: K1 + K2 + K3, plus the ascending active list
// through k_compact when d_active is given.  d_n_active (optional) receives
// the number of active neurons.
int llg_fused_enqueue(LlgDevice *d, LlgObject *wup, LlgObject *wout, LlgObject *bias,
                      LlgObject *b, const float *d_a, const float *d_x, float thr, int act,
                      float *d_out, int32_t *d_active, int32_t *d_n_active, uint8_t *ws,
                      const float *d_out_add) {
    if (int rc = llg_check_act(d, act)) return rc;
    const RowFmt &f = b->fmt;
    const int ff = wout->rows, rank = wup->rows;
    const int n_tiles = (ff + 63) / 64;
    if (xs_bytes(f) + (size_t)(rank + 136) * 4 > 64 * 1024)
        return llg_set_error(d, LLG_E_ARG, "predict_sparse: hidden size %d too large", f.cols);
    if ((n_tiles + down_groups(ff) - 1) / down_groups(ff) > 64)
        return llg_set_error(d, LLG_E_ARG, "predict_sparse: d_ff %d too large", ff);
    hipStream_t st = llg_dev_stream(d);
    int2 *pairs = reinterpret_cast<int2 *>(ws + llg_predict_ws_bytes(rank, ff));
    int32_t *tile_cnt = reinterpret_cast<int32_t *>(ws + llg_predict_ws_bytes(rank, ff) +
                                                    llg_align((long long)n_tiles * 64 * 8, 256));
    float *partial;
    unsigned long long *mask;
    int psplit;
    // K1 also clears out, the atomic target of K3 (or, with d_out_add, adds
    // d_out_add to it: out then ends as out + d_out_add + the FFN output)
    int rc = llg_pred_hidden_enqueue(d, wup, d_a, ws, &partial, &mask, &psplit, d_out, f.cols,
                                     nullptr, 0, nullptr, d_out_add);
    if (rc) return rc;
    if (psplit != PRED_SPLIT_N)
        return llg_set_error(d, LLG_E_ARG, "predict_sparse: hidden split %d != %d", psplit,
                             PRED_SPLIT_N);
    const float *d_bias = bias ? reinterpret_cast<const float *>(bias->d) : nullptr;
    switch (f.type) {
    case LLG_TYPE_Q4_0:
        launch_fused<LLG_TYPE_Q4_0>(st, wout, partial, d_bias, thr, b, d_x, act, mask, pairs,
                                    tile_cnt, d_n_active, d_out);
        break;
    case LLG_TYPE_Q8_0:
        launch_fused<LLG_TYPE_Q8_0>(st, wout, partial, d_bias, thr, b, d_x, act, mask, pairs,
                                    tile_cnt, d_n_active, d_out);
        break;
    case LLG_TYPE_F16:
        launch_fused<LLG_TYPE_F16>(st, wout, partial, d_bias, thr, b, d_x, act, mask, pairs,
                                   tile_cnt, d_n_active, d_out);
        break;
    case LLG_TYPE_F32:
        launch_fused<LLG_TYPE_F32>(st, wout, partial, d_bias, thr, b, d_x, act, mask, pairs,
                                   tile_cnt, d_n_active, d_out);
        break;
    default:
        return llg_set_error(d, LLG_E_TYPE, "predict_sparse: unsupported type %d", f.type);
    }
    LLG_LAUNCH_CHECK(d, "predict_sparse");
    if (d_active) return llg_compact_enqueue(d, mask, n_tiles, d_active, nullptr);
    return 0;
}
