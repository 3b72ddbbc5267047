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
//   k_moe_down     part[s][c][d] = down_e[d] . h[s] over column chunk c of h
//   k_moe_dec_combine
//                  out[d] = sum_s w_s * (sum_c part[s][c][d]), slots in the
//                  chosen order and chunks in order, starting from 0
//                  (moe_forward.go:71-77, 141-148): every sum has a fixed
//                  order, so results are the same on every run
// Expert e's rows are e*eff + j of gate/up and e*hidden + d of down, the
// addressing of ReadContiguousRows (flash/storage.go:72-94).
// Batches of 16 or more tokens over Q4_0 experts go to the grouped MFMA GEMM
// path (llg_moe_gemm.hip); smaller batches and other types use the kernels
// below token by token.
#include <algorithm>

#include "llg_common.hpp"
#include "llg_internal.hpp"

#define MOE_MAX_EXP 64
#define MOE_MAX_K 8

__device__ __forceinline__ float moe_lane(float v, int e) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), e));
}

// Softmax + stable descending top-k over `lg` (n_exp <= 64 values), one
// wavefront, lane e holding expert e.  The sequential parts keep the
// reference's order: max scan and fp32 sum from expert 0 (forward.go:463-479),
// wsum from slot 0 (moe_forward.go:62-68).  sort.Slice on n <= 12 is an
// insertion sort, i.e. stable: expert e's slot is the number of experts with a
// larger score plus those with an equal score and a lower index.  A NaN or
// +Inf logit makes every score NaN; the insertion sort then keeps index order.
__device__ void moe_route_wave(const float *lg, int n_exp, int k, int32_t *ids, float *w) {
    const int lane = threadIdx.x & 63;
    const float v = lane < n_exp ? lg[lane] : 0.0f;
    float mx = moe_lane(v, 0);
    for (int e = 1; e < n_exp; e++) {
        const float o = moe_lane(v, e);
        if (o > mx) mx = o;
    }
    float p = (float)exp((double)(v - mx));
    float sum = 0.0f;
    for (int e = 0; e < n_exp; e++) sum += moe_lane(p, e);
    p /= sum;
    int rank = 0;
    for (int e = 0; e < n_exp; e++) {
        const float o = moe_lane(p, e);
        rank += (o > p || (o == p && e < lane)) ? 1 : 0;
    }
    if (p != p) rank = lane;
    const bool mine = lane < n_exp && rank < k;
    float wsum = 0.0f;
    for (int s = 0; s < k; s++) {
        const unsigned long long m = __ballot(lane < n_exp && rank == s);
        wsum += moe_lane(p, __builtin_ctzll(m));
    }
    if (wsum < 1e-9f) wsum = 1.0f;
    if (mine) {
        ids[rank] = lane;
        w[rank] = p / wsum;
    }
}

// One workgroup per token; wavefront e computes logit e.  A lane's float4
// loads of router row and x are issued together (8 per lane per pass, clamped
// addresses, masked use), so a 4096-wide row costs two round trips.
__global__ __launch_bounds__(512) void k_moe_router(const uint8_t *__restrict__ router,
                                                    long long stride, int hidden, int n_exp, int k,
                                                    const float *__restrict__ x,
                                                    const float *__restrict__ given_logits,
                                                    int32_t *__restrict__ ids,
                                                    float *__restrict__ w) {
    __shared__ float lg[MOE_MAX_EXP];
    const int t = blockIdx.x;
    const int lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (given_logits) {
        for (int e = threadIdx.x; e < n_exp; e += blockDim.x) lg[e] = given_logits[(size_t)t * n_exp + e];
    } else {
        const float4 *xt = reinterpret_cast<const float4 *>(x + (size_t)t * hidden);
        const int n4 = hidden / 4;
        for (int e = wave; e < n_exp; e += nw) {
            const float4 *row = reinterpret_cast<const float4 *>(router + (long long)e * stride);
            float s = 0.0f;
            for (int c0 = 0; c0 < n4; c0 += 512) {
                float4 rv[8], xv[8];
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const int i = min(c0 + lane + 64 * q, n4 - 1);
                    rv[q] = row[i];
                    xv[q] = xt[i];
                }
#pragma unroll
                for (int q = 0; q < 8; q++)
                    if (c0 + lane + 64 * q < n4)
                        s += rv[q].x * xv[q].x + rv[q].y * xv[q].y + rv[q].z * xv[q].z +
                             rv[q].w * xv[q].w;
            }
            s = llg_wave_sum(s);
            if (lane == 0) lg[e] = s;
        }
    }
    __syncthreads();
    if (threadIdx.x < 64) moe_route_wave(lg, n_exp, k, ids + (size_t)t * k, w + (size_t)t * k);
}

// Dot products of NR rows against the staged vector xs (MOE_XS floats per
// 32-element block, block sum at [32]) over blocks [0, nb): lane l takes
// blocks l, l+64, ...; the loads of NB blocks x NR rows are issued together.
// The first batch is loaded by moe_rows_issue before the caller stages xs.
#define MOE_XS 36
template <int T, int NR, int NB>
struct MoeRows {
    BlockRaw<T> r[NB][NR];
    __device__ __forceinline__ void issue(const uint8_t *const (&rp)[NR], const RowFmt &f,
                                          int b0, int nb) {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int i = 0; i < NB; i++)
#pragma unroll
            for (int q = 0; q < NR; q++)
                llg_block_load<T>(r[i][q], rp[q], f, b0 + min(lane + 64 * i, nb - 1));
    }
    __device__ __forceinline__ void use(const float *xs, int b0, int nb, float (&s)[NR]) const {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int bl = lane + 64 * i;
            if (bl >= nb) continue;
            const float *xb = xs + (b0 + bl) * MOE_XS;
            const float4 *x4 = reinterpret_cast<const float4 *>(xb);
#pragma unroll
            for (int q = 0; q < NR; q++) s[q] += llg_raw_dot<T>(r[i][q], x4, xb[32]);
        }
    }
};

template <int T, int NR, int NB>
__device__ __forceinline__ void moe_rows_dot(const uint8_t *const (&rp)[NR], const RowFmt &f,
                                             int nb, const float *xs, float (&s)[NR],
                                             MoeRows<T, NR, NB> &m) {
    // m holds the loads of blocks [0, 64*NB); the rest stream in batches
    m.use(xs, 0, min(nb, 64 * NB), s);
    for (int b0 = 64 * NB; b0 < nb; b0 += 64 * NB) {
        m.issue(rp, f, b0, nb - b0);
        m.use(xs, b0, min(nb - b0, 64 * NB), s);
    }
}

// h[ts][j] = silu(gate_e[j] . x_t) * (up_e[j] . x_t), ts = token*k + slot,
// e = ids[ts] (moe_forward.go:101-132).  Workgroup: one ts, MOE_GU_TILE
// consecutive j; each wavefront owns MOE_GU_J j (2*MOE_GU_J rows: gate, up)
// whose loads are issued before x_t is staged.
#define MOE_GU_J 4
#define MOE_GU_TILE (4 * MOE_GU_J)
template <int T, int NB>
__global__ __launch_bounds__(256) void k_moe_gateup(const uint8_t *__restrict__ gate,
                                                    const uint8_t *__restrict__ up,
                                                    long long stride, RowFmt f, int eff, int k,
                                                    const int32_t *__restrict__ ids,
                                                    const float *__restrict__ x,
                                                    float *__restrict__ hbuf) {
    extern __shared__ float xs[];
    const int n_tiles = (eff + MOE_GU_TILE - 1) / MOE_GU_TILE;
    const int ts = blockIdx.x / n_tiles;
    const int j0 = (blockIdx.x % n_tiles) * MOE_GU_TILE +
                   MOE_GU_J * __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int e = ids[ts];
    const int t = ts / k;
    const uint8_t *rp[2 * MOE_GU_J];
#pragma unroll
    for (int q = 0; q < MOE_GU_J; q++) {  // rows past eff reload the last row, dropped
        const long long r = (long long)e * eff + min(j0 + q, eff - 1);
        rp[q] = gate + r * stride;
        rp[MOE_GU_J + q] = up + r * stride;
    }
    MoeRows<T, 2 * MOE_GU_J, NB> m;
    m.issue(rp, f, 0, f.nb);
    llg_stage_x_sum<MOE_XS, 5>(xs, x + (size_t)t * f.cols, f.nb);  // 256 threads: 160 blocks
    __syncthreads();
    if (j0 >= eff) return;
    float s[2 * MOE_GU_J];
#pragma unroll
    for (int q = 0; q < 2 * MOE_GU_J; q++) s[q] = 0.0f;
    moe_rows_dot<T, 2 * MOE_GU_J, NB>(rp, f, f.nb, xs, s, m);
#pragma unroll
    for (int q = 0; q < 2 * MOE_GU_J; q++) s[q] = llg_wave_sum(s[q]);
    if (lane == 0) {
#pragma unroll
        for (int q = 0; q < MOE_GU_J; q++) {
            if (j0 + q >= eff) break;
            const float g = s[q], u = s[MOE_GU_J + q];
            const float silu = g / (1.0f + (float)exp(-(double)g));  // moe_forward.go:130
            hbuf[(size_t)ts * eff + j0 + q] = silu * u;
        }
    }
}

// part[ts][ch][d] = down_e[d] . h[ts] over column chunk ch of h
// (moe_forward.go:141-148); k_moe_dec_combine adds the chunks and slots.
// Workgroup: one ts, MOE_DN_TILE consecutive d, one chunk of at most
// MOE_DN_CHUNK blocks of h staged in LDS; wavefront: MOE_DN_R rows.
#define MOE_DN_R 4
#define MOE_DN_TILE (4 * MOE_DN_R)
#define MOE_DN_CHUNK 160
template <int T, int NB>
__global__ __launch_bounds__(256) void k_moe_down(const uint8_t *__restrict__ down,
                                                  long long stride, RowFmt f, int hidden, int k,
                                                  int chunk_blocks,
                                                  const int32_t *__restrict__ ids,
                                                  const float *__restrict__ hbuf,
                                                  float *__restrict__ part) {
    extern __shared__ float xs[];
    const int n_chunks = (f.nb + chunk_blocks - 1) / chunk_blocks;
    const int n_tiles = (hidden + MOE_DN_TILE - 1) / MOE_DN_TILE;
    const int ch = blockIdx.x % n_chunks;
    const int tile = (blockIdx.x / n_chunks) % n_tiles;
    const int ts = blockIdx.x / (n_chunks * n_tiles);
    const int d0 = tile * MOE_DN_TILE + MOE_DN_R * __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int cb0 = ch * chunk_blocks;
    const int cnb = min(chunk_blocks, f.nb - cb0);
    const int e = ids[ts];
    const uint8_t *rp[MOE_DN_R];
#pragma unroll
    for (int q = 0; q < MOE_DN_R; q++)  // rows past hidden reload the last row, dropped
        rp[q] = down + ((long long)e * hidden + min(d0 + q, hidden - 1)) * stride;
    MoeRows<T, MOE_DN_R, NB> m;
    m.issue(rp, f, cb0, cnb);
    llg_stage_x_sum<MOE_XS, 5>(xs, hbuf + (size_t)ts * f.cols + (size_t)cb0 * 32, cnb);
    __syncthreads();
    if (d0 >= hidden) return;
    float s[MOE_DN_R];
#pragma unroll
    for (int q = 0; q < MOE_DN_R; q++) s[q] = 0.0f;
    m.use(xs, 0, min(cnb, 64 * NB), s);
    for (int b0 = 64 * NB; b0 < cnb; b0 += 64 * NB) {
        m.issue(rp, f, cb0 + b0, cnb - b0);
        m.use(xs, b0, min(cnb - b0, 64 * NB), s);
    }
#pragma unroll
    for (int q = 0; q < MOE_DN_R; q++) s[q] = llg_wave_sum(s[q]);
    if (lane == 0) {
        float *pr = part + ((size_t)ts * n_chunks + ch) * hidden;
#pragma unroll
        for (int q = 0; q < MOE_DN_R; q++)
            if (d0 + q < hidden) pr[d0 + q] = s[q];
    }
}

// ---------------------------------------------------------------------------
// Persistent decode forms (Q4_0/Q8_0, rows of at most 128 blocks for gate/up).
// A launch fills the chip once (MOE_P_BLOCKS workgroups per CU); wavefront w
// of W owns the contiguous item range [w*I/W, (w+1)*I/W), so the work is
// balanced to one item.  Each wavefront keeps its lanes' slice of the input
// vector in registers (blocks lane and lane+64 of the row, with their sums)
// and double-buffers the weight bytes: the loads of item i+1 are in flight
// while item i is reduced.  No LDS and no barriers.
// ---------------------------------------------------------------------------
#define MOE_P_BLOCKS 2

// Lane slice of a vector: NBL blocks (lane + 64*b of the chunk starting at
// block c0), 8 float4 and the 32-element sum each; blocks past nb are zero.
template <int NBL>
struct XSlice {
    float4 v[NBL][8];
    float sum[NBL];
};
template <int NBL>
__device__ __forceinline__ void xslice_load(XSlice<NBL> &xs, const float *__restrict__ x, int c0,
                                            int nb) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int b = 0; b < NBL; b++) {
        const int blk = c0 + lane + 64 * b;
        const float4 *p = reinterpret_cast<const float4 *>(x + (size_t)min(blk, nb - 1) * 32);
#pragma unroll
        for (int q = 0; q < 8; q++) xs.v[b][q] = p[q];
    }
#pragma unroll
    for (int b = 0; b < NBL; b++) {
        const bool ok = c0 + lane + 64 * b < nb;
        float t = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            if (!ok) xs.v[b][q] = make_float4(0.f, 0.f, 0.f, 0.f);
            t += (xs.v[b][q].x + xs.v[b][q].y) + (xs.v[b][q].z + xs.v[b][q].w);
        }
        xs.sum[b] = t;
    }
}

// gate/up item = 2 consecutive j of one ts (4 rows: gate j, j+1, up j, j+1).
template <int T>
__device__ __forceinline__ void gu_issue(BlockRaw<T> (&r)[2][4], const uint8_t *__restrict__ gate,
                                         const uint8_t *__restrict__ up, long long stride,
                                         const RowFmt &f, long long row, int bl0, int bl1) {
    const uint8_t *p[4] = {gate + row * stride, gate + (row + 1) * stride, up + row * stride,
                           up + (row + 1) * stride};
#pragma unroll
    for (int q = 0; q < 4; q++) {
        llg_block_load<T>(r[0][q], p[q], f, bl0);
        llg_block_load<T>(r[1][q], p[q], f, bl1);
    }
}

template <int T>
__device__ __forceinline__ void gu_finish(const BlockRaw<T> (&r)[2][4], const XSlice<2> &xs,
                                          bool ok0, bool ok1, float *__restrict__ h2) {
    float s[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float d0 = llg_raw_dot<T>(r[0][q], xs.v[0], xs.sum[0]);
        const float d1 = llg_raw_dot<T>(r[1][q], xs.v[1], xs.sum[1]);
        s[q] = (ok0 ? d0 : 0.0f) + (ok1 ? d1 : 0.0f);
    }
#pragma unroll
    for (int q = 0; q < 4; q++) s[q] = llg_wave_sum(s[q]);
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const float g = s[q], u = s[2 + q];
            const float silu = g / (1.0f + (float)exp(-(double)g));  // moe_forward.go:130
            h2[q] = silu * u;
        }
    }
}

// Lanes past the row's nb blocks reload its last block (in-bounds loads, no
// per-lane branch) and drop the product.
template <int T>
__global__ __launch_bounds__(256, MOE_P_BLOCKS) void k_moe_gateup_p(
    const uint8_t *__restrict__ gate, const uint8_t *__restrict__ up, long long stride, RowFmt f,
    int eff, int k, int n_items, const int32_t *__restrict__ ids,
    const float *__restrict__ x, float *__restrict__ hbuf) {
    const int lane = threadIdx.x & 63;
    const long long W = (long long)gridDim.x * 4;
    const long long w = (long long)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i0 = (int)(w * n_items / W), i1 = (int)((w + 1) * n_items / W);
    if (i0 >= i1) return;
    const int per_ts = eff >> 1;
    const int bl0 = min(lane, f.nb - 1), bl1 = min(lane + 64, f.nb - 1);
    const bool ok0 = lane < f.nb, ok1 = lane + 64 < f.nb;
    BlockRaw<T> ra[2][4], rb[2][4];
    int ts_a = (int)(i0 / per_ts), ts_b;
    int e = ids[ts_a], ts_e = ts_a;
    gu_issue<T>(ra, gate, up, stride, f, (long long)e * eff + 2 * (i0 % per_ts), bl0, bl1);
    XSlice<2> xs;
    int t_x = ts_a / k;
    xslice_load<2>(xs, x + (size_t)t_x * f.cols, 0, f.nb);
    // The next item's loads go out without a branch (past the range the last
    // item is loaded again and not used), after any reload of x: the waits
    // before an item's products then never cover the next item's loads (a
    // load under a branch makes the compiler wait for all of them).
    for (int i = i0;;) {
        // A holds item i
        if (ts_a / k != t_x) xslice_load<2>(xs, x + (size_t)(t_x = ts_a / k) * f.cols, 0, f.nb);
        {
            const int in = min(i + 1, i1 - 1);
            ts_b = (int)(in / per_ts);
            if (ts_b != ts_e) e = ids[ts_e = ts_b];
            gu_issue<T>(rb, gate, up, stride, f, (long long)e * eff + 2 * (in % per_ts), bl0, bl1);
        }
        gu_finish<T>(ra, xs, ok0, ok1, hbuf + (size_t)ts_a * eff + 2 * (i % per_ts));
        if (++i >= i1) break;
        // B holds item i
        if (ts_b / k != t_x) xslice_load<2>(xs, x + (size_t)(t_x = ts_b / k) * f.cols, 0, f.nb);
        {
            const int in = min(i + 1, i1 - 1);
            ts_a = (int)(in / per_ts);
            if (ts_a != ts_e) e = ids[ts_e = ts_a];
            gu_issue<T>(ra, gate, up, stride, f, (long long)e * eff + 2 * (in % per_ts), bl0, bl1);
        }
        gu_finish<T>(rb, xs, ok0, ok1, hbuf + (size_t)ts_b * eff + 2 * (i % per_ts));
        if (++i >= i1) break;
    }
}

// down item = MOE_DN_P consecutive d of one (ts, chunk of 64 blocks of h):
// item index = (ts * n_chunks + chunk) * (hidden / MOE_DN_P) + d / MOE_DN_P,
// so a wavefront's range mostly shares one h slice.  The item's dot products
// go to part[ts][chunk][d]; k_moe_dec_combine adds chunks and slots.
#define MOE_DN_P 8
template <int T>
__device__ __forceinline__ void dn_issue(BlockRaw<T> (&r)[MOE_DN_P],
                                         const uint8_t *__restrict__ down, long long stride,
                                         const RowFmt &f, long long row, int bl) {
#pragma unroll
    for (int q = 0; q < MOE_DN_P; q++) llg_block_load<T>(r[q], down + (row + q) * stride, f, bl);
}

template <int T>
__device__ __forceinline__ void dn_finish(const BlockRaw<T> (&r)[MOE_DN_P], const XSlice<1> &hs,
                                          bool ok, float *__restrict__ o) {
    float s[MOE_DN_P];
#pragma unroll
    for (int q = 0; q < MOE_DN_P; q++) {
        const float d = llg_raw_dot<T>(r[q], hs.v[0], hs.sum[0]);
        s[q] = ok ? d : 0.0f;  // lanes past the row's last block
    }
#pragma unroll
    for (int q = 0; q < MOE_DN_P; q++) s[q] = llg_wave_sum(s[q]);
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int q = 0; q < MOE_DN_P; q++) o[q] = s[q];
    }
}

template <int T>
__global__ __launch_bounds__(256, MOE_P_BLOCKS) void k_moe_down_p(
    const uint8_t *__restrict__ down, long long stride, RowFmt f, int hidden, int k, int n_items,
    const int32_t *__restrict__ ids, const float *__restrict__ hbuf, float *__restrict__ part) {
    const int lane = threadIdx.x & 63;
    const long long W = (long long)gridDim.x * 4;
    const long long w = (long long)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i0 = (int)(w * n_items / W), i1 = (int)((w + 1) * n_items / W);
    if (i0 >= i1) return;
    const int n_chunks = (f.nb + 63) >> 6;
    const int per_chunk = hidden / MOE_DN_P;
    BlockRaw<T> ra[MOE_DN_P], rb[MOE_DN_P];
    // item i -> sc = i / per_chunk = ts * n_chunks + chunk, dg = i % per_chunk
    int sc_a = i0 / per_chunk, sc_b = 0;
    int ts_e = sc_a / n_chunks, e = ids[ts_e];
    dn_issue<T>(ra, down, stride, f, (long long)e * hidden + MOE_DN_P * (i0 - sc_a * per_chunk),
                min((sc_a - ts_e * n_chunks) * 64 + lane, f.nb - 1));
    int sc_h = sc_a, ts_h = ts_e;
    XSlice<1> hs;
    xslice_load<1>(hs, hbuf + (size_t)ts_h * f.cols, (sc_h - ts_h * n_chunks) * 64, f.nb);
    // next item's loads without a branch, after any reload of h (as in
    // k_moe_gateup_p)
    for (int i = i0;;) {
        if (sc_a != sc_h) {
            sc_h = sc_a;
            ts_h = sc_a / n_chunks;
            xslice_load<1>(hs, hbuf + (size_t)ts_h * f.cols, (sc_h - ts_h * n_chunks) * 64, f.nb);
        }
        {
            const int in = min(i + 1, i1 - 1);
            sc_b = in / per_chunk;
            const int tsb = sc_b / n_chunks;
            if (tsb != ts_e) e = ids[ts_e = tsb];
            dn_issue<T>(rb, down, stride, f, (long long)e * hidden + MOE_DN_P * (in - sc_b * per_chunk),
                        min((sc_b - tsb * n_chunks) * 64 + lane, f.nb - 1));
        }
        dn_finish<T>(ra, hs, (sc_h - ts_h * n_chunks) * 64 + lane < f.nb,
                     part + (size_t)sc_h * hidden + MOE_DN_P * (i - sc_a * per_chunk));
        if (++i >= i1) break;
        if (sc_b != sc_h) {
            sc_h = sc_b;
            ts_h = sc_b / n_chunks;
            xslice_load<1>(hs, hbuf + (size_t)ts_h * f.cols, (sc_h - ts_h * n_chunks) * 64, f.nb);
        }
        {
            const int in = min(i + 1, i1 - 1);
            sc_a = in / per_chunk;
            const int tsa = sc_a / n_chunks;
            if (tsa != ts_e) e = ids[ts_e = tsa];
            dn_issue<T>(ra, down, stride, f, (long long)e * hidden + MOE_DN_P * (in - sc_a * per_chunk),
                        min((sc_a - tsa * n_chunks) * 64 + lane, f.nb - 1));
        }
        dn_finish<T>(rb, hs, (sc_h - ts_h * n_chunks) * 64 + lane < f.nb,
                     part + (size_t)sc_h * hidden + MOE_DN_P * (i - sc_b * per_chunk));
        if (++i >= i1) break;
    }
}

// out[t][d] = sum over the slots s of w[t][s] * (sum over the chunks c of
// part[t*k + s][c][d]), slots in order from 0 and chunks in order
// (moe_forward.go:71-77): one thread per 4 outputs.
__global__ void k_moe_dec_combine(const float *__restrict__ part, const float *__restrict__ w,
                                  int k, int n_tok, int hidden, int n_chunks,
                                  float *__restrict__ out) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;  // float4 index
    const int h4 = hidden / 4;
    if (i >= (long long)n_tok * h4) return;
    const int t = (int)(i / h4), d4 = (int)(i % h4);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int sl = 0; sl < k; sl++) {
        const float ws = w[t * k + sl];
        const float4 *pr = reinterpret_cast<const float4 *>(part + (size_t)(t * k + sl) * n_chunks * hidden);
        float4 y = pr[d4];
        for (int c = 1; c < n_chunks; c++) {
            const float4 q = pr[(size_t)c * h4 + d4];
            y.x += q.x;
            y.y += q.y;
            y.z += q.z;
            y.w += q.w;
        }
        acc.x += ws * y.x;
        acc.y += ws * y.y;
        acc.z += ws * y.z;
        acc.w += ws * y.w;
    }
    reinterpret_cast<float4 *>(out)[i] = acc;
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
    if ((size_t)a->gate->fmt.nb * MOE_XS * 4 > 160 * 1024)  // x is staged whole in LDS
        return llg_set_error(d, LLG_E_ARG, "moeFFN: hidden=%d too long", a->hidden);
    return 0;
}

static bool use_gemm(const MoeArgs &a, int n_tok) {
    return llg_moe_gemm_supported(a.gate->fmt.type, a.hidden, a.eff, n_tok);
}

// Column chunks of h the decode down kernels split a row into (64 blocks for
// the persistent form, up to MOE_DN_CHUNK for the tile form).
static int moe_dec_chunks(const MoeArgs &a, bool persistent) {
    const int nb = a.down->fmt.nb;
    if (persistent) return (nb + 63) / 64;
    return (nb + MOE_DN_CHUNK - 1) / MOE_DN_CHUNK;
}

static size_t moe_hbuf_bytes(const MoeArgs &a, int n_tok) {
    return (size_t)llg_align((long long)n_tok * a.k * a.eff * 4, 256);
}

static size_t moe_ws_bytes(const MoeArgs &a, int n_tok) {
    const size_t head = (size_t)llg_align((long long)n_tok * a.k * 4, 256) * 2;
    if (use_gemm(a, n_tok))
        return head + llg_moe_gemm_ws_bytes(n_tok, a.k, a.n_exp, a.hidden, a.eff);
    // h, then the down partials (the larger chunk count of the two forms)
    return head + moe_hbuf_bytes(a, n_tok) +
           (size_t)n_tok * a.k * moe_dec_chunks(a, true) * a.hidden * 4;
}

static void moe_launch_combine(hipStream_t st, const MoeArgs &a, int n_tok, const float *w,
                               const float *part, int n_chunks, float *out) {
    const long long n4 = (long long)n_tok * a.hidden / 4;
    hipLaunchKernelGGL(k_moe_dec_combine, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st,
                       part, w, a.k, n_tok, a.hidden, n_chunks, out);
}

template <int T, int NB>
static void moe_launch_experts_nb(hipStream_t st, const MoeArgs &a, int n_tok, const int32_t *ids,
                                  const float *w, const float *x, float *hbuf, float *part,
                                  float *out) {
    const long long nts = (long long)n_tok * a.k;
    const long long g1 = nts * ((a.eff + MOE_GU_TILE - 1) / MOE_GU_TILE);
    hipLaunchKernelGGL((k_moe_gateup<T, NB>), dim3((unsigned)g1), dim3(256),
                       (size_t)a.gate->fmt.nb * MOE_XS * 4, st, a.gate->d, a.up->d, a.gate->stride,
                       a.gate->fmt, a.eff, a.k, ids, x, hbuf);
    const int nb = a.down->fmt.nb;
    const int n_chunks = moe_dec_chunks(a, false);
    const int cb = (nb + n_chunks - 1) / n_chunks;
    const long long g2 = nts * ((a.hidden + MOE_DN_TILE - 1) / MOE_DN_TILE) * n_chunks;
    hipLaunchKernelGGL((k_moe_down<T, 3>), dim3((unsigned)g2), dim3(256), (size_t)cb * MOE_XS * 4,
                       st, a.down->d, a.down->stride, a.down->fmt, a.hidden, a.k, cb, ids, hbuf,
                       part);
    moe_launch_combine(st, a, n_tok, w, part, n_chunks, out);
}

// Q4_0/Q8_0 with hidden <= 4096 take the persistent kernels; other shapes and
// types the workgroup-per-tile kernels above.
template <int T>
static void moe_launch_experts(hipStream_t st, int cus, const MoeArgs &a, int n_tok,
                               const int32_t *ids, const float *w, const float *x, float *hbuf,
                               float *part, float *out) {
    if constexpr (T == LLG_TYPE_Q4_0 || T == LLG_TYPE_Q8_0) {
        const long long n_dn = (long long)n_tok * a.k * ((a.down->fmt.nb + 63) / 64) * a.hidden / MOE_DN_P;
        if (a.gate->fmt.nb <= 128 && a.hidden % MOE_DN_P == 0 && n_dn < (1LL << 31) &&
            (long long)n_tok * a.k * a.eff < (1LL << 31)) {
            const long long nts = (long long)n_tok * a.k;
            const long long gu_items = nts * (a.eff / 2);
            const int n_chunks = (a.down->fmt.nb + 63) / 64;
            const long long dn_items = nts * n_chunks * (a.hidden / MOE_DN_P);
            const long long full = (long long)cus * MOE_P_BLOCKS;
            const long long g1 = std::min(full, (gu_items + 3) / 4);
            const long long g2 = std::min(full, (dn_items + 3) / 4);
            hipLaunchKernelGGL(k_moe_gateup_p<T>, dim3((unsigned)g1), dim3(256), 0, st, a.gate->d,
                               a.up->d, a.gate->stride, a.gate->fmt, a.eff, a.k, (int)gu_items, ids, x,
                               hbuf);
            hipLaunchKernelGGL(k_moe_down_p<T>, dim3((unsigned)g2), dim3(256), 0, st, a.down->d,
                               a.down->stride, a.down->fmt, a.hidden, a.k, (int)dn_items, ids, hbuf,
                               part);
            moe_launch_combine(st, a, n_tok, w, part, n_chunks, out);
            return;
        }
    }
    if (a.gate->fmt.nb <= 64)
        moe_launch_experts_nb<T, 1>(st, a, n_tok, ids, w, x, hbuf, part, out);
    else
        moe_launch_experts_nb<T, 2>(st, a, n_tok, ids, w, x, hbuf, part, out);
}

static int moe_enqueue(LlgDevice *d, const MoeArgs &a, const float *d_x, int n_tok, float *d_out,
                       int32_t *d_ids, float *d_w, uint8_t *ws) {
    hipStream_t st = llg_dev_stream(d);
    const long long kb = llg_align((long long)n_tok * a.k * 4, 256);
    int32_t *ids = d_ids ? d_ids : reinterpret_cast<int32_t *>(ws);
    float *w = d_w ? d_w : reinterpret_cast<float *>(ws + kb);
    float *hbuf = reinterpret_cast<float *>(ws + 2 * kb);
    float *part = reinterpret_cast<float *>(ws + 2 * kb + moe_hbuf_bytes(a, n_tok));
    hipLaunchKernelGGL(k_moe_router, dim3(n_tok), dim3(512), 0, st, a.router->d, a.router->stride,
                       a.hidden, a.n_exp, a.k, d_x, (const float *)nullptr, ids, w);
    LLG_LAUNCH_CHECK(d, "moe_router");
    if (use_gemm(a, n_tok))  // batched tokens: grouped MFMA GEMMs
        return llg_moe_gemm_enqueue(d, a.gate, a.up, a.down, a.n_exp, a.k, a.hidden, a.eff, d_x,
                                    n_tok, ids, w, d_out, ws + 2 * kb);
    switch (a.gate->fmt.type) {
    case LLG_TYPE_Q4_0:
        moe_launch_experts<LLG_TYPE_Q4_0>(st, llg_cu_count(d), a, n_tok, ids, w, d_x, hbuf, part, d_out);
        break;
    case LLG_TYPE_Q8_0:
        moe_launch_experts<LLG_TYPE_Q8_0>(st, llg_cu_count(d), a, n_tok, ids, w, d_x, hbuf, part, d_out);
        break;
    case LLG_TYPE_F16:
        moe_launch_experts<LLG_TYPE_F16>(st, llg_cu_count(d), a, n_tok, ids, w, d_x, hbuf, part, d_out);
        break;
    case LLG_TYPE_F32:
        moe_launch_experts<LLG_TYPE_F32>(st, llg_cu_count(d), a, n_tok, ids, w, d_x, hbuf, part, d_out);
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
