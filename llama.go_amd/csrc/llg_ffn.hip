// llg_ffn.hip -- dense dequant-matvec FFN (inference/forward.go:318-353,
// tensor/ops.go:39-60) and the sparse-FFN entry points (kernels in
// llg_sparse.hip).
//
// k_matvec_q: y[r] = act(sum_b block_dot(row r, b, x)).  A workgroup owns a
// tile of `tile_rows` rows and one column chunk of at most MV_CHUNK blocks; it
// stages that chunk of x in LDS (36-float stride per 32-float block, so 16
// lanes reading one block each hit distinct banks).  Each wavefront takes
// MV_ROWS rows at a time and issues the loads of all their blocks before
// using any (two layouts of the blocks over the lanes, below).  Tiles are 8
// rows (one pass of 4 wavefronts), 16 or 32 for very tall matrices; a matrix
// of 2048-8191 whole rows instead gets one workgroup per CU (the balanced
// launch, below).  With one chunk the row sum is final and the activation is
// applied.  With several chunks, each workgroup hands its partial sums over
// as tagged 64-bit slots, (1 << 32) | bits, one per (chunk, row)
// (llg_dev_mvslots: zero between launches), and the last workgroups of the
// same grid reduce them (mv_reduce): they come after every chunk workgroup,
// add the chunks in order, apply the activation, store y and clear the
// slots.  A slot not filled within MV_POLLS polls is computed by the reducer
// itself from x in memory (the chunk workgroup's blocks, block sums and
// order), so the wait always ends.  Without slots (more than MV_HAND_MAX
// chunks, or the attention-merge instance) the partial sums go to
// part[chunk][row] and k_chunk_sum adds them.
// Either way the chunks are added in a fixed order, so results are the same
// on every run.
//
// Gated (G): y[r] = silu(gate_r . x) * (up_r . x) (ffnSwiGLU, forward.go:
// 368-389) with gate = w and up = w2; a wavefront's two row slots hold gate
// row r and up row r, so it takes one output row per pass.
#include "llg_common.hpp"
#include "llg_internal.hpp"
#include "llg_pred_tile.hpp"

#define MV_ROWS 2
#define MV_TILE_SMALL 8   // rows per workgroup: one pass of 4 wavefronts x MV_ROWS ...
#define MV_MAX_WG 8192    // ... doubled (up to 32) while the grid has more workgroups than this
#define MV_SMALL_ROWS 8192
#define MV_BAL_MIN 2048   // balanced launch from this many rows (at least 4 wavefronts per CU)
#define MV_CHUNK 160      // max blocks of x staged per workgroup
#define MV_XS 36          // staged floats per 32-float block
#define MV_BATCH 3        // pair layout: blocks per lane per row and step
#define MV_NI 5           // flat layout: slots per lane per step (MV_ROWS x MV_CHUNK / 64, rounded up)
#define MV_HAND_MAX 4       // chunks reduced inside the launch (more: k_chunk_sum); 4 keeps
                            // the Q4_0 instance at 96 registers (5 wavefronts per SIMD)
#define MV_POLLS (1 << 16)  // a reducer's polls of its slots before it computes a sum itself

// Row rq's partial sum over chunk c from x in memory, by the whole
// wavefront: the blocks each lane of a chunk workgroup's wavefront takes in
// that chunk (pair layout, or the flat layout of Q8_0 with q the row's slot
// in its row pair), in the same order, each with the staged block sum
// (llg_block_xsum), then llg_wave_sum: the value that workgroup hands over.
template <int T>
__device__ __forceinline__ float mv_chunk_direct(const uint8_t *__restrict__ w, long long stride,
                                                 const RowFmt &f, int chunk_blocks,
                                                 const float *__restrict__ x, int c, int rq,
                                                 int q) {
    const int lane = threadIdx.x & 63;
    const int c0 = c * chunk_blocks, cn = min(chunk_blocks, f.nb - c0);
    const uint8_t *row = w + (long long)rq * stride;
    float s = 0.0f;
    auto one = [&](int b) {
        BlockRaw<T> blk;
        llg_block_load<T>(blk, row, f, c0 + b);
        const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)(c0 + b) * 32);
        s += llg_raw_dot<T>(blk, x4, llg_block_xsum(x4));
    };
    if constexpr (T == LLG_TYPE_Q8_0) {
        for (int i = 0; i < MV_NI; i++) {
            const int k = lane + 64 * i;
            if (k < MV_ROWS * cn && (k >= cn) == (q == 1)) one(k - (q ? cn : 0));
        }
    } else {
        for (int i = 0; i < MV_BATCH; i++)
            if (lane + 64 * i < cn) one(lane + 64 * i);
    }
    return llg_wave_sum(s);
}

// A reducer workgroup rb: thread t takes row rb * blockDim.x + t, polls its
// n_chunks slots (all in each poll), adds chunk 0, 1, ... in order (as
// k_chunk_sum), applies the activation, stores y and zeroes the slots.
// check (llg_dev_check): every chunk sum computed here after the wait.
template <int T>
__device__ __forceinline__ void mv_reduce(const uint8_t *__restrict__ w, long long stride,
                                          const RowFmt &f, int rows, int chunk_blocks,
                                          int n_chunks, const float *__restrict__ x, int act,
                                          float *__restrict__ y, uint64_t *__restrict__ slots,
                                          int rb, int check) {
    const int lane = threadIdx.x & 63;
    const int r = rb * (int)blockDim.x + (int)threadIdx.x;
    const int rc = min(r, rows - 1);
    uint64_t v[MV_HAND_MAX];
    auto load = [&]() {  // every slot (a chunk past the last rereads it)
#pragma unroll
        for (int c = 0; c < MV_HAND_MAX; c++)
            v[c] = llg_slot_get(slots + (size_t)min(c, n_chunks - 1) * rows + rc);
    };
    auto ready = [&]() {
        bool ok = true;
#pragma unroll
        for (int c = 0; c < MV_HAND_MAX; c++) ok = ok && (uint32_t)(v[c] >> 32) == 1u;
        return ok;
    };
    load();
    for (int polls = 0; !__all(ready()) && polls < MV_POLLS; polls++) {
        __builtin_amdgcn_s_sleep(1);
        load();
    }
    float p[MV_HAND_MAX];
#pragma unroll
    for (int c = 0; c < MV_HAND_MAX; c++) {
        p[c] = __uint_as_float((uint32_t)v[c]);
        if (c >= n_chunks) continue;  // uniform
        unsigned long long miss = __ballot(r < rows && (check || (uint32_t)(v[c] >> 32) != 1u));
        while (miss) {  // wavefront-uniform
            const int l = __ffsll((long long)miss) - 1;
            miss &= miss - 1;
            const int rr = __builtin_amdgcn_readlane(r, l);
            // tiles start at even rows, so the row's slot in its pair is its parity
            const float sv = mv_chunk_direct<T>(w, stride, f, chunk_blocks, x, c, rr, rr & 1);
            if (lane == l) p[c] = sv;
        }
    }
    float sum = p[0];
#pragma unroll
    for (int c = 1; c < MV_HAND_MAX; c++)
        if (c < n_chunks) sum += p[c];
    if (r < rows) {
        y[r] = act >= 0 ? llg_act(act, sum) : sum;
#pragma unroll
        for (int c = 0; c < MV_HAND_MAX; c++)
            if (c < n_chunks) llg_slot_put(slots + (size_t)c * rows + r, 0u, 0.0f);
    }
}

// LNP > 0: x is the LayerNorm of a residual sum, staged with LNP float4 groups
// per thread (llg_stage_ln); LNP = 0: x is read from memory.  NT: the largest
// workgroup the instance is launched with.
//
// PF: the predictor fold (LlgPredFold, one chunk only): wavefront w of
// workgroup b takes fold tasks t = w * gridDim.x + b, b + grid * waves, ...
// (spread over the workgroups), the first one's loads requested with the
// first rows'; the row sums go to pf.resid (+=) and, if y is set, to y.
#define MV_PFL 3  // float4 loads per lane of a fold task (split_blocks <= 24)
template <int T, int LNP, bool G = false, int NT = 256, bool PF = false, bool AC = false>
__global__ __launch_bounds__(NT) void k_matvec_q(const uint8_t *__restrict__ w, long long stride,
                                                  RowFmt f, int rows, int tile_rows,
                                                  int chunk_blocks,
                                                  const float *__restrict__ x, int act,
                                                  float *__restrict__ y, float *__restrict__ part,
                                                  LlgLnArgs ln,
                                                  const uint8_t *__restrict__ w2 = nullptr,
                                                  LlgPredFold pf = LlgPredFold{},
                                                  LlgAttnParts ap = LlgAttnParts{},
                                                  uint64_t *__restrict__ slots = nullptr,
                                                  int check = 0) {
    static_assert(!G || (LNP == 0 && MV_ROWS == 2), "gated rows pair gate and up");
    static_assert(!PF || (LNP == 0 && !G), "the fold rides on a plain matvec");
    static_assert(!AC || (LNP == 0 && !G), "the attention merge replaces the plain x");
    constexpr int RW = G ? 1 : MV_ROWS;  // output rows per wavefront pass
    extern __shared__ float xs[];
    __shared__ float red[2 * (NT / 64)];
    const int n_chunks = (f.nb + chunk_blocks - 1) / chunk_blocks;
    // chunked plain rows with slots: the workgroups past the tiles reduce
    constexpr bool CAN_HAND = LNP == 0 && !G && !PF && !AC;
    const bool hand = CAN_HAND && n_chunks > 1 && slots != nullptr;
    if constexpr (CAN_HAND) {
        const int n_work = (rows + tile_rows - 1) / tile_rows * n_chunks;
        if (hand && (int)blockIdx.x >= n_work) {
            mv_reduce<T>(w, stride, f, rows, chunk_blocks, n_chunks, x, act, y, slots,
                         (int)blockIdx.x - n_work, check);
            return;
        }
    }
    const int tile = blockIdx.x / n_chunks;
    const int ch = blockIdx.x % n_chunks;
    const int cb0 = ch * chunk_blocks;
    const int cnb = min(chunk_blocks, f.nb - cb0);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform per wavefront
    const int r_end = min(rows, (tile + 1) * tile_rows);
    const int r_first = tile * tile_rows + wave * RW;
    // The loads of a pass are all requested, then used; loads are never under
    // a per-lane condition (that serialises them): a slot past the pass
    // reloads the chunk's last block and drops it, a row past the end reloads
    // the last row.  The first loads are requested right after those of x (or
    // of the LayerNorm inputs), so x is staged while they are in flight.
    //
    // Two layouts of a pass over MV_ROWS rows x cnb blocks:
    // - pair (Q4_0, F16, F32): lane l takes blocks l, l + 64, l + 128 of both
    //   rows, so each x block read from LDS serves both dots;
    // - flat (Q8_0): slot k = kb + lane + 64 i is block k - cnb * q of row slot
    //   q = (k >= cnb), so a 142-block row pair takes 5 dots per lane rather
    //   than 3 x 2 with most lanes idle in the third.  It makes the Q8_0
    //   matvecs about 5% faster; Q4_0 loses 4% (its dot is VALU-heavy, and
    //   each flat dot reads its own x block) and F16 gains nothing.
    static_assert(MV_ROWS == 2, "a flat slot's row is k >= cnb");
    constexpr bool FLAT = T == LLG_TYPE_Q8_0;
    constexpr int NR = FLAT ? MV_NI : MV_BATCH * MV_ROWS;  // blocks loaded per lane per step
    BlockRaw<T> r[NR];
    // row slot q of the pass at r0: row r0 + q of w, or (gated) row r0 of gate / up
    auto row_ptr = [&](int r0_, int q) {
        if constexpr (G) return (q ? w2 : w) + (long long)min(r0_, r_end - 1) * stride;
        else return w + (long long)min(r0_ + q, r_end - 1) * stride;
    };
    const int n_slots = FLAT ? MV_ROWS * cnb : cnb;  // what the kb steps run over
    auto issue_to = [&](BlockRaw<T>(&dst)[NR], int r0_, int kb) {
        if constexpr (FLAT) {
            const uint8_t *p0 = row_ptr(r0_, 0), *p1 = row_ptr(r0_, 1);
#pragma unroll
            for (int i = 0; i < MV_NI; i++) {
                const int k = kb + lane + 64 * i;
                const bool q = k >= cnb;
                llg_block_load<T>(dst[i], q ? p1 : p0, f, cb0 + min(k - (q ? cnb : 0), cnb - 1));
            }
        } else {
#pragma unroll
            for (int i = 0; i < MV_BATCH; i++)
#pragma unroll
                for (int q = 0; q < MV_ROWS; q++)
                    llg_block_load<T>(dst[i * MV_ROWS + q], row_ptr(r0_, q), f,
                                      cb0 + min(kb + lane + 64 * i, cnb - 1));
        }
    };
    auto issue = [&](int r0_, int kb) { issue_to(r, r0_, kb); };
    // fold tasks of this wavefront: t0, t0 + fstep, ... < n_tasks
    const int n_tasks = PF ? pf.rank * pf.n_split : 0;
    const int fstep = gridDim.x * (int)(blockDim.x >> 6);
    const int ft0 = wave * gridDim.x + blockIdx.x;
    float4 pr[PF ? MV_PFL : 1];
    // float4 groups of chunk sp (0 for a chunk past the row's end)
    auto fold_nq = [&](int sp) { return max(0, min(pf.split_blocks, f.nb - sp * pf.split_blocks)) * 8; };
    auto fold_issue = [&](int t) {
        const int j = t / pf.n_split, sp = t % pf.n_split;
        const int nq = fold_nq(sp);
        const float4 *row = reinterpret_cast<const float4 *>(pf.p + (size_t)j * f.cols) +
                            (nq > 0 ? (size_t)sp * pf.split_blocks * 8 : 0);
#pragma unroll
        for (int k = 0; k < MV_PFL; k++) pr[k] = row[min(lane + 64 * k, max(nq, 1) - 1)];
    };
    auto issue_first = [&]() {
        // Every wavefront calls this once, right after requesting its staging
        // loads: the barrier (no wait on memory) puts the staging loads of the
        // whole workgroup ahead of any weight load.  A CU returns vector loads
        // in request order, so otherwise a wavefront's x (or LayerNorm inputs)
        // would arrive behind the weights of the wavefronts before it.
        // The fold task's loads go before the weights: the fold is computed
        // first, and its wait would otherwise cover every weight load.
        __builtin_amdgcn_s_barrier();
        if constexpr (PF)
            if (ft0 < n_tasks) fold_issue(ft0);
        issue(min(r_first, r_end - 1), 0);
    };
    if constexpr (LNP > 0)  // x is the LayerNorm of the residual sum (one chunk: cb0 = 0)
        llg_stage_ln<MV_XS, LNP>(xs, ln, red, issue_first);
    else if constexpr (AC)
        // Q8_0's 1024-thread instance has registers for one group per round
        llg_stage_attn<MV_XS, T == LLG_TYPE_Q8_0 ? 1 : 2>(xs, ap, cb0, cnb, issue_first);
    else
        llg_stage_x_sum<MV_XS, (MV_CHUNK * 8 + NT - 1) / NT>(xs, x + (size_t)cb0 * 32, cnb,
                                                             issue_first);
    __syncthreads();
    // the fold task t from pr (x staged)
    auto fold_dot = [&](int t) {
        if constexpr (PF) {
            const int j = t / pf.n_split, sp = t % pf.n_split;
            const int nq = fold_nq(sp);
            const float *xb = xs + (size_t)sp * pf.split_blocks * MV_XS;
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < MV_PFL; k++) {
                const int q = lane + 64 * k;
                if (q < nq) {
                    const float4 xv =
                        *reinterpret_cast<const float4 *>(xb + (q >> 3) * MV_XS + (q & 7) * 4);
                    acc += pr[k].x * xv.x;
                    acc += pr[k].y * xv.y;
                    acc += pr[k].z * xv.z;
                    acc += pr[k].w * xv.w;
                }
            }
            acc = llg_wave_sum(acc);
            if (lane == 0) pf.part[sp * pf.rank + j] = acc;
        }
    };
    // the first task's loads went out before the weights: its wait leaves them in flight
    if constexpr (PF)
        if (ft0 < n_tasks) fold_dot(ft0);
    // a wavefront's further fold tasks (more tasks than wavefronts), after its
    // rows: a load loop ahead of the dots would make them wait for every block
    auto fold_rest = [&]() {
        if constexpr (PF)
            for (int t = ft0 + fstep; t < n_tasks; t += fstep) {
                fold_issue(t);
                fold_dot(t);
            }
    };
    // the dots of one kb step of the pass at r0 from the blocks in src
    auto dots = [&](const BlockRaw<T>(&src)[NR], int kb, int r0, float(&sv)[MV_ROWS]) {
        if constexpr (FLAT) {
#pragma unroll
            for (int i = 0; i < MV_NI; i++) {
                const int k = kb + lane + 64 * i;
                if (k >= n_slots) continue;
                const bool q = k >= cnb;
                const float *xb = xs + (k - (q ? cnb : 0)) * MV_XS;
                const float d = llg_raw_dot<T>(src[i], reinterpret_cast<const float4 *>(xb), xb[32]);
                if (q)
                    sv[1] += d;
                else
                    sv[0] += d;
            }
        } else {
#pragma unroll
            for (int i = 0; i < MV_BATCH; i++) {
                const int bl = kb + lane + 64 * i;
                if (bl >= cnb) continue;
                const float *xb = xs + bl * MV_XS;
                const float4 *x4 = reinterpret_cast<const float4 *>(xb);
#pragma unroll
                for (int q = 0; q < MV_ROWS; q++)
                    if (r0 + (G ? 0 : q) < r_end)
                        sv[q] += llg_raw_dot<T>(src[i * MV_ROWS + q], x4, xb[32]);
            }
        }
    };
    // the row sums of the pass at r0: activation and store, or the chunk's partials
    auto finish = [&](float(&sv)[MV_ROWS], int r0) {
        if constexpr (G) {  // silu(gate) * up in fp32 (forward.go:370-383)
            const float g = llg_wave_sum(sv[0]), u = llg_wave_sum(sv[1]);
            if (lane == 0 && r0 < r_end) y[r0] = llg_act(LLG_ACT_SILU, g) * u;
            return;
        }
#pragma unroll
        for (int q = 0; q < MV_ROWS; q++) {
            const float v = llg_wave_sum(sv[q]);
            if (lane == 0 && r0 + q < r_end) {
                if (n_chunks == 1) {
                    const float o = act >= 0 ? llg_act(act, v) : v;
                    if constexpr (PF) pf.resid[r0 + q] = pf.resid[r0 + q] + o;  // x += attnOut
                    if (!PF || y) y[r0 + q] = o;
                } else if (hand) {
                    llg_slot_put(slots + (size_t)ch * rows + r0 + q, 1u, v);
                } else {
                    part[(size_t)ch * rows + r0 + q] = v;
                }
            }
        }
    };
    const int step = (int)(blockDim.x >> 6) * RW;
    constexpr int KSTEP = 64 * (FLAT ? MV_NI : MV_BATCH);
    if (n_slots <= KSTEP && r_first + step >= r_end) {
        // One pass of one step (every balanced launch), without the loops: at
        // a loop head the compiler waits for every outstanding load, so the
        // first dot would wait for the last block.  Here each dot waits for
        // its own blocks only.
        if (r_first < r_end) {
            float sv[MV_ROWS] = {0.0f, 0.0f};
            dots(r, 0, r_first, sv);
            finish(sv, r_first);
        }
        fold_rest();
        return;
    }
    for (int r0 = r_first; r0 < r_end; r0 += step) {
        float sv[MV_ROWS] = {0.0f, 0.0f};
        for (int kb = 0; kb < n_slots; kb += KSTEP) {
            if (r0 != r_first || kb != 0) issue(r0, kb);
            dots(r, kb, r0, sv);
        }
        finish(sv, r0);
    }
    fold_rest();
}

// y[r] = act(sum over the chunks c of part[c][r]), chunks in order.
__global__ void k_chunk_sum(const float *__restrict__ part, int n_chunks, int rows, int act,
                            float *__restrict__ y) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    float v = part[r];
    for (int c = 1; c < n_chunks; c++) v += part[(size_t)c * rows + r];
    y[r] = act >= 0 ? llg_act(act, v) : v;
}

// Floats of partial sums a matvec over w needs (0 when its rows fit one chunk).
static size_t mv_part_floats(const RowFmt &f, int rows, int act);

static int mv_chunk_blocks(const RowFmt &f, int act) {
    // An activation needs the whole row in one workgroup.
    if (act >= 0 || f.nb <= MV_CHUNK) return f.nb;
    const int n_chunks = (f.nb + MV_CHUNK - 1) / MV_CHUNK;
    return (f.nb + n_chunks - 1) / n_chunks;
}

static size_t mv_part_floats(const RowFmt &f, int rows, int act) {
    const int cb = mv_chunk_blocks(f, act);
    const int n_chunks = (f.nb + cb - 1) / cb;
    return n_chunks > 1 ? (size_t)n_chunks * rows : 0;
}

// part: room for mv_part_floats (the partial sums of a chunked matvec).
// ln (optional): the staged x is the LayerNorm of a residual sum (llg_stage_ln).
// up (optional): gated rows, y = silu(w . x) * (up . x) (act is ignored).
// Launch parameters of one k_matvec_q call.
struct MvArgs {
    dim3 grid;
    int threads;
    size_t lds;
    hipStream_t st;
    const LlgObject *w;
    int tile_rows, cb;
    const float *x;
    int act;
    float *y, *part;
    LlgLnArgs ln;
    const uint8_t *w2;
    LlgPredFold pf;
    LlgAttnParts ap;
    uint64_t *slots;  // chunked rows reduced in the launch (llg_dev_mvslots)
    int check;        // llg_dev_check
};

template <int T, int LNP, bool G, int NT, bool PF, bool AC>
static void mv_go(const MvArgs &a) {
    hipLaunchKernelGGL((k_matvec_q<T, LNP, G, NT, PF, AC>), a.grid, dim3(a.threads), a.lds, a.st,
                       a.w->d, a.w->stride, a.w->fmt, a.w->rows, a.tile_rows, a.cb, a.x, a.act,
                       a.y, a.part, a.ln, a.w2, a.pf, a.ap, a.slots, a.check);
}

// Instances with NT = 1024 workgroups (the balanced launch) exist for the
// types whose blocks fit the 128 registers of a 16-wavefront workgroup:
// Q4_0 with up to 4 LayerNorm groups per thread, Q8_0 with up to 2.
template <int T>
constexpr int mv_bal_lnp() {
    return T == LLG_TYPE_Q4_0 ? 4 : T == LLG_TYPE_Q8_0 ? 2 : -1;
}

template <int T, int NT, int LNP>
static void mv_plain(const MvArgs &a, bool pf, bool ac) {
    if constexpr (LNP > 0) {
        mv_go<T, LNP, false, NT, false, false>(a);
    } else {
        if (pf && ac) mv_go<T, 0, false, NT, true, true>(a);
        else if (pf) mv_go<T, 0, false, NT, true, false>(a);
        else if (ac) mv_go<T, 0, false, NT, false, true>(a);
        else mv_go<T, 0, false, NT, false, false>(a);
    }
}

template <int T>
static void mv_dispatch(const MvArgs &a, bool bal, bool gated, bool pf, bool ac, int lnp) {
    if (gated) return mv_go<T, 0, true, 256, false, false>(a);
    if constexpr (mv_bal_lnp<T>() >= 0) {
        if (bal) {
            if (lnp == 0) mv_plain<T, 1024, 0>(a, pf, ac);
            else if (lnp <= 2) mv_plain<T, 1024, 2>(a, pf, ac);
            else if constexpr (mv_bal_lnp<T>() >= 4) mv_plain<T, 1024, 4>(a, pf, ac);
            return;
        }
    }
    if (lnp == 0) mv_plain<T, 256, 0>(a, pf, ac);
    else if (lnp <= 2) mv_plain<T, 256, 2>(a, pf, ac);
    else if (lnp <= 4) mv_plain<T, 256, 4>(a, pf, ac);
    else if (lnp <= 5) mv_plain<T, 256, 5>(a, pf, ac);
    else if (lnp <= 8) mv_plain<T, 256, 8>(a, pf, ac);
    else mv_plain<T, 256, 16>(a, pf, ac);
}

static int mv_bal_lnp_rt(int type) {
    switch (type) {
    case LLG_TYPE_Q4_0: return mv_bal_lnp<LLG_TYPE_Q4_0>();
    case LLG_TYPE_Q8_0: return mv_bal_lnp<LLG_TYPE_Q8_0>();
    default: return -1;
    }
}

// pf (optional): the predictor fold (whole rows in one workgroup, no LayerNorm).
// ap (optional): x is the attention output in split form (d_x unused).
static int matvec_launch(LlgDevice *d, const LlgObject *w, const float *d_x, int act, float *d_y,
                         float *part, const LlgLnArgs *ln = nullptr,
                         const LlgObject *up = nullptr, const LlgPredFold *pf = nullptr,
                         const LlgAttnParts *ap = nullptr) {
    const RowFmt &f = w->fmt;
    if (up) act = LLG_ACT_SILU;  // whole rows in one workgroup
    const int cb = ln ? f.nb : mv_chunk_blocks(f, act);
    const int n_chunks = (f.nb + cb - 1) / cb;
    const size_t lds = (size_t)cb * MV_XS * 4;
    if (lds > 160 * 1024)
        return llg_set_error(d, LLG_E_ARG, "matvec: row of %d elements too long", f.cols);
    // chunked plain rows (k_matvec_q's CAN_HAND instances): reduced in the
    // launch through slots; the attention-merge instance, or more than
    // MV_HAND_MAX chunks: k_chunk_sum from part
    const bool hand = n_chunks > 1 && n_chunks <= MV_HAND_MAX && !ln && !up && !pf && !ap;
    if (n_chunks > 1 && !hand && !part)
        return llg_set_error(d, LLG_E_ARG, "matvec: chunked rows need a partial buffer");
    if (pf && (n_chunks > 1 || ln || up || act >= 0 || pf->n_split < 1 ||
               pf->split_blocks * 8 > 64 * MV_PFL ||
               (long long)pf->split_blocks * pf->n_split < f.nb))
        return llg_set_error(d, LLG_E_ARG, "matvec: predictor fold needs whole plain rows");
    if (ap && (ln || up || ap->n_split < 1 || ap->n_split > LLG_ATTN_SPLIT_MAX ||
               ap->n_heads * ap->head_dim != f.cols || ap->head_dim % 4))
        return llg_set_error(d, LLG_E_ARG, "matvec: attention parts do not match the rows");
    MvArgs a;
    a.st = llg_dev_stream(d);
    a.w = w;
    a.cb = cb;
    a.lds = lds;
    a.x = d_x;
    a.act = act;
    a.y = d_y;
    a.part = part;
    a.ln = ln ? *ln : LlgLnArgs{};
    a.w2 = up ? up->d : nullptr;
    a.pf = pf ? *pf : LlgPredFold{};
    a.ap = ap ? *ap : LlgAttnParts{};
    a.slots = nullptr;
    a.check = llg_dev_check(d);
    if (hand) {
        int rc = 0;
        a.slots = llg_dev_mvslots(d, (size_t)n_chunks * w->rows * 8, &rc);
        if (rc) return rc;
    }
    // Rows per workgroup: one pass per wavefront (8 rows) gives the most
    // loads in flight; very tall matrices take 16 or 32 rows so that the grid
    // stays within MV_MAX_WG workgroups (an 18176-row Q4_0 matvec: 13.6 us at
    // 8 rows, 15.2 at 16, 16.8 at 32; 65024 rows: 36.0 at 8, 36.2 at 16).
    int tr = MV_TILE_SMALL;
    while (tr < 32 && (long long)(w->rows + tr - 1) / tr * n_chunks > MV_MAX_WG) tr *= 2;
    a.tile_rows = tr / (up ? 2 : 1);
    a.threads = 256;
    int lnp = ln ? (ln->n / 4 + a.threads - 1) / a.threads : 0;
    // Balanced: a matrix of MV_BAL_MIN..MV_SMALL_ROWS whole rows goes to at
    // most one workgroup per CU, each a single pass of MV_ROWS rows per
    // wavefront, so x (or the LayerNorm inputs) is staged once per CU rather
    // than by two or three workgroups of 8 rows.
    bool bal = false;
    if (!up && n_chunks == 1 && w->rows >= MV_BAL_MIN && w->rows < MV_SMALL_ROWS) {
        const int cus = llg_cu_count(d);
        const int rpw = MV_ROWS * ((w->rows + MV_ROWS * cus - 1) / (MV_ROWS * cus));
        const int th = 64 * (rpw / MV_ROWS);
        const int lnp_b = ln ? (ln->n / 4 + th - 1) / th : 0;
        if (th >= 256 && th <= 1024 && lnp_b <= mv_bal_lnp_rt(f.type)) {
            bal = true;
            a.tile_rows = rpw;
            a.threads = th;
            lnp = lnp_b;
        }
    }
    a.grid = dim3((w->rows + a.tile_rows - 1) / a.tile_rows * n_chunks +
                  (hand ? (w->rows + a.threads - 1) / a.threads : 0));
    switch (f.type) {
    case LLG_TYPE_Q4_0:
        mv_dispatch<LLG_TYPE_Q4_0>(a, bal, up != nullptr, pf != nullptr, ap != nullptr, lnp);
        break;
    case LLG_TYPE_Q8_0:
        mv_dispatch<LLG_TYPE_Q8_0>(a, bal, up != nullptr, pf != nullptr, ap != nullptr, lnp);
        break;
    case LLG_TYPE_F16:
        mv_dispatch<LLG_TYPE_F16>(a, bal, up != nullptr, pf != nullptr, ap != nullptr, lnp);
        break;
    case LLG_TYPE_F32:
        mv_dispatch<LLG_TYPE_F32>(a, bal, up != nullptr, pf != nullptr, ap != nullptr, lnp);
        break;
    default:
        return llg_set_error(d, LLG_E_TYPE, "matvec: unsupported type %d", f.type);
    }
    LLG_LAUNCH_CHECK(d, "matvec_q");
    if (n_chunks > 1 && !hand) {
        hipLaunchKernelGGL(k_chunk_sum, dim3((w->rows + 255) / 256), dim3(256), 0, a.st,
                           (const float *)part, n_chunks, w->rows, act, d_y);
        LLG_LAUNCH_CHECK(d, "matvec chunk sum");
    }
    return 0;
}

int llg_matvec_ln_enqueue(LlgDevice *d, const LlgObject *w, const LlgLnArgs &ln, float *d_y) {
    if (ln.n != w->fmt.cols)
        return llg_set_error(d, LLG_E_ARG, "matvec: LayerNorm length %d != %d", ln.n, w->fmt.cols);
    if (ln.n > 256 * 16 * 4)
        return llg_set_error(d, LLG_E_ARG, "matvec: LayerNorm length %d above 16384", ln.n);
    if (ln.stats && (ln.a1 || ln.a2 || ln.n % 32 || ln.n > 32 * 64 * LLG_LN_STATS_PER))
        return llg_set_error(d, LLG_E_ARG, "matvec: block statistics for a LayerNorm of %d", ln.n);
    return matvec_launch(d, w, nullptr, -1, d_y, nullptr, &ln);
}

int llg_matvec_enqueue(LlgDevice *d, const LlgObject *w, const float *d_x, int act, float *d_y,
                       float *part) {
    return matvec_launch(d, w, d_x, act, d_y, part);
}

bool llg_matvec_fold_ok(const LlgObject *w) { return mv_chunk_blocks(w->fmt, -1) == w->fmt.nb; }

int llg_matvec_attn_enqueue(LlgDevice *d, const LlgObject *w, const LlgAttnParts &ap, float *d_y,
                            float *part, const LlgPredFold *pf) {
    return matvec_launch(d, w, nullptr, -1, d_y, part, nullptr, nullptr, pf, &ap);
}

size_t llg_matvec_part_bytes(const LlgObject *w, int act) {
    return mv_part_floats(w->fmt, w->rows, act) * 4;
}

// Workspace of the dense FFN: the hidden row (ff floats), then the down
// matvec's partial sums.
static size_t dense_ws_bytes(const LlgObject *up, const LlgObject *down) {
    return (size_t)llg_align((long long)up->rows * 4, 256) + llg_matvec_part_bytes(down, -1);
}

// Dense FFN: hid = act(up . x) (whole rows), then out = down . hid.
static int dense_enqueue(LlgDevice *d, const LlgObject *up, const LlgObject *down,
                         const float *d_x, int act, uint8_t *ws, float *d_out) {
    if (int rc = llg_check_act(d, act)) return rc;
    float *hid = reinterpret_cast<float *>(ws);
    float *part = reinterpret_cast<float *>(ws + llg_align((long long)up->rows * 4, 256));
    int rc = matvec_launch(d, up, d_x, act, hid, nullptr);
    if (rc) return rc;
    return matvec_launch(d, down, hid, -1, d_out, part);
}

// SwiGLU dense FFN (forward.go:368-389): hid = silu(gate . x) * (up . x),
// then out = down . hid.
static int swiglu_enqueue(LlgDevice *d, const LlgObject *gate, const LlgObject *up,
                          const LlgObject *down, const float *d_x, uint8_t *ws, float *d_out) {
    float *hid = reinterpret_cast<float *>(ws);
    float *part = reinterpret_cast<float *>(ws + llg_align((long long)up->rows * 4, 256));
    int rc = matvec_launch(d, gate, d_x, LLG_ACT_SILU, hid, nullptr, nullptr, up);
    if (rc) return rc;
    return matvec_launch(d, down, hid, -1, d_out, part);
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
                              b->rows, b->rows, act, d_out, ws);
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
    if ((rc = llg_check_act(d, act))) return rc;
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
                            b->rows, act, (float *)(ws + o_out), ws + o_ws);
    if (rc) return rc;
    if ((rc = llg_d2h(d, out, ws + o_out, (size_t)hd * 4))) return rc;
    return llg_sync_dev(d);
}

static int check_fused(LlgDevice *d, int64_t hwup, int64_t hwout, int64_t hbias, int64_t hb,
                       LlgObject **wup, LlgObject **wout, LlgObject **bias, LlgObject **b) {
    int rc = llg_check_predictor(d, hwup, hwout, hbias, wup, wout, bias);
    if (rc) return rc;
    if ((rc = check_bundle(d, hb, b))) return rc;
    if ((*wout)->rows != (*b)->rows || (*wup)->fmt.cols != (*b)->fmt.cols)
        return llg_set_error(d, LLG_E_ARG, "predict_sparse: predictor/bundle shape mismatch");
    return 0;
}

int llg_hipd_ffn_predict_sparse(LlgHipDevice h, int64_t hwup, int64_t hwout, int64_t hbias,
                                int64_t hb, const float *d_a, const float *d_x, float thr,
                                int act, float *d_out, int32_t *d_active, int32_t *d_n_active) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *wup, *wout, *bias, *b;
    int rc = check_fused(d, hwup, hwout, hbias, hb, &wup, &wout, &bias, &b);
    if (rc) return rc;
    if (!d_a || !d_x || !d_out) return llg_set_error(d, LLG_E_ARG, "predict_sparse: null pointer");
    uint8_t *ws = (uint8_t *)llg_ws(d, llg_fused_ws_bytes(wup->rows, wout->rows, b->fmt.nb), &rc);
    if (rc) return rc;
    uint8_t *sync = llg_dev_sync(d, &rc);
    if (rc) return rc;
    return llg_fused_enqueue(d, wup, wout, bias, b, d_a, d_x, thr, act, d_out, d_active,
                             d_n_active, ws, sync);
}

// The same path with its workspace in the GPU's fixed scratch array: no
// allocation.  The scratch starts with the sync area (zero when the library
// loads; its slots carry an epoch, so it is never cleared), then the
// workspace, whose every slot the kernels read is written earlier in the
// same call.
int llg_hipd_ffn_predict_sparse_noalloc(LlgHipDevice h, int64_t hwup, int64_t hwout,
                                        int64_t hbias, int64_t hb, const float *d_a,
                                        const float *d_x, float thr, int act, float *d_out,
                                        int32_t *d_active, int32_t *d_n_active) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *wup, *wout, *bias, *b;
    int rc = check_fused(d, hwup, hwout, hbias, hb, &wup, &wout, &bias, &b);
    if (rc) return rc;
    if (!d_a || !d_x || !d_out) return llg_set_error(d, LLG_E_ARG, "predict_sparse: null pointer");
    uint8_t *sync = llg_dev_scratch(
        d, LLG_SYNC_BYTES + llg_fused_ws_bytes(wup->rows, wout->rows, b->fmt.nb), &rc);
    if (!sync) return rc;
    return llg_fused_enqueue(d, wup, wout, bias, b, d_a, d_x, thr, act, d_out, d_active,
                             d_n_active, sync + LLG_SYNC_BYTES, sync);
}

int llg_hip_ffn_predict_sparse(LlgHipDevice h, int64_t hwup, int64_t hwout, int64_t hbias,
                               int64_t hb, const float *a, const float *x, float thr, int act,
                               float *out, int32_t *active, int *n_active) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *wup, *wout, *bias, *b;
    int rc = check_fused(d, hwup, hwout, hbias, hb, &wup, &wout, &bias, &b);
    if (rc) return rc;
    if (!a || !x || !out) return llg_set_error(d, LLG_E_ARG, "predict_sparse: null pointer");
    const int hd = b->fmt.cols, ff = b->rows;
    const long long o_a = 0;
    const long long o_x = llg_align((long long)hd * 4, 256);
    const long long o_out = o_x + llg_align((long long)hd * 4, 256);
    const long long o_act = o_out + llg_align((long long)hd * 4, 256);
    const long long o_n = o_act + llg_align((long long)ff * 4, 256);
    const long long o_ws = o_n + 256;
    uint8_t *ws = (uint8_t *)llg_ws(d, o_ws + llg_fused_ws_bytes(wup->rows, ff, b->fmt.nb), &rc);
    if (rc) return rc;
    uint8_t *sync = llg_dev_sync(d, &rc);
    if (rc) return rc;
    if ((rc = llg_h2d(d, ws + o_a, a, (size_t)hd * 4))) return rc;
    if ((rc = llg_h2d(d, ws + o_x, x, (size_t)hd * 4))) return rc;
    rc = llg_fused_enqueue(d, wup, wout, bias, b, (const float *)(ws + o_a),
                           (const float *)(ws + o_x), thr, act, (float *)(ws + o_out),
                           active ? (int32_t *)(ws + o_act) : nullptr, (int32_t *)(ws + o_n),
                           ws + o_ws, sync);
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
    int rc2;
    float *part = nullptr;
    if (const size_t pb = llg_matvec_part_bytes(w, -1)) {
        part = (float *)llg_ws(d, pb, &rc2);
        if (rc2) return rc2;
    }
    return llg_matvec_enqueue(d, w, d_x, -1, d_y, part);
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
    const long long o_p = o_y + llg_align((long long)w->rows * 4, 256);
    uint8_t *ws = (uint8_t *)llg_ws(d, o_p + llg_matvec_part_bytes(w, -1), &rc);
    if (rc) return rc;
    if ((rc = llg_h2d(d, ws, x, (size_t)w->fmt.cols * 4))) return rc;
    if ((rc = llg_matvec_enqueue(d, w, (const float *)ws, -1, (float *)(ws + o_y),
                                 (float *)(ws + o_p))))
        return rc;
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
    uint8_t *ws = (uint8_t *)llg_ws(d, dense_ws_bytes(up, down), &rc);
    if (rc) return rc;
    return dense_enqueue(d, up, down, d_x, act, ws, d_out);
}

int llg_hip_ffn_dense(LlgHipDevice h, int64_t hu, int64_t hdn, const float *x, int act,
                      float *out) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *up, *down;
    int rc = check_dense(d, hu, hdn, &up, &down);
    if (rc) return rc;
    if (!x || !out) return llg_set_error(d, LLG_E_ARG, "ffn_dense: null pointer");
    const int hd = up->fmt.cols;
    const long long o_out = llg_align((long long)hd * 4, 256);
    const long long o_h = o_out + llg_align((long long)hd * 4, 256);
    uint8_t *ws = (uint8_t *)llg_ws(d, o_h + dense_ws_bytes(up, down), &rc);
    if (rc) return rc;
    if ((rc = llg_h2d(d, ws, x, (size_t)hd * 4))) return rc;
    if ((rc = dense_enqueue(d, up, down, (const float *)ws, act, ws + o_h,
                            (float *)(ws + o_out))))
        return rc;
    if ((rc = llg_d2h(d, out, ws + o_out, (size_t)hd * 4))) return rc;
    return llg_sync_dev(d);
}

static int check_swiglu(LlgDevice *d, int64_t hg, int64_t hu, int64_t hdn, LlgObject **gate,
                        LlgObject **up, LlgObject **down) {
    int rc = check_dense(d, hu, hdn, up, down);
    if (rc) return rc;
    *gate = llg_get(d, hg, LLG_KIND_MATRIX);
    if (!*gate) return llg_set_error(d, LLG_E_HANDLE, "ffn_swiglu: unknown gate handle");
    if ((*gate)->rows != (*up)->rows || (*gate)->fmt.cols != (*up)->fmt.cols ||
        (*gate)->fmt.type != (*up)->fmt.type || (*gate)->stride != (*up)->stride)
        return llg_set_error(d, LLG_E_ARG, "ffn_swiglu: gate [%d x %d] differs from up [%d x %d]",
                             (*gate)->rows, (*gate)->fmt.cols, (*up)->rows, (*up)->fmt.cols);
    return 0;
}

int llg_hipd_ffn_swiglu(LlgHipDevice h, int64_t hg, int64_t hu, int64_t hdn, const float *d_x,
                        float *d_out) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *gate, *up, *down;
    int rc = check_swiglu(d, hg, hu, hdn, &gate, &up, &down);
    if (rc) return rc;
    if (!d_x || !d_out) return llg_set_error(d, LLG_E_ARG, "ffn_swiglu: null pointer");
    uint8_t *ws = (uint8_t *)llg_ws(d, dense_ws_bytes(up, down), &rc);
    if (rc) return rc;
    return swiglu_enqueue(d, gate, up, down, d_x, ws, d_out);
}

int llg_hip_ffn_swiglu(LlgHipDevice h, int64_t hg, int64_t hu, int64_t hdn, const float *x,
                       float *out) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *gate, *up, *down;
    int rc = check_swiglu(d, hg, hu, hdn, &gate, &up, &down);
    if (rc) return rc;
    if (!x || !out) return llg_set_error(d, LLG_E_ARG, "ffn_swiglu: null pointer");
    const int hd = up->fmt.cols;
    const long long o_out = llg_align((long long)hd * 4, 256);
    const long long o_h = o_out + llg_align((long long)hd * 4, 256);
    uint8_t *ws = (uint8_t *)llg_ws(d, o_h + dense_ws_bytes(up, down), &rc);
    if (rc) return rc;
    if ((rc = llg_h2d(d, ws, x, (size_t)hd * 4))) return rc;
    if ((rc = swiglu_enqueue(d, gate, up, down, (const float *)ws, ws + o_h,
                             (float *)(ws + o_out))))
        return rc;
    if ((rc = llg_d2h(d, out, ws + o_out, (size_t)hd * 4))) return rc;
    return llg_sync_dev(d);
}

}  // extern "C"
