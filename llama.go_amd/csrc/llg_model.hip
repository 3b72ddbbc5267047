// llg_model.hip -- Falcon-architecture decode around the sparse FFN
// (inference/ffn_flash.go:115-185 ForwardFlash, inference/forward.go:106-314,
// kvcache/kvcache.go:25-82, cmd/generate.go:88-121).
//
// One token through the model, all on the device stream.  The residual
// stream lives in one buffer r:
//   k_embed           r = dequant(embedding row of the token)    (forward.go:449-454)
//   per layer l:
//     k_matvec_q      qkv = [Wq; Wk; Wv] . normed (forward.go:211-222), where
//                     every workgroup first forms normed = LayerNorm(r)
//                     (tensor/ops.go:138-165) itself (llg_stage_ln)
//     k_attn          NeoX RoPE of q and k (forward.go:483-497), K/V appended at
//                     row pos of the layer's cache (kvcache.go:42-52), softmax
//                     attention of every query head over rows 0..pos of its KV
//                     head (forward.go:258-301), split over workgroups by rows;
//                     each split also forms P . acc for its head, P = WUp . Wo
//                     formed once at load (below)
//     k_tile_wo_ffn   its first workgroups merge those products over the splits
//                     and heads into the predictor's hidden units, handed to
//                     the tile workgroups inside the launch; the tiles: ffnFlash
//                     path 2 (ffn_flash.go:157-163, 225-231), logits from the
//                     hidden units, the active up rows on normed, partial down
//                     sums; its last workgroups: attn_out = Wo . attn (forward.
//                     go:305), added into r (x += attnOut, ffn_flash.go:161)
//     k_tile_reduce   the down sums added into r (x += ffnOut, :164-166), so r
//                     ends as the next layer's residual
//
// The predictor fold.  The reference's predictor input is attn_out = Wo .
// attn, and its first product WUp . attn_out (predictor.go:57) is linear in
// attn, so it equals P . attn with P = WUp . Wo ([rank x n_heads head_dim]).
// k_fold_pred forms P once per layer at load, in fp64 sums rounded once to
// f32.  The attention splits apply P to their unnormalised outputs and the
// tile launch merges the products as the splits merge, so the hidden units
// need neither attn_out nor the merged attn, which removes a launch and two
// dependent reads per layer.  The hidden values differ from WUp . attn_out by
// fp32 rounding only (a few ulps).  A model whose Wo is not Q4_0/Q8_0 or
// whose head size is not a multiple of 8 keeps Wo (with the fold) as its own
// launch before the tile launch, and one whose Wo rows are too long for one
// workgroup's staged x also keeps the separate hidden kernel on attn_out.
//   k_out_norm        output LayerNorm of r from its block     (ffn_flash.go:126-129)
//                     statistics (k_resid_norm without them)
//   k_matvec_q        logits = LMHead . normed                 (ffn_flash.go:130)
//   k_argmax          next token = first index of the maximum  (generate.go:197-205)
// The token comes from device memory, so a greedy decode loop never waits on
// the host.
#include <algorithm>
#include <vector>

#include "llg_common.hpp"
#include "llg_internal.hpp"

#define NORM_THREADS 1024
#define ATTN_THREADS 1024

struct LlgModelLayer {
    LlgObject *norm_w, *norm_b, *wqkv, *wo, *pwup, *pwout, *bundle;
    float thr;
    float *pfold;  // P = WUp . Wo [rank x n_heads head_dim], or null (no fold)
};

struct LlgModel {
    int n_layers, hidden, n_heads, n_kv, head_dim, ff, vocab, max_seq, rank, act;
    int cus;  // compute units of the device
    float rope_base, eps;
    LlgObject *embed, *out_w, *out_b, *lm_head;
    std::vector<LlgModelLayer> layers;
    // device buffers, carved out of the object's allocation
    float *x, *normed, *qkv, *attn, *attn_out, *logits, *kv, *pred_logits;  // x: the residual
    float *mvpart;  // partial sums of a column-chunked Wo or LM-head matvec
    float *attn_ml;  // attention splits' (max, sum); attn holds their acc rows
    float2 *rope;  // [max_seq x head_dim/2] (cos, sin)
    // per 32 elements of x, (sum, M2) as the kernel that last wrote x left them
    // (k_embed, then each layer's partial-sum kernel), for the next QKV
    // LayerNorm prologue; null when hidden is not a multiple of 32 or above
    // what the prologue merges per wavefront
    float2 *rstats;
    int32_t *token, *n_active, *act_scratch;
    uint8_t *ws;
    // the device's sync area when every layer runs Wo and the predictor fold
    // inside its tile launch (llg_fused_wo_enqueue), else null
    uint8_t *sync;
    // with sync: the attention splits' predictor products [split][head][rank]
    float *pd;
};

// The objects a model reads, each once per use (llg_ref / llg_unref pairs).
template <class F>
static void model_objects(LlgModel *m, F &&f) {
    f(m->embed);
    f(m->lm_head);
    f(m->out_w);
    f(m->out_b);
    for (LlgModelLayer &L : m->layers)
        for (LlgObject *o : {L.norm_w, L.norm_b, L.wqkv, L.wo, L.pwup, L.pwout, L.bundle}) f(o);
}

void llg_model_destroy(LlgDevice *d, LlgObject *o) {
    LlgModel *m = reinterpret_cast<LlgModel *>(o->ext);
    if (!m) return;
    model_objects(m, [&](LlgObject *x) { llg_unref(d, x); });
    delete m;
    o->ext = nullptr;
}

// ---------------------------------------------------------------------------
// x = dequant(embedding row of the token), 4 elements per thread; with stats
// (cols a multiple of 32) also each 32-element block's (sum, M2), from the 8
// lanes that hold it.
#define EMBED_THREADS 256
__global__ __launch_bounds__(EMBED_THREADS) void k_embed(
    const uint8_t *__restrict__ emb, long long stride, RowFmt f,
    const int32_t *__restrict__ token, int vocab, float *__restrict__ x,
    float2 *__restrict__ stats) {
    // a token id outside the table would be a slice-bounds panic in the
    // reference; the host entry points reject it, the device loop only feeds
    // argmax results (< vocab)
    const int t = min(max(*token, 0), vocab - 1);
    const uint8_t *row = emb + (long long)t * stride;
    const int c0 = 4 * (blockIdx.x * EMBED_THREADS + threadIdx.x);
    float e[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        e[k] = c0 + k < f.cols ? llg_dequant_elem(row, f, c0 + k) : 0.0f;
        if (c0 + k < f.cols) x[c0 + k] = e[k];
    }
    if (stats) {  // uniform: every lane takes part in the block sums
        const float2 bs = llg_block32_stats(make_float4(e[0], e[1], e[2], e[3]));
        if ((threadIdx.x & 7) == 0 && c0 < f.cols) stats[c0 >> 5] = bs;
    }
}


// x = (x + a1) + a2 (either may be null); out = LayerNorm(x) * w + b.  Each
// thread keeps NP elements in registers (hidden <= NORM_THREADS * NP); all
// loads of a thread are issued together.
#define NORM_PER 16  // largest NP instantiated
template <int NP>
__global__ __launch_bounds__(NORM_THREADS) void k_resid_norm(
    float *__restrict__ x, const float *__restrict__ a1, const float *__restrict__ a2,
    const float *__restrict__ w, const float *__restrict__ b, int n, float eps,
    float *__restrict__ out) {
    __shared__ float red[NORM_THREADS / 64];
    float v[NP], p1[NP], p2[NP];
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < NP; k++) {
        const int i = min(tid + k * NORM_THREADS, n - 1);
        v[k] = x[i];
        p1[k] = a1 ? a1[i] : 0.0f;
        p2[k] = a2 ? a2[i] : 0.0f;
    }
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NP; k++) {
        const int i = tid + k * NORM_THREADS;
        if (a1) v[k] = v[k] + p1[k];
        if (a2) v[k] = v[k] + p2[k];
        if (i < n) {
            if (a1 || a2) x[i] = v[k];
            s += v[k];
        }
    }
    const float mean = llg_block_sum(s, red) / (float)n;
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < NP; k++) {
        const float dv = v[k] - mean;
        if (tid + k * NORM_THREADS < n) q += dv * dv;
    }
    const float var = llg_block_sum(q, red) / (float)n;
    const float std_ = (float)sqrt((double)var + (double)eps);  // ops.go:159
#pragma unroll
    for (int k = 0; k < NP; k++) {
        const int i = tid + k * NORM_THREADS;
        if (i < n) out[i] = (v[k] - mean) / std_ * w[i] + b[i];
    }
}

// The output LayerNorm of r (ffn_flash.go:126-129) from r's block
// statistics (each 32-element block's (sum, M2), left by the last layer's
// k_tile_reduce), merged as in the QKV prologue (llg_stage_ln): every
// wavefront merges the pairs in the same order, so no workgroup reduction is
// needed and the row is spread over several workgroups, one float4 group per
// thread.  n: a multiple of 32, at most 32 * 64 * LLG_LN_STATS_PER.
#define ONORM_THREADS 256
__global__ __launch_bounds__(ONORM_THREADS) void k_out_norm(const float *__restrict__ x,
                                                            const float2 *__restrict__ stats,
                                                            const float *__restrict__ w,
                                                            const float *__restrict__ b, int n,
                                                            float eps, float *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int nbk = n / 32, n4 = n / 4;
    const int g = blockIdx.x * ONORM_THREADS + threadIdx.x;
    const int i = min(g, n4 - 1);
    const float4 v = reinterpret_cast<const float4 *>(x)[i];
    const float4 wv = reinterpret_cast<const float4 *>(w)[i];
    const float4 bv = reinterpret_cast<const float4 *>(b)[i];
    float2 st[LLG_LN_STATS_PER];
#pragma unroll
    for (int k = 0; k < LLG_LN_STATS_PER; k++) st[k] = stats[min(lane + 64 * k, nbk - 1)];
    float sm = 0.0f;
#pragma unroll
    for (int k = 0; k < LLG_LN_STATS_PER; k++)
        if (lane + 64 * k < nbk) sm += st[k].x;
    const float mean = llg_wave_sum(sm) / (float)n;
    float m2 = 0.0f;
#pragma unroll
    for (int k = 0; k < LLG_LN_STATS_PER; k++)
        if (lane + 64 * k < nbk) {
            const float d = st[k].x / 32.0f - mean;
            m2 += st[k].y + 32.0f * d * d;
        }
    const float var = llg_wave_sum(m2) / (float)n;
    const float std_ = (float)sqrt((double)var + (double)eps);  // ops.go:159
    if (g < n4)
        reinterpret_cast<float4 *>(out)[i] =
            make_float4((v.x - mean) / std_ * wv.x + bv.x, (v.y - mean) / std_ * wv.y + bv.y,
                        (v.z - mean) / std_ * wv.z + bv.z, (v.w - mean) / std_ * wv.w + bv.w);
}

// Sum over each 16-lane row (all lanes of the row get the total).
__device__ __forceinline__ float row16_sum(float v) {
    v = llg_quad_sum(v);
    v += llg_dpp<0x124>(v);  // row_ror:4
    v += llg_dpp<0x128>(v);  // row_ror:8
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// RoPE angles of every position (forward.go:487-489): freq = pos / base^(2i/hd)
// in double, cos and sin rounded to float.  Built once per model, so the
// attention kernel reads two floats where it would evaluate pow/cos/sin.  A
// base <= 0 means no RoPE (forward.go:249): the table holds the identity
// rotation (cos 1, sin 0).
__global__ void k_rope_table(float2 *__restrict__ tab, int max_seq, int half, float base) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= max_seq * half) return;
    if (!(base > 0.0f)) {
        tab[j] = make_float2(1.0f, 0.0f);
        return;
    }
    const int pos = j / half, i = j % half;
    const double fr = (double)pos / pow((double)base, (double)(2 * i) / (double)(2 * half));
    tab[j] = make_float2((float)cos(fr), (float)sin(fr));
}

// P = WUp . dequant(Wo) of one layer: [rank x hidden] . [hidden x cols], fp64
// sums rounded once to f32.  32 x 32 output tiles through LDS, 256 threads of
// 2 x 2 outputs each.  Runs once per layer at load.
#define FOLD_T 32
__global__ __launch_bounds__(256) void k_fold_pred(const uint8_t *__restrict__ wup,
                                                   long long wup_stride, int rank, int hidden,
                                                   const uint8_t *__restrict__ wo,
                                                   long long wo_stride, RowFmt wf,
                                                   float *__restrict__ pf) {
    __shared__ double a[FOLD_T][FOLD_T + 1], b[FOLD_T][FOLD_T + 1];
    const int cols = wf.cols;
    const int j0 = blockIdx.y * FOLD_T, c0 = blockIdx.x * FOLD_T;
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    double acc[2][2] = {{0.0, 0.0}, {0.0, 0.0}};
    for (int k0 = 0; k0 < hidden; k0 += FOLD_T) {
        for (int i = threadIdx.x; i < FOLD_T * FOLD_T; i += 256) {
            const int r = i / FOLD_T, q = i % FOLD_T;
            const int j = j0 + r, k = k0 + q;
            a[r][q] = j < rank && k < hidden
                          ? (double)reinterpret_cast<const float *>(wup + (long long)j * wup_stride)[k]
                          : 0.0;
            const int kk = k0 + r, c = c0 + q;
            b[r][q] = kk < hidden && c < cols
                          ? (double)llg_dequant_elem(wo + (long long)kk * wo_stride, wf, c)
                          : 0.0;
        }
        __syncthreads();
        for (int k = 0; k < FOLD_T; k++) {
            const double a0 = a[2 * ty][k], a1 = a[2 * ty + 1][k];
            const double b0 = b[k][2 * tx], b1 = b[k][2 * tx + 1];
            acc[0][0] += a0 * b0;
            acc[0][1] += a0 * b1;
            acc[1][0] += a1 * b0;
            acc[1][1] += a1 * b1;
        }
        __syncthreads();
    }
    for (int u = 0; u < 2; u++)
        for (int v = 0; v < 2; v++) {
            const int j = j0 + 2 * ty + u, c = c0 + 2 * tx + v;
            if (j < rank && c < cols) pf[(size_t)j * cols + c] = (float)acc[u][v];
        }
}

// One workgroup per query head; HD = head_dim (64 or 128).  LP = HD/4 lanes
// hold one cached row (a float4 each), so a wavefront covers PW = 64/LP
// positions per load and U loads: a round of the workgroup covers
// PR = 16 * PW * U positions, wavefront w taking the PW*U consecutive rows
// from w*PW*U.  Every key and value row of a round is requested before
// anything waits: the first round's loads go out before q, k and v of this
// token are read and rotated, so the cache and the QKV output arrive
// together.  Row pos is this token's rotated key and its value, taken from
// LDS (the cache row is written by the group's first query head for later
// tokens, so no workgroup waits on another).
//
// Softmax (forward.go:463-479) in one pass: each position group keeps the
// running max m, the sum l of exp(score - m) and acc = sum exp(score - m) v
// over its rows; groups merge by rescaling to the larger max (exp(-inf) = 0
// for empty groups), wavefronts in LDS in wavefront order, so the result is
// the same on every run.  The exponentials are fp32 expf of the fp32
// difference; the reference rounds a double exp to float, which differs by
// about an ulp.
//
// The rows 0..pos of a head are split over n_split workgroups (blockIdx =
// head * n_split + split), so long caches spread over more CUs; each leaves
// its (acc, m, l) (LlgAttnParts) and the Wo matvec merges the splits while
// it stages its x (out = sum acc e / sum l e, e = exp(m - max m)).
template <int HD>
struct AttnShape {
    static constexpr int LP = HD / 4;                    // lanes per position
    static constexpr int PW = 64 / LP;                   // positions per wavefront load
    static constexpr int NW = ATTN_THREADS / 64;         // wavefronts
    static constexpr int per_round(int u) { return NW * PW * u; }
};

// Value of lane u of each LP-lane position group (LP = 16: 16-lane rows;
// LP = 32: 32-lane halves), by ds_swizzle in bit mode.
template <int LP, int U>
__device__ __forceinline__ float group_lane(float v) {
    constexpr int pattern = LP == 16 ? (0x10 | (U << 5)) : (U << 5);
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), pattern));
}

template <int LP, int U, int K = 0>
__device__ __forceinline__ void group_bcast(float v, float (&p)[U]) {
    if constexpr (K < U) {
        p[K] = group_lane<LP, K>(v);
        group_bcast<LP, U, K + 1>(v, p);
    }
}

// (m, l, acc) <- merge of (m, l, acc) and (mo, lo, ao): rescaled to the larger max.
__device__ __forceinline__ void attn_merge(float &m, float &l, float4 &acc, float mo, float lo,
                                           float4 ao) {
    const float M = fmaxf(m, mo);
    const float a = m == -INFINITY ? 0.0f : expf(m - M);
    const float b = mo == -INFINITY ? 0.0f : expf(mo - M);
    l = l * a + lo * b;
    acc.x = acc.x * a + ao.x * b;
    acc.y = acc.y * a + ao.y * b;
    acc.z = acc.z * a + ao.z * b;
    acc.w = acc.w * a + ao.w * b;
    m = M;
}

template <int HD, int U>
__global__ __launch_bounds__(ATTN_THREADS) void k_attn(const float *__restrict__ qkv, int n_heads,
                                                       int n_kv, int pos,
                                                       const float2 *__restrict__ rope,
                                                       int max_seq, float *__restrict__ kv,
                                                       int n_split, float *__restrict__ acc_out,
                                                       float *__restrict__ ml_out,
                                                       const float *__restrict__ pfold, int rank,
                                                       float *__restrict__ pd_out) {
    using S = AttnShape<HD>;
    constexpr int LP = S::LP, PW = S::PW, NW = S::NW, PR = NW * PW * U;
    static_assert(U <= LP, "lane u of a group computes the exponential of load u");
    __shared__ __attribute__((aligned(16))) float qh[HD], kh[HD], vh[HD];
    __shared__ __attribute__((aligned(16))) float wacc[NW][HD];
    __shared__ float wm[NW], wl[NW];
    const int h = blockIdx.x / n_split, sp = blockIdx.x % n_split;
    const int chunk = (pos + n_split) / n_split;  // rows 0..pos over n_split workgroups
    const int row0 = sp * chunk, row1 = min(pos + 1, row0 + chunk);  // this one's rows [row0, row1)
    const int kvh = h * n_kv / n_heads;  // forward.go:266
    const int kv_dim = n_kv * HD, row4 = kv_dim / 4;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sub = lane % LP, slot = lane / LP;
    const float4 *kc4 = reinterpret_cast<const float4 *>(kv + (size_t)kvh * HD) + sub;
    const float4 *vc4 =
        reinterpret_cast<const float4 *>(kv + (size_t)max_seq * kv_dim + (size_t)kvh * HD) + sub;
    const int t0 = row0 + wave * PW * U + slot;  // + round * PR + u * PW
    float4 kk[U], vv[U];
    auto issue = [&](int r) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int t = max(0, min(r * PR + t0 + u * PW, pos - 1));  // row pos comes from LDS
            kk[u] = kc4[(size_t)t * row4];
            vv[u] = vc4[(size_t)t * row4];
        }
    };
    issue(0);
    // the predictor fold's columns of this head (P = WUp . Wo): thread (j,
    // seg) of the first pass takes P[j][h HD + 8 seg .. + 8], requested now
    constexpr int TPU = HD / 8, UPP = ATTN_THREADS / TPU;  // threads per unit, units per pass
    const int fj = tid / TPU, fseg = tid % TPU;
    float4 pf[2];
    if (pfold) {
        const float4 *pr4 = reinterpret_cast<const float4 *>(
            pfold + (size_t)min(fj, rank - 1) * (n_heads * HD) + (size_t)h * HD + 8 * fseg);
        pf[0] = pr4[0];
        pf[1] = pr4[1];
    }
    const float *q = qkv + (size_t)h * HD;
    const float *kcur = qkv + (size_t)n_heads * HD + (size_t)kvh * HD;
    const float *vcur = kcur + kv_dim;
    // the group's first query head appends row pos (kvcache.go:42-52)
    const bool first = h == kvh * (n_heads / n_kv) && sp == 0;
    if (tid < HD / 2) {  // RoPE, pairs (i, i + HD/2) (forward.go:483-497)
        const int i = tid;
        const float2 cs = rope[(size_t)pos * (HD / 2) + i];
        const float c = cs.x, s = cs.y;
        const float q0 = q[i], q1 = q[i + HD / 2], k0 = kcur[i], k1 = kcur[i + HD / 2];
        const float r0 = k0 * c - k1 * s, r1 = k0 * s + k1 * c;
        qh[i] = q0 * c - q1 * s;
        qh[i + HD / 2] = q0 * s + q1 * c;
        kh[i] = r0;
        kh[i + HD / 2] = r1;
        if (first) {
            kv[(size_t)pos * kv_dim + (size_t)kvh * HD + i] = r0;
            kv[(size_t)pos * kv_dim + (size_t)kvh * HD + i + HD / 2] = r1;
        }
    } else if (tid >= 64 && tid < 64 + HD) {
        const int i = tid - 64;
        const float v = vcur[i];
        vh[i] = v;
        if (first) kv[(size_t)max_seq * kv_dim + (size_t)pos * kv_dim + (size_t)kvh * HD + i] = v;
    }
    __syncthreads();
    const float scale = (float)(1.0 / sqrt((double)HD));  // forward.go:255
    const float4 qv = reinterpret_cast<const float4 *>(qh)[sub];
    const float4 kn = reinterpret_cast<const float4 *>(kh)[sub];
    const float4 vn = reinterpret_cast<const float4 *>(vh)[sub];
    float m = -INFINITY, l = 0.0f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    const int n_rounds = (max(row1 - row0, 0) + PR - 1) / PR;
    for (int r = 0; r < n_rounds; r++) {
        if (r > 0) issue(r);
        float sc[U];
        float mr = -INFINITY;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int t = r * PR + t0 + u * PW;
            const float4 k4 = t == pos ? kn : kk[u];
            float dot = qv.x * k4.x + qv.y * k4.y + qv.z * k4.z + qv.w * k4.w;
            dot = row16_sum(dot);
            if (LP == 32) dot += __shfl_xor(dot, 16, 64);
            sc[u] = dot * scale;
            if (t < row1) mr = fmaxf(mr, sc[u]);
        }
        // lane `sub` of the group takes the exponential of load u = sub
        float mine = sc[0];
#pragma unroll
        for (int u = 1; u < U; u++)
            if (sub == u) mine = sc[u];
        const bool valid = sub < U && r * PR + t0 + sub * PW < row1;
        const float pm = valid ? expf(mine - mr) : 0.0f;
        float p[U];
        group_bcast<LP, U>(pm, p);
        float lr = 0.0f;
        float4 ar = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int t = r * PR + t0 + u * PW;
            const float4 v4 = t == pos ? vn : vv[u];
            lr += p[u];
            ar.x += p[u] * v4.x;
            ar.y += p[u] * v4.y;
            ar.z += p[u] * v4.z;
            ar.w += p[u] * v4.w;
        }
        if (r == 0) {
            m = mr;
            l = lr;
            acc = ar;
        } else if (mr != -INFINITY) {
            attn_merge(m, l, acc, mr, lr, ar);
        }
    }
    // the PW groups of a wavefront, then the wavefronts in order
#pragma unroll
    for (int o = LP; o < 64; o <<= 1) {
        const float mo = __shfl_xor(m, o, 64), lo = __shfl_xor(l, o, 64);
        const float4 ao = make_float4(__shfl_xor(acc.x, o, 64), __shfl_xor(acc.y, o, 64),
                                      __shfl_xor(acc.z, o, 64), __shfl_xor(acc.w, o, 64));
        attn_merge(m, l, acc, mo, lo, ao);
    }
    if (lane < LP) reinterpret_cast<float4 *>(&wacc[wave][0])[lane] = acc;
    if (lane == 0) {
        wm[wave] = m;
        wl[wave] = l;
    }
    __syncthreads();
    if (tid < HD) {  // this workgroup's (acc, m, l), merged with the other splits by the reader
        static_assert(NW <= 64, "one wavefront partial per lane");
        float M = wm[0];
#pragma unroll
        for (int w = 1; w < NW; w++) M = fmaxf(M, wm[w]);
        // lane w takes partial w's weight once; the sums read it back with
        // readlane in the order w = 0, 1, ... (the same values and order as
        // every thread forming all NW exponentials itself)
        const float mw = wm[min(lane, NW - 1)];
        const float ew = mw == -INFINITY ? 0.0f : expf(mw - M);
        float L = 0.0f, R = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float e = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ew), w));
            L += wl[w] * e;
            R += wacc[w][tid] * e;
        }
        acc_out[((size_t)sp * n_heads + h) * HD + tid] = R;
        if (tid == 0) {
            ml_out[((size_t)sp * n_heads + h) * 2] = M;
            ml_out[((size_t)sp * n_heads + h) * 2 + 1] = L;
        }
        if (pfold) qh[tid] = R;  // q is no longer read
    }
    if (pfold) {
        // pd[j] = P[j][h HD ..] . R (this split's unnormalised output): 8
        // products per thread in order, then the TPU threads of a unit by a
        // butterfly, so every run adds in the same order
        __syncthreads();
        float4 w0 = pf[0], w1 = pf[1];
        for (int j0 = 0; j0 < rank; j0 += UPP) {
            if (j0 > 0) {
                const float4 *pr4 = reinterpret_cast<const float4 *>(
                    pfold + (size_t)min(j0 + fj, rank - 1) * (n_heads * HD) + (size_t)h * HD + 8 * fseg);
                w0 = pr4[0];
                w1 = pr4[1];
            }
            const float4 r0 = *reinterpret_cast<const float4 *>(&qh[8 * fseg]);
            const float4 r1 = *reinterpret_cast<const float4 *>(&qh[8 * fseg + 4]);
            float d = w0.x * r0.x;
            d += w0.y * r0.y;
            d += w0.z * r0.z;
            d += w0.w * r0.w;
            d += w1.x * r1.x;
            d += w1.y * r1.y;
            d += w1.z * r1.z;
            d += w1.w * r1.w;
#pragma unroll
            for (int o = 1; o < TPU; o <<= 1) d += __shfl_xor(d, o, 64);
            if (fseg == 0 && j0 + fj < rank)
                pd_out[((size_t)sp * n_heads + h) * rank + j0 + fj] = d;
        }
    }
}

// First index of the maximum (generate.go:197-205: strict '>' from index 0,
// so a NaN at index 0 wins and later NaNs never do).  One workgroup; each
// thread requests all of its float4 groups (up to AM_U per pass) before
// using any, so a 65024-entry vocabulary takes one memory round.  Two
// branch-free passes over the registers: the maximum M (fmaxf skips NaN),
// then the smallest index holding M.
#define AM_U 16
#define AM_THREADS 1024
__global__ __launch_bounds__(AM_THREADS) void k_argmax(const float *__restrict__ v, int n,
                                                       int32_t *__restrict__ out) {
    __shared__ float mv_s[AM_THREADS / 64];
    __shared__ int mi_s[AM_THREADS / 64];
    const int n4 = n >> 2;
    const float4 *v4 = reinterpret_cast<const float4 *>(v);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // pass 1: the maximum.  Up to AM_U * AM_THREADS float4 groups stay in
    // registers for pass 2; a longer row is read again there.
    constexpr int CH = AM_U * AM_THREADS;
    float4 xs[AM_U];
    auto load = [&](int c0) {
#pragma unroll
        for (int k = 0; k < AM_U; k++) xs[k] = v4[max(0, min(c0 + tid + k * AM_THREADS, n4 - 1))];
    };
    const float tail = tid < (n & 3) ? v[4 * n4 + tid] : -INFINITY;
    float m = tail;
    for (int c0 = 0; c0 < n4; c0 += CH) {
        load(c0);
#pragma unroll
        for (int k = 0; k < AM_U; k++)
            if (c0 + tid + k * AM_THREADS < n4)
                m = fmaxf(m, fmaxf(fmaxf(xs[k].x, xs[k].y), fmaxf(xs[k].z, xs[k].w)));
    }
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if (lane == 0) mv_s[wave] = m;
    __syncthreads();
    float M = mv_s[0];
#pragma unroll
    for (int w = 1; w < AM_THREADS / 64; w++) M = fmaxf(M, mv_s[w]);
    // pass 2: first index holding M (chunks from the last, so the first wins)
    int bi = n;
    for (int c0 = (n4 - 1) / CH * CH; c0 >= 0; c0 -= CH) {
        if (n4 > CH) load(c0);
#pragma unroll
        for (int k = AM_U - 1; k >= 0; k--) {
            const int j = c0 + tid + k * AM_THREADS;
            if (j < n4) {
                bi = xs[k].w == M ? 4 * j + 3 : bi;
                bi = xs[k].z == M ? 4 * j + 2 : bi;
                bi = xs[k].y == M ? 4 * j + 1 : bi;
                bi = xs[k].x == M ? 4 * j : bi;
            }
        }
    }
    if (tid < (n & 3) && tail == M) bi = min(bi, 4 * n4 + tid);
    for (int o = 32; o > 0; o >>= 1) bi = min(bi, __shfl_xor(bi, o, 64));
    if (lane == 0) mi_s[wave] = bi;
    __syncthreads();
    if (tid == 0) {
        int b = mi_s[0];
        for (int w = 1; w < AM_THREADS / 64; w++) b = min(b, mi_s[w]);
        const float v0 = v[0];
        *out = (v0 != v0 || b >= n) ? 0 : b;
    }
}

// ---------------------------------------------------------------------------
static LlgModel *get_model(LlgDevice *d, int64_t h) {
    LlgObject *o = llg_get(d, h, LLG_KIND_MODEL);
    return o ? reinterpret_cast<LlgModel *>(o->ext) : nullptr;
}

static size_t model_ws_bytes(const LlgModel &m) {
    return std::max(llg_fused_ws_bytes(m.rank, m.ff, (m.hidden + 31) / 32),
                    (size_t)llg_predict_ws_bytes(m.rank, m.ff));
}

// Rows per attention workgroup above which a head's rows are split further:
// up to LLG_ATTN_SPLIT_MAX workgroups per head, and no more workgroups than
// CUs (a CU given two would take twice as long as the rest).
#define ATTN_SPLIT_ROWS 160
static int attn_splits(const LlgModel &m, int pos) {
    const int by_rows = (pos + ATTN_SPLIT_ROWS) / ATTN_SPLIT_ROWS;
    const int by_cus = std::max(1, m.cus / m.n_heads);
    return std::min(std::min(LLG_ATTN_SPLIT_MAX, by_cus), by_rows);
}

// The attention launch for rows 0..pos: attn_splits workgroups per head, and
// the fewest loads per lane U whose round covers a workgroup's rows, else
// rounds of the largest.
template <int HD>
// pfold (optional): the layer's P, whose per-split products go to m.pd.
static void launch_attn(hipStream_t st, const LlgModel &m, int pos, float *kvl,
                        const float *pfold) {
    using S = AttnShape<HD>;
    const int ns = attn_splits(m, pos);
    const int n = (pos + ns) / ns;
    const dim3 grid(m.n_heads * ns);
#define ATT(U)                                                                                     \
    hipLaunchKernelGGL((k_attn<HD, U>), grid, dim3(ATTN_THREADS), 0, st, m.qkv, m.n_heads,        \
                       m.n_kv, pos, m.rope, m.max_seq, kvl, ns, m.attn, m.attn_ml, pfold,       \
                       m.rank, m.pd)
    if (n <= S::per_round(1)) ATT(1);
    else if (n <= S::per_round(2)) ATT(2);
    else if (n <= S::per_round(4)) ATT(4);
    else if (n <= S::per_round(6)) ATT(6);
    else if (n <= S::per_round(8)) ATT(8);
    else ATT(10);
#undef ATT
}

static LlgAttnParts attn_parts(const LlgModel &m, int pos) {
    LlgAttnParts ap;
    ap.acc = m.attn;
    ap.ml = m.attn_ml;
    ap.n_split = attn_splits(m, pos);
    ap.n_heads = m.n_heads;
    ap.head_dim = m.head_dim;
    return ap;
}

// One token: embed -> layers -> norm -> LM head -> argmax, on the stream.
// token_in: device int32 (the token to embed); token_out: device int32 (the
// greedy next token); n_active_out: device int32[n_layers] or null;
// pred_logits: device float[n_layers x ff] or null (each layer's predictor
// logits, from an extra predict-only pass, for threshold calibration).
static int model_step(LlgDevice *d, LlgModel &m, const int32_t *token_in, int pos,
                      int32_t *token_out, int32_t *n_active_out, float *pred_logits) {
    hipStream_t st = llg_dev_stream(d);
    const int qkv_rows = (m.n_heads + 2 * m.n_kv) * m.head_dim;
    (void)qkv_rows;
    float *r = m.x;  // the residual stream
    hipLaunchKernelGGL(k_embed, dim3((m.hidden + 4 * EMBED_THREADS - 1) / (4 * EMBED_THREADS)),
                       dim3(EMBED_THREADS), 0, st, m.embed->d, m.embed->stride, m.embed->fmt,
                       token_in, m.vocab, r, m.rstats);
    for (int l = 0; l < m.n_layers; l++) {
        const LlgModelLayer &L = m.layers[l];
        LlgLnArgs ln;
        ln.x_in = r;
        ln.x_out = nullptr;
        ln.a1 = nullptr;
        ln.a2 = nullptr;
        ln.w = reinterpret_cast<const float *>(L.norm_w->d);
        ln.b = reinterpret_cast<const float *>(L.norm_b->d);
        ln.normed_out = m.normed;
        ln.stats = m.rstats;
        ln.eps = m.eps;
        ln.n = m.hidden;
        int rc = llg_matvec_ln_enqueue(d, L.wqkv, ln, m.qkv);
        if (rc) return rc;
        float *kvl = m.kv + (size_t)l * 2 * m.max_seq * m.n_kv * m.head_dim;
        // with Wo in the tile launch, the attention kernel also forms the
        // predictor's per-split products P . acc
        const float *pf = L.pfold && m.sync && !pred_logits ? L.pfold : nullptr;
        if (m.head_dim == 64)
            launch_attn<64>(st, m, pos, kvl, pf);
        else
            launch_attn<128>(st, m, pos, kvl, pf);
        LLG_LAUNCH_CHECK(d, "model attention");
        if (L.pfold && m.sync && !pred_logits) {
            // one tile launch: r += Wo . attn and the hidden partials P . attn
            // in its first workgroups, then the tiles; the reduce adds the FFN
            // output into r
            if ((rc = llg_fused_wo_enqueue(d, L.wo, attn_parts(m, pos), m.pd, L.pwout, nullptr,
                                           L.bundle, m.normed, L.thr, m.act, r,
                                           n_active_out ? n_active_out + l : nullptr, m.ws,
                                           m.sync, m.rstats)))
                return rc;
            continue;
        }
        if (L.pfold) {  // Wo with the predictor fold: r += attn_out, hidden partials in ws
            LlgPredFold pf;
            unsigned long long *mask;
            llg_pred_ws_layout(m.ws, m.rank, &pf.part, &mask);
            pf.p = L.pfold;
            pf.resid = r;
            pf.rank = m.rank;
            pf.n_split = llg_pred_split();
            pf.split_blocks = (L.wo->fmt.nb + pf.n_split - 1) / pf.n_split;
            if ((rc = llg_matvec_attn_enqueue(d, L.wo, attn_parts(m, pos), nullptr, m.mvpart,
                                              &pf)))
                return rc;
            if (pred_logits &&
                (rc = llg_pred_logits_enqueue(d, L.pwout, nullptr, L.thr, m.ws, m.act_scratch,
                                              m.act_scratch + m.ff,
                                              pred_logits + (size_t)l * m.ff)))
                return rc;
            rc = llg_fused_tail_enqueue(d, L.pwout, nullptr, L.bundle, m.normed, L.thr, m.act, r,
                                        nullptr, n_active_out ? n_active_out + l : nullptr, m.ws,
                                        true, m.rstats);
            if (rc) return rc;
            continue;
        }
        if ((rc = llg_matvec_attn_enqueue(d, L.wo, attn_parts(m, pos), m.attn_out, m.mvpart,
                                          nullptr)))
            return rc;
        if (pred_logits &&
            (rc = llg_predict_enqueue(d, L.pwup, L.pwout, nullptr, m.attn_out, L.thr, m.act_scratch,
                                      m.act_scratch + m.ff, pred_logits + (size_t)l * m.ff, m.ws)))
            return rc;
        // ffnFlash path 2: predictor on the attention output, FFN on normed
        // r += attn_out by its first kernel, then r += the FFN output
        rc = llg_fused_enqueue(d, L.pwup, L.pwout, nullptr, L.bundle, m.attn_out, m.normed, L.thr,
                               m.act, r, nullptr, n_active_out ? n_active_out + l : nullptr, m.ws,
                               nullptr, m.attn_out, m.rstats);
        if (rc) return rc;
    }
    const float *fw = reinterpret_cast<const float *>(m.out_w->d);
    const float *fb = reinterpret_cast<const float *>(m.out_b->d);
    if (m.rstats) {  // r's block statistics are there (the last layer's reduce left them)
        hipLaunchKernelGGL(k_out_norm, dim3((m.hidden / 4 + ONORM_THREADS - 1) / ONORM_THREADS),
                           dim3(ONORM_THREADS), 0, st, r, (const float2 *)m.rstats, fw, fb,
                           m.hidden, m.eps, m.normed);
        int rc = llg_matvec_enqueue(d, m.lm_head, m.normed, -1, m.logits, m.mvpart);
        if (rc) return rc;
        hipLaunchKernelGGL(k_argmax, dim3(1), dim3(AM_THREADS), 0, st, m.logits, m.vocab, token_out);
        LLG_LAUNCH_CHECK(d, "model step");
        return 0;
    }
    const int np = (m.hidden + NORM_THREADS - 1) / NORM_THREADS;
#define RN(NP)                                                                                    \
    hipLaunchKernelGGL((k_resid_norm<NP>), dim3(1), dim3(NORM_THREADS), 0, st, r,                 \
                       (const float *)nullptr, (const float *)nullptr, fw, fb, m.hidden, m.eps,   \
                       m.normed)
    if (np <= 2) RN(2);
    else if (np <= 4) RN(4);
    else if (np <= 6) RN(6);
    else if (np <= 8) RN(8);
    else RN(16);
#undef RN
    int rc = llg_matvec_enqueue(d, m.lm_head, m.normed, -1, m.logits, m.mvpart);
    if (rc) return rc;
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(AM_THREADS), 0, st, m.logits, m.vocab, token_out);
    LLG_LAUNCH_CHECK(d, "model step");
    return 0;
}

static LlgObject *get_f32_vec(LlgDevice *d, int64_t h, int n) {
    LlgObject *o = llg_get(d, h, LLG_KIND_MATRIX);
    if (!o || o->fmt.type != LLG_TYPE_F32 || o->rows != 1 || o->fmt.cols != n) return nullptr;
    return o;
}

extern "C" {

int llg_hip_falcon_create(LlgHipDevice h, const int32_t *dims, float rope_base, float norm_eps,
                          int act, int64_t embed, const int64_t *layer_handles,
                          const float *thresholds, int64_t out_norm_w, int64_t out_norm_b,
                          int64_t lm_head, int64_t *model) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    if (!dims || !layer_handles || !thresholds || !model)
        return llg_set_error(d, LLG_E_ARG, "falcon_create: null argument");
    LlgModel *m = new LlgModel();
    m->n_layers = dims[0];
    m->hidden = dims[1];
    m->n_heads = dims[2];
    m->n_kv = dims[3];
    m->head_dim = dims[4];
    m->ff = dims[5];
    m->vocab = dims[6];
    m->max_seq = dims[7];
    m->rope_base = rope_base;
    m->eps = norm_eps;
    m->cus = llg_cu_count(d);
    m->act = act;
    auto fail = [&](int code, const char *msg) {
        delete m;
        return llg_set_error(d, code, "falcon_create: %s", msg);
    };
    if (m->n_layers < 1 || m->hidden < 32 || m->n_heads < 1 || m->n_kv < 1 ||
        m->n_heads % m->n_kv || m->vocab < 1 || m->max_seq < 1 || m->ff < 1)
        return fail(LLG_E_HPARAM, "invalid dimensions");
    if (m->head_dim != 64 && m->head_dim != 128) return fail(LLG_E_HPARAM, "head_dim must be 64 or 128");
    if (!llg_act_ok(m->act)) return fail(LLG_E_ARG, "activation must be ReLU, GELU or SiLU");
    if (m->hidden > NORM_THREADS * NORM_PER) return fail(LLG_E_HPARAM, "hidden above 16384");
    if ((size_t)m->max_seq * 4 > 64 * 1024) return fail(LLG_E_HPARAM, "max_seq above 16384");
    const int qkv_rows = (m->n_heads + 2 * m->n_kv) * m->head_dim;
    m->embed = llg_get(d, embed, LLG_KIND_MATRIX);
    m->lm_head = llg_get(d, lm_head, LLG_KIND_MATRIX);
    m->out_w = get_f32_vec(d, out_norm_w, m->hidden);
    m->out_b = get_f32_vec(d, out_norm_b, m->hidden);
    if (!m->embed || m->embed->rows != m->vocab || m->embed->fmt.cols != m->hidden)
        return fail(LLG_E_ARG, "embedding must be [vocab x hidden]");
    if (!m->lm_head || m->lm_head->rows != m->vocab || m->lm_head->fmt.cols != m->hidden)
        return fail(LLG_E_ARG, "lm head must be [vocab x hidden]");
    if (!m->out_w || !m->out_b) return fail(LLG_E_ARG, "output norm must be F32 [1 x hidden]");
    m->rank = -1;
    for (int l = 0; l < m->n_layers; l++) {
        const int64_t *lh = layer_handles + 7 * l;
        LlgModelLayer L;
        L.norm_w = get_f32_vec(d, lh[0], m->hidden);
        L.norm_b = get_f32_vec(d, lh[1], m->hidden);
        L.wqkv = llg_get(d, lh[2], LLG_KIND_MATRIX);
        L.wo = llg_get(d, lh[3], LLG_KIND_MATRIX);
        L.pwup = llg_get(d, lh[4], LLG_KIND_MATRIX);
        L.pwout = llg_get(d, lh[5], LLG_KIND_MATRIX);
        L.bundle = llg_get(d, lh[6], LLG_KIND_BUNDLE);
        L.thr = thresholds[l];
        L.pfold = nullptr;
        if (!L.norm_w || !L.norm_b) return fail(LLG_E_ARG, "layer norm must be F32 [1 x hidden]");
        if (!L.wqkv || L.wqkv->rows != qkv_rows || L.wqkv->fmt.cols != m->hidden)
            return fail(LLG_E_ARG, "wqkv must be [(n_heads + 2 n_kv) head_dim x hidden]");
        if (!L.wo || L.wo->rows != m->hidden || L.wo->fmt.cols != m->n_heads * m->head_dim)
            return fail(LLG_E_ARG, "wo must be [hidden x n_heads head_dim]");
        if (!L.bundle || L.bundle->rows != m->ff || L.bundle->fmt.cols != m->hidden)
            return fail(LLG_E_ARG, "bundle must hold ff neurons of hidden");
        if (!L.pwup || !L.pwout || L.pwup->fmt.type != LLG_TYPE_F32 ||
            L.pwout->fmt.type != LLG_TYPE_F32 || L.pwup->fmt.cols != m->hidden ||
            L.pwout->rows != m->ff || L.pwout->fmt.cols != L.pwup->rows)
            return fail(LLG_E_ARG, "predictor must be F32 WUp [rank x hidden], WOut [ff x rank]");
        if (m->rank < 0) m->rank = L.pwup->rows;
        if (L.pwup->rows != m->rank) return fail(LLG_E_ARG, "predictor rank differs between layers");
        m->layers.push_back(L);
    }
    // device buffers
    const size_t kv_dim = (size_t)m->n_kv * m->head_dim;
    const size_t v_h = llg_align((long long)m->hidden * 4, 256);
    const size_t v_qkv = llg_align((long long)qkv_rows * 4, 256);
    const size_t v_att = llg_align((long long)LLG_ATTN_SPLIT_MAX * m->n_heads * m->head_dim * 4, 256);
    const size_t v_aml = llg_align((long long)LLG_ATTN_SPLIT_MAX * m->n_heads * 2 * 4, 256);
    const size_t v_log = llg_align((long long)m->vocab * 4, 256);
    const size_t v_kv = llg_align((long long)m->n_layers * 2 * m->max_seq * kv_dim * 4, 256);
    const size_t v_i = llg_align((long long)(m->n_layers + 4) * 4, 256);
    const size_t v_ff = llg_align((long long)(m->ff + 4) * 4, 256);
    const size_t v_pl = llg_align((long long)m->n_layers * m->ff * 4, 256);
    const size_t v_rope = llg_align((long long)m->max_seq * m->head_dim / 2 * 8, 256);
    const bool use_stats = m->hidden % 32 == 0 && m->hidden <= 32 * 64 * LLG_LN_STATS_PER;
    const size_t v_st = use_stats ? llg_align((long long)(m->hidden / 32) * 8, 256) : 0;
    const size_t wsb = model_ws_bytes(*m);
    const int attn_dim = m->n_heads * m->head_dim;
    bool fold = true;
    for (const LlgModelLayer &L : m->layers) fold = fold && llg_matvec_fold_ok(L.wo);
    const size_t v_pf1 = llg_align((long long)m->rank * attn_dim * 4, 256);
    const size_t v_pf = fold ? (size_t)m->n_layers * v_pf1 : 0;
    size_t v_mp = llg_matvec_part_bytes(m->lm_head, -1);
    for (const LlgModelLayer &L : m->layers) v_mp = std::max(v_mp, llg_matvec_part_bytes(L.wo, -1));
    v_mp = llg_align((long long)v_mp, 256);
    bool in_tile = fold && use_stats && m->head_dim % 8 == 0;
    for (const LlgModelLayer &L : m->layers)
        in_tile = in_tile && llg_fused_wo_ok(L.wo, m->rank, m->hidden);
    const size_t v_pd =
        in_tile ? llg_align((long long)LLG_ATTN_SPLIT_MAX * m->n_heads * m->rank * 4, 256) : 0;
    const size_t total =
        3 * v_h + v_qkv + v_att + v_aml + v_log + v_kv + v_i + v_ff + v_pl + v_rope + v_st + v_mp +
        v_pf + v_pd + wsb;
    uint8_t *buf = nullptr;
    if (hipMalloc(&buf, total) != hipSuccess) return fail(LLG_E_NOMEM, "buffer allocation failed");
    uint8_t *p = buf;
    m->x = reinterpret_cast<float *>(p); p += v_h;
    m->normed = reinterpret_cast<float *>(p); p += v_h;
    m->attn_out = reinterpret_cast<float *>(p); p += v_h;
    m->qkv = reinterpret_cast<float *>(p); p += v_qkv;
    m->attn = reinterpret_cast<float *>(p); p += v_att;
    m->attn_ml = reinterpret_cast<float *>(p); p += v_aml;
    m->logits = reinterpret_cast<float *>(p); p += v_log;
    m->kv = reinterpret_cast<float *>(p); p += v_kv;
    m->token = reinterpret_cast<int32_t *>(p);
    m->n_active = m->token + 4;
    p += v_i;
    m->act_scratch = reinterpret_cast<int32_t *>(p);
    p += v_ff;
    m->pred_logits = reinterpret_cast<float *>(p);
    p += v_pl;
    m->rope = reinterpret_cast<float2 *>(p);
    p += v_rope;
    m->rstats = use_stats ? reinterpret_cast<float2 *>(p) : nullptr;
    p += v_st;
    m->mvpart = v_mp ? reinterpret_cast<float *>(p) : nullptr;
    p += v_mp;
    for (LlgModelLayer &L : m->layers) {
        L.pfold = fold ? reinterpret_cast<float *>(p) : nullptr;
        p += fold ? v_pf1 : 0;
    }
    m->pd = in_tile ? reinterpret_cast<float *>(p) : nullptr;
    p += v_pd;
    m->ws = p;
    if (in_tile) {  // the sync area is taken (and cleared) here, outside any capture
        int rc = 0;
        m->sync = llg_dev_sync(d, &rc);
        if (rc) {
            (void)hipFree(buf);
            delete m;
            return rc;
        }
    }
    hipStream_t st = llg_dev_stream(d);
    hipError_t e = hipMemsetAsync(buf, 0, total, st);
    const int n_rope = m->max_seq * (m->head_dim / 2);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(k_rope_table, dim3((n_rope + 255) / 256), dim3(256), 0, st, m->rope,
                           m->max_seq, m->head_dim / 2, m->rope_base);
        e = hipGetLastError();
    }
    for (const LlgModelLayer &L : m->layers) {
        if (e != hipSuccess || !L.pfold) break;
        const dim3 grid((attn_dim + FOLD_T - 1) / FOLD_T, (m->rank + FOLD_T - 1) / FOLD_T);
        hipLaunchKernelGGL(k_fold_pred, grid, dim3(256), 0, st, L.pwup->d, L.pwup->stride, m->rank,
                           m->hidden, L.wo->d, L.wo->stride, L.wo->fmt, L.pfold);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        (void)hipFree(buf);
        delete m;
        return llg_hip_error(d, e, "falcon_create");
    }
    model_objects(m, [](LlgObject *x) { llg_ref(x); });
    LlgObject *o = new LlgObject();
    o->kind = LLG_KIND_MODEL;
    o->d = buf;
    o->bytes = total;
    o->rows = m->n_layers;
    o->fmt = m->embed->fmt;
    o->stride = 0;
    o->ext = m;
    *model = llg_register(d, o);
    return 0;
}

int llg_hip_falcon_set_thresholds(LlgHipDevice h, int64_t hm, const float *thresholds) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgModel *m = get_model(d, hm);
    if (!m) return llg_set_error(d, LLG_E_HANDLE, "falcon: unknown model");
    if (!thresholds) return llg_set_error(d, LLG_E_ARG, "falcon: null thresholds");
    for (int l = 0; l < m->n_layers; l++) m->layers[l].thr = thresholds[l];
    return 0;
}

int llg_hip_falcon_forward(LlgHipDevice h, int64_t hm, int32_t token, int pos, float *logits,
                           int32_t *next_token, int32_t *n_active, float *pred_logits) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgModel *m = get_model(d, hm);
    if (!m) return llg_set_error(d, LLG_E_HANDLE, "falcon: unknown model");
    if (token < 0 || token >= m->vocab)
        return llg_set_error(d, LLG_E_RANGE, "falcon: token %d outside [0,%d)", token, m->vocab);
    if (pos < 0 || pos >= m->max_seq)
        return llg_set_error(d, LLG_E_RANGE, "falcon: position %d outside [0,%d)", pos, m->max_seq);
    int rc;
    if ((rc = llg_h2d(d, m->token, &token, 4))) return rc;
    if ((rc = model_step(d, *m, m->token, pos, m->token + 1, n_active ? m->n_active : nullptr,
                         pred_logits ? m->pred_logits : nullptr)))
        return rc;
    if (pred_logits &&
        (rc = llg_d2h(d, pred_logits, m->pred_logits, (size_t)m->n_layers * m->ff * 4)))
        return rc;
    if (logits && (rc = llg_d2h(d, logits, m->logits, (size_t)m->vocab * 4))) return rc;
    if (next_token && (rc = llg_d2h(d, next_token, m->token + 1, 4))) return rc;
    if (n_active && (rc = llg_d2h(d, n_active, m->n_active, (size_t)m->n_layers * 4))) return rc;
    return llg_sync_dev(d);
}

int llg_hipd_falcon_step(LlgHipDevice h, int64_t hm, const int32_t *d_token, int pos,
                         int32_t *d_next_token, float *d_logits) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgModel *m = get_model(d, hm);
    if (!m) return llg_set_error(d, LLG_E_HANDLE, "falcon: unknown model");
    if (!d_token || !d_next_token) return llg_set_error(d, LLG_E_ARG, "falcon: null token pointer");
    if (pos < 0 || pos >= m->max_seq)
        return llg_set_error(d, LLG_E_RANGE, "falcon: position %d outside [0,%d)", pos, m->max_seq);
    int rc = model_step(d, *m, d_token, pos, d_next_token, nullptr, nullptr);
    if (rc) return rc;
    if (d_logits)
        LLG_HIP_TRY(d, hipMemcpyAsync(d_logits, m->logits, (size_t)m->vocab * 4,
                                      hipMemcpyDeviceToDevice, llg_dev_stream(d)));
    return 0;
}

}  // extern "C"
