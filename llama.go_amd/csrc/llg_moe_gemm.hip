// llg_moe_gemm.hip -- MoE FFN for a batch of tokens (prefill) as grouped
// MFMA GEMMs (inference/moe_forward.go:32-150 applied to every token; the
// reference runs them one token at a time, cmd/generate.go:88-96).
//
//   1. k_moe_router (llg_moe.hip): ids / weights per token
//   2. k_moe_group: counting sort of the (token, slot) pairs by expert, the
//      pair <-> row maps, and a list of 64-row M-tiles (expert, first row, rows)
//   3. k_moe_x16: X -> f16, each 8-group of K stored in the order
//      [0,4,1,5,2,6,3,7] (the order in which the Q4_0 B fragment unpacks)
//   4. k_moe_gemm<0>: G = X_e . gate_e^T, U = X_e . up_e^T on v_mfma_f32_16x16x32_f16,
//      epilogue H = silu(G) * U (moe_forward.go:128-132) stored f16, same K order
//   5. k_moe_gemm<1>: Y = H_e . down_e^T
//   6. k_moe_combine: out[t] = sum_s w[t][s] * Y[row(t, s)], in slot order
//      from 0 (moe_forward.go:71-77)
//
// MFMA operands (16x16x32 f16): lane l holds 8 halves of A row l%16 and of B
// column l%16 for the K-group l/16; C lane l holds column l%16, rows
// 4*(l/16) .. +3.  A and B use the same K permutation, so the dot products are
// unchanged.  B is a Q4_0 block per K step: lane (column j, group g) takes
// 32-bit word g of the block (nibble p = element 8g + p), forms the f16 pairs
// (1024 + q_p, 1024 + q_{p+4}) with one and/or, subtracts 1032 (exact) and
// multiplies by the block scale.  Tiles: 64 rows x 128 columns per workgroup
// (per weight matrix), 4 wavefronts of 64 x 32, K chunks of 128 staged in LDS
// (double buffered; the next chunk is loaded into registers while the current
// one is multiplied).
#include "llg_common.hpp"
#include "llg_internal.hpp"

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

#define GM_BM 64
#define GM_BN 128
#define GM_KC 128                 // K per chunk
#define GM_KB (GM_KC / 32)        // Q4_0 blocks per chunk
#define GM_AST (GM_KC + 8)        // LDS A row stride (halves)
#define GM_BST 80                 // LDS B nibble row stride (bytes): conflict-free reads

// ---------------------------------------------------------------------------
// Grouping: pairs p = t*k + s sorted by expert (order within an expert is not
// significant: each row's result depends only on its own token).
// tiles[i] = (expert, first row, rows); n_tiles[0] = count.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_moe_group(const int32_t *__restrict__ ids, int n_pairs,
                                                    int n_exp, int32_t *__restrict__ row_pair,
                                                    int32_t *__restrict__ pair_row,
                                                    int4 *__restrict__ tiles,
                                                    int32_t *__restrict__ n_tiles) {
    __shared__ int cnt[64], off[65], fill[64];
    const int tid = threadIdx.x;
    if (tid < 64) {
        cnt[tid] = 0;
        fill[tid] = 0;
    }
    __syncthreads();
    for (int p = tid; p < n_pairs; p += blockDim.x) atomicAdd(&cnt[ids[p]], 1);
    __syncthreads();
    if (tid == 0) {
        int o = 0, nt = 0;
        for (int e = 0; e < n_exp; e++) {
            off[e] = o;
            for (int r = 0; r < cnt[e]; r += GM_BM)
                tiles[nt++] = make_int4(e, o + r, min(GM_BM, cnt[e] - r), 0);
            o += cnt[e];
        }
        off[n_exp] = o;
        *n_tiles = nt;
    }
    __syncthreads();
    for (int p = tid; p < n_pairs; p += blockDim.x) {
        const int e = ids[p];
        const int r = off[e] + atomicAdd(&fill[e], 1);
        row_pair[r] = p;
        pair_row[p] = r;
    }
}

// X (fp32, [n_tok x K]) -> f16 with each 8-group in the order [0,4,1,5,2,6,3,7].
__global__ void k_moe_x16(const float *__restrict__ x, long long n8, _Float16 *__restrict__ x16) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;  // 8-group index
    if (i >= n8) return;
    const float4 a = reinterpret_cast<const float4 *>(x)[2 * i];
    const float4 b = reinterpret_cast<const float4 *>(x)[2 * i + 1];
    half8_t h;
    h[0] = (_Float16)a.x;
    h[1] = (_Float16)b.x;
    h[2] = (_Float16)a.y;
    h[3] = (_Float16)b.y;
    h[4] = (_Float16)a.z;
    h[5] = (_Float16)b.z;
    h[6] = (_Float16)a.w;
    h[7] = (_Float16)b.w;
    reinterpret_cast<half8_t *>(x16)[i] = h;
}

// B fragment: word g of a Q4_0 block (nibble p = element 8g+p) times scale d,
// as f16 in the order [e0,e4,e1,e5,e2,e6,e3,e7].
__device__ __forceinline__ half8_t q4_frag(uint32_t w, _Float16 d) {
    const half2_t off = {(_Float16)1032.0f, (_Float16)1032.0f};
    const half2_t dd = {d, d};
    half8_t r;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t bits = ((w >> (4 * t)) & 0x000F000Fu) | 0x64006400u;  // 1024 + q
        half2_t v = __builtin_bit_cast(half2_t, bits);
        v = (v - off) * dd;
        r[2 * t] = v[0];
        r[2 * t + 1] = v[1];
    }
    return r;
}

// MODE 0: gate+up with SwiGLU epilogue -> H (f16, permuted K order, [rows x N]).
// MODE 1: down -> Y (f32, [rows x N]).
// A rows: MODE 0 gathers X16 row row_pair[r] / k (the pair's token); MODE 1
// reads H row r.
template <int MODE>
__global__ __launch_bounds__(256, 2) void k_moe_gemm(
    const int4 *__restrict__ tiles, const int32_t *__restrict__ n_tiles_p,
    const int32_t *__restrict__ row_pair, int k_slots, const _Float16 *__restrict__ A,
    const uint8_t *__restrict__ W0, const uint8_t *__restrict__ W1, long long wstride,
    int d_off, int rows_per_expert, int K, int N, _Float16 *__restrict__ H,
    float *__restrict__ Y) {
    constexpr int NM = MODE == 0 ? 2 : 1;  // weight matrices
    constexpr int BROWS = GM_BN * NM;      // B rows per chunk
    __shared__ __attribute__((aligned(16))) _Float16 As[2][GM_BM * GM_AST];
    __shared__ __attribute__((aligned(16))) uint8_t Bq[2][BROWS * GM_BST];
    __shared__ __attribute__((aligned(16))) _Float16 Bd[2][BROWS * GM_KB];
    const int n_ntiles = N / GM_BN;
    const int nt = blockIdx.x % n_ntiles;
    const int mt = blockIdx.x / n_ntiles;
    if (mt >= *n_tiles_p) return;
    const int4 tile = tiles[mt];
    const int e = tile.x, row0 = tile.y, nrows = tile.z;
    const int n0 = nt * GM_BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // Per-thread load assignment.  A: 64 rows x 16 uint4 per chunk -> 4 per
    // thread (rows past the tile reload the tile's last row; results dropped).
    constexpr int BQ = BROWS * GM_KB / 256;  // B nibble uint4 per thread (4 or 2)
    long long a_off[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int idx = tid + 256 * q;
        const int r = idx >> 4, part = idx & 15;
        const int rr = min(r, nrows - 1);
        const long long arow = MODE == 0 ? row_pair[row0 + rr] / k_slots : row0 + rr;
        a_off[q] = arow * K + part * 8;
    }
    long long b_off[BQ];
#pragma unroll
    for (int q = 0; q < BQ; q++) {
        const int idx = tid + 256 * q;
        const int rb = idx / GM_KB, blk = idx % GM_KB;
        const int n = rb % GM_BN;
        b_off[q] = ((long long)e * rows_per_expert + n0 + n) * wstride + blk * 16;
    }
    const uint8_t *W0b = W0, *W1b = MODE == 0 ? W1 : W0;
    const long long d_row = ((long long)e * rows_per_expert + n0 + (tid % GM_BN)) * wstride + d_off;
    const uint8_t *Wd = (MODE == 0 && tid >= GM_BN) ? W1b : W0b;

    uint4 ra[4], rbq[BQ];
    uint2 rd = make_uint2(0, 0);
#define GM_LOAD(c)                                                                               \
    do {                                                                                         \
        _Pragma("unroll") for (int q = 0; q < 4; q++) ra[q] =                                   \
            *reinterpret_cast<const uint4 *>(A + a_off[q] + (long long)(c) * GM_KC);             \
        _Pragma("unroll") for (int q = 0; q < BQ; q++) {                                         \
            const uint8_t *W = (MODE == 0 && (tid + 256 * q) / GM_KB >= GM_BN) ? W1b : W0b;      \
            rbq[q] = *reinterpret_cast<const uint4 *>(W + b_off[q] + (long long)(c) * GM_KB * 16); \
        }                                                                                        \
        if (tid < BROWS) rd = *reinterpret_cast<const uint2 *>(Wd + d_row + (c) * GM_KB * 2);    \
    } while (0)
#define GM_STORE(buf)                                                                            \
    do {                                                                                         \
        _Pragma("unroll") for (int q = 0; q < 4; q++) {                                         \
            const int idx = tid + 256 * q;                                                       \
            *reinterpret_cast<uint4 *>(&As[buf][(idx >> 4) * GM_AST + (idx & 15) * 8]) = ra[q];  \
        }                                                                                        \
        _Pragma("unroll") for (int q = 0; q < BQ; q++) {                                         \
            const int idx = tid + 256 * q;                                                       \
            *reinterpret_cast<uint4 *>(&Bq[buf][(idx / GM_KB) * GM_BST + (idx % GM_KB) * 16]) =  \
                rbq[q];                                                                          \
        }                                                                                        \
        if (tid < BROWS) *reinterpret_cast<uint2 *>(&Bd[buf][tid * GM_KB]) = rd;                \
    } while (0)

    floatx4_t acc[NM][4][2];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) acc[m][i][j] = {0.f, 0.f, 0.f, 0.f};

    const int nc = K / GM_KC;
    GM_LOAD(0);
    GM_STORE(0);
    __syncthreads();
    const int li = lane & 15, lg = lane >> 4;
    for (int c = 0; c < nc; c++) {
        const int buf = c & 1;
        GM_LOAD(min(c + 1, nc - 1));  // the last iteration reloads its own chunk (unused)
#pragma unroll
        for (int s = 0; s < GM_KB; s++) {
            half8_t a[4];
#pragma unroll
            for (int ms = 0; ms < 4; ms++)
                a[ms] = *reinterpret_cast<const half8_t *>(
                    &As[buf][(ms * 16 + li) * GM_AST + s * 32 + lg * 8]);
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int ns = 0; ns < 2; ns++) {
                    const int rb = m * GM_BN + wave * 32 + ns * 16 + li;
                    const uint32_t w =
                        *reinterpret_cast<const uint32_t *>(&Bq[buf][rb * GM_BST + s * 16 + lg * 4]);
                    const half8_t b = q4_frag(w, Bd[buf][rb * GM_KB + s]);
#pragma unroll
                    for (int ms = 0; ms < 4; ms++)
                        acc[m][ms][ns] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            a[ms], b, acc[m][ms][ns], 0, 0, 0);
                }
        }
        if (c + 1 < nc) GM_STORE(buf ^ 1);
        __syncthreads();
    }
#undef GM_LOAD
#undef GM_STORE

    // epilogue
#pragma unroll
    for (int ms = 0; ms < 4; ms++)
#pragma unroll
        for (int ns = 0; ns < 2; ns++) {
            const int n = n0 + wave * 32 + ns * 16 + li;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int m = ms * 16 + lg * 4 + v;
                if (m >= nrows) continue;
                const long long r = row0 + m;
                if (MODE == 0) {
                    const float g = acc[0][ms][ns][v], u = acc[1][ms][ns][v];
                    const float h = g / (1.0f + (float)exp(-(double)g)) * u;  // moe_forward.go:130
                    const int slot = (n & ~7) | ((n & 3) << 1) | ((n >> 2) & 1);
                    H[r * N + slot] = (_Float16)h;
                } else {
                    Y[r * N + n] = acc[0][ms][ns][v];
                }
            }
        }
}

// out[t][d] = sum_s w[t][s] * Y[pair_row[t*k+s]][d], summed from 0 in slot order.
__global__ void k_moe_combine(const float *__restrict__ Y, const int32_t *__restrict__ pair_row,
                              const float *__restrict__ w, int k, int n_tok, int hidden,
                              float *__restrict__ out) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;  // float4 index
    const long long n4 = (long long)n_tok * hidden / 4;
    if (i >= n4) return;
    const int t = (int)(i / (hidden / 4));
    const int d4 = (int)(i % (hidden / 4));
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < k; s++) {
        const float ws = w[t * k + s];
        const float4 y = reinterpret_cast<const float4 *>(Y + (long long)pair_row[t * k + s] * hidden)[d4];
        acc.x += ws * y.x;
        acc.y += ws * y.y;
        acc.z += ws * y.z;
        acc.w += ws * y.w;
    }
    reinterpret_cast<float4 *>(out)[i] = acc;
}

// ---------------------------------------------------------------------------
size_t llg_moe_gemm_ws_bytes(int n_tok, int k, int n_exp, int hidden, int eff) {
    const long long np = (long long)n_tok * k;
    const long long nt = np / GM_BM + n_exp + 1;
    return (size_t)(llg_align(np * 4, 256) * 2 + llg_align(nt * 16, 256) + 256 +
                    llg_align((long long)n_tok * hidden * 2, 256) +
                    llg_align(np * eff * 2, 256) + llg_align(np * hidden * 4, 256));
}

bool llg_moe_gemm_supported(int type, int hidden, int eff, int n_tok) {
    return type == LLG_TYPE_Q4_0 && n_tok >= 16 && hidden % GM_BN == 0 && eff % GM_BN == 0 &&
           hidden % GM_KC == 0 && eff % GM_KC == 0;
}

int llg_moe_gemm_enqueue(LlgDevice *d, const LlgObject *gate, const LlgObject *up,
                         const LlgObject *down, int n_exp, int k, int hidden, int eff,
                         const float *d_x, int n_tok, const int32_t *ids, const float *w,
                         float *d_out, uint8_t *ws) {
    hipStream_t st = llg_dev_stream(d);
    const long long np = (long long)n_tok * k;
    const long long nt_max = np / GM_BM + n_exp + 1;
    uint8_t *p = ws;
    int32_t *row_pair = reinterpret_cast<int32_t *>(p);
    p += llg_align(np * 4, 256);
    int32_t *pair_row = reinterpret_cast<int32_t *>(p);
    p += llg_align(np * 4, 256);
    int4 *tiles = reinterpret_cast<int4 *>(p);
    p += llg_align(nt_max * 16, 256);
    int32_t *n_tiles = reinterpret_cast<int32_t *>(p);
    p += 256;
    _Float16 *x16 = reinterpret_cast<_Float16 *>(p);
    p += llg_align((long long)n_tok * hidden * 2, 256);
    _Float16 *H = reinterpret_cast<_Float16 *>(p);
    p += llg_align(np * eff * 2, 256);
    float *Y = reinterpret_cast<float *>(p);

    hipLaunchKernelGGL(k_moe_group, dim3(1), dim3(1024), 0, st, ids, (int)np, n_exp, row_pair,
                       pair_row, tiles, n_tiles);
    const long long n8 = (long long)n_tok * hidden / 8;
    hipLaunchKernelGGL(k_moe_x16, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st, d_x, n8,
                       x16);
    hipLaunchKernelGGL((k_moe_gemm<0>), dim3((unsigned)(nt_max * (eff / GM_BN))), dim3(256), 0, st,
                       tiles, n_tiles, row_pair, k, x16, gate->d, up->d, gate->stride,
                       gate->fmt.d_off, eff, hidden, eff, H, (float *)nullptr);
    hipLaunchKernelGGL((k_moe_gemm<1>), dim3((unsigned)(nt_max * (hidden / GM_BN))), dim3(256), 0,
                       st, tiles, n_tiles, row_pair, k, H, down->d, (const uint8_t *)nullptr,
                       down->stride, down->fmt.d_off, hidden, eff, hidden, (_Float16 *)nullptr, Y);
    const long long n4 = (long long)n_tok * hidden / 4;
    hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, Y,
                       pair_row, w, k, n_tok, hidden, d_out);
    LLG_LAUNCH_CHECK(d, "moe grouped gemm");
    return 0;
}
