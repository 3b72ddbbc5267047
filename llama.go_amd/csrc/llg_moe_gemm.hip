// llg_moe_gemm.hip -- MoE FFN for a batch of tokens (prefill) as grouped
// MFMA GEMMs (inference/moe_forward.go:32-150 applied to every token; the
// reference runs them one token at a time, cmd/generate.go:88-96).
//
//   1. k_moe_router (llg_moe.hip): ids / weights per token
//   2. k_moe_group: counting sort of the (token, slot) pairs by expert, the
//      pair <-> row maps, and a list of M-tiles (expert, first row, rows):
//      each expert's rows in the fewest tiles of at most 80 rows, balanced
//   3. k_moe_x16: X -> f16 in the MFMA K order (k_order)
//   4. k_moe_gemm<0>: G = X_e . gate_e^T, U = X_e . up_e^T on v_mfma_f32_16x16x32_f16,
//      epilogue H = silu(G) * U (moe_forward.go:128-132) stored f16, same K order
//   5. k_moe_gemm<1>: Y = H_e . down_e^T
//   6. k_moe_combine: out[t] = sum_s w[t][s] * Y[row(t, s)], in slot order
//      from 0 (moe_forward.go:71-77)
//
// MFMA operands (16x16x32 f16): lane l holds 8 halves of A row l%16 and of B
// column l%16 for the K-group l/16; C lane l holds column l%16, rows
// 4*(l/16) .. +3.  A and B use the same K permutation, so the dot products are
// unchanged: in each 128-wide chunk (4 Q4_0 blocks), MFMA step j gives lane
// group g word j of block g, so a lane's 16-byte load of one block holds its
// B fragments for all 4 steps of the chunk.  The B fragment is built from the
// word with two and-or's per nibble pair (q4_frag), an exact subtraction of
// the offset and a multiply by the block scale.  The weights are read from
// a fragment-major copy of each matrix (k_gm_pack, made once per matrix at its
// first use), where the B fragments of one 16-column group and K chunk are
// 1152 contiguous bytes, so each B load instruction reads whole cache lines.
// Tiles: up to 80 rows per
// workgroup, 4 wavefronts of all the tile's rows each; a gate/up wavefront owns 32 columns
// of gate and the same 32 of up, a down wavefront 64 columns, so each A
// fragment feeds 4 MFMAs.  A in K chunks of 128 staged in LDS (double
// buffered; the next chunk is loaded into registers while the current one is
// multiplied); B straight into registers, one chunk ahead.
#include <type_traits>

#include "llg_common.hpp"
#include "llg_internal.hpp"

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

#define GM_BM 80
#define GM_MS (GM_BM / 16)  // 16-row MFMA groups of a tile
#define GM_KC 128                 // K per chunk
#define GM_KB (GM_KC / 32)        // Q4_0 blocks per chunk
#define GM_AST (GM_KC + 8)        // LDS A row stride (halves)
#ifndef GM_BD
#define GM_BD 1                   // chunks of B loads in flight ahead of use
#endif
#define GM_STORE_STEP 2           // MFMA step of a chunk before which the next A is stored

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
            // the fewest tiles of at most GM_BM rows (each streams the
            // expert's weights once), their sizes within one of each other
            const int n = (cnt[e] + GM_BM - 1) / GM_BM;
            for (int i = 0, r = 0; i < n; i++) {
                const int rows = cnt[e] / n + (i < cnt[e] % n ? 1 : 0);
                tiles[nt++] = make_int4(e, o + r, rows, 0);
                r += rows;
            }
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

// X (fp32, [n_tok x K]) -> f16 in the MFMA K order (k_order; K is a
// multiple of 128, so chunks never straddle rows): 8-group i goes to 8-group
// (i & ~15) | (i & 3) << 2 | (i >> 2) & 3, its elements in the order
// [0,4,1,5,2,6,3,7].
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
    const long long dst = (i & ~15ll) | ((i & 3) << 2) | ((i >> 2) & 3);
    reinterpret_cast<half8_t *>(x16)[dst] = h;
}

// The fragment-major copy of a Q4_0 matrix (rows a multiple of 16, columns of
// GM_KC): 16-row group g and K chunk c (GM_KB blocks) take the 1152 bytes at
// (g * nck + c) * 1152: lane l's 16 quant bytes (row 16 g + l % 16, block
// GM_KB c + l / 16) at l * 16, then the lanes' block scales at 1024 + 2 l.
// That is a wavefront's B fragments for the chunk's 4 MFMA steps (and their
// scales) in the lane order of k_moe_gemm's loads.  One thread per (g, c, l).
#define GM_FRAG_BYTES 1152
__global__ void k_gm_pack(const uint8_t *__restrict__ src, long long stride, int d_off, int nck,
                          long long n_units, uint8_t *__restrict__ dst) {
    const long long u = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= n_units) return;
    const int l = (int)(u & 63);
    const long long gc = u >> 6;  // g * nck + c
    const long long g = gc / nck;
    const int c = (int)(gc % nck);
    const uint8_t *row = src + (g * 16 + (l & 15)) * stride;
    const int blk = GM_KB * c + (l >> 4);
    uint8_t *o = dst + gc * GM_FRAG_BYTES;
    *reinterpret_cast<uint4 *>(o + l * 16) = *reinterpret_cast<const uint4 *>(row + blk * 16);
    *reinterpret_cast<unsigned short *>(o + 1024 + l * 2) =
        *reinterpret_cast<const unsigned short *>(row + d_off + blk * 2);
}

// The fragment-major copy of w, made (on the stream) at the first call.
static const uint8_t *gm_tiled(LlgDevice *d, const LlgObject *w, int *rc) {
    *rc = 0;
    if (w->tiled) return w->tiled;
    const int nck = w->fmt.cols / GM_KC;
    const size_t bytes = (size_t)w->rows / 16 * nck * GM_FRAG_BYTES;
    uint8_t *t = nullptr;
    if (hipMalloc(&t, bytes) != hipSuccess) {
        *rc = llg_set_error(d, LLG_E_NOMEM, "moe gemm: fragment-major copy (%zu bytes)", bytes);
        return nullptr;
    }
    const long long n_units = (long long)w->rows / 16 * nck * 64;
    hipLaunchKernelGGL(k_gm_pack, dim3((unsigned)((n_units + 255) / 256)), dim3(256), 0,
                       llg_dev_stream(d), w->d, w->stride, w->fmt.d_off, nck, n_units, t);
    if (hipError_t e = hipGetLastError(); e != hipSuccess) {
        hipFree(t);
        *rc = llg_hip_error(d, e, "moe gemm: fragment-major copy");
        return nullptr;
    }
    w->tiled = t;
    return t;
}

// (a & m) | o in one instruction
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(o));
    return r;
}

// B fragment: word g of a Q4_0 block (nibble p = element 8g+p) times scale d,
// as f16 in the order [e0,e4,e1,e5,e2,e6,e3,e7].  A nibble at bits 0-3 of an
// f16 under exponent bits 0x6400 is the exact value 1024 + q; one at bits 4-7
// under 0x5400 is 64 + q (ulp 1/16).  So the two nibble pairs of each byte
// pair need one shift between them, and subtracting 1032 or 72 gives q - 8
// exactly before the scale.
__device__ __forceinline__ half8_t q4_frag(uint32_t w, _Float16 d) {
    const half2_t off_lo = {(_Float16)1032.0f, (_Float16)1032.0f};
    const half2_t off_hi = {(_Float16)72.0f, (_Float16)72.0f};
    const half2_t dd = {d, d};
    const uint32_t w8 = w >> 8;
    const uint32_t m_lo = 0x000F000Fu, m_hi = 0x00F000F0u, e_lo = 0x64006400u, e_hi = 0x54005400u;
    const half2_t v0 = (__builtin_bit_cast(half2_t, and_or(w, m_lo, e_lo)) - off_lo) * dd;
    const half2_t v1 = (__builtin_bit_cast(half2_t, and_or(w, m_hi, e_hi)) - off_hi) * dd;
    const half2_t v2 = (__builtin_bit_cast(half2_t, and_or(w8, m_lo, e_lo)) - off_lo) * dd;
    const half2_t v3 = (__builtin_bit_cast(half2_t, and_or(w8, m_hi, e_hi)) - off_hi) * dd;
    half8_t r;
    r[0] = v0[0];
    r[1] = v0[1];
    r[2] = v1[0];
    r[3] = v1[1];
    r[4] = v2[0];
    r[5] = v2[1];
    r[6] = v3[0];
    r[7] = v3[1];
    return r;
}

// Position of element k of a row in the MFMA K order: within each 128-wide
// chunk, MFMA step j (0..3) takes word j (elements 8j..8j+7) of block g for
// lane group g, so the 8-group of word j of block g sits at 8-group j*4 + g;
// inside it, nibble order [0,4,1,5,2,6,3,7] (q4_frag's).
__device__ __forceinline__ int k_order(int k) {
    const int gi = k >> 3;  // 8-group
    const int dst = (gi & ~15) | ((gi & 3) << 2) | ((gi >> 2) & 3);
    const int p = k & 7;
    return dst * 8 + ((p & 3) << 1) + (p >> 2);
}

// MODE 0: gate+up with SwiGLU epilogue -> H (f16, MFMA K order, [rows x N]).
// MODE 1: down -> Y (f32, [rows x N]), K split into ksplit equal slices: slice
// q writes its partial product to Y + q * ystride (the combine adds them).
// blockIdx = (M tile * N tiles + N tile) * ksplit + slice.
// A rows: MODE 0 gathers X16 row row_pair[r] / k (the pair's token); MODE 1
// reads H row r.  A goes through LDS (every wavefront reads all the rows); B
// is private to a wavefront (its columns), so each lane loads its own
// block of each column straight into registers: lane (column n, group g)
// takes the 16 quant bytes and the scale of block 4c + g of chunk c, whose
// word j is the lane's B fragment at MFMA step j.
// Columns per wavefront of each weight matrix: gate/up 32 of gate and 32 of
// up, down 64, so both take 4 B fragments per K step and every A fragment read
// from LDS feeds 4 MFMAs.
template <int MODE>
constexpr int gm_wave_cols() {
    return MODE == 0 ? 32 : 64;
}

template <int MODE>
__global__ __launch_bounds__(256, 2) void k_moe_gemm(
    const int4 *__restrict__ tiles, const int32_t *__restrict__ n_tiles_p,
    const int32_t *__restrict__ row_pair, int k_slots, const _Float16 *__restrict__ A,
    const uint8_t *__restrict__ W0, const uint8_t *__restrict__ W1, int rows_per_expert, int K,
    int N, _Float16 *__restrict__ H,
    float *__restrict__ Y, int ksplit, long long ystride) {
    constexpr int NF = 4;                     // B fragments per wavefront per K step
    constexpr int WC = gm_wave_cols<MODE>();  // columns per wavefront per matrix
    __shared__ __attribute__((aligned(16))) _Float16 As[2][GM_BM * GM_AST];
    const int n_ntiles = N / (4 * WC);
    const int ks = blockIdx.x % ksplit;
    const int nt = (blockIdx.x / ksplit) % n_ntiles;
    const int mt = blockIdx.x / ksplit / n_ntiles;
    if (mt >= *n_tiles_p) return;
    const int4 tile = tiles[mt];
    const int e = tile.x, row0 = tile.y, nrows = tile.z;
    const int n0 = nt * 4 * WC;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;

    // The tile's rows take NMS = ceil(nrows / 16) of the GM_MS 16-row MFMA
    // groups; the body is instantiated per NMS and chosen once per workgroup,
    // so a ragged tile issues no MFMAs, A loads or stores for its empty groups
    // and each instance stays straight-line code.
    auto body = [&](auto nms_c) __attribute__((always_inline)) {
    constexpr int NMS = decltype(nms_c)::value;
    // A: GM_BM rows x 16 uint4 per chunk -> thread load q covers rows 16 q ..
    // 16 q + 15, so only q < NMS are needed (rows past the tile reload the
    // tile's last row; their results are dropped).
    long long a_off[GM_MS];
#pragma unroll
    for (int q = 0; q < NMS; q++) {
        const int idx = tid + 256 * q;
        const int r = idx >> 4, part = idx & 15;
        const int rr = min(r, nrows - 1);
        const long long arow = MODE == 0 ? row_pair[row0 + rr] / k_slots : row0 + rr;
        a_off[q] = arow * K + part * 8;
    }
    // B: fragment f = (matrix m, 16-column group ns) -> columns
    // n0 + wave*WC + ns*16 .. + 15 of matrix m (gate/up: m = f / 2, ns = f % 2;
    // down: m = 0, ns = f), the 16-row group of the fragment-major copy whose
    // chunk c holds the lane's block 4c + lg of column n0 + wave*WC + ns*16 + li
    // at lane * 16 (its scale at 1024 + lane * 2).
    const int nck = K / GM_KC;
    const uint8_t *brow[NF];
#pragma unroll
    for (int f = 0; f < NF; f++) {
        const int m = MODE == 0 ? f / 2 : 0, ns = MODE == 0 ? f % 2 : f;
        const uint8_t *W = m == 1 ? W1 : W0;
        const long long g = ((long long)e * rows_per_expert + n0 + wave * WC + ns * 16) / 16;
        brow[f] = W + g * nck * GM_FRAG_BYTES;
    }

    constexpr int NB = GM_BD + 1;                  // B register slots
    constexpr int UNR = NB % 2 == 0 ? NB : 2 * NB;  // loop unroll: static A buffer and B slot
    u32x4_t ra[GM_MS];
    u32x4_t bq[NB][NF];
    _Float16 bd[NB][NF];  // block scales as loaded (no conversion that would wait for them)
#define GM_LOAD_A(c)                                                                             \
    _Pragma("unroll") for (int q = 0; q < NMS; q++) ra[q] =                                     \
        *reinterpret_cast<const u32x4_t *>(A + a_off[q] + (long long)(c) * GM_KC)
#define GM_LOAD_B(c, slot)                                                                       \
    _Pragma("unroll") for (int f = 0; f < NF; f++) {                                             \
        const uint8_t *fr = brow[f] + (long long)(c) * GM_FRAG_BYTES;                            \
        bq[slot][f] = *reinterpret_cast<const u32x4_t *>(fr + lane * 16);                        \
        bd[slot][f] = *reinterpret_cast<const _Float16 *>(fr + 1024 + lane * 2);                 \
    }
#define GM_STORE_A(buf)                                                                          \
    _Pragma("unroll") for (int q = 0; q < NMS; q++) {                                           \
        const int idx = tid + 256 * q;                                                           \
        *reinterpret_cast<u32x4_t *>(&As[buf][(idx >> 4) * GM_AST + (idx & 15) * 8]) = ra[q];    \
    }

    floatx4_t acc[NF][NMS];  // [fragment][16-row group]
#pragma unroll
    for (int f = 0; f < NF; f++)
#pragma unroll
        for (int i = 0; i < NMS; i++) acc[f][i] = {0.f, 0.f, 0.f, 0.f};

    const int ncs = K / GM_KC / ksplit;  // chunks of this slice: c0 .. ce - 1
    const int c0 = ks * ncs, ce = c0 + ncs;
    GM_LOAD_A(c0);
#pragma unroll
    for (int i = 0; i < GM_BD; i++) GM_LOAD_B(min(c0 + i, ce - 1), i);
    GM_STORE_A(0);
    __syncthreads();
    // chunk c (the i-th of the slice): A in As[i & 1], B in slot i % NB.  First
    // the loads of A for chunk c + 1 and of B for chunk c + GM_BD are issued
    // (past the end, the last chunk is reloaded and not used).  A for chunk
    // c + 1 goes to the free buffer after the chunk's second step (the buffer
    // was last read in chunk c - 1, before the barrier that ended it): storing
    // it at the end of the chunk, or under a condition, let the compiler move
    // its loads down to the store and wait for every outstanding load there,
    // the next chunks' B included.
    auto chunk = [&](int c, int buf, int slot) __attribute__((always_inline)) {
        GM_LOAD_A(min(c + 1, ce - 1));
        GM_LOAD_B(min(c + GM_BD, ce - 1), (slot + GM_BD) % NB);
        __builtin_amdgcn_sched_barrier(0);  // the loads stay ahead of the steps
#pragma unroll
        for (int s = 0; s < 4; s++) {
            if (s == GM_STORE_STEP) {  // the last chunk stores its reload, unread
                __builtin_amdgcn_sched_barrier(0);
                GM_STORE_A(buf ^ 1);
                __builtin_amdgcn_sched_barrier(0);
            }
            half8_t a[NMS];
#pragma unroll
            for (int ms = 0; ms < NMS; ms++)
                a[ms] = *reinterpret_cast<const half8_t *>(
                    &As[buf][(ms * 16 + li) * GM_AST + s * 32 + lg * 8]);
#pragma unroll
            for (int f = 0; f < NF; f++) {
                const uint32_t w = bq[slot][f][s];
                const half8_t b = q4_frag(w, bd[slot][f]);
#pragma unroll
                for (int ms = 0; ms < NMS; ms++)
                    acc[f][ms] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[ms], b, acc[f][ms], 0, 0, 0);
            }
        }
        __syncthreads();
    };
    for (int c = c0; c < ce; c += UNR) {
#pragma unroll
        for (int i = 0; i < UNR; i++)
            if (c + i < ce) chunk(c + i, i & 1, i % NB);
    }
#undef GM_LOAD_A
#undef GM_LOAD_B
#undef GM_STORE_A

    // epilogue: gate/up pairs fragment ns (gate) with ns + 2 (up)
    constexpr int NS = MODE == 0 ? 2 : 4;  // 16-column groups per wavefront
#pragma unroll
    for (int ms = 0; ms < NMS; ms++)
#pragma unroll
        for (int ns = 0; ns < NS; ns++) {
            const int n = n0 + wave * WC + ns * 16 + li;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int m = ms * 16 + lg * 4 + v;
                if (m >= nrows) continue;
                const long long r = row0 + m;
                if (MODE == 0) {
                    const float g = acc[ns][ms][v], u = acc[ns + 2][ms][v];
                    const float h = g / (1.0f + (float)exp(-(double)g)) * u;  // moe_forward.go:130
                    H[r * N + k_order(n)] = (_Float16)h;
                } else {
                    Y[ks * ystride + r * N + n] = acc[ns][ms][v];
                }
            }
        }
    };
    switch ((nrows + 15) / 16) {
    case 1: body(std::integral_constant<int, 1>{}); break;
    case 2: body(std::integral_constant<int, 2>{}); break;
    case 3: body(std::integral_constant<int, 3>{}); break;
    case 4: body(std::integral_constant<int, 4>{}); break;
    default: body(std::integral_constant<int, 5>{}); break;
    }
}

// out[t][d] = sum_s w[t][s] * Y[pair_row[t*k+s]][d], summed from 0 in slot order;
// Y of a pair is the sum of its ksplit K-slice partials, in slice order.
__global__ void k_moe_combine(const float *__restrict__ Y, const int32_t *__restrict__ pair_row,
                              const float *__restrict__ w, int k, int n_tok, int hidden,
                              int ksplit, long long ystride, float *__restrict__ out) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;  // float4 index
    const long long n4 = (long long)n_tok * hidden / 4;
    if (i >= n4) return;
    const int t = (int)(i / (hidden / 4));
    const int d4 = (int)(i % (hidden / 4));
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < k; s++) {
        const float ws = w[t * k + s];
        const float *yr = Y + (long long)pair_row[t * k + s] * hidden;
        float4 y = reinterpret_cast<const float4 *>(yr)[d4];
        for (int q = 1; q < ksplit; q++) {
            const float4 p = reinterpret_cast<const float4 *>(yr + q * ystride)[d4];
            y.x += p.x;
            y.y += p.y;
            y.z += p.z;
            y.w += p.w;
        }
        acc.x += ws * y.x;
        acc.y += ws * y.y;
        acc.z += ws * y.z;
        acc.w += ws * y.w;
    }
    reinterpret_cast<float4 *>(out)[i] = acc;
}

// K slices of the down GEMM: 4 (or 2) when the chunks divide evenly, so that
// the launch has enough independent workgroups to keep loads in flight.
static int down_split(int eff) {
    const int nc = eff / GM_KC;
    return nc % 4 == 0 ? 4 : nc % 2 == 0 ? 2 : 1;
}

// ---------------------------------------------------------------------------
size_t llg_moe_gemm_ws_bytes(int n_tok, int k, int n_exp, int hidden, int eff) {
    const long long np = (long long)n_tok * k;
    const long long nt = np / GM_BM + n_exp + 1;
    return (size_t)(llg_align(np * 4, 256) * 2 + llg_align(nt * 16, 256) + 256 +
                    llg_align((long long)n_tok * hidden * 2, 256) +
                    llg_align(np * eff * 2, 256) + down_split(eff) * llg_align(np * hidden * 4, 256));
}

bool llg_moe_gemm_supported(int type, int hidden, int eff, int n_tok) {
    return type == LLG_TYPE_Q4_0 && n_tok >= 16 && hidden % (4 * gm_wave_cols<1>()) == 0 &&
           eff % (4 * gm_wave_cols<0>()) == 0 &&
           hidden % GM_KC == 0 && eff % GM_KC == 0;
}

int llg_moe_gemm_enqueue(LlgDevice *d, const LlgObject *gate, const LlgObject *up,
                         const LlgObject *down, int n_exp, int k, int hidden, int eff,
                         const float *d_x, int n_tok, const int32_t *ids, const float *w,
                         float *d_out, uint8_t *ws) {
    int rc = 0;
    const uint8_t *tg = gm_tiled(d, gate, &rc);
    const uint8_t *tu = rc ? nullptr : gm_tiled(d, up, &rc);
    const uint8_t *td = rc ? nullptr : gm_tiled(d, down, &rc);
    if (rc) return rc;
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
    hipLaunchKernelGGL((k_moe_gemm<0>), dim3((unsigned)(nt_max * (eff / (4 * gm_wave_cols<0>())))),
                       dim3(256), 0, st,
                       tiles, n_tiles, row_pair, k, x16, tg, tu, eff, hidden, eff, H,
                       (float *)nullptr, 1, 0ll);
    const int ksplit = down_split(eff);
    const long long ystride = llg_align(np * hidden * 4, 256) / 4;
    hipLaunchKernelGGL((k_moe_gemm<1>),
                       dim3((unsigned)(nt_max * (hidden / (4 * gm_wave_cols<1>())) * ksplit)),
                       dim3(256), 0, st, tiles, n_tiles, row_pair, k, H, td,
                       (const uint8_t *)nullptr, hidden, eff, hidden, (_Float16 *)nullptr, Y,
                       ksplit, ystride);
    const long long n4 = (long long)n_tok * hidden / 4;
    hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, Y,
                       pair_row, w, k, n_tok, hidden, ksplit, ystride, d_out);
    LLG_LAUNCH_CHECK(d, "moe grouped gemm");
    return 0;
}
