// llg_common.hpp -- shared host/device definitions for the gfx950 sparse-FFN library.
//
// HBM row layout ("row format").  A GGUF row of `cols` elements
// (gguf/types.go:90-102: ByteSize = cols/32 * 18 for Q4_0, * 34 for Q8_0) is
// stored per row as struct-of-arrays so that every lane can issue 16-byte
// aligned loads:
//   Q4_0: [ qs: nb x 16 B ][ d: nb x 2 B (f16) ][ pad to 128 B ]
//   Q8_0: [ qs: nb x 32 B ][ d: nb x 2 B (f16) ][ pad to 128 B ]
//   F16 : [ cols x 2 B ][ pad ]      F32: [ cols x 4 B ][ pad ]
// where nb = cols / 32.  The bytes of each block are the GGUF bytes
// unchanged; only the scale and the quants of one row are split apart.  For
// Q4_0 the reference decodes element 2i from the low nibble and element 2i+1
// from the high nibble of byte i (tensor/dtype.go:73-79), so nibble p of the
// little-endian 32-bit word w of a block is element 8w + p.
//
// A bundle (flash/bundle.go:22-24) stores, per neuron, the up row followed by
// the down row, each in the row format above: one contiguous span of
// 2 * stride bytes per neuron.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/llg_hip.h"

typedef _Float16 half2_llg __attribute__((ext_vector_type(2)));

#define LLG_ROW_ALIGN 128

struct RowFmt {
    int type;        // ggml type code
    int cols;        // elements per row
    int nb;          // 32-element blocks per row (cols / 32, rounded up for F16/F32)
    int d_off;       // byte offset of the f16 scales inside a row (Q4_0 / Q8_0)
    long long stride;  // bytes per row in HBM
};

static inline long long llg_align(long long v, long long a) { return (v + a - 1) / a * a; }

// Returns 0 and fills *f, or an LLG_E_* code (types.go:93-100 semantics).
static inline int llg_row_fmt(int type, int cols, RowFmt *f) {
    if (cols <= 0) return LLG_E_ARG;
    f->type = type;
    f->cols = cols;
    switch (type) {
    case LLG_TYPE_Q4_0:
        if (cols % 32) return LLG_E_ALIGN;
        f->nb = cols / 32;
        f->d_off = f->nb * 16;
        f->stride = llg_align((long long)f->nb * 18, LLG_ROW_ALIGN);
        return 0;
    case LLG_TYPE_Q8_0:
        if (cols % 32) return LLG_E_ALIGN;
        f->nb = cols / 32;
        f->d_off = f->nb * 32;
        f->stride = llg_align((long long)f->nb * 34, LLG_ROW_ALIGN);
        return 0;
    case LLG_TYPE_F16:
        f->nb = (cols + 31) / 32;
        f->d_off = 0;
        f->stride = llg_align((long long)cols * 2, LLG_ROW_ALIGN);
        return 0;
    case LLG_TYPE_F32:
        f->nb = (cols + 31) / 32;
        f->d_off = 0;
        f->stride = llg_align((long long)cols * 4, LLG_ROW_ALIGN);
        return 0;
    default:
        return LLG_E_TYPE;
    }
}

// GGUF bytes per row: gguf/types.go:90-102.
static inline long long llg_gguf_row_bytes(int type, int cols) {
    switch (type) {
    case LLG_TYPE_Q4_0: return (long long)(cols / 32) * 18;
    case LLG_TYPE_Q8_0: return (long long)(cols / 32) * 34;
    case LLG_TYPE_F16: return (long long)cols * 2;
    case LLG_TYPE_F32: return (long long)cols * 4;
    default: return -1;
    }
}

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------

// f16 -> f32 with the reference's semantics (tensor/dtype.go:417-443):
// subnormals normalised, +-Inf kept, every NaN becomes sign|0x7FC00000.
__device__ __forceinline__ float llg_f16_ref(uint32_t h) {
    uint32_t sign = (h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1F;
    uint32_t m = h & 0x3FF;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            // normalise: shift the leading one into bit 10
            int lz = __clz(m) - 21;  // m < 0x400, so clz(m) >= 22; lz = shifts needed
            m = (m << lz) & 0x3FF;
            bits = sign | ((uint32_t)(113 - lz) << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = sign | (m ? 0x7FC00000u : 0x7F800000u);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    return __uint_as_float(bits);
}

// Hardware f16 -> f32 (identical to llg_f16_ref for every non-NaN input).
__device__ __forceinline__ float llg_f16(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)h));
}

// DPP lane moves (GFX9 encodings): quad_perm xor-1 = 0xB1, xor-2 = 0x4E;
// row_ror:n = 0x120 + n rotates within each row of 16 lanes.
template <int CTRL>
__device__ __forceinline__ float llg_dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over the 4 lanes of each quad, in every lane of the quad.
__device__ __forceinline__ float llg_quad_sum(float v) {
    v += llg_dpp<0xB1>(v);
    v += llg_dpp<0x4E>(v);
    return v;
}

// Sum over the wavefront, returned in every lane: quad and row sums through
// DPP, then the four row sums read out with v_readlane.
__device__ __forceinline__ float llg_wave_sum(float v) {
    v = llg_quad_sum(v);
    v += llg_dpp<0x124>(v);  // row_ror:4
    v += llg_dpp<0x128>(v);  // row_ror:8
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

// Activations, with the reference's rounding: ops.go:168-189.
__device__ __forceinline__ float llg_act(int act, float v) {
    if (act == LLG_ACT_SILU) {
        return v / (1.0f + (float)exp(-(double)v));
    } else if (act == LLG_ACT_GELU) {
        const float c = 0.7978845608028654f;
        const float k = 0.044715f;
        float inner = c * (v + k * v * v * v);
        return 0.5f * v * (1.0f + (float)tanh((double)inner));
    }
    return v < 0.0f ? 0.0f : v;  // NaN and -0.0 pass through, as ops.go:170
}

// One 32-element block b of a row: dot with x[32] (x given as 8 float4).
template <int T>
__device__ __forceinline__ float llg_block_dot(const uint8_t *__restrict__ row, const RowFmt &f,
                                               int b, const float4 *__restrict__ x4);

template <>
__device__ __forceinline__ float llg_block_dot<LLG_TYPE_Q4_0>(const uint8_t *__restrict__ row,
                                                               const RowFmt &f, int b,
                                                               const float4 *__restrict__ x4) {
    const uint4 q = *reinterpret_cast<const uint4 *>(row + (size_t)b * 16);
    const float d = llg_f16(*reinterpret_cast<const unsigned short *>(row + f.d_off + b * 2));
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 xa = x4[2 * i], xb = x4[2 * i + 1];
        const uint32_t v = w[i];
        s += (float)((int)((v >> 0) & 15) - 8) * xa.x;
        s += (float)((int)((v >> 4) & 15) - 8) * xa.y;
        s += (float)((int)((v >> 8) & 15) - 8) * xa.z;
        s += (float)((int)((v >> 12) & 15) - 8) * xa.w;
        s += (float)((int)((v >> 16) & 15) - 8) * xb.x;
        s += (float)((int)((v >> 20) & 15) - 8) * xb.y;
        s += (float)((int)((v >> 24) & 15) - 8) * xb.z;
        s += (float)((int)((v >> 28) & 15) - 8) * xb.w;
    }
    return s * d;
}

template <>
__device__ __forceinline__ float llg_block_dot<LLG_TYPE_Q8_0>(const uint8_t *__restrict__ row,
                                                               const RowFmt &f, int b,
                                                               const float4 *__restrict__ x4) {
    const uint4 qa = *reinterpret_cast<const uint4 *>(row + (size_t)b * 32);
    const uint4 qb = *reinterpret_cast<const uint4 *>(row + (size_t)b * 32 + 16);
    const float d = llg_f16(*reinterpret_cast<const unsigned short *>(row + f.d_off + b * 2));
    const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 xv = x4[i];
        const uint32_t v = w[i];
        s += (float)(int8_t)(v & 0xFF) * xv.x;
        s += (float)(int8_t)((v >> 8) & 0xFF) * xv.y;
        s += (float)(int8_t)((v >> 16) & 0xFF) * xv.z;
        s += (float)(int8_t)(v >> 24) * xv.w;
    }
    return s * d;
}

template <>
__device__ __forceinline__ float llg_block_dot<LLG_TYPE_F16>(const uint8_t *__restrict__ row,
                                                              const RowFmt &f, int b,
                                                              const float4 *__restrict__ x4) {
    const uint4 *p = reinterpret_cast<const uint4 *>(row + (size_t)b * 64);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint4 q = p[i];
        const float4 xa = x4[2 * i], xb = x4[2 * i + 1];
        s += llg_f16(q.x & 0xFFFF) * xa.x;
        s += llg_f16(q.x >> 16) * xa.y;
        s += llg_f16(q.y & 0xFFFF) * xa.z;
        s += llg_f16(q.y >> 16) * xa.w;
        s += llg_f16(q.z & 0xFFFF) * xb.x;
        s += llg_f16(q.z >> 16) * xb.y;
        s += llg_f16(q.w & 0xFFFF) * xb.z;
        s += llg_f16(q.w >> 16) * xb.w;
    }
    return s;
}

template <>
__device__ __forceinline__ float llg_block_dot<LLG_TYPE_F32>(const uint8_t *__restrict__ row,
                                                              const RowFmt &f, int b,
                                                              const float4 *__restrict__ x4) {
    const float4 *p = reinterpret_cast<const float4 *>(row + (size_t)b * 128);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 w = p[i];
        const float4 xv = x4[i];
        s += w.x * xv.x;
        s += w.y * xv.y;
        s += w.z * xv.z;
        s += w.w * xv.w;
    }
    return s;
}

// acc[0..31] += u * dequant(block b of row).
template <int T>
__device__ __forceinline__ void llg_block_axpy(const uint8_t *__restrict__ row, const RowFmt &f,
                                               int b, float u, float *acc);

template <>
__device__ __forceinline__ void llg_block_axpy<LLG_TYPE_Q4_0>(const uint8_t *__restrict__ row,
                                                               const RowFmt &f, int b, float u,
                                                               float *acc) {
    const uint4 q = *reinterpret_cast<const uint4 *>(row + (size_t)b * 16);
    const float s = u * llg_f16(*reinterpret_cast<const unsigned short *>(row + f.d_off + b * 2));
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int p = 0; p < 8; p++)
            acc[8 * i + p] += s * (float)((int)((w[i] >> (4 * p)) & 15) - 8);
}

template <>
__device__ __forceinline__ void llg_block_axpy<LLG_TYPE_Q8_0>(const uint8_t *__restrict__ row,
                                                               const RowFmt &f, int b, float u,
                                                               float *acc) {
    const uint4 qa = *reinterpret_cast<const uint4 *>(row + (size_t)b * 32);
    const uint4 qb = *reinterpret_cast<const uint4 *>(row + (size_t)b * 32 + 16);
    const float s = u * llg_f16(*reinterpret_cast<const unsigned short *>(row + f.d_off + b * 2));
    const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int p = 0; p < 4; p++) acc[4 * i + p] += s * (float)(int8_t)((w[i] >> (8 * p)) & 0xFF);
}

template <>
__device__ __forceinline__ void llg_block_axpy<LLG_TYPE_F16>(const uint8_t *__restrict__ row,
                                                              const RowFmt &f, int b, float u,
                                                              float *acc) {
    const uint4 *p = reinterpret_cast<const uint4 *>(row + (size_t)b * 64);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint4 q = p[i];
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            acc[8 * i + 2 * k] += u * llg_f16(w[k] & 0xFFFF);
            acc[8 * i + 2 * k + 1] += u * llg_f16(w[k] >> 16);
        }
    }
}

template <>
__device__ __forceinline__ void llg_block_axpy<LLG_TYPE_F32>(const uint8_t *__restrict__ row,
                                                              const RowFmt &f, int b, float u,
                                                              float *acc) {
    const float4 *p = reinterpret_cast<const float4 *>(row + (size_t)b * 128);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 w = p[i];
        acc[4 * i + 0] += u * w.x;
        acc[4 * i + 1] += u * w.y;
        acc[4 * i + 2] += u * w.z;
        acc[4 * i + 3] += u * w.w;
    }
}

// Element c of a row in the row format, bit-exact (tensor/dtype.go:12-82).
__device__ __forceinline__ float llg_dequant_elem(const uint8_t *row, const RowFmt &f, int c) {
    switch (f.type) {
    case LLG_TYPE_Q4_0: {
        const int b = c >> 5, e = c & 31;
        const uint8_t byte = row[b * 16 + (e >> 1)];
        const int q = (e & 1) ? (byte >> 4) : (byte & 15);
        const uint32_t hb = row[f.d_off + 2 * b] | (row[f.d_off + 2 * b + 1] << 8);
        return (float)(q - 8) * llg_f16_ref(hb);
    }
    case LLG_TYPE_Q8_0: {
        const int b = c >> 5, e = c & 31;
        const int8_t q = (int8_t)row[b * 32 + e];
        const uint32_t hb = row[f.d_off + 2 * b] | (row[f.d_off + 2 * b + 1] << 8);
        return (float)q * llg_f16_ref(hb);
    }
    case LLG_TYPE_F16: {
        const uint32_t hb = row[2 * c] | (row[2 * c + 1] << 8);
        return llg_f16_ref(hb);
    }
    default:
        return reinterpret_cast<const float *>(row)[c];
    }
}

// ---------------------------------------------------------------------------
// Split load / compute forms of one 32-element block.  Kernels load the raw
// bytes of all the blocks a lane owns first (BlockRaw), so their memory
// requests are in flight together, and only then dequantize and use them.
// ---------------------------------------------------------------------------
template <int T>
struct BlockRaw;
template <>
struct BlockRaw<LLG_TYPE_Q4_0> {
    uint4 q;
    unsigned short d;
};
template <>
struct BlockRaw<LLG_TYPE_Q8_0> {
    uint4 q0, q1;
    unsigned short d;
};
template <>
struct BlockRaw<LLG_TYPE_F16> {
    uint4 q[4];
};
template <>
struct BlockRaw<LLG_TYPE_F32> {
    float4 q[8];
};

// r, or (keep false) a block whose dot is 0 for finite x: the scale (or
// the values) zeroed by a select, so a dot can run unconditionally on every
// lane and the compiler has no branch to move the block's loads into.
template <int T>
__device__ __forceinline__ void llg_block_keep(BlockRaw<T> &r, bool keep) {
    if constexpr (T == LLG_TYPE_Q4_0 || T == LLG_TYPE_Q8_0) {
        r.d = keep ? r.d : (unsigned short)0;
    } else if constexpr (T == LLG_TYPE_F16) {
#pragma unroll
        for (int i = 0; i < 4; i++) r.q[i] = keep ? r.q[i] : make_uint4(0u, 0u, 0u, 0u);
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) r.q[i] = keep ? r.q[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

template <int T>
__device__ __forceinline__ void llg_block_load(BlockRaw<T> &r, const uint8_t *__restrict__ row,
                                               const RowFmt &f, int b);
template <>
__device__ __forceinline__ void llg_block_load<LLG_TYPE_Q4_0>(BlockRaw<LLG_TYPE_Q4_0> &r,
                                                               const uint8_t *__restrict__ row,
                                                               const RowFmt &f, int b) {
    r.q = *reinterpret_cast<const uint4 *>(row + (size_t)b * 16);
    r.d = *reinterpret_cast<const unsigned short *>(row + f.d_off + b * 2);
}
template <>
__device__ __forceinline__ void llg_block_load<LLG_TYPE_Q8_0>(BlockRaw<LLG_TYPE_Q8_0> &r,
                                                               const uint8_t *__restrict__ row,
                                                               const RowFmt &f, int b) {
    r.q0 = *reinterpret_cast<const uint4 *>(row + (size_t)b * 32);
    r.q1 = *reinterpret_cast<const uint4 *>(row + (size_t)b * 32 + 16);
    r.d = *reinterpret_cast<const unsigned short *>(row + f.d_off + b * 2);
}
template <>
__device__ __forceinline__ void llg_block_load<LLG_TYPE_F16>(BlockRaw<LLG_TYPE_F16> &r,
                                                              const uint8_t *__restrict__ row,
                                                              const RowFmt &f, int b) {
    const uint4 *p = reinterpret_cast<const uint4 *>(row + (size_t)b * 64);
#pragma unroll
    for (int i = 0; i < 4; i++) r.q[i] = p[i];
}
template <>
__device__ __forceinline__ void llg_block_load<LLG_TYPE_F32>(BlockRaw<LLG_TYPE_F32> &r,
                                                              const uint8_t *__restrict__ row,
                                                              const RowFmt &f, int b) {
    const float4 *p = reinterpret_cast<const float4 *>(row + (size_t)b * 128);
#pragma unroll
    for (int i = 0; i < 8; i++) r.q[i] = p[i];
}

// dot(dequant(block), x[32]) from loaded bytes; xsum = sum of the 32 x values.
// Q4_0 sums (64 + q) * x over f16 values built from the nibbles and subtracts
// 72 * xsum once; Q8_0 flips the sign bit of every byte (q + 128 in [0, 255])
// and subtracts 128 * xsum.  F16/F32 ignore xsum.  The offset term is an
// explicit fused multiply-add (as are the F16/F32 products), so a dot rounds
// the same in every kernel that inlines it: left to the compiler, 72 * xsum
// shared by two rows' dots stayed a separate multiply, fused elsewhere.  The
// Q8_0 products are the row's own and contract the same everywhere.
template <int T>
__device__ __forceinline__ float llg_raw_dot(const BlockRaw<T> &r, const float4 *x4, float xsum);
// (a & m) | o in one instruction
__device__ __forceinline__ uint32_t llg_and_or(uint32_t a, uint32_t m, uint32_t o) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(o));
    return r;
}

template <>
__device__ __forceinline__ float llg_raw_dot<LLG_TYPE_Q4_0>(const BlockRaw<LLG_TYPE_Q4_0> &r,
                                                             const float4 *x4, float xsum) {
    // Nibble p of word i is element 8i + p.  A nibble at bits 4-7 of an f16
    // whose other bits are 0x5400 is exactly 64 + q, so one shift and one
    // and-or give the pair (64 + q_p, 64 + q_{p+4}) of a word, and the f16
    // values multiply fp32 x directly (v_fma_mix_f32).  The sum of
    // (64 + q) x less 72 xsum is the sum of (q - 8) x.
    const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    const uint32_t m = 0x00F000F0u, e = 0x54005400u;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 xa = x4[2 * i], xb = x4[2 * i + 1];
        const half2_llg p0 = __builtin_bit_cast(half2_llg, llg_and_or(w[i] << 4, m, e));
        const half2_llg p1 = __builtin_bit_cast(half2_llg, llg_and_or(w[i], m, e));
        const half2_llg p2 = __builtin_bit_cast(half2_llg, llg_and_or(w[i] >> 4, m, e));
        const half2_llg p3 = __builtin_bit_cast(half2_llg, llg_and_or(w[i] >> 8, m, e));
        s = __builtin_fmaf((float)p0[0], xa.x, s);
        s = __builtin_fmaf((float)p1[0], xa.y, s);
        s = __builtin_fmaf((float)p2[0], xa.z, s);
        s = __builtin_fmaf((float)p3[0], xa.w, s);
        s = __builtin_fmaf((float)p0[1], xb.x, s);
        s = __builtin_fmaf((float)p1[1], xb.y, s);
        s = __builtin_fmaf((float)p2[1], xb.z, s);
        s = __builtin_fmaf((float)p3[1], xb.w, s);
    }
    return __builtin_fmaf(-72.0f, xsum, s) * llg_f16(r.d);
}
template <>
__device__ __forceinline__ float llg_raw_dot<LLG_TYPE_Q8_0>(const BlockRaw<LLG_TYPE_Q8_0> &r,
                                                             const float4 *x4, float xsum) {
    const uint32_t w[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 xv = x4[i];
        const uint32_t v = w[i] ^ 0x80808080u;  // byte = q + 128
        s += (float)(v & 0xFF) * xv.x;
        s += (float)((v >> 8) & 0xFF) * xv.y;
        s += (float)((v >> 16) & 0xFF) * xv.z;
        s += (float)(v >> 24) * xv.w;
    }
    return __builtin_fmaf(-128.0f, xsum, s) * llg_f16(r.d);
}
template <>
__device__ __forceinline__ float llg_raw_dot<LLG_TYPE_F16>(const BlockRaw<LLG_TYPE_F16> &r,
                                                            const float4 *x4, float xsum) {
    (void)xsum;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint4 q = r.q[i];
        const float4 xa = x4[2 * i], xb = x4[2 * i + 1];
        s = __builtin_fmaf(llg_f16(q.x & 0xFFFF), xa.x, s);
        s = __builtin_fmaf(llg_f16(q.x >> 16), xa.y, s);
        s = __builtin_fmaf(llg_f16(q.y & 0xFFFF), xa.z, s);
        s = __builtin_fmaf(llg_f16(q.y >> 16), xa.w, s);
        s = __builtin_fmaf(llg_f16(q.z & 0xFFFF), xb.x, s);
        s = __builtin_fmaf(llg_f16(q.z >> 16), xb.y, s);
        s = __builtin_fmaf(llg_f16(q.w & 0xFFFF), xb.z, s);
        s = __builtin_fmaf(llg_f16(q.w >> 16), xb.w, s);
    }
    return s;
}
template <>
__device__ __forceinline__ float llg_raw_dot<LLG_TYPE_F32>(const BlockRaw<LLG_TYPE_F32> &r,
                                                            const float4 *x4, float xsum) {
    (void)xsum;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 xv = x4[i];
        s = __builtin_fmaf(r.q[i].x, xv.x, s);
        s = __builtin_fmaf(r.q[i].y, xv.y, s);
        s = __builtin_fmaf(r.q[i].z, xv.z, s);
        s = __builtin_fmaf(r.q[i].w, xv.w, s);
    }
    return s;
}

// acc[0..31] += u * dequant(block) from loaded bytes, with the block's offset
// folded into *corr: for Q4_0 acc gets u*d*q (q in [0, 15]) and corr 8*u*d;
// for Q8_0 acc gets u*d*(q + 128) and corr 128*u*d.  The caller subtracts
// corr from every acc element once, after its last block.
template <int T>
__device__ __forceinline__ void llg_raw_axpy(const BlockRaw<T> &r, float u, float *acc,
                                             float &corr);
template <>
__device__ __forceinline__ void llg_raw_axpy<LLG_TYPE_Q4_0>(const BlockRaw<LLG_TYPE_Q4_0> &r,
                                                             float u, float *acc, float &corr) {
    const float s = u * llg_f16(r.d);
    corr += 8.0f * s;
    const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            acc[8 * i + 2 * k] += s * (float)((lo >> (8 * k)) & 0xFF);
            acc[8 * i + 2 * k + 1] += s * (float)((hi >> (8 * k)) & 0xFF);
        }
    }
}
template <>
__device__ __forceinline__ void llg_raw_axpy<LLG_TYPE_Q8_0>(const BlockRaw<LLG_TYPE_Q8_0> &r,
                                                             float u, float *acc, float &corr) {
    const float s = u * llg_f16(r.d);
    corr += 128.0f * s;
    const uint32_t w[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t v = w[i] ^ 0x80808080u;
#pragma unroll
        for (int k = 0; k < 4; k++) acc[4 * i + k] += s * (float)((v >> (8 * k)) & 0xFF);
    }
}
template <>
__device__ __forceinline__ void llg_raw_axpy<LLG_TYPE_F16>(const BlockRaw<LLG_TYPE_F16> &r,
                                                            float u, float *acc, float &corr) {
    (void)corr;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t w[4] = {r.q[i].x, r.q[i].y, r.q[i].z, r.q[i].w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            acc[8 * i + 2 * k] += u * llg_f16(w[k] & 0xFFFF);
            acc[8 * i + 2 * k + 1] += u * llg_f16(w[k] >> 16);
        }
    }
}
template <>
__device__ __forceinline__ void llg_raw_axpy<LLG_TYPE_F32>(const BlockRaw<LLG_TYPE_F32> &r,
                                                            float u, float *acc, float &corr) {
    (void)corr;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        acc[4 * i + 0] += u * r.q[i].x;
        acc[4 * i + 1] += u * r.q[i].y;
        acc[4 * i + 2] += u * r.q[i].z;
        acc[4 * i + 3] += u * r.q[i].w;
    }
}

// Stage x[nb*32] into LDS, XS (>= 33) floats per block: the block's 32 values
// then, at offset 32, their sum (the xsum of llg_raw_dot).  Loads are
// coalesced float4s, 8 consecutive lanes per block, up to 8 per thread issued
// before any store; each block's sum is reduced over its 8 lanes with DPP
// (quad steps, then row_half_mirror = 0x141 pairs the two quads of 8 lanes).
// The loop bound is uniform per wavefront, so every DPP sees full lanes.
//
// issue(): called once, right after the first group of x loads is issued and
// before any of them is used.  Vector loads complete in issue order, so loads
// a caller issues there (e.g. its weight bytes) stay in flight while x is
// staged, instead of x waiting behind them.
struct LlgNoIssue {
    __device__ void operator()() const {}
};

template <int XS>
__device__ __forceinline__ void llg_x_sum_store(float *xs, const float4 &v, int i, int n4) {
    float sum = (v.x + v.y) + (v.z + v.w);
    sum = llg_quad_sum(sum);
    sum += llg_dpp<0x141>(sum);
    if (i < n4) {
        reinterpret_cast<float4 *>(xs + (i >> 3) * XS)[i & 7] = v;
        if ((i & 7) == 0) xs[(i >> 3) * XS + 32] = sum;
    }
}

// The block sum llg_x_sum_store leaves, formed by one lane from the block's
// 8 float4 groups (s_k = (x + y) + (z + w) of group k): the quad sums of
// lanes 0-3 and 4-7 in their DPP order, then the half-row mirror's add.
__device__ __forceinline__ float llg_block_xsum(const float4 *__restrict__ x4) {
    float s[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const float4 v = x4[k];
        s[k] = (v.x + v.y) + (v.z + v.w);
    }
    return ((s[0] + s[1]) + (s[2] + s[3])) + ((s[6] + s[7]) + (s[4] + s[5]));
}

// KN: float4 rounds of the one-pass form (the row must fit KN * blockDim.x
// float4, else the looped form runs).  Callers pass the fewest that cover
// their rows: a clamped round past the row's end rereads its last float4 and
// costs the CU's address unit as much as a real one, ahead of every later
// wavefront's x.
template <int XS, int KN = 8, class Issue = LlgNoIssue>
__device__ __forceinline__ void llg_stage_x_sum(float *xs, const float *__restrict__ x, int nb,
                                                Issue &&issue = Issue()) {
    static_assert(XS >= 33, "room for the block sum");
    static_assert(KN >= 1 && KN <= 8, "rounds of the one-pass form");
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const int n4 = nb * 8;
    const int lane = threadIdx.x & 63;
    const int base0 = threadIdx.x - lane;
    if (n4 <= KN * (int)blockDim.x) {
        // one pass, straight-line: the wait before the stores covers the x
        // loads only (clamped addresses, so no load sits under a branch)
        float4 v[KN];
#pragma unroll
        for (int k = 0; k < KN; k++) v[k] = x4[min(base0 + k * (int)blockDim.x + lane, n4 - 1)];
        __builtin_amdgcn_sched_barrier(0);  // keep the caller's loads behind these
        issue();
#pragma unroll
        for (int k = 0; k < KN; k++)
            llg_x_sum_store<XS>(xs, v[k], base0 + k * blockDim.x + lane, n4);
        return;
    }
    issue();
    for (int base = base0; base < n4; base += 8 * blockDim.x) {
        float4 v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = x4[min(base + k * (int)blockDim.x + lane, n4 - 1)];
#pragma unroll
        for (int k = 0; k < 8; k++) llg_x_sum_store<XS>(xs, v[k], base + k * blockDim.x + lane, n4);
    }
}

// Attention output in split form: the positions of each head are divided
// over n_split workgroups, each leaving acc = sum_t exp(s_t - m) v_t and
// (m, l = sum_t exp(s_t - m)) over its rows (m = -inf, l = 0 for none).
struct LlgAttnParts {
    const float *acc;  // [n_split][n_heads * head_dim]
    const float *ml;   // [n_split][n_heads][2]
    int n_split, n_heads, head_dim;
};
#define LLG_ATTN_SPLIT_MAX 4

// One float4 of the merged attention output from its splits' acc and (m, l)
// (the slots past n_split are ignored).
__device__ __forceinline__ float4 llg_attn_merge4(const float4 (&a)[LLG_ATTN_SPLIT_MAX],
                                                  const float2 (&ml)[LLG_ATTN_SPLIT_MAX],
                                                  int n_split) {
    float M = ml[0].x;
#pragma unroll
    for (int s = 1; s < LLG_ATTN_SPLIT_MAX; s++)
        if (s < n_split) M = fmaxf(M, ml[s].x);
    float L = 0.0f;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int s = 0; s < LLG_ATTN_SPLIT_MAX; s++)
        if (s < n_split) {
            const float e = ml[s].x == -INFINITY ? 0.0f : expf(ml[s].x - M);
            L += ml[s].y * e;
            v.x += a[s].x * e;
            v.y += a[s].y * e;
            v.z += a[s].z * e;
            v.w += a[s].w * e;
        }
    const float rl = 1.0f / L;
    v.x *= rl;
    v.y *= rl;
    v.z *= rl;
    v.w *= rl;
    return v;
}

// Float4 j of the merged attention output, read from the splits directly,
// one split at a time (few registers): the operations of llg_attn_merge4 in
// the same order, so the same value.
__device__ __forceinline__ float4 llg_attn_merged4(const LlgAttnParts &ap, int j) {
    const int cols = ap.n_heads * ap.head_dim, h = 4 * j / ap.head_dim;
    const float2 *ml = reinterpret_cast<const float2 *>(ap.ml) + h;
    const float4 *a = reinterpret_cast<const float4 *>(ap.acc) + j;
    float M = ml[0].x;
#pragma unroll 1
    for (int s = 1; s < ap.n_split; s++) M = fmaxf(M, ml[s * ap.n_heads].x);
    float L = 0.0f;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 1
    for (int s = 0; s < ap.n_split; s++) {
        const float2 m = ml[s * ap.n_heads];
        const float4 x = a[(size_t)s * cols >> 2];
        const float e = m.x == -INFINITY ? 0.0f : expf(m.x - M);
        L += m.y * e;
        v.x += x.x * e;
        v.y += x.y * e;
        v.z += x.z * e;
        v.w += x.w * e;
    }
    const float rl = 1.0f / L;
    v.x *= rl;
    v.y *= rl;
    v.z *= rl;
    v.w *= rl;
    return v;
}

// Stage the merged attention output, x[c] = sum_s acc_s[c] e_s / sum_s l_s e_s
// with e_s = exp(m_s - max_s m_s) for the head of column c (0 for an empty
// split), like llg_stage_x_sum (the nb blocks from block cb0).  Each thread
// requests its columns of every split (KB float4 groups at a time) before
// merging them; issue() runs after the first requests.  KB: float4 groups
// per thread in a round.
template <int XS, int KB = 2, class Issue = LlgNoIssue>
__device__ __forceinline__ void llg_stage_attn(float *xs, const LlgAttnParts &ap, int cb0, int nb,
                                               Issue &&issue = Issue()) {
    static_assert(XS >= 33, "room for the block sum");
    const int n4 = nb * 8, cols = ap.n_heads * ap.head_dim;
    const int lane = threadIdx.x & 63, base0 = threadIdx.x - lane, bd = blockDim.x;
    const float4 *acc4 = reinterpret_cast<const float4 *>(ap.acc);
    const float2 *ml2 = reinterpret_cast<const float2 *>(ap.ml);
    float4 a[KB][LLG_ATTN_SPLIT_MAX];
    float2 ml[KB][LLG_ATTN_SPLIT_MAX];
    // Every split slot is loaded (a slot past n_split reads split 0 again
    // and is skipped in the merge), and the first round by every wavefront
    // with clamped indices: straight-line loads stay ahead of the caller's.
    auto load = [&](int k0) {
#pragma unroll
        for (int k = 0; k < KB; k++) {
            const int i = min(base0 + (k0 + k) * bd + lane, n4 - 1);
            const int c = cb0 * 32 + 4 * i;
            const int h = c / ap.head_dim;
#pragma unroll
            for (int s = 0; s < LLG_ATTN_SPLIT_MAX; s++) {
                const int sc = s < ap.n_split ? s : 0;
                a[k][s] = acc4[((size_t)sc * cols + c) >> 2];
                ml[k][s] = ml2[sc * ap.n_heads + h];
            }
        }
    };
    auto merge = [&](int k0) {
#pragma unroll
        for (int k = 0; k < KB; k++)
            llg_x_sum_store<XS>(xs, llg_attn_merge4(a[k], ml[k], ap.n_split),
                                base0 + (k0 + k) * bd + lane, n4);
    };
    load(0);
    __builtin_amdgcn_sched_barrier(0);  // keep the caller's loads behind these
    issue();
    merge(0);
    for (int k0 = KB; base0 + k0 * bd < n4; k0 += KB) {
        load(k0);
        merge(k0);
    }
}

// Sum over the workgroup (every thread gets it); red: LDS, one float per
// wavefront.  Contains two barriers.
__device__ __forceinline__ float llg_block_sum(float v, float *red) {
    v = llg_wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();  // red may still be read from a previous call
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < nw; i++) s += red[i];
    return s;
}

// llg_block_sum over a slot no thread has read yet (red: one float per
// wavefront): one barrier.
__device__ __forceinline__ float llg_block_sum_fresh(float v, float *red) {
    v = llg_wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < nw; i++) s += red[i];
    return s;
}

// Residual add + LayerNorm as the prologue of a matvec over the normed row
// (tensor/ops.go:138-165, residual order of ffn_flash.go:161-166):
// v = (x_in + a1) + a2 (a1, a2 may be null), normed = (v - mean) / std * w + b
// with std = sqrt(var + eps) in double.  The normed row is staged in LDS with
// XS floats per 32-element block and the block sum at [32], like
// llg_stage_x_sum; workgroup 0 also writes v to x_out and normed to
// normed_out.  n is a multiple of 32.
//
// stats (optional, with a1 = a2 = null and n <= 32 * LLG_LN_STATS_PER * 64):
// per 32-element block b of x_in, (sum, sum of squared deviations from the
// block mean), as written by the kernel that produced x_in.  Every wavefront
// then merges them itself (the parallel form of the two-pass variance:
// mean = sum / n, M2 = sum_b M2_b + 32 (mean_b - mean)^2), so the prologue
// needs no workgroup reduction.
#define LLG_LN_STATS_PER 4
struct LlgLnArgs {
    const float *x_in, *a1, *a2, *w, *b;
    float *x_out, *normed_out;
    const float2 *stats;
    float eps;
    int n;
};

// (sum, M2) of the 32 values v[0..3] held by each of 8 consecutive lanes
// (lanes 8 j .. 8 j + 7 hold one block): the lane-pair sums in a fixed
// butterfly order, so every lane of the group gets the same result.
__device__ __forceinline__ float2 llg_block32_stats(const float4 &v) {
    float s = (v.x + v.y) + (v.z + v.w);
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 4, 64);
    const float m = s / 32.0f;
    const float d0 = v.x - m, d1 = v.y - m, d2 = v.z - m, d3 = v.w - m;
    float q = (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
    q += __shfl_xor(q, 1, 64);
    q += __shfl_xor(q, 2, 64);
    q += __shfl_xor(q, 4, 64);
    return make_float2(s, q);
}

// A matvec over attn with the predictor's first matrix folded in: p is
// WUp . Wo ([rank x cols] f32), and wavefront task (j, s) stores
// part[s * rank + j] = p[j, chunk s] . x[chunk s] (n_split chunks of
// split_blocks 32-float blocks, the last shorter); the matvec's row sums are
// added into resid (resid[r] += y[r]).
struct LlgPredFold {
    const float *p;
    float *part;
    float *resid;
    int rank, n_split, split_blocks;
};

// NP = float4 groups per thread (n <= 4 * NP * blockDim.x): every load of the
// residual terms and of w and b is issued before the first use, so the
// prologue costs one memory round trip plus the two block reductions (one
// barrier each: red holds 2 floats per wavefront, unread before the call).
// issue() as in llg_stage_x_sum.
template <int XS, int NP, class Issue = LlgNoIssue>
__device__ __forceinline__ void llg_stage_ln(float *xs, const LlgLnArgs &a, float *red,
                                             Issue &&issue = Issue()) {
    const int n4 = a.n >> 2;
    const int tid = threadIdx.x, bd = blockDim.x;
    const float4 *x4 = reinterpret_cast<const float4 *>(a.x_in);
    const float4 *p4 = reinterpret_cast<const float4 *>(a.a1);
    const float4 *q4 = reinterpret_cast<const float4 *>(a.a2);
    const float4 *w4 = reinterpret_cast<const float4 *>(a.w);
    const float4 *b4 = reinterpret_cast<const float4 *>(a.b);
    const bool w0 = blockIdx.x == 0;
    const int lane = tid & 63, nbk = a.n >> 5;
    float4 v[NP], p[NP], q[NP], wv[NP], bv[NP];
    float2 st[LLG_LN_STATS_PER];
#pragma unroll
    for (int k = 0; k < NP; k++) {
        const int i = min(tid + k * bd, n4 - 1);
        v[k] = x4[i];
        if (p4) p[k] = p4[i];
        if (q4) q[k] = q4[i];
        wv[k] = w4[i];
        bv[k] = b4[i];
    }
    if (a.stats) {
#pragma unroll
        for (int k = 0; k < LLG_LN_STATS_PER; k++) st[k] = a.stats[min(lane + 64 * k, nbk - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the caller's loads behind these
    issue();
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NP; k++) {
        const int i = tid + k * bd;
        if (p4) {
            v[k].x = v[k].x + p[k].x; v[k].y = v[k].y + p[k].y;
            v[k].z = v[k].z + p[k].z; v[k].w = v[k].w + p[k].w;
        }
        if (q4) {
            v[k].x = v[k].x + q[k].x; v[k].y = v[k].y + q[k].y;
            v[k].z = v[k].z + q[k].z; v[k].w = v[k].w + q[k].w;
        }
        if (i < n4) {
            s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
            if (w0 && a.x_out) reinterpret_cast<float4 *>(a.x_out)[i] = v[k];
        }
    }
    float mean, var;
    if (a.stats) {
        // this wavefront merges the block statistics (same order in every one)
        float sm = 0.0f;
#pragma unroll
        for (int k = 0; k < LLG_LN_STATS_PER; k++)
            if (lane + 64 * k < nbk) sm += st[k].x;
        mean = llg_wave_sum(sm) / (float)a.n;
        float m2 = 0.0f;
#pragma unroll
        for (int k = 0; k < LLG_LN_STATS_PER; k++)
            if (lane + 64 * k < nbk) {
                const float d = st[k].x / 32.0f - mean;
                m2 += st[k].y + 32.0f * d * d;
            }
        var = llg_wave_sum(m2) / (float)a.n;
    } else {
        mean = llg_block_sum_fresh(s, red) / (float)a.n;
        float qs = 0.0f;
#pragma unroll
        for (int k = 0; k < NP; k++) {
            const float d0 = v[k].x - mean, d1 = v[k].y - mean, d2 = v[k].z - mean,
                        d3 = v[k].w - mean;
            if (tid + k * bd < n4) qs += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
        }
        var = llg_block_sum_fresh(qs, red + (blockDim.x >> 6)) / (float)a.n;
    }
    const float sd = (float)sqrt((double)var + (double)a.eps);
#pragma unroll
    for (int k = 0; k < NP; k++) {
        const int i = tid + k * bd;
        float4 o;
        o.x = (v[k].x - mean) / sd * wv[k].x + bv[k].x;
        o.y = (v[k].y - mean) / sd * wv[k].y + bv[k].y;
        o.z = (v[k].z - mean) / sd * wv[k].z + bv[k].z;
        o.w = (v[k].w - mean) / sd * wv[k].w + bv[k].w;
        float bs = (o.x + o.y) + (o.z + o.w);
        bs = llg_quad_sum(bs);
        bs += llg_dpp<0x141>(bs);  // the 8 float4 of one 32-element block
        if (i < n4) {
            reinterpret_cast<float4 *>(xs + (i >> 3) * XS)[i & 7] = o;
            if ((i & 7) == 0) xs[(i >> 3) * XS + 32] = bs;
            if (w0 && a.normed_out) reinterpret_cast<float4 *>(a.normed_out)[i] = o;
        }
    }
}

// ---------------------------------------------------------------------------
// Host-side runtime objects (defined in llg_runtime.hip)
// ---------------------------------------------------------------------------
#ifdef __cplusplus
#include <string>


enum LlgKind { LLG_KIND_MATRIX = 1, LLG_KIND_BUNDLE = 2, LLG_KIND_WINDOW = 3, LLG_KIND_MODEL = 4 };

// Objects are value-initialized (new LlgObject()).  A window or model holds
// the objects it reads (llg_ref); releasing a held object only retires its
// handle, and its memory goes when the last holder does (llg_unref).
struct LlgObject {
    int kind;
    int64_t id_self;
    uint8_t *d;          // device bytes
    size_t bytes;
    RowFmt fmt;          // row format (matrix rows, or each half of a bundle)
    int rows;            // matrix rows, or bundle neurons (ff)
    long long stride;    // matrix: bytes per row; bundle: bytes per neuron (2 * fmt.stride)
    void *ext;           // kind-specific state (window, model)
    // Q4_0 matrix: the grouped GEMM's fragment-major copy (llg_moe_gemm.hip),
    // made at its first use and freed with the object; null until then
    mutable uint8_t *tiled;
    int refs;            // windows / models holding this object
    bool released;       // handle retired; freed when refs reaches 0
};

struct LlgDevice;

// Runtime services used by every translation unit.
LlgDevice *llg_dev(LlgHipDevice h);
hipStream_t llg_dev_stream(LlgDevice *d);
int llg_set_error(LlgDevice *d, int code, const char *fmt, ...);
int llg_hip_error(LlgDevice *d, hipError_t e, const char *what);
LlgObject *llg_get(LlgDevice *d, int64_t h, int kind);  // live handles only
int64_t llg_register(LlgDevice *d, LlgObject *o);
void llg_ref(LlgObject *o);
void llg_unref(LlgDevice *d, LlgObject *o);
// Device workspace of at least `bytes`, valid until the next llg_ws call that
// grows it (growth synchronises the device before freeing the old buffer).
void *llg_ws(LlgDevice *d, size_t bytes, int *rc);
// The device address of this GPU's fixed scratch array (allocation-free entry
// points), or null with *rc set when `bytes` exceeds LLG_SCRATCH_BYTES
// (LLG_E_SCRATCH) or the address lookup at init failed.
#define LLG_SCRATCH_BYTES (8 * 1024 * 1024)
uint8_t *llg_dev_scratch(LlgDevice *d, size_t bytes, int *rc);
// Sync area of a fused predictor launch (llg_pred_tile.hpp): a 256-byte head
// (the epoch word) and LLG_SYNC_COPIES copies of one 64-bit slot per hidden
// unit, for ranks up to LLG_SYNC_SLOTS.  It starts zeroed and keeps its
// contents between calls.
#define LLG_SYNC_HEAD 256
#define LLG_SYNC_SLOTS 1024
#define LLG_SYNC_COPIES 8
#define LLG_SYNC_BYTES (LLG_SYNC_HEAD + 8 * LLG_SYNC_SLOTS * LLG_SYNC_COPIES)
// The handle's own sync area (allocated and zeroed on the stream at first
// use), or null with *rc set.
uint8_t *llg_dev_sync(LlgDevice *d, int *rc);
// Hand-off slots of the chunked matvecs (k_matvec_q): at least `bytes`,
// zeroed at allocation, and every slot is zero again at the end of each
// launch that uses it.  Growth synchronises the stream first; null with *rc
// set on failure.
uint64_t *llg_dev_mvslots(LlgDevice *d, size_t bytes, int *rc);
// Nonzero when the handle was created with LLG_CHECK_HANDOFF set (a test
// setting): every consumer of an in-launch hand-off still waits for and
// clears its slots, then computes each handed-over value itself and uses its
// own, so that a test can compare the fallback path with the slots bit for bit.
int llg_dev_check(LlgDevice *d);
// Copy host -> device workspace slot / device -> host, on the stream.
int llg_h2d(LlgDevice *d, void *dst, const void *src, size_t bytes);
int llg_d2h(LlgDevice *d, void *dst, const void *src, size_t bytes);
int llg_sync_dev(LlgDevice *d);
int llg_device_id(LlgDevice *d);
int llg_cu_count(LlgDevice *d);

#define LLG_LAUNCH_CHECK(dev, what)                                     \
    do {                                                                \
        hipError_t _e = hipGetLastError();                              \
        if (_e != hipSuccess) return llg_hip_error((dev), _e, (what)); \
    } while (0)

#define LLG_HIP_TRY(dev, expr)                                          \
    do {                                                                \
        hipError_t _e = (expr);                                         \
        if (_e != hipSuccess) return llg_hip_error((dev), _e, #expr);   \
    } while (0)
#endif
