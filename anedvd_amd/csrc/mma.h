// mma.h -- device helpers shared by the expert kernels (k_mm.hip, k_pf.hip):
// MFMA operand types, the exact byte -> f16 conversion, raw buffer loads and the
// addressing of the tile layout's planes.
#pragma once

#include "common.h"

namespace anedvd {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ inline int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ inline f32x4 mfma(half8 a, half8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }

// Bytes (b0, b1) and (b2, b3) of `b` under the f16 exponent byte 0x64: the pairs
// (1024 + b0, 1024 + b1) and (1024 + b2, 1024 + b3), exact.
__device__ inline uint32_t pair01(uint32_t b) { return __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u); }
__device__ inline uint32_t pair23(uint32_t b) { return __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u); }

// 1024 + each byte of lo then hi, as 8 halves in byte order.
__device__ inline half8 bytes_h8(uint32_t lo, uint32_t hi)
{
    const u32x4 w = {pair01(lo), pair23(lo), pair01(hi), pair23(hi)};
    half8 h;
    __builtin_memcpy(&h, &w, 16);
    return h;
}

// The 8 nibbles of v as exact f16 integers 0..15, in bytes_h8's order (the low
// nibbles of bytes 0..3, then the high nibbles).  A byte n < 16 read as OCP e4m3
// is n * 2^-9 (the denormals and the first binade are evenly spaced 2^-9 apart),
// and the converter scales by the exponent of its f32 operand, 2^9: one
// v_cvt_scalef32_pk_f16_fp8 per pair of values.
__device__ inline half8 nibbles_h8(uint32_t v)
{
    typedef _Float16 h2v __attribute__((ext_vector_type(2)));
    const uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
    const h2v a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, false);
    const h2v b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, true);
    const h2v c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, false);
    const h2v d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, true);
    return __builtin_shufflevector(__builtin_shufflevector(a, b, 0, 1, 2, 3), __builtin_shufflevector(c, d, 0, 1, 2, 3),
                                   0, 1, 2, 3, 4, 5, 6, 7);
}

// Bit b (b < 4) of x -> bit 4 of byte b: the fifth bits of four packed values
// (one full-rate 24-bit multiply spreads them 7 bits apart per step).
__device__ inline uint32_t bit4_of_bytes(uint32_t x) { return ((x & 0xFu) * 0x00204081u & 0x01010101u) << 4; }
// The same to bit 2 (Q3_K's third bits).
__device__ inline uint32_t bit2_of_bytes(uint32_t x) { return ((x & 0xFu) * 0x00204081u & 0x01010101u) << 2; }

__device__ inline uint32_t pick4(u32x4 v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

// Raw buffer loads: a wave-uniform descriptor (base, size), a per-lane byte offset
// that stays fixed while a wavefront streams, and a scalar per-step offset -- no
// per-step 64-bit address arithmetic, and loads outside the buffer return 0.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format
constexpr int kNT = 2;                  // non-temporal: weights are streamed once

__device__ inline rsrc_t make_rsrc(const void *p, size_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)(uint32_t)bytes, kRsrcWord3);
}

// The planes of one matrix (expert) of a QMat.
struct Planes {
    rsrc_t q, s, h, d;
    int steps, units, nrb;  // nrb: row blocks of the matrix
};

__device__ inline Planes planes(const QMat &m, int mat)
{
    Planes p;
    p.q = make_rsrc(m.q + (size_t)mat * m.q_stride, m.q_stride);
    p.s = make_rsrc(m.s + (size_t)mat * m.s_stride, m.s_stride);
    p.h = make_rsrc(m.h ? m.h + (size_t)mat * m.h_stride : m.q, m.h_stride);
    p.d = make_rsrc(m.d ? m.d + (size_t)mat * m.d_stride : m.q, m.d_stride);
    p.steps = m.steps;
    p.units = m.units;
    p.nrb = m.rows / kRowBlock;
    return p;
}

// Byte offset of (row block rb, step s) in a per-lane plane of `bytes` per lane,
// and of (rb, unit u) in a per-row plane of `bytes` per row (tile layout).
__device__ inline int lane_plane_off(const Planes &p, int rb, int s, int bytes) { return (rb * p.steps + s) * 256 * bytes; }
__device__ inline int row_plane_off(const Planes &p, int rb, int u, int bytes) { return (rb * p.units + u) * 64 * bytes; }

__device__ inline half8 as_h8(u32x4 v)
{
    half8 h;
    __builtin_memcpy(&h, &v, 16);
    return h;
}

// getScaleMinK4 (gguf.zig:948-958) over the 12 scale bytes held in 3 dwords, j at
// run time.
__device__ inline int scale_byte(uint32_t s1, uint32_t s2, uint32_t s3, int i)
{
    const uint32_t w = i < 4 ? s1 : i < 8 ? s2 : s3;
    return (int)((w >> (8 * (i & 3))) & 0xFFu);
}

__device__ inline void scale_min_k4(int j, uint32_t s1, uint32_t s2, uint32_t s3, int &d, int &m)
{
    if (j < 4) {
        d = scale_byte(s1, s2, s3, j) & 63;
        m = scale_byte(s1, s2, s3, j + 4) & 63;
    } else {
        const int b = scale_byte(s1, s2, s3, j + 4);
        d = (b & 0xF) | ((scale_byte(s1, s2, s3, j - 4) >> 6) << 4);
        m = (b >> 4) | ((scale_byte(s1, s2, s3, j) >> 6) << 4);
    }
}

__device__ inline float gelu_tanh(float x)
{
    const float c = 0.7978845608028654f;
    return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

// moeExpertAccumF32's activation: g / (1 + exp(-g)) (cpu.zig:434-437), or gelu.  The
// quotient is g times the hardware reciprocal (within 1 ulp) rather than an IEEE
// division, which costs a dozen instructions per value in the epilogues.
__device__ inline float gate_act(float g, int use_gelu)
{
    return use_gelu ? gelu_tanh(g) : g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

}  // namespace anedvd
