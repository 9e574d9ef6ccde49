// common.h -- shared definitions of the gfx950 MoE library: types, status,
// GGUF block geometry and the HBM tile layout the kernels read.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/anedvd_moe.h"

namespace anedvd {

typedef _Float16 half_t;
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- errors

void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

#define ANEDVD_HIP(call)                                                                   \
    do {                                                                                   \
        hipError_t e_ = (call);                                                            \
        if (e_ != hipSuccess) {                                                            \
            ::anedvd::set_error("%s failed: %s (%s:%d)", #call, hipGetErrorString(e_),     \
                                __FILE__, __LINE__);                                       \
            return ANEDVD_E_HIP;                                                           \
        }                                                                                  \
    } while (0)

#define ANEDVD_TRY(expr)              \
    do {                              \
        int rc_ = (expr);             \
        if (rc_ != ANEDVD_OK) return rc_; \
    } while (0)

// ------------------------------------------------- GGUF block geometry

// GgmlType.blockElems / blockBytes (gguf.zig:49-77).  0 = unknown type.
__host__ __device__ inline int block_elems(int t)
{
    switch (t) {
    case ANEDVD_F32: case ANEDVD_F16: case ANEDVD_BF16: return 1;
    case ANEDVD_Q4_0: case ANEDVD_Q4_1: case ANEDVD_Q5_0: case ANEDVD_Q5_1: case ANEDVD_Q8_0: case ANEDVD_Q8_1: return 32;
    case ANEDVD_Q2_K: case ANEDVD_Q3_K: case ANEDVD_Q4_K: case ANEDVD_Q5_K: case ANEDVD_Q6_K: case ANEDVD_Q8_K: return 256;
    default: return 0;
    }
}

__host__ __device__ inline int block_bytes(int t)
{
    switch (t) {
    case ANEDVD_F32: return 4;
    case ANEDVD_F16: case ANEDVD_BF16: return 2;
    case ANEDVD_Q4_0: return 18;
    case ANEDVD_Q4_1: return 20;
    case ANEDVD_Q5_0: return 22;
    case ANEDVD_Q5_1: return 24;
    case ANEDVD_Q8_0: return 34;
    case ANEDVD_Q8_1: return 36;
    case ANEDVD_Q2_K: return 84;
    case ANEDVD_Q3_K: return 110;
    case ANEDVD_Q4_K: return 144;
    case ANEDVD_Q5_K: return 176;
    case ANEDVD_Q6_K: return 210;
    case ANEDVD_Q8_K: return 292;
    default: return 0;
    }
}

// ------------------------------------------------------------ tile layout
//
// A quantised matrix [rows][cols] (blocks along cols) is stored "row per lane":
// rows are cut into row groups of 64, one row per wavefront lane, and the
// column axis into units of UNIT elements (whole GGUF blocks).  For each
// (row group, unit) the quant bytes of the 64 rows are interleaved in 16-byte
// chunks, [chunk][lane][16 B], so one global_load_dwordx4 of a wavefront reads
// 1 KiB contiguous; the per-lane scale bytes of the unit follow in a separate
// plane, [lane][SB bytes].  Byte count per weight is unchanged:
//
//   type   UNIT  chunks/unit  scale bytes/unit   bytes per UNIT weights
//   Q8_0    64     4 (64 B)     4 (2 x f16 d)      68  = 2 x 34
//   Q4_0    64     2 (32 B)     4 (2 x f16 d)      36  = 2 x 18
//   Q4_K   256     9 (144 B)    0                  144 (d, dmin, scales, qs)
//   Q6_K   256    13 (208 B)    2 (f16 d)          210 (ql, qh, scales | d)
//
// Within a unit the chunks keep GGUF block byte order (Q8_0 chunk c is bytes
// 16c..16c+15 of the two blocks' quants, each stored biased as q ^ 0x80 = q + 128;
// Q4_K chunk 0 is d/dmin/scales and chunks 1..8 are qs; Q6_K chunks 0..7 ql,
// 8..11 qh, 12 scales).
struct Fmt {
    int unit;      // elements per unit
    int chunks;    // 16-byte quant chunks per lane per unit
    int sbytes;    // scale-plane bytes per lane per unit
};

__host__ __device__ inline Fmt tile_fmt(int t)
{
    switch (t) {
    case ANEDVD_Q8_0: return Fmt{64, 4, 4};
    case ANEDVD_Q4_0: return Fmt{64, 2, 4};
    case ANEDVD_Q4_K: return Fmt{256, 9, 0};
    case ANEDVD_Q6_K: return Fmt{256, 13, 2};
    default: return Fmt{0, 0, 0};
    }
}

constexpr int kRowGroup = 64;

// One stacked matrix set (all experts of one projection) in tile layout.
struct QMat {
    int type;
    int rows, cols, n;        // n stacked matrices (experts)
    uint8_t *q;               // quant plane, n * rows * cols * chunks*16/unit bytes
    uint8_t *s;               // scale plane (may be null when sbytes == 0)
    size_t q_stride, s_stride;  // bytes per matrix in each plane
    int units;                // cols / unit
};

__host__ __device__ inline size_t tile_q_off(const Fmt &f, int units, int rg, int u, int c, int lane)
{
    return ((((size_t)rg * units + u) * f.chunks + c) * kRowGroup + lane) * 16;
}

__host__ __device__ inline size_t tile_s_off(const Fmt &f, int units, int rg, int u, int lane)
{
    return (((size_t)rg * units + u) * kRowGroup + lane) * (size_t)f.sbytes;
}

// GEMV activation order: within every 4 consecutive elements, (0, 2, 1, 3), so
// that the f16 pairs (e0, e2) and (e1, e3) a lane builds from one dword of four
// quants meet their activations as one aligned pair.
__host__ __device__ inline int pair_perm(int e) { return (e & ~3) | ((e & 1) << 1) | ((e >> 1) & 1); }

// IEEE binary16 bits -> f32, exact.
__host__ __device__ inline float f16_bits_to_f32(uint16_t h)
{
    half_t v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}

// ------------------------------------------------- GEMV activation format
//
// The decode kernels read activations as f16 scaled by a power of two per
// (row, 64-element group), stored pair-permuted, with a float4 per group
// {sum of the lower 32 f16 values, sum of the upper 32, the power of two that
// undoes the scale, 0}.  Power-of-two scaling is exact; it keeps every group's
// largest value in [2^14, 2^15), far from f16 overflow and subnormals.

__device__ inline float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ inline float pow2_scale(float maxabs)
{
    if (!(maxabs > 0.0f) || !(maxabs < __builtin_inff())) return 1.0f;
    int e;
    frexpf(maxabs, &e);  // maxabs = m * 2^e, m in [0.5, 1)
    return ldexpf(1.0f, max(-100, min(15 - e, 100)));
}

// One wavefront converts one 64-element group: lane i holds element i.
__device__ inline void act_group(float v, int lane, half_t *__restrict__ q, float4 *__restrict__ side)
{
    const float sc = pow2_scale(wave_max(fabsf(v)));
    const half_t hv = (half_t)(v * sc);
    q[pair_perm(lane)] = hv;
    float s = (float)hv;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    const float s_hi = __shfl(s, 32, 64);
    if (lane == 0) *side = make_float4(s, s_hi, 1.0f / sc, 0.0f);
}

}  // namespace anedvd
