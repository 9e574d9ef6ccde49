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

// -------------------------------------------------------- MMA tile layout
//
// A quantised matrix [rows][cols] (blocks along cols) is stored for the 16x16x32
// f16 MFMA: rows in blocks of 64 (4 tiles of 16 rows), columns in steps of 64.
// For (row block rb, step s, tile t) the 64 lanes of a wavefront hold, lane
// l = 16 g + n, row 64 rb + 16 t + n and the 16 columns {64 s + 32 j + 8 g + i :
// j = 0, 1; i = 0..7} in the order (j, i): the B operands of two MFMAs (j), so one
// load per lane per tile feeds both.
//   quant plane [rb][s][t][lane][QB bytes]
//   h plane     [rb][s][t][lane] 4 bytes (Q6_K only): byte b, bits 4j + 2h and
//               4j + 2h + 1, hold the high 2 bits of value (j, b + 4h)
//   scale plane [rb][u][t][16 rows][SB bytes], u = the step's scale unit (one
//               step for Q8_0 / Q4_0, a 256-column super-block for Q4_K / Q6_K)
//   d plane     [rb][u][t][16 rows] f16 (Q6_K only)
//
//   type  QB  the lane's 16 values                                   SB
//   Q8_0  16  byte 8j + i = q + 128                                   4  (d of blocks j = 0, 1)
//   Q4_0   8  dword j, byte b: low nibble = (j, b), high = (j, b+4)   4  (d x 2)
//   Q4_K   8  as Q4_0, the super-block's 4-bit quants                16  (d, dmin, 12 scale bytes)
//   Q6_K   8  as Q4_0, the low 4 bits (high 2 in the h plane)        16  (int8 scales) + d plane
//
// Bytes per weight are those of the GGUF blocks (Q8_0 1.0625, Q4_0 0.5625,
// Q4_K 0.5625, Q6_K 0.8203); every dequantised value is kept (the repack only
// moves bits).
struct Fmt {
    int qb;     // quant bytes per lane per (step, tile)
    int sb;     // scale bytes per row per scale unit
    int spu;    // steps per scale unit
    int blk;    // GGUF block elements
};

__host__ __device__ inline Fmt tile_fmt(int t)
{
    switch (t) {
    case ANEDVD_Q8_0: return Fmt{16, 4, 1, 32};
    case ANEDVD_Q8_1: return Fmt{16, 4, 1, 32};
    case ANEDVD_Q4_0: return Fmt{8, 4, 1, 32};
    case ANEDVD_Q4_1: return Fmt{8, 8, 1, 32};
    case ANEDVD_Q5_0: return Fmt{8, 4, 1, 32};
    case ANEDVD_Q5_1: return Fmt{8, 8, 1, 32};
    case ANEDVD_Q2_K: return Fmt{4, 16, 4, 256};
    case ANEDVD_Q3_K: return Fmt{4, 16, 4, 256};
    case ANEDVD_Q4_K: return Fmt{8, 16, 4, 256};
    case ANEDVD_Q5_K: return Fmt{8, 16, 4, 256};
    case ANEDVD_Q6_K: return Fmt{8, 16, 4, 256};
    case ANEDVD_F16: return Fmt{32, 0, 1, 1};  // the f16 values themselves, no scales
    default: return Fmt{0, 0, 0, 0};
    }
}

constexpr int kRowBlock = 64;
constexpr int kStep = 64;

// One stacked matrix set (all experts of one projection) in tile layout.
struct QMat {
    int type;
    int rows, cols, n;            // n stacked matrices (experts)
    int steps, units;             // cols / 64, steps / steps-per-unit
    uint8_t *q, *s, *h, *d;       // quant, scale, high-bit (tile_hb) and super-block scale (tile_db) planes
    size_t q_stride, s_stride, h_stride, d_stride;  // bytes per matrix in each plane
};

__host__ __device__ inline size_t tile_q_off(const Fmt &f, int steps, int rb, int s, int t, int lane)
{
    return ((((size_t)rb * steps + s) * 4 + t) * 64 + lane) * (size_t)f.qb;
}

__host__ __device__ inline size_t tile_s_off(const Fmt &f, int units, int rb, int u, int t, int n)
{
    return ((((size_t)rb * units + u) * 4 + t) * 16 + n) * (size_t)f.sb;
}

// High-bit plane bytes per lane per (step, tile): Q6_K 2 bits per value, the
// 5-bit formats and Q3_K 1.
__host__ __device__ inline int tile_hb(int type)
{
    return type == ANEDVD_Q6_K ? 4
           : (type == ANEDVD_Q5_K || type == ANEDVD_Q5_0 || type == ANEDVD_Q5_1 || type == ANEDVD_Q3_K) ? 2
                                                                                                          : 0;
}

// Super-block scale (d plane) bytes per row per scale unit: Q6_K and Q3_K d, Q2_K d and dmin.
__host__ __device__ inline int tile_db(int type)
{
    return (type == ANEDVD_Q6_K || type == ANEDVD_Q3_K) ? 2 : type == ANEDVD_Q2_K ? 4 : 0;
}

__host__ __device__ inline size_t tile_h_off(int steps, int rb, int s, int t, int lane, int hb)
{
    return ((((size_t)rb * steps + s) * 4 + t) * 64 + lane) * (size_t)hb;
}

__host__ __device__ inline size_t tile_d_off(int units, int rb, int u, int t, int n, int db)
{
    return ((((size_t)rb * units + u) * 4 + t) * 16 + n) * (size_t)db;
}

// Column of lane group g's value (j, i) within a 64-column step.
__host__ __device__ inline int mma_col(int g, int j, int i) { return 32 * j + 8 * g + i; }

// MFMA activation format: element e of a 64-column group is stored at position
// 16 g + 8 j + i (e = 32 j + 8 g + i), so lane group g reads its 16 A values as 32
// contiguous bytes.
__host__ __device__ inline int mma_pos(int e) { return 16 * ((e & 31) >> 3) + 8 * (e >> 5) + (e & 7); }

// IEEE binary16 bits -> f32, exact.
__host__ __device__ inline float f16_bits_to_f32(uint16_t h)
{
    half_t v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}

// ------------------------------------------------- MFMA activation format
//
// The expert kernels read activations as f16 scaled by a power of two per (row,
// 64-element group), stored in mma_pos order, with the power of two that undoes
// the scale in a float array ds[group][row] (row-contiguous per group).  Power-of-
// two scaling is exact; it keeps every group's largest value in [2^14, 2^15), far
// from f16 overflow and subnormals.

// cpu.sigmoid (cpu.zig:1223-1230): the clamped logistic of the shared expert's gate.
__device__ inline float shared_sigmoid(float g)
{
    if (g >= 0.0f) return 1.0f / (1.0f + __expf(-fminf(g, 80.0f)));
    const float ex = __expf(fmaxf(g, -80.0f));
    return ex / (1.0f + ex);
}

// 2^p with p = 15 - e for maxabs = m 2^e, m in [0.5, 1), clamped to [-100, 100]: the
// largest magnitude lands in [2^14, 2^15).  For a normal maxabs with biased exponent
// field E, e = E - 126; a subnormal one (E = 0) clamps to 2^100 as its true exponent
// would.  Read off the bits: no frexp, no ldexp.
__device__ inline float pow2_scale(float maxabs)
{
    if (!(maxabs > 0.0f) || !(maxabs < __builtin_inff())) return 1.0f;
    const int E = (__float_as_int(maxabs) >> 23) & 0xFF;
    const int p = max(-100, min(141 - E, 100));
    return __int_as_float((p + 127) << 23);
}

// 1 / s for a power of two s = 2^p, |p| <= 126: 2^-p, exact, from the exponent bits.
__device__ inline float pow2_recip(float s) { return __int_as_float(0x7F000000 - __float_as_int(s)); }

template <int CTRL>
__device__ inline float dpp_f32(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ inline float row_max_f32(float v)
{
    v = fmaxf(v, dpp_f32<0xB1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f32<0x4E>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f32<0x141>(v));  // row_half_mirror
    v = fmaxf(v, dpp_f32<0x140>(v));  // row_mirror
    return v;
}

// Wavefront-wide max (fmaxf: NaN only if every lane's is): DPP inside each row of
// 16 lanes, readlane across the four rows; every lane gets the result.
__device__ inline float wave_max(float v)
{
    v = row_max_f32(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// One wavefront converts one 64-element group: lane e holds element e.
__device__ inline void act_group(float v, int lane, half_t *__restrict__ q, float *__restrict__ ds)
{
    const float sc = pow2_scale(wave_max(fabsf(v)));
    q[mma_pos(lane)] = (half_t)(v * sc);
    if (lane == 0) *ds = 1.0f / sc;
}

}  // namespace anedvd
