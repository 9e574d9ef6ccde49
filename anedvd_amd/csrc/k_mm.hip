// k_mm.hip -- expert products on the MFMA units: GGUF dequant fused into the
// SwiGLU gate/up and down products, for the token groups the dispatch built.
//
// Semantics follow cpu.moeExpertAccumF32 (cpu.zig:416-452): g = W_g h,
// u = W_u h, a = (g / (1 + exp(-g))) * u, y = W_d a; the combine adds p * y per
// slot.  Block dequantisation follows gguf.zig's dequantQ8_0 (827-840),
// dequantQ4_0 (763-776), dequantQ4K (960-996) and dequantQ6K (1036-1059).
//
// Design.  Weights stay in HBM in the MMA tile layout (common.h); a wavefront
// owns 64 weight rows (four 16-row tiles) and streams their K span in steps of 64
// columns, one global load per lane per tile per step.  Each lane turns its 16
// quants into the f16 B operands of two v_mfma_f32_16x16x32_f16 (byte permutes
// under the exponent byte 0x64 give 1024 + q exactly); the A operand is 16 tokens
// of the group (padded by repeating the last token), read straight from the
// L2-resident activations, so the weights are read once per 16 tokens and no
// LDS staging or barrier sits in the stream.  Each MFMA covers one 32-column
// block of one 16-row tile, so the block's scale (and Q4_K's min term, with the
// block sums of the activations from an MFMA against ones) is applied to its
// f32 result together with the activations' per-64-column descale.  Q6_K's
// 16-column sub-block scales are folded into its f16 weights (each lane's 8
// columns share one sub-block); sc * (q - 32) rounds only when its magnitude
// exceeds 2048 (relative error <= 2^-12).
//
// The K axis is split over ks workgroups when a call has too few rows to fill
// the 256 CUs; the partial sums are added in a fixed order by a later launch, so
// results do not depend on scheduling.
#include <stdlib.h>

#include <algorithm>

#include "common.h"
#include "kernels.h"
#include "mma.h"

namespace anedvd {

constexpr int kWaves = 4;
#ifndef ANEDVD_WG_TARGET
#define ANEDVD_WG_TARGET 1024
#endif
// Mean group size (tokens per expert) from which the planner takes the grouped
// GEMM (k_pf.hip) instead of the decode kernels.
#ifndef ANEDVD_STAGED_MIN
#define ANEDVD_STAGED_MIN 32
#endif
// Mean group size from which the grouped GEMM takes 128-token workgroups (types
// with such a kernel only).
#ifndef ANEDVD_PF_WIDE_MIN
#define ANEDVD_PF_WIDE_MIN 64
#endif
// Groups of at most this many tokens (one 16-token tile) leave the grouped GEMM's
// work list for its small-group workgroups (the same launch, after the grouped
// ones), which read their activations straight from memory instead of staging
// them in LDS; only while the mean group is below ANEDVD_SMALL_MEAN (skewed
// routing of many experts: most groups then hold a few tokens).  0 turns the
// split off.
#ifndef ANEDVD_SMALL_GROUP
#define ANEDVD_SMALL_GROUP 16
#endif
#ifndef ANEDVD_SMALL_MEAN
#define ANEDVD_SMALL_MEAN 64
#endif
constexpr int kCUs = 256;  // MI355X compute units
#ifdef ANEDVD_MM_WPE
#define MM_ATTR __attribute__((amdgpu_waves_per_eu(ANEDVD_MM_WPE)))
#else
#define MM_ATTR
#endif

// ------------------------------------------------------------------ decoders
//
// A decoder loads one step of its wavefront's four tiles (load), takes what
// stays valid for a whole scale unit (begin), and yields the B operand of (tile
// t, block j) with the block's scale d and min coefficient mn (operand); the
// MFMA result r then contributes d * r - mn * (activation block sum).
//
// A load's per-lane offset is one VGPR shared by the four tiles; the tile's
// constant offset goes into the scalar offset.  (Written as VGPR sums, the
// hoisted loop invariants took a register per tile: 6-8 more VGPRs per kernel.)

// F16 experts (the eager path's weights, cpu.moeExpertAccum with matmulF16,
// cpu.zig:1141-1185): the tile holds the values themselves, the B operand without
// any conversion.
struct MF16 {
    static constexpr int kSpu = 1;
    static constexpr bool kMin = false;
    struct Raw {
        u32x4 q[4][2];
    };
    struct State {};
    __device__ static inline void load(Raw &r, const Planes &p, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(p, rb, s, 32);
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int j = 0; j < 2; j++)
                r.q[t][j] = __builtin_amdgcn_raw_buffer_load_b128(p.q, 32 * lane, qo + 2048 * t + 16 * j, kNT);
    }
    __device__ static inline void begin(const Raw &, State &, int) {}
    __device__ static inline void operand(const Raw &r, const State &, int, int, int t, int j, half8 &b, float &d,
                                          float &mn)
    {
        b = as_h8(r.q[t][j]);
        d = 1.0f;
        mn = 0.0f;
    }
};

struct MQ8_0 {
    static constexpr int kSpu = 1;
    static constexpr bool kMin = false;
    struct Raw {
        u32x4 q[4];
        uint32_t s[4];
    };
    struct State {};
    __device__ static inline void load(Raw &r, const Planes &p, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(p, rb, s, 16), so = row_plane_off(p, rb, s, 4);
#pragma unroll
        for (int t = 0; t < 4; t++) r.q[t] = __builtin_amdgcn_raw_buffer_load_b128(p.q, 16 * lane, qo + 1024 * t, kNT);
#pragma unroll
        for (int t = 0; t < 4; t++) r.s[t] = __builtin_amdgcn_raw_buffer_load_b32(p.s, 4 * (lane & 15), so + 64 * t, kNT);
    }
    __device__ static inline void begin(const Raw &, State &, int) {}
    __device__ static inline void operand(const Raw &r, const State &, int, int, int t, int j, half8 &b, float &d,
                                          float &mn)
    {
        b = bytes_h8(r.q[t][2 * j], r.q[t][2 * j + 1]) - (half_t)1152.0f;  // the tile stores q + 128
        d = f16_bits_to_f32((uint16_t)(r.s[t] >> (16 * j)));
        mn = 0.0f;
    }
};

struct MQ4_0 {
    static constexpr int kSpu = 1;
    static constexpr bool kMin = false;
    struct Raw {
        u32x2 q[4];
        uint32_t s[4];
    };
    struct State {};
    __device__ static inline void load(Raw &r, const Planes &p, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(p, rb, s, 8), so = row_plane_off(p, rb, s, 4);
#pragma unroll
        for (int t = 0; t < 4; t++) r.q[t] = __builtin_amdgcn_raw_buffer_load_b64(p.q, 8 * lane, qo + 512 * t, kNT);
#pragma unroll
        for (int t = 0; t < 4; t++) r.s[t] = __builtin_amdgcn_raw_buffer_load_b32(p.s, 4 * (lane & 15), so + 64 * t, kNT);
    }
    __device__ static inline void begin(const Raw &, State &, int) {}
    __device__ static inline void operand(const Raw &r, const State &, int, int, int t, int j, half8 &b, float &d,
                                          float &mn)
    {
        const uint32_t v = r.q[t][j];
        b = nibbles_h8(v) - (half_t)8.0f;  // n - 8, exact
        d = f16_bits_to_f32((uint16_t)(r.s[t] >> (16 * j)));
        mn = 0.0f;
    }
};

// Q4_1 / Q5_1 (y = d q + m, gguf.zig:778-822) and Q5_0 (y = d (q - 16)): 32-element
// blocks, the step's two blocks' d (and m) in the scale plane, the 5-bit formats'
// fifth bits in the high-bit plane.  The min coefficient is -m.
template <bool kFive, bool kHasMin>
struct MQLegacy {
    static constexpr int kSpu = 1;
    static constexpr bool kMin = kHasMin;
    struct Raw {
        u32x2 q[4];
        uint32_t h[kFive ? 4 : 1];
        u32x2 s[4];  // (d0 | m0 << 16, d1 | m1 << 16) with a min, else (d0 | d1 << 16, -)
    };
    struct State {};
    __device__ static inline void load(Raw &r, const Planes &p, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(p, rb, s, 8), so = row_plane_off(p, rb, s, kHasMin ? 8 : 4);
#pragma unroll
        for (int t = 0; t < 4; t++) r.q[t] = __builtin_amdgcn_raw_buffer_load_b64(p.q, 8 * lane, qo + 512 * t, kNT);
        if constexpr (kFive) {
            const int ho = lane_plane_off(p, rb, s, 2);
#pragma unroll
            for (int t = 0; t < 4; t++) r.h[t] = __builtin_amdgcn_raw_buffer_load_b16(p.h, 2 * lane, ho + 128 * t, kNT);
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            if constexpr (kHasMin)
                r.s[t] = __builtin_amdgcn_raw_buffer_load_b64(p.s, 8 * (lane & 15), so + 128 * t, kNT);
            else
                r.s[t].x = __builtin_amdgcn_raw_buffer_load_b32(p.s, 4 * (lane & 15), so + 64 * t, kNT);
        }
    }
    __device__ static inline void begin(const Raw &, State &, int) {}
    __device__ static inline void operand(const Raw &r, const State &, int, int, int t, int j, half8 &b, float &d,
                                          float &mn)
    {
        const uint32_t v = r.q[t][j];
        if constexpr (kFive) {
            const uint32_t lo = (v & 0x0F0F0F0Fu) | bit4_of_bytes(r.h[t] >> (8 * j));
            const uint32_t hi = ((v >> 4) & 0x0F0F0F0Fu) | bit4_of_bytes(r.h[t] >> (8 * j + 4));
            // Q5_0 values are q - 16; Q5_1's the raw quant
            b = bytes_h8(lo, hi) - (half_t)(kHasMin ? 1024.0f : 1040.0f);
        } else {
            b = nibbles_h8(v);
        }
        if constexpr (kHasMin) {
            const uint32_t dm = r.s[t][j];
            d = f16_bits_to_f32((uint16_t)(dm & 0xFFFFu));
            mn = -f16_bits_to_f32((uint16_t)(dm >> 16));
        } else {
            d = f16_bits_to_f32((uint16_t)(r.s[t].x >> (16 * j)));
            mn = 0.0f;
        }
    }
};
using MQ4_1 = MQLegacy<false, true>;
using MQ5_0 = MQLegacy<true, false>;
using MQ5_1 = MQLegacy<true, true>;

// Q4_K: step s covers sub-blocks 2 (s % 4) + j; y = d1 n - m1 with d1 = d * sc,
// m1 = dmin * m.
struct MQ4_K {
    static constexpr int kSpu = 4;
    static constexpr bool kMin = true;
    struct Raw {
        u32x2 q[4];
        u32x4 sc[4];  // d, dmin, scales of the row's super-block (first step of a unit)
    };
    struct State {
        u32x4 sc[4];
    };
    __device__ static inline void load(Raw &r, const Planes &p, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(p, rb, s, 8);
#pragma unroll
        for (int t = 0; t < 4; t++) r.q[t] = __builtin_amdgcn_raw_buffer_load_b64(p.q, 8 * lane, qo + 512 * t, kNT);
        if ((s & 3) == 0) {
            const int so = row_plane_off(p, rb, s >> 2, 16);
#pragma unroll
            for (int t = 0; t < 4; t++)
                r.sc[t] = __builtin_amdgcn_raw_buffer_load_b128(p.s, 16 * (lane & 15), so + 256 * t, kNT);
        }
    }
    __device__ static inline void begin(const Raw &r, State &st, int s)
    {
        if ((s & 3) == 0) {
#pragma unroll
            for (int t = 0; t < 4; t++) st.sc[t] = r.sc[t];
        }
    }
    __device__ static inline void operand(const Raw &r, const State &st, int s, int, int t, int j, half8 &b, float &d,
                                          float &mn)
    {
        const uint32_t v = r.q[t][j];
        b = nibbles_h8(v);  // n
        const u32x4 sc = st.sc[t];
        int a, m;
        scale_min_k4(2 * (s & 3) + j, sc.y, sc.z, sc.w, a, m);
        d = f16_bits_to_f32((uint16_t)(sc.x & 0xFFFFu)) * (float)a;
        mn = f16_bits_to_f32((uint16_t)(sc.x >> 16)) * (float)m;
    }
};

// Q5_K: the Q4_K scheme on 5-bit values, the fifth bit from the high-bit plane.
struct MQ5_K {
    static constexpr int kSpu = 4;
    static constexpr bool kMin = true;
    struct Raw {
        u32x2 q[4];
        uint32_t h[4];
        u32x4 sc[4];  // d, dmin, scales of the row's super-block (first step of a unit)
    };
    using State = MQ4_K::State;
    __device__ static inline void load(Raw &r, const Planes &p, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(p, rb, s, 8), ho = lane_plane_off(p, rb, s, 2);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            r.q[t] = __builtin_amdgcn_raw_buffer_load_b64(p.q, 8 * lane, qo + 512 * t, kNT);
            r.h[t] = __builtin_amdgcn_raw_buffer_load_b16(p.h, 2 * lane, ho + 128 * t, kNT);
        }
        if ((s & 3) == 0) {
            const int so = row_plane_off(p, rb, s >> 2, 16);
#pragma unroll
            for (int t = 0; t < 4; t++)
                r.sc[t] = __builtin_amdgcn_raw_buffer_load_b128(p.s, 16 * (lane & 15), so + 256 * t, kNT);
        }
    }
    __device__ static inline void begin(const Raw &r, State &st, int s)
    {
        if ((s & 3) == 0) {
#pragma unroll
            for (int t = 0; t < 4; t++) st.sc[t] = r.sc[t];
        }
    }
    __device__ static inline void operand(const Raw &r, const State &st, int s, int, int t, int j, half8 &b, float &d,
                                          float &mn)
    {
        const uint32_t v = r.q[t][j], hb = r.h[t];
        const uint32_t lo = (v & 0x0F0F0F0Fu) | bit4_of_bytes(hb >> (8 * j));
        const uint32_t hi = ((v >> 4) & 0x0F0F0F0Fu) | bit4_of_bytes(hb >> (8 * j + 4));
        b = bytes_h8(lo, hi) - (half_t)1024.0f;  // q in [0, 31]
        const u32x4 sc = st.sc[t];
        int a, m;
        scale_min_k4(2 * (s & 3) + j, sc.y, sc.z, sc.w, a, m);
        d = f16_bits_to_f32((uint16_t)(sc.x & 0xFFFFu)) * (float)a;
        mn = f16_bits_to_f32((uint16_t)(sc.x >> 16)) * (float)m;
    }
};

// Q2_K (gguf.zig:855-889) and Q3_K (gguf.zig:891-946): 2-bit fields, four per
// byte (value (j, 4 hh + b) in bits 2 (2 j + hh) of byte b), 16-element sub-blocks
// (the lane's 8 columns of block j lie in sub-block 4 (s % 4) + 2 j + g / 2).
// Q3_K: the third bit from the high-bit plane, the int8 sub-block scale folded
// into the exact f16 weight (u - 4) sc and the super-block d applied to the
// result.  Q2_K: y = dl v - ml with dl = d (sc & 15), ml = dmin (sc >> 4), formed
// per lane in f32 and rounded to f16 with the weight (one rounding of each).
template <bool kThree>
struct MQ23K {
    static constexpr int kSpu = 4;
    static constexpr bool kMin = false;
    struct Raw {
        uint32_t q[4];
        uint32_t h[kThree ? 4 : 1];
        u32x4 sc[4];     // sub-block scales (first step of a unit)
        uint32_t dm[4];  // d (Q3_K) or d | dmin << 16 (Q2_K) (first step of a unit)
    };
    struct State {
        u32x4 sc[4];
        float d[4], dmin[4];
    };
    __device__ static inline void load(Raw &r, const Planes &p, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(p, rb, s, 4);
#pragma unroll
        for (int t = 0; t < 4; t++) r.q[t] = __builtin_amdgcn_raw_buffer_load_b32(p.q, 4 * lane, qo + 256 * t, kNT);
        if constexpr (kThree) {
            const int ho = lane_plane_off(p, rb, s, 2);
#pragma unroll
            for (int t = 0; t < 4; t++) r.h[t] = __builtin_amdgcn_raw_buffer_load_b16(p.h, 2 * lane, ho + 128 * t, kNT);
        }
        if ((s & 3) == 0) {
            const int so = row_plane_off(p, rb, s >> 2, 16), dof = row_plane_off(p, rb, s >> 2, kThree ? 2 : 4);
#pragma unroll
            for (int t = 0; t < 4; t++) {
                r.sc[t] = __builtin_amdgcn_raw_buffer_load_b128(p.s, 16 * (lane & 15), so + 256 * t, kNT);
                if constexpr (kThree)
                    r.dm[t] = __builtin_amdgcn_raw_buffer_load_b16(p.d, 2 * (lane & 15), dof + 32 * t, kNT);
                else
                    r.dm[t] = __builtin_amdgcn_raw_buffer_load_b32(p.d, 4 * (lane & 15), dof + 64 * t, kNT);
            }
        }
    }
    __device__ static inline void begin(const Raw &r, State &st, int s)
    {
        if ((s & 3) == 0) {
#pragma unroll
            for (int t = 0; t < 4; t++) {
                st.sc[t] = r.sc[t];
                st.d[t] = f16_bits_to_f32((uint16_t)(r.dm[t] & 0xFFFFu));
                st.dmin[t] = f16_bits_to_f32((uint16_t)(r.dm[t] >> 16));
            }
        }
    }
    __device__ static inline void operand(const Raw &r, const State &st, int s, int lane, int t, int j, half8 &b,
                                          float &d, float &mn)
    {
        const uint32_t w = r.q[t];
        uint32_t lo = (w >> (4 * j)) & 0x03030303u, hi = (w >> (4 * j + 2)) & 0x03030303u;
        const int sub = 4 * (s & 3) + 2 * j + (lane >> 5);
        const uint32_t scb = (pick4(st.sc[t], sub >> 2) >> (8 * (sub & 3))) & 0xFFu;
        mn = 0.0f;
        if constexpr (kThree) {
            lo |= bit2_of_bytes(r.h[t] >> (8 * j));
            hi |= bit2_of_bytes(r.h[t] >> (8 * j + 4));
            b = (bytes_h8(lo, hi) - (half_t)1028.0f) * (half_t)(float)(int)(int8_t)scb;  // (u - 4) sc, exact
            d = st.d[t];
        } else {
            const float dl = st.d[t] * (float)(scb & 0xFu), ml = st.dmin[t] * (float)(scb >> 4);
            b = (bytes_h8(lo, hi) - (half_t)1024.0f) * (half_t)dl - (half_t)ml;
            d = 1.0f;
        }
    }
};
using MQ2_K = MQ23K<false>;
using MQ3_K = MQ23K<true>;

// Q6_K: the lane's 8 columns of block j lie in sub-block 4 (s % 4) + 2 j + g / 2;
// its int8 scale is folded into the f16 weights and the super-block's d applied
// to the result.
struct MQ6_K {
    static constexpr int kSpu = 4;
    static constexpr bool kMin = false;
    struct Raw {
        u32x2 q[4];
        uint32_t h[4];
        u32x4 sc[4];    // int8 scales (first step of a unit)
        uint16_t d[4];  // f16 d (first step of a unit)
    };
    struct State {
        u32x4 sc[4];
        float d[4];
    };
    __device__ static inline void load(Raw &r, const Planes &p, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(p, rb, s, 8), ho = lane_plane_off(p, rb, s, 4);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            r.q[t] = __builtin_amdgcn_raw_buffer_load_b64(p.q, 8 * lane, qo + 512 * t, kNT);
            r.h[t] = __builtin_amdgcn_raw_buffer_load_b32(p.h, 4 * lane, ho + 256 * t, kNT);
        }
        if ((s & 3) == 0) {
            const int so = row_plane_off(p, rb, s >> 2, 16), dof = row_plane_off(p, rb, s >> 2, 2);
#pragma unroll
            for (int t = 0; t < 4; t++) {
                r.sc[t] = __builtin_amdgcn_raw_buffer_load_b128(p.s, 16 * (lane & 15), so + 256 * t, kNT);
                r.d[t] = __builtin_amdgcn_raw_buffer_load_b16(p.d, 2 * (lane & 15), dof + 32 * t, kNT);
            }
        }
    }
    __device__ static inline void begin(const Raw &r, State &st, int s)
    {
        if ((s & 3) == 0) {
#pragma unroll
            for (int t = 0; t < 4; t++) {
                st.sc[t] = r.sc[t];
                st.d[t] = f16_bits_to_f32(r.d[t]);
            }
        }
    }
    __device__ static inline void operand(const Raw &r, const State &st, int s, int lane, int t, int j, half8 &b,
                                          float &d, float &mn)
    {
        const uint32_t v = r.q[t][j], hb = r.h[t];
        const uint32_t lo = (v & 0x0F0F0F0Fu) | (((hb >> (4 * j)) & 0x03030303u) << 4);
        const uint32_t hi = ((v >> 4) & 0x0F0F0F0Fu) | (((hb >> (4 * j + 2)) & 0x03030303u) << 4);
        const int sub = 4 * (s & 3) + 2 * j + (lane >> 5);
        const int sc = (int)(int8_t)((pick4(st.sc[t], sub >> 2) >> (8 * (sub & 3))) & 0xFFu);
        b = (bytes_h8(lo, hi) - (half_t)1056.0f) * (half_t)(float)sc;  // sc * (q - 32)
        d = st.d[t];
        mn = 0.0f;
    }
};

// ------------------------------------------------------------------ core
//
// A wavefront computes 64 weight rows (four 16-row tiles) against MT tiles of 16
// tokens: acc[mt][t][i] = sum_k W[64 rb + 16 t + l % 16][k] * x[token 4 (l / 16) + i
// of tile mt][k], lane l.  Each step's weights are decoded once and used by all MT
// token tiles, so a 64-token chunk (MT = 4) reads and decodes the weights a quarter
// as often as four 16-token passes.
//
// Activation descales come in two forms:
//   kRow  one power of two per token row (the layer input x): the MFMA results
//         accumulate with the weight scale only, and the row's descale is
//         applied once after the K loop;
//   kStep one per (row, 64-column group) (the SwiGLU activations, written group
//         by group): each step's descales of the lane's four result tokens --
//         consecutive positions -- come in with one 16-byte load per token tile.
enum DsMode { kRow, kStepDs };

template <int MT, int MODE>
struct AStep {
    half8 a0[MT], a1[MT];
    f32x4 dv[MODE == kStepDs ? MT : 1];
};

// Where a lane's activations come from: its A row's byte offset (token l % 16 of
// tile mt, plus lane group g's 32 bytes) in the f16 values and, for kStepDs, the
// byte offset of its first result token's descale within a group (ld4 bytes per
// group).
template <int MT>
struct AOp {
    rsrc_t q, ds;
    int qoff[MT];
    int doff[MT];
    int ld4;
};

// The same operands from LDS: the fused-reduce down kernel's prologue writes its
// 16 MT rows there, for its steps [s0, s0 + n) only (rows of rowb bytes in the
// activation format; descales [step][16 MT]).
template <int MT>
struct AOpL {
    const char *q;
    const float *ds;
    int qoff[MT];  // byte offset of the lane's row and lane group
    int doff[MT];  // float offset of its first result token's descale within a step
    int s0;
};

template <int MT, int MODE>
__device__ inline void load_a(AStep<MT, MODE> &x, const AOpL<MT> &a, int s)
{
    const int o = (s - a.s0) * 2 * kStep;
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        x.a0[mt] = *(const half8 *)(a.q + a.qoff[mt] + o);
        x.a1[mt] = *(const half8 *)(a.q + a.qoff[mt] + o + 16);
    }
    if (MODE == kStepDs) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++) x.dv[mt] = *(const f32x4 *)(a.ds + (s - a.s0) * 16 * MT + a.doff[mt]);
    }
}

template <int MT, int MODE>
__device__ inline void load_a(AStep<MT, MODE> &x, const AOp<MT> &a, int s)
{
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        x.a0[mt] = as_h8(__builtin_amdgcn_raw_buffer_load_b128(a.q, a.qoff[mt], s * 2 * kStep, 0));
        x.a1[mt] = as_h8(__builtin_amdgcn_raw_buffer_load_b128(a.q, a.qoff[mt], s * 2 * kStep + 16, 0));
    }
    if (MODE == kStepDs) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(a.ds, a.doff[mt], s * a.ld4, 0);
            __builtin_memcpy(&x.dv[mt], &v, 16);
        }
    }
}

// acc[mt][t][i] += the step's contribution.
template <class D, int MT, int MODE>
__device__ inline void mm_step(const typename D::Raw &w, typename D::State &st, const AStep<MT, MODE> &x, int s,
                               int lane, f32x4 (*acc)[4])
{
    const half8 ones = (half8)(half_t)1.0f;
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    D::begin(w, st, s);
    f32x4 sum[MT][2];
    if (D::kMin) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            sum[mt][0] = mfma(x.a0[mt], ones, zero);
            sum[mt][1] = mfma(x.a1[mt], ones, zero);
        }
    }
#pragma unroll
    for (int t = 0; t < 4; t++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            half8 b;
            float d, mn;
            D::operand(w, st, s, lane, t, j, b, d, mn);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const f32x4 r = mfma(j ? x.a1[mt] : x.a0[mt], b, zero);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if (MODE == kRow) {
                        acc[mt][t][i] = __builtin_fmaf(d, r[i], acc[mt][t][i]);
                        if (D::kMin) acc[mt][t][i] = __builtin_fmaf(-mn, sum[mt][j][i], acc[mt][t][i]);
                    } else {
                        const float v = D::kMin ? d * r[i] - mn * sum[mt][j][i] : d * r[i];
                        acc[mt][t][i] = __builtin_fmaf(x.dv[mt][i], v, acc[mt][t][i]);
                    }
                }
            }
        }
    }
}

// Streams steps [s0, s1) of the wavefront's four tiles (row block rb of the
// matrix whose planes are W).
//
// Weights and activations are loaded one step ahead of the MFMAs that use them (two
// register buffers in rotation), the activations first, so that waiting for them
// never waits for the later weight loads.  (Weights two steps ahead, through three
// buffers, measured slower: at 5 and 4 wavefronts per SIMD alike, the Q8_0 down
// kernel was no faster at 64 tokens and 3-9 % slower at 1 and 8.)
//
// Loads are unconditional, so every trip through the loop issues the same loads
// in the same order and the compiler's wait counts stay exact (a skipped load would
// make them conservative at the loop head and serialise the prefetch).  Past the
// wavefront's last step, weight loads go to step `so`, whose offsets land exactly
// at the end of the matrix's planes: out of range, so they read 0 without touching
// memory.  Activation loads repeat the last step (L2 hits).  sched_barrier keeps
// the scheduler from sinking the prefetches down to their uses.
template <class D, int MT, int MODE, class AS>
__device__ inline void mm_steps(const Planes &W, int rb, int s0, int s1, int lane, const AS &A, f32x4 (*acc)[4])
{
    if (s0 >= s1) return;
    const int sl = s1 - 1, so = (W.nrb - rb) * W.steps;
    auto ws = [&](int x) { return x < s1 ? x : so; };
    typename D::State st;
    typename D::Raw w0, w1;
    AStep<MT, MODE> x0, x1;
    load_a(x0, A, s0);
    D::load(w0, W, rb, s0, lane);
    for (int s = s0; s < s1; s += 2) {
        load_a(x1, A, min(s + 1, sl));
        D::load(w1, W, rb, ws(s + 1), lane);
        __builtin_amdgcn_sched_barrier(0);
        mm_step<D, MT, MODE>(w0, st, x0, s, lane, acc);
        if (s + 1 >= s1) break;
        load_a(x0, A, min(s + 2, sl));
        D::load(w0, W, rb, ws(s + 2), lane);
        __builtin_amdgcn_sched_barrier(0);
        mm_step<D, MT, MODE>(w1, st, x1, s + 1, lane, acc);
    }
}

struct MmArgs {
    QMat w0, w1;     // gate and up (gate/up), or down (w0)
    ActQ x;          // input activations: tokens (gate/up) or positions (down)
    Dispatch d;
    float *part;     // gate/up K partials [KS][P][2][I] when KS > 1
    ActQ act;        // gate/up output [P][I]
    float *ypart;    // down output [KS][P][H], rows in (token, slot) order
    int H, I, KS, P, use_gelu;
    int KSg;         // down with KSg > 1: its input is gate/up's KSg partials in `part`, finished in LDS
    int kk;          // slots per token row of ypart
    int nchunk;      // chunk rows of the grid: blockIdx.x = chunk + nchunk * (row block, K share)
};

// The token chunk `ci` of the dispatch's list: expert e, first position p0 and nt
// (1..16 MT) tokens; false past the end of the list.
template <int MT>
__device__ inline bool chunk_of(const Dispatch &d, int ci, int &e, int &p0, int &nt)
{
    const int n = d.meta[3];
    const uint64_t c = d.chunks[ci];  // ci < the list's capacity: loaded beside the count
    if (ci >= n) return false;
    e = (int)(c & 0xFFu);
    nt = (int)((c >> 8) & 0xFFu);
    p0 = (int)(c >> 16);
    return true;
}

// ------------------------------------------------------------ gate / up

// Grid nchunk * I/64 * KS workgroups of 256 threads; one per (token chunk of 16 MT,
// 64-row block, K share), chunks fastest.  Wave w: matrix w >> 1 (gate, up), half w & 1 of
// the workgroup's K units; the four are summed through LDS and wave 0 applies
// SiLU(g) * u to its 64 rows x 16 MT tokens.
template <class D, int MT>
__global__ __launch_bounds__(256) MM_ATTR void k_mm_gateup(MmArgs a)
{
    __shared__ f32x4 xch[3][MT][4][64];
    int e, p0, nt;
    if (!chunk_of<MT>(a.d, (int)(blockIdx.x % a.nchunk), e, p0, nt)) return;  // uniform over the workgroup
    const int rbk = (int)(blockIdx.x / a.nchunk), rb = rbk / a.KS, ks = rbk % a.KS;
    const int units = a.H / kStep / D::kSpu, upw = units / a.KS, u0 = ks * upw;
    const int wv = wave_id(), lane = threadIdx.x & 63;
    const int mat = wv >> 1, half = wv & 1;
    const int hu = (upw + 1) / 2;
    const int ub = u0 + half * hu, ue = min(u0 + upw, ub + hu);
    const Planes W = planes(mat ? a.w1 : a.w0, e);
    const int n = lane & 15, gq = lane >> 4;
    AOp<MT> A;
    A.q = make_rsrc(a.x.q, (size_t)a.x.ld * a.H * 2);  // x: ld = tokens
    A.ds = make_rsrc(a.x.ds, (size_t)(a.H / kStep) * a.x.ld * 4);
    A.ld4 = a.x.ld * 4;
    float dvr[MT][4];  // x's per-row descales of the lane's result tokens
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        A.qoff[mt] = a.d.rows[p0 + min(16 * mt + n, nt - 1)] * a.H * 2 + 32 * gq;
        A.doff[mt] = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) dvr[mt][i] = a.x.ds[a.d.rows[p0 + min(16 * mt + 4 * gq + i, nt - 1)]];
    }
    f32x4 acc[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[mt][t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    mm_steps<D, MT, kRow>(W, rb, ub * D::kSpu, ue * D::kSpu, lane, A, acc);
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[mt][t][i] *= dvr[mt][i];
    if (wv) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int t = 0; t < 4; t++) xch[wv - 1][mt][t][lane] = acc[mt][t];
    }
    __syncthreads();
    if (wv) return;
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        f32x4 gs[4], us[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            gs[t] = acc[mt][t] + xch[0][mt][t][lane];
            us[t] = xch[1][mt][t][lane] + xch[2][mt][t][lane];
        }
        if (a.KS == 1) {
            // SiLU(g) * u, quantised per token over these 64 rows (one 64-column
            // group of the down input): the 16 lanes of a DPP row hold them.
            f32x4 v[4];
            float mx[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    v[t][i] = gate_act(gs[t][i], a.use_gelu) * us[t][i];
                    mx[i] = fmaxf(mx[i], fabsf(v[t][i]));
                }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = 16 * mt + 4 * gq + i;
                const float sc = pow2_scale(row_max_f32(mx[i]));
                if (m < nt) {
                    const size_t pos = (size_t)p0 + m;
                    half_t *dst = a.act.q + pos * a.I + (size_t)kStep * rb;
#pragma unroll
                    for (int t = 0; t < 4; t++) dst[mma_pos(16 * t + n)] = (half_t)(v[t][i] * sc);
                    if (n == 0) a.act.ds[(size_t)rb * a.act.ld + pos] = 1.0f / sc;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = 16 * mt + 4 * gq + i;
                if (m < nt) {
                    float *pp = a.part + (((size_t)ks * a.P + p0 + m) * 2) * a.I + (size_t)kStep * rb + n;
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        pp[16 * t] = gs[t][i];
                        pp[a.I + 16 * t] = us[t][i];
                    }
                }
            }
        }
    }
}

// Finishes a K-split gate/up: one wavefront per (position, 64-row group) adds the
// KS partials in ks order, applies SiLU(g) * u and writes the activations.  Grid:
// P * I/64 wavefronts, 4 per workgroup.
__global__ __launch_bounds__(256) void k_act_reduce(MmArgs a)
{
    const size_t w = (size_t)blockIdx.x * 4 + wave_id();
    const int G = a.I / kStep, lane = threadIdx.x & 63;
    if (w >= (size_t)a.P * G) return;
    const int pos = (int)(w / G), rg = (int)(w % G);
    float g = 0.0f, u = 0.0f;
    for (int s = 0; s < a.KS; s++) {
        const float *pp = a.part + (((size_t)s * a.P + pos) * 2) * a.I + (size_t)kStep * rg + lane;
        g += pp[0];
        u += pp[a.I];
    }
    act_group(gate_act(g, a.use_gelu) * u, lane, a.act.q + (size_t)pos * a.I + (size_t)kStep * rg,
              a.act.ds + (size_t)rg * a.act.ld + pos);
}

// ---------------------------------------------------------------- down

// Grid nchunk * ceil(H/256) * KS workgroups of 256 threads, chunks fastest; wave w
// owns row block 4 x + w of the output (x the workgroup's row-block group), the
// workgroup's K units and token chunk.  The chunk's positions
// are consecutive, so tokens past the group's end read other groups' (or, past
// the last position, out-of-range zero) activations and are not stored.  Position
// p's result goes to row rows[p] * kk + slots[p] of the output.
//
// kPart: gate/up split its K over KSg workgroups and left the partials in `part`.
// The workgroup finishes the activations it reads itself, k_act_reduce's sums in
// the same order (so the same bits), for its chunk's tokens and its K range only,
// into LDS (dynamic: 16 MT rows of its steps, and their descales); the K loop then
// reads them from there.  No launch between gate/up and down.
template <class D, int MT, bool kPart>
__global__ __launch_bounds__(256) MM_ATTR void k_mm_down(MmArgs a)
{
    int e, p0, nt;
    if (!chunk_of<MT>(a.d, (int)(blockIdx.x % a.nchunk), e, p0, nt)) return;
    const int wv = wave_id(), lane = threadIdx.x & 63;
    const int rbk = (int)(blockIdx.x / a.nchunk);
    const int rb = kWaves * (rbk / a.KS) + wv, ks = rbk % a.KS;
    const int units = a.I / kStep / D::kSpu, upw = units / a.KS, u0 = ks * upw;
    const int n = lane & 15, gq = lane >> 4;
    const Planes W = planes(a.w0, e);
    int orow[MT][4];  // output rows of the lane's positions (loaded before the K loop)
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = min(16 * mt + 4 * gq + i, nt - 1);
            orow[mt][i] = a.d.rows[p0 + m] * a.kk + a.d.slots[p0 + m];
        }
    f32x4 acc[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[mt][t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (kPart) {
        extern __shared__ __attribute__((aligned(16))) char lds_act[];
        const int sw = upw * D::kSpu, s0 = u0 * D::kSpu;  // the workgroup's steps
        const int rowb = sw * 2 * kStep;
        float *lds_ds = reinterpret_cast<float *>(lds_act + 16 * MT * rowb);
        for (int i = threadIdx.x; i < (16 * MT - nt) * rowb / 16; i += 256)
            reinterpret_cast<u32x4 *>(lds_act + nt * rowb)[i] = (u32x4){0u, 0u, 0u, 0u};
        for (int i = threadIdx.x; i < sw * 16 * MT; i += 256)
            if (i % (16 * MT) >= nt) lds_ds[i] = 0.0f;
        // four (token, step) pieces per wavefront at once, one per 16-lane row (lane
        // l: columns 4 l .. 4 l + 3): the KSg partials of gate and up summed in
        // partial order, SiLU(g) * u, the piece's power of two from the row's
        // largest magnitude -- act_group's values, max and rounding
        const size_t qs = (size_t)a.P * 2 * a.I;
        const int l = lane & 15;
        for (int t0 = 4 * wv; t0 < nt * sw; t0 += 4 * kWaves) {  // uniform per wavefront
            const int t = t0 + (lane >> 4);
            const bool live = t < nt * sw;
            const int tt = live ? t : t0;
            const int m = tt / sw, g = tt - m * sw;
            const float *pp = a.part + ((size_t)(p0 + m) * 2) * a.I + (size_t)kStep * (s0 + g) + 4 * l;
            float gs[4] = {0.0f, 0.0f, 0.0f, 0.0f}, us[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int q = 0; q < a.KSg; q++) {
                const float4 x = *reinterpret_cast<const float4 *>(pp + q * qs);
                const float4 y = *reinterpret_cast<const float4 *>(pp + q * qs + a.I);
                gs[0] += x.x; gs[1] += x.y; gs[2] += x.z; gs[3] += x.w;
                us[0] += y.x; us[1] += y.y; us[2] += y.z; us[3] += y.w;
            }
            float v[4], mx = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[i] = gate_act(gs[i], a.use_gelu) * us[i];
                mx = fmaxf(mx, fabsf(v[i]));
            }
            const float sc = pow2_scale(row_max_f32(mx));
            if (live) {
                half_t *dq = reinterpret_cast<half_t *>(lds_act + m * rowb + g * 2 * kStep);
#pragma unroll
                for (int i = 0; i < 4; i++) dq[mma_pos(4 * l + i)] = (half_t)(v[i] * sc);
                if (l == 0) lds_ds[g * 16 * MT + m] = 1.0f / sc;
            }
        }
        __syncthreads();
        if (rb >= a.H / kRowBlock) return;  // no barriers after this one
        AOpL<MT> A;
        A.q = lds_act;
        A.ds = lds_ds;
        A.s0 = s0;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            A.qoff[mt] = (16 * mt + n) * rowb + 32 * gq;
            A.doff[mt] = 16 * mt + 4 * gq;
        }
        mm_steps<D, MT, kStepDs>(W, rb, s0, s0 + sw, lane, A, acc);
    } else {
        if (rb >= a.H / kRowBlock) return;  // no barriers in this kernel
        AOp<MT> A;
        A.q = make_rsrc(a.x.q, (size_t)a.P * a.I * 2);
        A.ds = make_rsrc(a.x.ds, (size_t)(a.I / kStep) * a.x.ld * 4);
        A.ld4 = a.x.ld * 4;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            A.qoff[mt] = (p0 + 16 * mt + n) * a.I * 2 + 32 * gq;
            A.doff[mt] = (p0 + 16 * mt + 4 * gq) * 4;
        }
        mm_steps<D, MT, kStepDs>(W, rb, u0 * D::kSpu, (u0 + upw) * D::kSpu, lane, A, acc);
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = 16 * mt + 4 * gq + i;
            if (m < nt) {
                float *yp = a.ypart + ((size_t)ks * a.P + orow[mt][i]) * a.H + (size_t)kRowBlock * rb + n;
#pragma unroll
                for (int t = 0; t < 4; t++) yp[16 * t] = acc[mt][t][i];
            }
        }
}

// ------------------------------------------------------------- combine

constexpr int kCombLanes = 8;   // slot lanes per output column group
constexpr int kCombCols = 32;   // float4 column groups per workgroup
constexpr int kMaxKS = 16;      // K partials the combine reads per position

// out[t][h] = sum over slots s of p[t][s] * y[t k + s][h] (+ scale[t] * shared),
// a deterministic gather, no atomics (main.zig:495-509 / engine.zig:725-777).  The
// rows of y are in (token, slot) order, so every load's address is known up front;
// inv[t k + s] < 0 (an expert id out of range, a row nothing wrote) only masks the
// slot's term.
// Thread (c, l) of a workgroup takes column group c and the slots s = l, l + 8,
// ...: it issues the KS partial loads of a slot together (one memory round trip
// per slot instead of one per partial), adds them in partial order and weights
// them; the eight slot-lane sums are then added in lane order through LDS.  The
// order of every addition is fixed, so results do not depend on scheduling.
// Grid: (ceil(H/4 / 32), T).
__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ ypart, const int32_t *__restrict__ inv,
                                                 const float *__restrict__ probs, int T, int k, int H, int KS, int P,
                                                 const float *__restrict__ shared, const float *__restrict__ shared_scale,
                                                 int sKS, const float *resid, float *out)
{
    __shared__ float4 part[kCombLanes + 1][kCombCols];  // slot-lane sums, then the shared term
    const int c = threadIdx.x % kCombCols, l = threadIdx.x / kCombCols;
    const int h = (blockIdx.x * kCombCols + c) * 4;
    const bool live = h < H;
    for (int t = blockIdx.y; t < T; t += gridDim.y) {  // uniform over the workgroup
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int s = l; s < k && live; s += kCombLanes) {
            const size_t ts = (size_t)t * k + s;
            const int pos = inv[ts];
            const float p = probs[ts];
            float4 z[kMaxKS];
#pragma unroll
            for (int q = 0; q < kMaxKS; q++)
                if (q < KS) z[q] = *(const float4 *)(ypart + ((size_t)q * P + ts) * H + h);
            float4 y = z[0];
#pragma unroll
            for (int q = 1; q < kMaxKS; q++)
                if (q < KS) {
                    y.x += z[q].x; y.y += z[q].y; y.z += z[q].z; y.w += z[q].w;
                }
            if (pos >= 0) {
                acc.x += p * y.x; acc.y += p * y.y; acc.z += p * y.z; acc.w += p * y.w;
            }
        }
        part[l][c] = acc;
        if (l == 0 && shared && live) {  // the shared expert's partials [sKS][T][H], then its scale
            const float sc = shared_scale ? shared_scale[t] : 1.0f;
            float4 z[kMaxKS];
#pragma unroll
            for (int q = 0; q < kMaxKS; q++)
                if (q < sKS) z[q] = *(const float4 *)(shared + ((size_t)q * T + t) * H + h);
            float4 y = z[0];
#pragma unroll
            for (int q = 1; q < kMaxKS; q++)
                if (q < sKS) {
                    y.x += z[q].x; y.y += z[q].y; y.z += z[q].z; y.w += z[q].w;
                }
            part[kCombLanes][c] = make_float4(sc * y.x, sc * y.y, sc * y.z, sc * y.w);
        }
        __syncthreads();
        if (l == 0 && live) {
            float4 r = part[0][c];
#pragma unroll
            for (int i = 1; i < kCombLanes + 1; i++) {
                if (i == kCombLanes && !shared) break;
                const float4 v = part[i][c];
                r.x += v.x; r.y += v.y; r.z += v.z; r.w += v.w;
            }
            if (resid) {  // x += proj (main.zig:519): the residual plus the whole block output
                const float4 x = *(const float4 *)(resid + (size_t)t * H + h);
                r = make_float4(x.x + r.x, x.y + r.y, x.z + r.z, x.w + r.w);
            }
            *(float4 *)(out + (size_t)t * H + h) = r;
        }
        __syncthreads();
    }
}

// Large calls: one thread per (token, 4 columns), slots in order, eight slots'
// loads issued together (indices clamped rather than branched on).  Grid: T * H/4
// threads.
template <int NS>
__global__ __launch_bounds__(256) void k_combine_rows(const float *__restrict__ ypart, const int32_t *__restrict__ inv,
                                                      const float *__restrict__ probs, int T, int k, int H, int KS,
                                                      int P, const float *__restrict__ shared,
                                                      const float *__restrict__ shared_scale, int sKS,
                                                      const float *resid, float *out)
{
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int H4 = H / 4;
    if (id >= (size_t)T * H4) return;
    const int t = (int)(id / H4), h = (int)(id % H4) * 4;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0; s0 < k; s0 += NS) {  // NS slots per pass, their loads issued together
        int pos[NS];
        float p[NS];
        bool ok[NS];
        float4 y[NS];
#pragma unroll
        for (int i = 0; i < NS; i++) {
            const int s = min(s0 + i, k - 1);
            pos[i] = (int)((size_t)t * k + s);
            const int iv = inv[pos[i]];
            p[i] = probs[pos[i]];
            ok[i] = s0 + i < k && iv >= 0;
            y[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        for (int q = 0; q < KS; q++) {
#pragma unroll
            for (int i = 0; i < NS; i++) {
                const float4 z = *(const float4 *)(ypart + ((size_t)q * P + pos[i]) * H + h);
                y[i].x += z.x; y[i].y += z.y; y[i].z += z.z; y[i].w += z.w;
            }
        }
#pragma unroll
        for (int i = 0; i < NS; i++)
            if (ok[i]) {
                acc.x += p[i] * y[i].x; acc.y += p[i] * y[i].y; acc.z += p[i] * y[i].z; acc.w += p[i] * y[i].w;
            }
    }
    if (shared) {
        const float sc = shared_scale ? shared_scale[t] : 1.0f;
        float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int q = 0; q < sKS; q++) {
            const float4 z = *(const float4 *)(shared + ((size_t)q * T + t) * H + h);
            y.x += z.x; y.y += z.y; y.z += z.z; y.w += z.w;
        }
        acc.x += sc * y.x; acc.y += sc * y.y; acc.z += sc * y.z; acc.w += sc * y.w;
    }
    if (resid) {
        const float4 x = *(const float4 *)(resid + (size_t)t * H + h);
        acc = make_float4(x.x + acc.x, x.y + acc.y, x.z + acc.z, x.w + acc.w);
    }
    *(float4 *)(out + (size_t)t * H + h) = acc;
}

// ------------------------------------------------------------- planning

static int steps_per_unit(int type) { return tile_fmt(type).spu; }

// Dynamic LDS of a kPart down workgroup: 16 rows of its steps in the activation
// format, and a descale per (step, row).
constexpr size_t kFuseLdsMax = 64 * 1024;
static size_t down_part_lds(int down_type, int I, int ks_dn)
{
    const int spu = steps_per_unit(down_type);
    const size_t sw = (size_t)(I / kStep / spu / ks_dn) * spu;
    return 16 * sw * 2 * kStep + sw * 16 * 4;
}

bool mm_supported(int type) { return tile_fmt(type).qb != 0; }

// Splits a K axis of `units` scale units over ks workgroups, ks dividing units
// and at most kMaxKS (the partials the combine reads): the smallest ks that gives
// `wg_per_ks * ks` >= ANEDVD_WG_TARGET workgroups while every wavefront keeps >=
// `min_steps` steps of `waves_per_k` shares, else the largest ks keeping them.
static int choose_ks(int units, int spu, long wg_per_ks, int waves_per_k, int min_steps)
{
    int best = 1;
    for (int ks = 1; ks <= std::min(units, kMaxKS); ks++) {
        if (units % ks) continue;
        const int steps = (units / ks) * spu / waves_per_k;
        if (ks > 1 && steps < min_steps) break;
        best = ks;
        if (wg_per_ks * ks >= ANEDVD_WG_TARGET) break;
    }
    return best;
}

MmPlan plan_mm(int gate_type, int down_type, int H, int I, int P, int max_u, int T)
{
    MmPlan p{};
    // The grouped GEMM (64-token chunks of a group, activations staged in LDS and
    // shared by four wavefronts) once the groups average 32 tokens and its gate/up
    // grid has a workgroup per CU at least; the chunks then give the grid its
    // parallelism and K is not split.  Below that, the decode kernels: 16-token
    // tiles, activations straight from L2, K split over workgroups.  (A single
    // shared expert at 32 tokens on the grouped GEMM would be 22 workgroups: it
    // measured 105 us against the decode kernels' split K.  Kernels that read the
    // activations from L2 per wavefront with folded scales and 32- or 64-token
    // chunks measured 233 against 192 us on the Qwen3 512-token prefill and 512
    // against 377 us on the DeepSeek 1024-token one: four wavefronts fetching the
    // same activations from L2 cost more than staging them once in LDS.)
    const long mean = P / std::max(max_u, 1);
    const long pf_wgs = (long)((P + 63) / 64) * (I / 128);
    if (mean >= ANEDVD_STAGED_MIN && grouped_supported(H, I) && pf_wgs >= 256) {
        p.kind = kMmStaged;
        // 128-token workgroups once the groups average 64 tokens: each dequantised
        // step then feeds eight token tiles instead of four.  (Mixtral 2048 tokens:
        // gate/up 1.31 -> 1.20 ms; DeepSeek-V2-Lite 1024: gate/up 220 -> 210 us,
        // down 130 -> 111 us.)
        const long wide_wgs = (long)((P + 127) / 128) * (I / 128);
        const bool wide = mean >= ANEDVD_PF_WIDE_MIN && wide_wgs >= 256;
        p.mt_gu = wide && grouped_wide(gate_type) ? 8 : 4;
        p.mt_dn = wide && grouped_wide_down(down_type) ? 8 : 4;
        // A long down K (>= 128 steps) splits in two when that shortens the grid's
        // rounds of resident workgroups (two per CU) by 10 %: a partial last round
        // is then half as long, for one more plane for the combine to add.
        // (Mixtral 2048 tokens: down 858 -> 700 us, combine 27 -> 45 us.)
        const long dn_wgs = (long)(P / (16 * p.mt_dn) + max_u) * (H / 256);
        const long r1 = (dn_wgs + 2 * kCUs - 1) / (2 * kCUs), r2 = (2 * dn_wgs + 2 * kCUs - 1) / (2 * kCUs);
        p.ks_dn = I / kStep >= 128 && 10 * r2 <= 18 * r1 && grouped_down_ks_ok(down_type, I, 2) ? 2 : 1;
        p.mt = std::max(p.mt_gu, p.mt_dn);
        p.contig = P >= 2 * 16 * p.mt * (long)max_u;  // experts average two chunks or more
        // (the decode down writes one K partial: the combine reads the same count for every row)
        p.small = mean < ANEDVD_SMALL_MEAN && p.ks_dn == 1 && p.mt == 4 ? std::min(ANEDVD_SMALL_GROUP, 16) : 0;
        p.nsmall = p.small ? max_u : 0;
    } else {
        p.kind = kMmDecode;
        p.mt = 1;
    }
    p.chunk = 16 * p.mt;
    p.nchunk = P / p.chunk + max_u;
    p.xper = p.kind == kMmStaged && p.contig ? (p.nchunk + 7) / 8 : 0;  // the grouped grid's work items per XCD
    if (p.kind != kMmDecode) {
        p.ks_gu = 1;
        return p;
    }
    p.ks_gu = choose_ks(H / kStep / steps_per_unit(gate_type), steps_per_unit(gate_type), (long)max_u * (I / kRowBlock),
                        2, 2);
    p.ks_dn = choose_ks(I / kStep / steps_per_unit(down_type), steps_per_unit(down_type),
                        (long)max_u * ((H / kRowBlock + kWaves - 1) / kWaves), 1, 2);
#ifdef ANEDVD_KS_DN
    if (max_u > 64 && (I / kStep / steps_per_unit(down_type)) % ANEDVD_KS_DN == 0) p.ks_dn = ANEDVD_KS_DN;
#endif
    // A K-split gate/up is finished inside the down kernel (k_mm_down<kPart>) when
    // a down workgroup's rows of its K range fit the LDS budget and its prologue
    // has at most 64 (token, step) pieces, four memory round trips (16 pieces each),
    // even if every token of the call sends a slot to the same expert (a chunk
    // holds at most min(T, 16) tokens).  Otherwise k_act_reduce finishes them.
    const int sw = I / kStep / steps_per_unit(down_type) / p.ks_dn * steps_per_unit(down_type);
    p.fuse = p.ks_gu > 1 && down_part_lds(down_type, I, p.ks_dn) <= kFuseLdsMax && std::min(T, 16) * sw <= 64;
    return p;
}

// ------------------------------------------------------------- launchers

template <class D, int MT>
static int launch_gateup_t(const MmArgs &a, hipStream_t st)
{
    const size_t wgs = (size_t)a.nchunk * (a.I / kRowBlock) * a.KS;
    hipLaunchKernelGGL((k_mm_gateup<D, MT>), dim3((unsigned)wgs), dim3(256), 0, st, a);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

template <class D, int MT>
static int launch_down_t(const MmArgs &a, hipStream_t st)
{
    static_assert(MT == 1, "the kPart LDS budget is sized for 16-token chunks");
    const size_t wgs = (size_t)a.nchunk * ((a.H / kRowBlock + kWaves - 1) / kWaves) * a.KS;
    if (a.KSg > 1) {
        const size_t lds = down_part_lds(a.w0.type, a.I, a.KS);
        hipLaunchKernelGGL((k_mm_down<D, MT, true>), dim3((unsigned)wgs), dim3(256), lds, st, a);
    } else {
        hipLaunchKernelGGL((k_mm_down<D, MT, false>), dim3((unsigned)wgs), dim3(256), 0, st, a);
    }
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

template <class D>
static int launch_gateup_d(const MmArgs &a, int, hipStream_t st)
{
    return launch_gateup_t<D, 1>(a, st);
}

template <class D>
static int launch_down_d(const MmArgs &a, int, hipStream_t st)
{
    return launch_down_t<D, 1>(a, st);
}

int launch_expert_gateup(const QMat &gate, const QMat &up, const ActQ &x, int H, int I, const Dispatch &d, int P,
                         const MmPlan &plan, float *part, const ActQ &act, int use_gelu, hipStream_t st)
{
    if (plan.kind == kMmStaged)
        return launch_grouped_gateup(gate, up, x, H, I, d, P, plan.mt_gu, plan.nchunk, plan.contig, plan.nsmall, act,
                                     use_gelu, st);
    if (gate.type != up.type) {
        set_error("expert gate/up: gate type %d and up type %d differ", gate.type, up.type);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
    MmArgs a{};
    a.w0 = gate;
    a.w1 = up;
    a.x = x;
    a.d = d;
    a.part = part;
    a.act = act;
    a.H = H;
    a.I = I;
    a.KS = plan.ks_gu;
    a.P = P;
    a.use_gelu = use_gelu;
    a.nchunk = plan.nchunk;
    int rc;
    switch (gate.type) {
    case ANEDVD_Q8_0:
    case ANEDVD_Q8_1: rc = launch_gateup_d<MQ8_0>(a, plan.mt, st); break;  // one tile layout
    case ANEDVD_F16: rc = launch_gateup_d<MF16>(a, plan.mt, st); break;
    case ANEDVD_Q4_0: rc = launch_gateup_d<MQ4_0>(a, plan.mt, st); break;
    case ANEDVD_Q4_1: rc = launch_gateup_d<MQ4_1>(a, plan.mt, st); break;
    case ANEDVD_Q5_0: rc = launch_gateup_d<MQ5_0>(a, plan.mt, st); break;
    case ANEDVD_Q5_1: rc = launch_gateup_d<MQ5_1>(a, plan.mt, st); break;
    case ANEDVD_Q2_K: rc = launch_gateup_d<MQ2_K>(a, plan.mt, st); break;
    case ANEDVD_Q3_K: rc = launch_gateup_d<MQ3_K>(a, plan.mt, st); break;
    case ANEDVD_Q4_K: rc = launch_gateup_d<MQ4_K>(a, plan.mt, st); break;
    case ANEDVD_Q5_K: rc = launch_gateup_d<MQ5_K>(a, plan.mt, st); break;
    case ANEDVD_Q6_K: rc = launch_gateup_d<MQ6_K>(a, plan.mt, st); break;
    default:
        set_error("expert gate/up: ggml type %d has no kernel", gate.type);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
    if (rc != ANEDVD_OK || plan.ks_gu == 1 || plan.fuse) return rc;  // fuse: the down kernel finishes them
    const size_t waves = (size_t)P * (I / kStep);
    hipLaunchKernelGGL(k_act_reduce, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, a);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

int launch_expert_down(const QMat &down, const ActQ &act, int H, int I, const Dispatch &d, int P,
                       const MmPlan &plan, const float *part, int use_gelu, float *ypart, int kk, hipStream_t st)
{
    if (!d.rows || !d.slots || !ypart || kk <= 0 || (plan.fuse && !part)) {
        set_error("down: the dispatch's rows and slots, the output and a fused gate/up's partials are needed (kk %d)",
                  kk);
        return ANEDVD_E_INVALID_ARG;
    }
    if (plan.kind == kMmStaged)
        return launch_grouped_down(down, act, H, I, d, P, plan.mt_dn, plan.nchunk, plan.contig, plan.nsmall, plan.ks_dn,
                                   ypart, kk, st);
    MmArgs a{};
    a.w0 = down;
    a.x = act;
    a.d = d;
    a.ypart = ypart;
    a.kk = kk;
    a.H = H;
    a.I = I;
    a.KS = plan.ks_dn;
    a.P = P;
    a.nchunk = plan.nchunk;
    if (plan.fuse) {
        a.part = const_cast<float *>(part);
        a.KSg = plan.ks_gu;
        a.use_gelu = use_gelu;
    }
    switch (down.type) {
    case ANEDVD_Q8_0:
    case ANEDVD_Q8_1: return launch_down_d<MQ8_0>(a, plan.mt, st);
    case ANEDVD_F16: return launch_down_d<MF16>(a, plan.mt, st);
    case ANEDVD_Q4_0: return launch_down_d<MQ4_0>(a, plan.mt, st);
    case ANEDVD_Q4_1: return launch_down_d<MQ4_1>(a, plan.mt, st);
    case ANEDVD_Q5_0: return launch_down_d<MQ5_0>(a, plan.mt, st);
    case ANEDVD_Q5_1: return launch_down_d<MQ5_1>(a, plan.mt, st);
    case ANEDVD_Q2_K: return launch_down_d<MQ2_K>(a, plan.mt, st);
    case ANEDVD_Q3_K: return launch_down_d<MQ3_K>(a, plan.mt, st);
    case ANEDVD_Q4_K: return launch_down_d<MQ4_K>(a, plan.mt, st);
    case ANEDVD_Q5_K: return launch_down_d<MQ5_K>(a, plan.mt, st);
    case ANEDVD_Q6_K: return launch_down_d<MQ6_K>(a, plan.mt, st);
    default:
        set_error("expert down: ggml type %d has no kernel", down.type);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
}

int launch_combine(const float *ypart, const int32_t *inv, const float *probs, int T, int k, int H, int KS, int P,
                   const float *shared, const float *shared_scale, int sKS, float *out, hipStream_t st,
                   const float *resid)
{
    if (T <= 0) return ANEDVD_OK;
    if (KS > kMaxKS || sKS > kMaxKS) {
        set_error("combine: %d K partials, at most %d", max(KS, sKS), kMaxKS);
        return ANEDVD_E_INVALID_ARG;
    }
    const size_t threads = (size_t)T * (H / 4);
    // From 32768 (token, column) threads on, one thread per column group with its
    // slots in order: the Qwen3 B=64 step (32768) 119.1-119.4 -> 117.7 us against the
    // slot-parallel kernel; at B=32 (16384) the slot-parallel one is as fast or faster.
    if (threads >= 32768) {
        const dim3 grid((unsigned)((threads + 255) / 256));
        if (k <= 2)  // as many slot loads per pass as there are slots (Mixtral: 2, not 8 clamped copies)
            hipLaunchKernelGGL(k_combine_rows<2>, grid, dim3(256), 0, st, ypart, inv, probs, T, k, H, KS, P, shared,
                               shared_scale, sKS, resid, out);
        else if (k <= 4)
            hipLaunchKernelGGL(k_combine_rows<4>, grid, dim3(256), 0, st, ypart, inv, probs, T, k, H, KS, P, shared,
                               shared_scale, sKS, resid, out);
        else
            hipLaunchKernelGGL(k_combine_rows<8>, grid, dim3(256), 0, st, ypart, inv, probs, T, k, H, KS, P, shared,
                               shared_scale, sKS, resid, out);
    } else {  // decode: spread the slots over lanes so each thread waits on one slot's loads
        const dim3 grid((unsigned)((H / 4 + kCombCols - 1) / kCombCols), (unsigned)std::min(T, 65535));
        hipLaunchKernelGGL(k_combine, grid, dim3(kCombLanes * kCombCols), 0, st, ypart, inv, probs, T, k, H, KS, P,
                           shared, shared_scale, sKS, resid, out);
    }
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

}  // namespace anedvd
