// fq.h -- the folded-scale decoders of the grouped GEMM (k_pf.hip), which
// dequantises a whole step once to f16 and reuses it for several 16-token tiles:
// the block and sub-block scales go into the f16 weights, so the MFMA accumulates
// the whole K with no per-block rescale.
#pragma once

#include "common.h"
#include "mma.h"

namespace anedvd {

// Weight steps loaded ahead of the one being multiplied, at least (the grouped
// loop may go deeper): the super-block formats two, the 32-element formats one.
#ifndef ANEDVD_PF_DEPTH_K
#define ANEDVD_PF_DEPTH_K 2
#endif
#ifndef ANEDVD_PF_DEPTH_L
#define ANEDVD_PF_DEPTH_L 1
#endif
constexpr int kPfTiles = 4;   // 16-row tiles per wavefront: each staged A read feeds four MFMAs
// Cache policy of the weight loads.  The grouped GEMM reads an expert's weight
// slice once per chunk of its group (the chunks of one row group run side by
// side on one XCD), so the loads keep the default policy and the later chunks hit
// in L2, where the decode kernels stream every weight once (non-temporal).
#ifndef ANEDVD_PF_WAUX
#define ANEDVD_PF_WAUX 0
#endif
constexpr int kPfAux = ANEDVD_PF_WAUX;

__device__ inline half_t h_bits(uint32_t b)
{
    const uint16_t u = (uint16_t)b;
    half_t h;
    __builtin_memcpy(&h, &u, 2);
    return h;
}

__device__ inline h2 as_h2(uint32_t b)
{
    h2 h;
    __builtin_memcpy(&h, &b, 4);
    return h;
}

__device__ inline uint32_t h2_bits(h2 h)
{
    uint32_t b;
    __builtin_memcpy(&b, &h, 4);
    return b;
}


// Where a wavefront's four 16-row tiles come from: tile tt is tile idx(tt) of row
// block rb of planes src(tt).  One matrix's whole 64-row block (Tiles1), or two
// tiles each of two matrices of the same shape (Tiles2: gate and up, tiles t0 and
// t0 + 1).  tt is a compile-time index in every use, so the choice folds away.
struct Tiles1 {
    Planes p;
    __device__ const Planes &src(int) const { return p; }
    __device__ int idx(int tt) const { return tt; }
};
struct Tiles2 {
    Planes g, u;
    int t0;
    __device__ const Planes &src(int tt) const { return tt < 2 ? g : u; }
    __device__ int idx(int tt) const { return t0 + (tt & 1); }
};

// ------------------------------------------------------------------ decoders
//
// A decoder loads one step of a wavefront's four row tiles: load() (kUnit 1 or 0:
// the caller knows at compile time whether step s starts a scale unit, which
// then loads the unit's scales; -1: decided from s);
// takes what stays valid for a whole scale unit on the unit's first step: begin();
// and yields the f16 B operand of (tile tt, block j) at step `ss` of the unit:
// bop().  Lane l = 16 g + n holds row n of the tile and the 8 columns 32 j + 8 g + i.

// F16 experts: the tile holds the values themselves.
struct FF16 {
    static constexpr int kSpu = 1;
    static constexpr bool kHoistA = false;  // 32 VGPRs of values per ring slot already
    static constexpr int kDepth = ANEDVD_PF_DEPTH_L;       // steps of weights in flight ahead
    static constexpr int kMinLoads = 8;                    // load instructions of every load() call
    struct Raw {
        u32x4 q[kPfTiles][2];
    };
    struct State {};
    template <int kUnit = -1, class TS>
    __device__ static inline void load(Raw &r, const TS &ts, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(ts.src(0), rb, s, 32);
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++)
#pragma unroll
            for (int j = 0; j < 2; j++)
                r.q[tt][j] = __builtin_amdgcn_raw_buffer_load_b128(ts.src(tt).q, 32 * lane, qo + 2048 * ts.idx(tt) + 16 * j,
                                                                   kPfAux);
    }
    __device__ static inline void begin(const Raw &, State &, int, int) {}
    __device__ static inline half8 bop(const Raw &r, const State &, int, int tt, int j, int) { return as_h8(r.q[tt][j]); }
};

struct FQ8_0 {
    static constexpr int kSpu = 1;
    static constexpr bool kHoistA = false;  // at 176 VGPRs two waves per SIMD instead of three
    static constexpr int kDepth = ANEDVD_PF_DEPTH_L;       // steps of weights in flight ahead
    static constexpr int kMinLoads = 8;
    struct Raw {
        u32x4 q[kPfTiles];
        uint32_t s[kPfTiles];
    };
    struct State {};
    template <int kUnit = -1, class TS>
    __device__ static inline void load(Raw &r, const TS &ts, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(ts.src(0), rb, s, 16), so = row_plane_off(ts.src(0), rb, s, 4);
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) {
            r.q[tt] = __builtin_amdgcn_raw_buffer_load_b128(ts.src(tt).q, 16 * lane, qo + 1024 * ts.idx(tt), kPfAux);
            r.s[tt] = __builtin_amdgcn_raw_buffer_load_b32(ts.src(tt).s, 4 * (lane & 15), so + 64 * ts.idx(tt), kPfAux);
        }
    }
    __device__ static inline void begin(const Raw &, State &, int, int) {}
    __device__ static inline half8 bop(const Raw &r, const State &, int, int tt, int j, int)
    {
        const half8 q = bytes_h8(r.q[tt][2 * j], r.q[tt][2 * j + 1]) - (half_t)1152.0f;  // exact q
        return q * h_bits(r.s[tt] >> (16 * j));  // d * q, rounded once
    }
};

struct FQ4_0 {
    static constexpr int kSpu = 1;
    static constexpr bool kHoistA = true;   // activation fragments read at the step's start
    static constexpr int kDepth = ANEDVD_PF_DEPTH_L;       // steps of weights in flight ahead
    static constexpr int kMinLoads = 8;
    struct Raw {
        u32x2 q[kPfTiles];
        uint32_t s[kPfTiles];
    };
    struct State {};
    template <int kUnit = -1, class TS>
    __device__ static inline void load(Raw &r, const TS &ts, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(ts.src(0), rb, s, 8), so = row_plane_off(ts.src(0), rb, s, 4);
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) {
            r.q[tt] = __builtin_amdgcn_raw_buffer_load_b64(ts.src(tt).q, 8 * lane, qo + 512 * ts.idx(tt), kPfAux);
            r.s[tt] = __builtin_amdgcn_raw_buffer_load_b32(ts.src(tt).s, 4 * (lane & 15), so + 64 * ts.idx(tt), kPfAux);
        }
    }
    __device__ static inline void begin(const Raw &, State &, int, int) {}
    __device__ static inline half8 bop(const Raw &r, const State &, int, int tt, int j, int)
    {
        const uint32_t v = r.q[tt][j];
        const half_t d = h_bits(r.s[tt] >> (16 * j));
        return nibbles_h8(v) * d + d * (half_t)-8.0f;  // n d - 8 d (exact) rounded once: (n - 8) d
    }
};

// Q4_1 / Q5_1: y = d q + m (gguf.zig:778-822), d q + m rounded once to f16; Q5_0:
// y = d (q - 16), rounded once.  The 5-bit formats' fifth bits come from the
// high-bit plane.
template <bool kFive, bool kHasMin>
struct FQLegacy {
    static constexpr int kSpu = 1;
    static constexpr bool kHoistA = !kFive;  // the 5-bit formats: three waves per SIMD without it
    static constexpr int kDepth = ANEDVD_PF_DEPTH_L;       // steps of weights in flight ahead
    static constexpr int kMinLoads = kFive ? 12 : 8;
    struct Raw {
        u32x2 q[kPfTiles];
        uint32_t h[kFive ? kPfTiles : 1];
        u32x2 s[kPfTiles];  // (d0 | m0 << 16, d1 | m1 << 16) with a min, else (d0 | d1 << 16, -)
    };
    struct State {};
    template <int kUnit = -1, class TS>
    __device__ static inline void load(Raw &r, const TS &ts, int rb, int s, int lane)
    {
        const Planes &p = ts.src(0);
        const int qo = lane_plane_off(p, rb, s, 8), so = row_plane_off(p, rb, s, kHasMin ? 8 : 4);
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) {
            const int ti = ts.idx(tt);
            r.q[tt] = __builtin_amdgcn_raw_buffer_load_b64(ts.src(tt).q, 8 * lane, qo + 512 * ti, kPfAux);
            if constexpr (kHasMin)
                r.s[tt] = __builtin_amdgcn_raw_buffer_load_b64(ts.src(tt).s, 8 * (lane & 15), so + 128 * ti, kPfAux);
            else
                r.s[tt].x = __builtin_amdgcn_raw_buffer_load_b32(ts.src(tt).s, 4 * (lane & 15), so + 64 * ti, kPfAux);
        }
        if constexpr (kFive) {
            const int ho = lane_plane_off(p, rb, s, 2);
#pragma unroll
            for (int tt = 0; tt < kPfTiles; tt++)
                r.h[tt] = __builtin_amdgcn_raw_buffer_load_b16(ts.src(tt).h, 2 * lane, ho + 128 * ts.idx(tt), kPfAux);
        }
    }
    __device__ static inline void begin(const Raw &, State &, int, int) {}
    __device__ static inline half8 bop(const Raw &r, const State &, int, int tt, int j, int)
    {
        const uint32_t v = r.q[tt][j];
        half8 q;  // exact
        if constexpr (kFive) {
            const uint32_t lo = (v & 0x0F0F0F0Fu) | bit4_of_bytes(r.h[tt] >> (8 * j));
            const uint32_t hi = ((v >> 4) & 0x0F0F0F0Fu) | bit4_of_bytes(r.h[tt] >> (8 * j + 4));
            q = bytes_h8(lo, hi) - (half_t)(kHasMin ? 1024.0f : 1040.0f);
        } else {
            q = nibbles_h8(v);
        }
        if constexpr (kHasMin) {
            const uint32_t dm = r.s[tt][j];
            return q * h_bits(dm) + h_bits(dm >> 16);
        } else {
            return q * h_bits(r.s[tt].x >> (16 * j));
        }
    }
};
using FQ4_1 = FQLegacy<false, true>;
using FQ5_0 = FQLegacy<true, false>;
using FQ5_1 = FQLegacy<true, true>;

// Q4_K: y = d1 * n - m1 (gguf.zig:960-996) with d1 = d * sc and m1 = dmin * m
// formed in f32 once per super-block and kept as f16; the nibble n is exact and
// the f16 FMA rounds once, so a weight is within 2^-10 of its scale.
struct FQ4_K {
    static constexpr int kSpu = 4;
    static constexpr bool kHoistA = true;   // activation fragments read at the step's start
    static constexpr int kDepth = ANEDVD_PF_DEPTH_K;       // steps of weights in flight ahead
    static constexpr int kMinLoads = 4;                    // the scales come on a unit's first step only
    struct Raw {
        u32x2 q[kPfTiles];
        u32x4 sc[kPfTiles];  // d, dmin, scales: loaded on a unit's first step
    };
    struct State {
        uint32_t dm[kPfTiles][8];  // f16 d1 | f16 (-m1) << 16 per (tile, sub-block)
    };
    template <int kUnit = -1, class TS>
    __device__ static inline void load(Raw &r, const TS &ts, int rb, int s, int lane)
    {
        const Planes &p = ts.src(0);
        const int qo = lane_plane_off(p, rb, s, 8);
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++)
            r.q[tt] = __builtin_amdgcn_raw_buffer_load_b64(ts.src(tt).q, 8 * lane, qo + 512 * ts.idx(tt), kPfAux);
        if (kUnit > 0 || (kUnit < 0 && (s & 3) == 0)) {
            const int so = row_plane_off(p, rb, s >> 2, 16);
#pragma unroll
            for (int tt = 0; tt < kPfTiles; tt++)
                r.sc[tt] = __builtin_amdgcn_raw_buffer_load_b128(ts.src(tt).s, 16 * (lane & 15), so + 256 * ts.idx(tt), kPfAux);
        }
    }
    // The 6-bit scales and mins of getScaleMinK4 (gguf.zig:948-958) for all eight
    // sub-blocks at once, a byte each: a_lo / m_lo for sub-blocks 0..3 (bytes 0..3
    // and 4..7 of the packed 12), a_hi / m_hi for 4..7 (the low or high nibble of
    // bytes 8..11 with the top two bits of bytes 0..3 or 4..7).  Each (a, m) pair
    // becomes the exact f16 pair (a, m) by the 0x64 exponent trick, and one packed
    // f16 multiply by (d, -dmin) gives (d a, -dmin m): the exact product rounded once,
    // as rounding the f32 product d * a to f16 does.
    __device__ static inline void begin(const Raw &r, State &st, int ss, int)
    {
        if (ss) return;
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) {
            const uint32_t y = r.sc[tt].y, z = r.sc[tt].z, w = r.sc[tt].w;
            const uint32_t a_lo = y & 0x3F3F3F3Fu, m_lo = z & 0x3F3F3F3Fu;
            const uint32_t a_hi = (w & 0x0F0F0F0Fu) | ((y >> 2) & 0x30303030u);
            const uint32_t m_hi = ((w >> 4) & 0x0F0F0F0Fu) | ((z >> 2) & 0x30303030u);
            // (a_j, m_j, a_j+1, m_j+1) byte pairs
            const uint32_t am[4] = {__builtin_amdgcn_perm(m_lo, a_lo, 0x05010400u),
                                    __builtin_amdgcn_perm(m_lo, a_lo, 0x07030602u),
                                    __builtin_amdgcn_perm(m_hi, a_hi, 0x05010400u),
                                    __builtin_amdgcn_perm(m_hi, a_hi, 0x07030602u)};
            const h2 dd = as_h2(r.sc[tt].x ^ 0x80000000u);  // (d, -dmin)
#pragma unroll
            for (int sub = 0; sub < 8; sub++) {
                const uint32_t biased = (sub & 1) ? pair23(am[sub >> 1]) : pair01(am[sub >> 1]);  // 1024 + a, 1024 + m
                const h2 dm = dd * (as_h2(biased) - (h2)1024.0f);
                st.dm[tt][sub] = h2_bits(dm);
            }
        }
    }
    __device__ static inline half8 bop(const Raw &r, const State &st, int ss, int tt, int j, int)
    {
        const uint32_t v = r.q[tt][j];
        const half8 nib = nibbles_h8(v);  // exact n
        const uint32_t dm = st.dm[tt][2 * ss + j];
        return nib * h_bits(dm) + h_bits(dm >> 16);
    }
};

// Q5_K: y = d1 q - m1 (gguf.zig:998-1034), the Q4_K scheme with the fifth bit of
// each value from the high-bit plane (2 bytes per lane per step).
struct FQ5_K {
    static constexpr int kSpu = 4;
    static constexpr bool kHoistA = true;   // activation fragments read at the step's start
    static constexpr int kDepth = ANEDVD_PF_DEPTH_K;       // steps of weights in flight ahead
    static constexpr int kMinLoads = 8;
    struct Raw {
        u32x2 q[kPfTiles];
        uint32_t h[kPfTiles];
        u32x4 sc[kPfTiles];  // d, dmin, scales: loaded on a unit's first step
    };
    using State = FQ4_K::State;
    template <int kUnit = -1, class TS>
    __device__ static inline void load(Raw &r, const TS &ts, int rb, int s, int lane)
    {
        const Planes &p = ts.src(0);
        const int qo = lane_plane_off(p, rb, s, 8), ho = lane_plane_off(p, rb, s, 2);
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) {
            r.q[tt] = __builtin_amdgcn_raw_buffer_load_b64(ts.src(tt).q, 8 * lane, qo + 512 * ts.idx(tt), kPfAux);
            r.h[tt] = __builtin_amdgcn_raw_buffer_load_b16(ts.src(tt).h, 2 * lane, ho + 128 * ts.idx(tt), kPfAux);
        }
        if (kUnit > 0 || (kUnit < 0 && (s & 3) == 0)) {
            const int so = row_plane_off(p, rb, s >> 2, 16);
#pragma unroll
            for (int tt = 0; tt < kPfTiles; tt++)
                r.sc[tt] = __builtin_amdgcn_raw_buffer_load_b128(ts.src(tt).s, 16 * (lane & 15), so + 256 * ts.idx(tt), kPfAux);
        }
    }
    __device__ static inline void begin(const Raw &r, State &st, int ss, int lane)
    {
        FQ4_K::Raw k;
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) k.sc[tt] = r.sc[tt];
        FQ4_K::begin(k, st, ss, lane);
    }
    __device__ static inline half8 bop(const Raw &r, const State &st, int ss, int tt, int j, int)
    {
        const uint32_t v = r.q[tt][j], hb = r.h[tt];
        const uint32_t lo = (v & 0x0F0F0F0Fu) | bit4_of_bytes(hb >> (8 * j));
        const uint32_t hi = ((v >> 4) & 0x0F0F0F0Fu) | bit4_of_bytes(hb >> (8 * j + 4));
        const half8 q = bytes_h8(lo, hi) - (half_t)1024.0f;  // exact q in [0, 31]
        const uint32_t dm = st.dm[tt][2 * ss + j];
        return q * h_bits(dm) + h_bits(dm >> 16);
    }
};

// Q2_K / Q3_K: 2-bit fields four per byte, 16-element sub-blocks (the lane's
// 8 columns of block j lie in sub-block 4 ss + 2 j + g / 2).  Q3_K: y = (d sc) (u - 4)
// with d sc formed in f32 and kept as f16, the product rounded once; Q2_K: y = dl v - ml
// with dl, ml formed in f32 and kept as f16, the f16 FMA rounding once.
template <bool kThree>
struct FQ23K {
    static constexpr int kSpu = 4;
    static constexpr bool kHoistA = true;   // activation fragments read at the step's start
    static constexpr int kDepth = ANEDVD_PF_DEPTH_K;       // steps of weights in flight ahead
    static constexpr int kMinLoads = kThree ? 8 : 4;
    struct Raw {
        uint32_t q[kPfTiles];
        uint32_t h[kThree ? kPfTiles : 1];
        u32x4 sc[kPfTiles];     // sub-block scales (a unit's first step)
        uint32_t dm[kPfTiles];  // d (Q3_K) or d | dmin << 16 (Q2_K) (a unit's first step)
    };
    struct State {
        half_t dl[kPfTiles][8], ml[kPfTiles][8];  // [tt][2 ss + j] of the lane's sub-block 4 ss + 2 j + g / 2
    };
    template <int kUnit = -1, class TS>
    __device__ static inline void load(Raw &r, const TS &ts, int rb, int s, int lane)
    {
        const Planes &p = ts.src(0);
        const int qo = lane_plane_off(p, rb, s, 4);
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) {
            const int ti = ts.idx(tt);
            r.q[tt] = __builtin_amdgcn_raw_buffer_load_b32(ts.src(tt).q, 4 * lane, qo + 256 * ti, kPfAux);
            if constexpr (kThree)
                r.h[tt] = __builtin_amdgcn_raw_buffer_load_b16(ts.src(tt).h, 2 * lane, lane_plane_off(p, rb, s, 2) + 128 * ti,
                                                               kPfAux);
        }
        if (kUnit > 0 || (kUnit < 0 && (s & 3) == 0)) {
            const int so = row_plane_off(p, rb, s >> 2, 16), dof = row_plane_off(p, rb, s >> 2, kThree ? 2 : 4);
#pragma unroll
            for (int tt = 0; tt < kPfTiles; tt++) {
                const int ti = ts.idx(tt);
                r.sc[tt] = __builtin_amdgcn_raw_buffer_load_b128(ts.src(tt).s, 16 * (lane & 15), so + 256 * ti, kPfAux);
                if constexpr (kThree)
                    r.dm[tt] = __builtin_amdgcn_raw_buffer_load_b16(ts.src(tt).d, 2 * (lane & 15), dof + 32 * ti, kPfAux);
                else
                    r.dm[tt] = __builtin_amdgcn_raw_buffer_load_b32(ts.src(tt).d, 4 * (lane & 15), dof + 64 * ti, kPfAux);
            }
        }
    }
    __device__ static inline void begin(const Raw &r, State &st, int ss, int lane)
    {
        if (ss) return;
        const int hg = lane >> 5;
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) {
            const float d = f16_bits_to_f32((uint16_t)(r.dm[tt] & 0xFFFFu));
            const float dmin = f16_bits_to_f32((uint16_t)(r.dm[tt] >> 16));
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int sub = 2 * k + hg;  // = 4 ss + 2 j + hg with k = 2 ss + j
                const uint32_t scb = (pick4(r.sc[tt], sub >> 2) >> (8 * (sub & 3))) & 0xFFu;
                if constexpr (kThree) {
                    st.dl[tt][k] = (half_t)(d * (float)(int)(int8_t)scb);
                } else {
                    st.dl[tt][k] = (half_t)(d * (float)(scb & 0xFu));
                    st.ml[tt][k] = (half_t)(dmin * (float)(scb >> 4));
                }
            }
        }
    }
    __device__ static inline half8 bop(const Raw &r, const State &st, int ss, int tt, int j, int)
    {
        const uint32_t w = r.q[tt];
        uint32_t lo = (w >> (4 * j)) & 0x03030303u, hi = (w >> (4 * j + 2)) & 0x03030303u;
        if constexpr (kThree) {
            lo |= bit2_of_bytes(r.h[tt] >> (8 * j));
            hi |= bit2_of_bytes(r.h[tt] >> (8 * j + 4));
            return (bytes_h8(lo, hi) - (half_t)1028.0f) * st.dl[tt][2 * ss + j];  // exact u - 4
        } else {
            return (bytes_h8(lo, hi) - (half_t)1024.0f) * st.dl[tt][2 * ss + j] - st.ml[tt][2 * ss + j];
        }
    }
};
using FQ2_K = FQ23K<false>;
using FQ3_K = FQ23K<true>;

// Q6_K: y = d * sc * q (gguf.zig:1036-1059) with d * sc formed in f32 once per
// super-block and kept as f16; q - 32 is exact and the product rounds once.  The
// lane's 8 columns of block j lie in sub-block 4 ss + 2 j + g / 2.
struct FQ6_K {
    static constexpr int kSpu = 4;
    static constexpr bool kHoistA = true;   // activation fragments read at the step's start
    static constexpr int kDepth = ANEDVD_PF_DEPTH_K;       // steps of weights in flight ahead
    static constexpr int kMinLoads = 8;
    struct Raw {
        u32x2 q[kPfTiles];
        uint32_t h[kPfTiles];
        u32x4 sc[kPfTiles];    // int8 scales (a unit's first step)
        uint16_t d[kPfTiles];  // f16 d (a unit's first step)
    };
    struct State {
        uint32_t dsc[kPfTiles][4];  // f16 pairs; [tt][k / 2] half k % 2 (k = 2 ss + j): d * sc of the lane's sub-block 2 k + g / 2
    };
    template <int kUnit = -1, class TS>
    __device__ static inline void load(Raw &r, const TS &ts, int rb, int s, int lane)
    {
        const Planes &p = ts.src(0);
        const int qo = lane_plane_off(p, rb, s, 8), ho = lane_plane_off(p, rb, s, 4);
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) {
            r.q[tt] = __builtin_amdgcn_raw_buffer_load_b64(ts.src(tt).q, 8 * lane, qo + 512 * ts.idx(tt), kPfAux);
            r.h[tt] = __builtin_amdgcn_raw_buffer_load_b32(ts.src(tt).h, 4 * lane, ho + 256 * ts.idx(tt), kPfAux);
        }
        if (kUnit > 0 || (kUnit < 0 && (s & 3) == 0)) {
            const int so = row_plane_off(p, rb, s >> 2, 16), dof = row_plane_off(p, rb, s >> 2, 2);
#pragma unroll
            for (int tt = 0; tt < kPfTiles; tt++) {
                const int ti = ts.idx(tt);
                r.sc[tt] = __builtin_amdgcn_raw_buffer_load_b128(ts.src(tt).s, 16 * (lane & 15), so + 256 * ti, kPfAux);
                r.d[tt] = __builtin_amdgcn_raw_buffer_load_b16(ts.src(tt).d, 2 * (lane & 15), dof + 32 * ti, kPfAux);
            }
        }
    }
    // d * sc for two sub-blocks at once: the int8 scales become exact f16 by the
    // 0x64 exponent trick (bias 1024 + 128), and one packed f16 multiply by (d, d)
    // gives the exact products rounded once, as rounding the f32 product does.
    __device__ static inline void begin(const Raw &r, State &st, int ss, int lane)
    {
        if (ss) return;
        const uint32_t sel = (lane >> 5) ? 0x04030401u : 0x04020400u;  // bytes g/2 and 2 + g/2 of a dword
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) {
            const h2 dd = as_h2((uint32_t)r.d[tt] * 0x10001u);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t u = pick4(r.sc[tt], q) ^ 0x80808080u;  // sc + 128
                const h2 v = as_h2(__builtin_amdgcn_perm(0x64646464u, u, sel)) - (h2)1152.0f;
                st.dsc[tt][q] = h2_bits(dd * v);
            }
        }
    }
    __device__ static inline half8 bop(const Raw &r, const State &st, int ss, int tt, int j, int)
    {
        const uint32_t v = r.q[tt][j], hb = r.h[tt];
        const uint32_t lo = (v & 0x0F0F0F0Fu) | (((hb >> (4 * j)) & 0x03030303u) << 4);
        const uint32_t hi = ((v >> 4) & 0x0F0F0F0Fu) | (((hb >> (4 * j + 2)) & 0x03030303u) << 4);
        const half8 q = bytes_h8(lo, hi) - (half_t)1056.0f;  // exact q - 32
        return q * h_bits(st.dsc[tt][ss] >> (16 * j));
    }
};

// Q6_K as the grouped down kernel reads it: activation fragments read where they
// are used and weights one step ahead, so the kernel holds three wavefronts per
// SIMD (168 VGPRs and 36 bytes per lane spilled).  Qwen3 Q4_K_M 512-token
// down launch 72.7 -> 63 us against two wavefronts with both deeper.
struct FQ6_KDown : FQ6_K {
    static constexpr bool kHoistA = false;
    static constexpr int kDepth = 1;
};


}  // namespace anedvd
