// k_pf.hip -- the grouped GEMM for prefill-sized expert groups.
//
// Same math as the decode kernels (cpu.moeExpertAccumF32, cpu.zig:416-452, over
// the gguf.zig block formats), organised for groups of tens to hundreds of tokens:
//   - a workgroup takes a 64-token chunk of one expert's group and 128 weight rows
//     of both gate and up (or 256 rows of down);
//   - the chunk's activations are staged in LDS once per 64-column step and shared
//     by the four wavefronts;
//   - each wavefront dequantises its four 16-row tiles once per step to f16 (Q8_0,
//     Q4_0: d * q rounded once; Q4_K, Q6_K: the quant exact, the sub-block scale
//     and min as f16, one rounding in the FMA) and runs them against the chunk's
//     16-token tiles, accumulating the whole K inside the MFMA;
//   - activations carry one power of two per row (x as converted; the SwiGLU
//     activations are rescaled to their row's largest descale while staged), so
//     nothing is rescaled inside the K loop.
#include "common.h"
#include "kernels.h"
#include "mma.h"

namespace anedvd {

// Weight and activation steps loaded ahead of the one being multiplied: the
// super-block formats (small register footprint per step, memory-bound prefill
// shapes) go deeper than Q8_0 / Q4_0, whose kernels keep three wavefronts per SIMD.
#ifndef ANEDVD_PF_DEPTH_K
#define ANEDVD_PF_DEPTH_K 2
#endif
#ifndef ANEDVD_PF_DEPTH_L
#define ANEDVD_PF_DEPTH_L 1
#endif
#ifndef ANEDVD_PF_STAGE_K
#define ANEDVD_PF_STAGE_K 2
#endif
#ifndef ANEDVD_PF_STAGE_L
#define ANEDVD_PF_STAGE_L 1
#endif
constexpr int kAStride = 72;  // halves per staged token row: 64 + 8 against LDS bank conflicts
constexpr int kPfTiles = 4;   // 16-row tiles per wavefront: each staged A read feeds four MFMAs

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


// ------------------------------------------------------------------ decoders
//
// A decoder loads one step of a wavefront's four row tiles (a 64-row block): load();
// takes what stays valid for a whole scale unit on the unit's first step: begin();
// and yields the f16 B operand of (tile tt, block j) at step `ss` of the unit:
// bop().  Lane l = 16 g + n holds row n of the tile and the 8 columns 32 j + 8 g + i.

// F16 experts: the tile holds the values themselves.
struct FF16 {
    static constexpr int kSpu = 1;
    static constexpr bool kHoistA = false;  // 32 VGPRs of values per ring slot already
    static constexpr int kDepth = ANEDVD_PF_DEPTH_L;       // steps of weights in flight ahead
    static constexpr int kStageDepth = ANEDVD_PF_STAGE_L;  // steps of activations in flight ahead
    struct Raw {
        u32x4 q[kPfTiles][2];
    };
    struct State {};
    __device__ static inline void load(Raw &r, const Planes &p, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(p, rb, s, 32);
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++)
#pragma unroll
            for (int j = 0; j < 2; j++)
                r.q[tt][j] = __builtin_amdgcn_raw_buffer_load_b128(p.q, 32 * lane, qo + 2048 * tt + 16 * j, kNT);
    }
    __device__ static inline void begin(const Raw &, State &, int, int) {}
    __device__ static inline half8 bop(const Raw &r, const State &, int, int tt, int j, int) { return as_h8(r.q[tt][j]); }
};

struct FQ8_0 {
    static constexpr int kSpu = 1;
    static constexpr bool kHoistA = false;  // at 176 VGPRs two waves per SIMD instead of three
    static constexpr int kDepth = ANEDVD_PF_DEPTH_L;       // steps of weights in flight ahead
    static constexpr int kStageDepth = ANEDVD_PF_STAGE_L;  // steps of activations in flight ahead
    struct Raw {
        u32x4 q[kPfTiles];
        uint32_t s[kPfTiles];
    };
    struct State {};
    __device__ static inline void load(Raw &r, const Planes &p, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(p, rb, s, 16), so = row_plane_off(p, rb, s, 4);
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) {
            r.q[tt] = __builtin_amdgcn_raw_buffer_load_b128(p.q, 16 * lane, qo + 1024 * tt, kNT);
            r.s[tt] = __builtin_amdgcn_raw_buffer_load_b32(p.s, 4 * (lane & 15), so + 64 * tt, kNT);
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
    static constexpr int kStageDepth = ANEDVD_PF_STAGE_L;  // steps of activations in flight ahead
    struct Raw {
        u32x2 q[kPfTiles];
        uint32_t s[kPfTiles];
    };
    struct State {};
    __device__ static inline void load(Raw &r, const Planes &p, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(p, rb, s, 8), so = row_plane_off(p, rb, s, 4);
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) {
            r.q[tt] = __builtin_amdgcn_raw_buffer_load_b64(p.q, 8 * lane, qo + 512 * tt, kNT);
            r.s[tt] = __builtin_amdgcn_raw_buffer_load_b32(p.s, 4 * (lane & 15), so + 64 * tt, kNT);
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
    static constexpr int kStageDepth = ANEDVD_PF_STAGE_L;  // steps of activations in flight ahead
    struct Raw {
        u32x2 q[kPfTiles];
        uint32_t h[kFive ? kPfTiles : 1];
        u32x2 s[kPfTiles];  // (d0 | m0 << 16, d1 | m1 << 16) with a min, else (d0 | d1 << 16, -)
    };
    struct State {};
    __device__ static inline void load(Raw &r, const Planes &p, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(p, rb, s, 8), so = row_plane_off(p, rb, s, kHasMin ? 8 : 4);
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) {
            r.q[tt] = __builtin_amdgcn_raw_buffer_load_b64(p.q, 8 * lane, qo + 512 * tt, kNT);
            if constexpr (kHasMin)
                r.s[tt] = __builtin_amdgcn_raw_buffer_load_b64(p.s, 8 * (lane & 15), so + 128 * tt, kNT);
            else
                r.s[tt].x = __builtin_amdgcn_raw_buffer_load_b32(p.s, 4 * (lane & 15), so + 64 * tt, kNT);
        }
        if constexpr (kFive) {
            const int ho = lane_plane_off(p, rb, s, 2);
#pragma unroll
            for (int tt = 0; tt < kPfTiles; tt++)
                r.h[tt] = __builtin_amdgcn_raw_buffer_load_b16(p.h, 2 * lane, ho + 128 * tt, kNT);
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
    static constexpr int kStageDepth = ANEDVD_PF_STAGE_K;  // steps of activations in flight ahead
    struct Raw {
        u32x2 q[kPfTiles];
        u32x4 sc[kPfTiles];  // d, dmin, scales: loaded on a unit's first step
    };
    struct State {
        uint32_t dm[kPfTiles][8];  // f16 d1 | f16 (-m1) << 16 per (tile, sub-block)
    };
    __device__ static inline void load(Raw &r, const Planes &p, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(p, rb, s, 8);
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) r.q[tt] = __builtin_amdgcn_raw_buffer_load_b64(p.q, 8 * lane, qo + 512 * tt, kNT);
        if ((s & 3) == 0) {
            const int so = row_plane_off(p, rb, s >> 2, 16);
#pragma unroll
            for (int tt = 0; tt < kPfTiles; tt++)
                r.sc[tt] = __builtin_amdgcn_raw_buffer_load_b128(p.s, 16 * (lane & 15), so + 256 * tt, kNT);
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
    static constexpr int kStageDepth = ANEDVD_PF_STAGE_K;  // steps of activations in flight ahead
    struct Raw {
        u32x2 q[kPfTiles];
        uint32_t h[kPfTiles];
        u32x4 sc[kPfTiles];  // d, dmin, scales: loaded on a unit's first step
    };
    using State = FQ4_K::State;
    __device__ static inline void load(Raw &r, const Planes &p, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(p, rb, s, 8), ho = lane_plane_off(p, rb, s, 2);
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) {
            r.q[tt] = __builtin_amdgcn_raw_buffer_load_b64(p.q, 8 * lane, qo + 512 * tt, kNT);
            r.h[tt] = __builtin_amdgcn_raw_buffer_load_b16(p.h, 2 * lane, ho + 128 * tt, kNT);
        }
        if ((s & 3) == 0) {
            const int so = row_plane_off(p, rb, s >> 2, 16);
#pragma unroll
            for (int tt = 0; tt < kPfTiles; tt++)
                r.sc[tt] = __builtin_amdgcn_raw_buffer_load_b128(p.s, 16 * (lane & 15), so + 256 * tt, kNT);
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
    static constexpr int kStageDepth = ANEDVD_PF_STAGE_K;  // steps of activations in flight ahead
    struct Raw {
        uint32_t q[kPfTiles];
        uint32_t h[kThree ? kPfTiles : 1];
        u32x4 sc[kPfTiles];     // sub-block scales (a unit's first step)
        uint32_t dm[kPfTiles];  // d (Q3_K) or d | dmin << 16 (Q2_K) (a unit's first step)
    };
    struct State {
        half_t dl[kPfTiles][8], ml[kPfTiles][8];  // [tt][2 ss + j] of the lane's sub-block 4 ss + 2 j + g / 2
    };
    __device__ static inline void load(Raw &r, const Planes &p, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(p, rb, s, 4);
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) {
            r.q[tt] = __builtin_amdgcn_raw_buffer_load_b32(p.q, 4 * lane, qo + 256 * tt, kNT);
            if constexpr (kThree)
                r.h[tt] = __builtin_amdgcn_raw_buffer_load_b16(p.h, 2 * lane, lane_plane_off(p, rb, s, 2) + 128 * tt, kNT);
        }
        if ((s & 3) == 0) {
            const int so = row_plane_off(p, rb, s >> 2, 16), dof = row_plane_off(p, rb, s >> 2, kThree ? 2 : 4);
#pragma unroll
            for (int tt = 0; tt < kPfTiles; tt++) {
                r.sc[tt] = __builtin_amdgcn_raw_buffer_load_b128(p.s, 16 * (lane & 15), so + 256 * tt, kNT);
                if constexpr (kThree)
                    r.dm[tt] = __builtin_amdgcn_raw_buffer_load_b16(p.d, 2 * (lane & 15), dof + 32 * tt, kNT);
                else
                    r.dm[tt] = __builtin_amdgcn_raw_buffer_load_b32(p.d, 4 * (lane & 15), dof + 64 * tt, kNT);
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
    static constexpr int kStageDepth = ANEDVD_PF_STAGE_K;  // steps of activations in flight ahead
    struct Raw {
        u32x2 q[kPfTiles];
        uint32_t h[kPfTiles];
        u32x4 sc[kPfTiles];    // int8 scales (a unit's first step)
        uint16_t d[kPfTiles];  // f16 d (a unit's first step)
    };
    struct State {
        uint32_t dsc[kPfTiles][4];  // f16 pairs; [tt][k / 2] half k % 2 (k = 2 ss + j): d * sc of the lane's sub-block 2 k + g / 2
    };
    __device__ static inline void load(Raw &r, const Planes &p, int rb, int s, int lane)
    {
        const int qo = lane_plane_off(p, rb, s, 8), ho = lane_plane_off(p, rb, s, 4);
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) {
            r.q[tt] = __builtin_amdgcn_raw_buffer_load_b64(p.q, 8 * lane, qo + 512 * tt, kNT);
            r.h[tt] = __builtin_amdgcn_raw_buffer_load_b32(p.h, 4 * lane, ho + 256 * tt, kNT);
        }
        if ((s & 3) == 0) {
            const int so = row_plane_off(p, rb, s >> 2, 16), dof = row_plane_off(p, rb, s >> 2, 2);
#pragma unroll
            for (int tt = 0; tt < kPfTiles; tt++) {
                r.sc[tt] = __builtin_amdgcn_raw_buffer_load_b128(p.s, 16 * (lane & 15), so + 256 * tt, kNT);
                r.d[tt] = __builtin_amdgcn_raw_buffer_load_b16(p.d, 2 * (lane & 15), dof + 32 * tt, kNT);
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

// ------------------------------------------------------------ staging

// Thread tid of a workgroup stages, per step, quarter q = tid / 64 of the step's
// 64 columns (32 bytes) of token rows r = tid % 64 + 64 h, h < R: consecutive lanes
// write consecutive rows, so the LDS writes of a wavefront hit distinct banks.  The
// global loads land in a ring of NB register slots, so a step's activations can be
// loaded several steps before they are written to LDS.
template <int R, int NB>
struct StageX {  // gate/up: token rows gathered through the dispatch; x has per-row descales
    static constexpr int kSlots = NB;
    rsrc_t q;
    int off[R];
    u32x4 v[NB][R][2];
    template <int B>
    __device__ inline void load(int s)
    {
#pragma unroll
        for (int h = 0; h < R; h++) {
            v[B][h][0] = __builtin_amdgcn_raw_buffer_load_b128(q, off[h], s * 2 * kStep, 0);
            v[B][h][1] = __builtin_amdgcn_raw_buffer_load_b128(q, off[h], s * 2 * kStep + 16, 0);
        }
    }
    template <int B>
    __device__ inline void store(half_t *dst) const  // dst: this thread's first row, its quarter
    {
#pragma unroll
        for (int h = 0; h < R; h++) {
            *(u32x4 *)(dst + h * 64 * kAStride) = v[B][h][0];
            *(u32x4 *)(dst + h * 64 * kAStride + 8) = v[B][h][1];
        }
    }
};

template <int R, int NB>
struct StageAct {  // down: consecutive positions, rescaled from their group's descale to the row's
    static constexpr int kSlots = NB;
    rsrc_t q, ds;
    int off[R], doff[R], ld4;
    float inv_ref[R];
    u32x4 v[NB][R][2];
    float dg[NB][R];
    template <int B>
    __device__ inline void load(int s)
    {
#pragma unroll
        for (int h = 0; h < R; h++) {
            v[B][h][0] = __builtin_amdgcn_raw_buffer_load_b128(q, off[h], s * 2 * kStep, 0);
            v[B][h][1] = __builtin_amdgcn_raw_buffer_load_b128(q, off[h], s * 2 * kStep + 16, 0);
            dg[B][h] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ds, doff[h], s * ld4, 0));
        }
    }
    template <int B>
    __device__ inline void store(half_t *dst) const
    {
#pragma unroll
        for (int h = 0; h < R; h++) {
            const half_t f = (half_t)(dg[B][h] * inv_ref[h]);  // a power of two <= 1
            *(half8 *)(dst + h * 64 * kAStride) = as_h8(v[B][h][0]) * f;
            *(half8 *)(dst + h * 64 * kAStride + 8) = as_h8(v[B][h][1]) * f;
        }
    }
};

// Register slot b chosen at run time; inside the unrolled step loop b is a
// constant and the branch folds away.
template <class S>
__device__ inline void stage_load(S &st, int b, int s)
{
    if (b == 0) st.template load<0>(s);
    else if (b == 1) st.template load<1 % S::kSlots>(s);
    else if (b == 2) st.template load<2 % S::kSlots>(s);
    else st.template load<3 % S::kSlots>(s);
}

template <class S>
__device__ inline void stage_store(const S &st, int b, half_t *dst)
{
    if (b == 0) st.template store<0>(dst);
    else if (b == 1) st.template store<1 % S::kSlots>(dst);
    else if (b == 2) st.template store<2 % S::kSlots>(dst);
    else st.template store<3 % S::kSlots>(dst);
}

// ------------------------------------------------------------ main loop

// Steps [0, steps) of the wavefront's four tiles of row block rb against the MT
// 16-token tiles staged in `abuf` (two buffers of 16 MT x kAStride halves):
// acc[tt][mt] = sum_k W[64 rb + 16 tt + l % 16][k] * A[16 mt + 4 (l / 16) + i][k].
// Weights are loaded F::kDepth steps ahead and activations F::kStageDepth steps
// ahead (rings of register slots); every thread of the workgroup takes part in the staging, so all of
// them reach the barriers.  Steps go in unrolled blocks of four (one scale unit of
// the super-block formats), so the slots and the LDS buffers alternate at
// compile-time indices.  Weight loads past the last step go out of range (zero, no
// memory traffic).
template <class F, int MT, class S>
__device__ inline void pf_loop(const Planes &W, int rb, int steps, int lane, S &stage, half_t *abuf,
                               int srow, int mt_live, f32x4 (*acc)[MT])
{
    constexpr int U = 4;
    constexpr int BUF = 16 * MT * kAStride;
    static_assert(U % F::kSpu == 0, "a scale unit must fit an unrolled block");
    const int n = lane & 15, g = lane >> 4;
    const int so = (W.nrb - rb) * W.steps;
    auto ws = [&](int x) { return x < steps ? x : so; };
    constexpr int D = F::kDepth, DA = F::kStageDepth;
    constexpr int R = D == 1 ? 2 : 4;    // ring of weight slots; divides the unrolled block
    constexpr int RA = DA == 1 ? 2 : 4;  // ring of staging slots
    static_assert(D >= 1 && D <= 3 && DA >= 1 && DA <= 3, "at most three steps ahead");
    static_assert(S::kSlots == RA, "staging ring");
    typename F::Raw w[R];
    typename F::State st;
    stage.template load<0>(0);
#pragma unroll
    for (int d = 0; d < D; d++) F::load(w[d], W, rb, ws(d), lane);
    stage.template store<0>(abuf + srow);
#pragma unroll
    for (int d = 1; d < DA; d++)
        if (d < steps) stage_load(stage, d, d);
    __syncthreads();
    for (int s0 = 0; s0 < steps; s0 += U) {
#pragma unroll
        for (int k = 0; k < U; k++) {
            const int s = s0 + k;
            if (s >= steps) break;  // uniform; only for a step count that is not a multiple of 4
            const bool more = s + 1 < steps;
            if (s + DA < steps) stage_load(stage, (k + DA) % RA, s + DA);
            F::load(w[(k + D) % R], W, rb, ws(s + D), lane);
            __builtin_amdgcn_sched_barrier(0);
            const int ss = k % F::kSpu;
            F::begin(w[k % R], st, ss, lane);
            const half_t *a = abuf + (k & 1) * BUF + n * kAStride + 16 * g;
            // The step's activation fragments, read before the dequantisation so their
            // LDS latency hides behind it (token tiles past the chunk's end read stale
            // rows of the buffer that no MFMA uses), or, for decoders whose registers
            // are tight, just before their MFMAs.
            half8 av[2][MT];
            if constexpr (F::kHoistA) {
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) av[j][mt] = *(const half8 *)(a + mt * 16 * kAStride + 8 * j);
            }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                half8 b[kPfTiles];
#pragma unroll
                for (int tt = 0; tt < kPfTiles; tt++) b[tt] = F::bop(w[k % R], st, ss, tt, j, lane);
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    if (mt >= mt_live) break;  // uniform: token tiles past the chunk's end stay zero
                    if constexpr (!F::kHoistA) av[j][mt] = *(const half8 *)(a + mt * 16 * kAStride + 8 * j);
#pragma unroll
                    for (int tt = 0; tt < kPfTiles; tt++) acc[tt][mt] = mfma(av[j][mt], b[tt], acc[tt][mt]);
                }
            }
            if (more) stage_store(stage, (k + 1) % RA, abuf + ((k + 1) & 1) * BUF + srow);
            __syncthreads();
        }
    }
}

struct PfArgs {
    QMat w0, w1;  // gate, up (or down in w0)
    ActQ x;       // gate/up input (tokens) or down input (positions)
    Dispatch d;
    ActQ act;     // gate/up output
    float *ypart; // down output [P][H], rows in (token, slot) order
    int H, I, P, nchunk, use_gelu;
    int kk;       // slots per token row of ypart
};

// The chunk `ci` of the dispatch's (16 MT)-token work list.
template <int MT>
__device__ inline bool pf_chunk(const Dispatch &d, int ci, int &e, int &p0, int &nt)
{
    const int n = d.meta[3];
    const uint64_t c = d.chunks[ci];  // ci < the list's capacity: loaded beside the count
    if (ci >= n) return false;
    e = (int)(c & 0xFFu);
    nt = (int)((c >> 8) & 0xFFu);
    p0 = (int)(c >> 16);
    return true;
}

// LDS of one workgroup: the two staged activation tiles during the K loop, then
// (gate/up) the gate and up results of 64 tokens x 64 rows at a time.
template <int MT>
struct PfLds {
    static constexpr int kA = 2 * 16 * MT * kAStride * 2;        // bytes
    static constexpr int kEpi = 2 * 64 * (kRowBlock + 1) * 4;    // bytes
    static constexpr int kBytes = kA > kEpi ? kA : kEpi;
};

// ------------------------------------------------------------ gate / up

// Grid nchunk * I/128 workgroups of 256 threads, chunks fastest.  Wave w: matrix
// w & 1 (gate, up) of row block 2 x + (w >> 1), x the workgroup's row-block pair.
// After the K loop the gate and up results of one row block at a time go through
// LDS (64 tokens x 64 rows each, as many passes as 64-token groups); each
// wavefront then applies SiLU(g) * u to 16 of the tokens and writes them in the
// activation format (one 64-column group per token).
template <class F, int MT>
__global__ __launch_bounds__(256) void k_pf_gateup(PfArgs a)
{
    constexpr int R = MT / 4;
    __shared__ float dvs[16 * MT];
    __shared__ __attribute__((aligned(16))) unsigned char smem[PfLds<MT>::kBytes];
    int e, p0, nt;
    if (!pf_chunk<MT>(a.d, (int)(blockIdx.x % a.nchunk), e, p0, nt)) return;  // uniform over the workgroup
    const int rbg = (int)(blockIdx.x / a.nchunk);
    const int wv = wave_id(), lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const int mat = wv & 1, half = wv >> 1, rb = 2 * rbg + half;
    const Planes W = planes(mat ? a.w1 : a.w0, e);
    half_t *abuf = (half_t *)smem;
    const int r = threadIdx.x & 63, q = threadIdx.x >> 6;
    StageX<R, F::kStageDepth == 1 ? 2 : 4> stage;
    stage.q = make_rsrc(a.x.q, (size_t)a.x.ld * a.H * 2);
#pragma unroll
    for (int h = 0; h < R; h++) stage.off[h] = a.d.rows[p0 + min(r + 64 * h, nt - 1)] * a.H * 2 + 32 * q;
    f32x4 acc[kPfTiles][MT];
#pragma unroll
    for (int tt = 0; tt < kPfTiles; tt++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[tt][mt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    // token m's descale for the epilogue, loaded by thread m before the K loop
    const float tdv = (int)threadIdx.x < 16 * MT ? a.x.ds[a.d.rows[p0 + min((int)threadIdx.x, nt - 1)]] : 0.0f;
    pf_loop<F, MT>(W, rb, a.H / kStep, lane, stage, abuf, r * kAStride + 16 * q,
                   __builtin_amdgcn_readfirstlane((nt + 15) / 16), acc);

    if ((int)threadIdx.x < 16 * MT) dvs[threadIdx.x] = tdv;
    __syncthreads();
    float dv[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) dv[mt][i] = dvs[16 * mt + 4 * g + i];
    // results * the tokens' descales -> LDS [mat][token][row]: one row block and 64
    // tokens per pass
    float *res = (float *)smem;
#pragma unroll
    for (int hb = 0; hb < 2; hb++) {
#pragma unroll
        for (int h = 0; h < R; h++) {
            if (half == hb) {
#pragma unroll
                for (int mq = 0; mq < 4; mq++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int m = 16 * mq + 4 * g + i;
#pragma unroll
                        for (int tt = 0; tt < kPfTiles; tt++)
                            res[(mat * 64 + m) * (kRowBlock + 1) + 16 * tt + n] = acc[tt][4 * h + mq][i] * dv[4 * h + mq][i];
                    }
            }
            __syncthreads();
            const int rbo = 2 * rbg + hb;
            for (int m = 16 * wv; m < 16 * wv + 16; m++) {  // uniform per wavefront
                const float gv = res[m * (kRowBlock + 1) + lane], uv = res[(64 + m) * (kRowBlock + 1) + lane];
                const float v = gate_act(gv, a.use_gelu) * uv;
                const float sc = pow2_scale(wave_max(fabsf(v)));
                if (64 * h + m < nt) {
                    const size_t pos = (size_t)p0 + 64 * h + m;
                    a.act.q[pos * a.I + (size_t)kStep * rbo + mma_pos(lane)] = (half_t)(v * sc);
                    if (lane == 0) a.act.ds[(size_t)rbo * a.act.ld + pos] = 1.0f / sc;
                }
            }
            __syncthreads();
        }
    }
}

// ---------------------------------------------------------------- down

// Grid nchunk * H/256 workgroups of 256 threads, chunks fastest.  Wave w: row block
// 4 x + w.  Before the K loop the workgroup finds each position's largest descale
// over the I/64 groups (the row reference); staging scales every group to it, and
// the results are multiplied by it once at the end.  Positions past the group's
// end are computed on the next group's (or, past the last position, the last
// position's) activations and not stored.
template <class F, int MT>
__global__ __launch_bounds__(256) void k_pf_down(PfArgs a)
{
    constexpr int R = MT / 4;
    __shared__ __attribute__((aligned(16))) unsigned char smem[PfLds<MT>::kA];
    __shared__ float ref[16 * MT];
    __shared__ int orow[16 * MT];  // output rows of the chunk's positions, (token, slot) order
    __shared__ float ref4[4][16 * MT];
    int e, p0, nt;
    if (!pf_chunk<MT>(a.d, (int)(blockIdx.x % a.nchunk), e, p0, nt)) return;
    const int rbg = (int)(blockIdx.x / a.nchunk);
    const int wv = wave_id(), lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const int rb = 4 * rbg + wv;
    const Planes W = planes(a.w0, e);
    const int G = a.I / kStep, ld = a.x.ld;
    {
        // the row references: thread (part, m) takes every 4th group of position m,
        // eight loads in flight at a time, and the four partial maxima meet in LDS
        static_assert(16 * MT * 4 == 256, "four threads per chunk position");
        const int m = threadIdx.x % (16 * MT), part = threadIdx.x / (16 * MT);
        const int pr = min(p0 + m, a.P - 1);
        if (part == 0) orow[m] = a.d.rows[pr] * a.kk + a.d.slots[pr];
        float mx = 0.0f;
        for (int g0 = part; g0 < G; g0 += 4 * 8) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = g0 + 4 * i < G ? a.x.ds[(size_t)(g0 + 4 * i) * ld + pr] : 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) mx = fmaxf(mx, v[i]);
        }
        ref4[part][m] = mx;
        __syncthreads();
        if (part == 0) ref[m] = fmaxf(fmaxf(ref4[0][m], ref4[1][m]), fmaxf(ref4[2][m], ref4[3][m]));
        __syncthreads();
    }
    const int r = threadIdx.x & 63, q = threadIdx.x >> 6;
    StageAct<R, F::kStageDepth == 1 ? 2 : 4> stage;
    stage.q = make_rsrc(a.x.q, (size_t)a.P * a.I * 2);
    stage.ds = make_rsrc(a.x.ds, (size_t)G * ld * 4);
    stage.ld4 = ld * 4;
#pragma unroll
    for (int h = 0; h < R; h++) {
        const int pos = min(p0 + r + 64 * h, a.P - 1);
        stage.off[h] = pos * a.I * 2 + 32 * q;
        stage.doff[h] = pos * 4;
        stage.inv_ref[h] = 1.0f / ref[r + 64 * h];
    }
    f32x4 acc[kPfTiles][MT];
#pragma unroll
    for (int tt = 0; tt < kPfTiles; tt++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[tt][mt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    pf_loop<F, MT>(W, rb, a.I / kStep, lane, stage, (half_t *)smem, r * kAStride + 16 * q,
                   __builtin_amdgcn_readfirstlane((nt + 15) / 16), acc);
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = 16 * mt + 4 * g + i;
            if (m < nt) {
                float *yp = a.ypart + (size_t)orow[m] * a.H + (size_t)kRowBlock * rb + n;
#pragma unroll
                for (int tt = 0; tt < kPfTiles; tt++) yp[16 * tt] = acc[tt][mt][i] * ref[m];
            }
        }
}

// ------------------------------------------------------------- launchers

bool grouped_supported(int H, int I) { return H % 256 == 0 && I % 128 == 0; }

template <class F, int MT>
static int launch_pf(const PfArgs &a, bool gateup, hipStream_t st)
{
    if (gateup) {
        const size_t wgs = (size_t)a.nchunk * (a.I / (2 * kRowBlock));
        hipLaunchKernelGGL((k_pf_gateup<F, MT>), dim3((unsigned)wgs), dim3(256), 0, st, a);
    } else {
        const size_t wgs = (size_t)a.nchunk * (a.H / (4 * kRowBlock));
        hipLaunchKernelGGL((k_pf_down<F, MT>), dim3((unsigned)wgs), dim3(256), 0, st, a);
    }
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

// 64-token chunks (mt = 4).  128-token chunks (MT = 8) compile too, but at 2-3
// waves per SIMD they measured slower on the Mixtral 2048-token prefill (2.84 ms
// against 2.36 ms), so the planner does not select them.
template <class F>
static int launch_pf_mt(const PfArgs &a, int, bool gateup, hipStream_t st)
{
    return launch_pf<F, 4>(a, gateup, st);
}

static int launch_pf_type(int type, const PfArgs &a, int mt, bool gateup, hipStream_t st)
{
    switch (type) {
    case ANEDVD_Q8_0:
    case ANEDVD_Q8_1: return launch_pf_mt<FQ8_0>(a, mt, gateup, st);  // one tile layout
    case ANEDVD_F16: return launch_pf_mt<FF16>(a, mt, gateup, st);
    case ANEDVD_Q4_0: return launch_pf_mt<FQ4_0>(a, mt, gateup, st);
    case ANEDVD_Q4_1: return launch_pf_mt<FQ4_1>(a, mt, gateup, st);
    case ANEDVD_Q5_0: return launch_pf_mt<FQ5_0>(a, mt, gateup, st);
    case ANEDVD_Q5_1: return launch_pf_mt<FQ5_1>(a, mt, gateup, st);
    case ANEDVD_Q2_K: return launch_pf_mt<FQ2_K>(a, mt, gateup, st);
    case ANEDVD_Q3_K: return launch_pf_mt<FQ3_K>(a, mt, gateup, st);
    case ANEDVD_Q4_K: return launch_pf_mt<FQ4_K>(a, mt, gateup, st);
    case ANEDVD_Q5_K: return launch_pf_mt<FQ5_K>(a, mt, gateup, st);
    case ANEDVD_Q6_K: return launch_pf_mt<FQ6_K>(a, mt, gateup, st);
    default:
        set_error("grouped GEMM: ggml type %d has no kernel", type);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
}

int launch_grouped_gateup(const QMat &gate, const QMat &up, const ActQ &x, int H, int I, const Dispatch &d, int P,
                          int mt, int nchunk, const ActQ &act, int use_gelu, hipStream_t st)
{
    if (gate.type != up.type) {
        set_error("grouped gate/up: gate type %d and up type %d differ", gate.type, up.type);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
    PfArgs a{};
    a.w0 = gate;
    a.w1 = up;
    a.x = x;
    a.d = d;
    a.act = act;
    a.H = H;
    a.I = I;
    a.P = P;
    a.nchunk = nchunk;
    a.use_gelu = use_gelu;
    return launch_pf_type(gate.type, a, mt, true, st);
}

int launch_grouped_down(const QMat &down, const ActQ &act, int H, int I, const Dispatch &d, int P, int mt,
                        int nchunk, float *ypart, int kk, hipStream_t st)
{
    PfArgs a{};
    a.w0 = down;
    a.x = act;
    a.d = d;
    a.ypart = ypart;
    a.kk = kk;
    a.H = H;
    a.I = I;
    a.P = P;
    a.nchunk = nchunk;
    return launch_pf_type(down.type, a, mt, false, st);
}

}  // namespace anedvd
