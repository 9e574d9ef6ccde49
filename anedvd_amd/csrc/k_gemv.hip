// k_gemv.hip -- decode-regime expert kernels: GGUF dequant fused into the
// SwiGLU gate/up and down products, for the token groups the dispatch built.
//
// Semantics follow cpu.moeExpertAccumF32 (cpu.zig:416-452): g = W_g h,
// u = W_u h, a = (g / (1 + exp(-g))) * u, y = W_d a; the combine adds p * y per
// slot.  Block dequantisation follows gguf.zig's dequantQ8_0 (827-840),
// dequantQ4_0 (763-776), dequantQ4K (960-996) and dequantQ6K (1036-1059).
//
// Bandwidth design (HBM-bound GEMV, no MFMA): one weight row per lane, 64 rows
// per wavefront, weights in the tile layout of common.h so that every
// global_load_dwordx4 of a wavefront reads 1 KiB contiguous.  A lane turns its
// quants into f16 integers with byte permutes under the exponent byte 0x64
// (1024 + q exactly), keeps them for every token of the group, and multiplies them
// with the group's activations (f16, power-of-two scaled per 64 elements, read
// from LDS as wave-uniform broadcasts) by v_dot2_f32_f16 into f32 sums.  The
// 1024-offset (Q4_0, Q4_K; 1152 for Q8_0's biased bytes) is removed from each
// block sum with the block's activation sum, the block scale (and Q4_K's min
// term) is applied to the f32 block sum, and the activation scale to the group.
// The K axis is split over ks workgroups when a call has too few rows to fill
// the 256 CUs; partial sums are added in a fixed order, so results do not depend
// on scheduling.
#include <stdlib.h>

#include "common.h"
#include "kernels.h"

namespace anedvd {

constexpr int kWaves = 4;

// Minimum wavefronts per SIMD the GEMV kernels are compiled for (a register cap);
// a build option for tuning.
#ifndef ANEDVD_GEMV_MIN_WAVES
#define ANEDVD_GEMV_MIN_WAVES 1
#endif

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ inline float fdot2(h2 a, h2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }

__device__ inline h2 as_h2(uint32_t u)
{
    h2 r;
    __builtin_memcpy(&r, &u, 4);
    return r;
}

// Bytes (b0, b2) and (b1, b3) of `b` under the f16 exponent byte 0x64: the pairs
// (1024 + b0, 1024 + b2) and (1024 + b1, 1024 + b3), exact.
__device__ inline h2 pair02(uint32_t b) { return as_h2(__builtin_amdgcn_perm(0x64646464u, b, 0x04020400u)); }
__device__ inline h2 pair13(uint32_t b) { return as_h2(__builtin_amdgcn_perm(0x64646464u, b, 0x04030401u)); }

template <class T>
__device__ inline T ld_stream(const T *p)
{
    return __builtin_nontemporal_load(p);
}

// ------------------------------------------------------------------ decoders
//
// A decoder streams one lane's share (its row) of one unit of the tile layout in
// kSteps steps of 64 weights.  load() fetches a step's bytes; convert() turns
// them into 32 f16 pairs (W) plus the step's scales, keeping per-unit scales in
// State across the unit's steps; dot() accumulates, for each of the nt tokens,
// the step's dot product with the staged activations into acc[token], already
// multiplied by the activations' power-of-two scale.  x points at the unit's
// first h2 for token 0 (token j at x + j*xs); sd at the unit's first 64-group
// record (token j at sd + j*ss).

// Sum of 16 f16 pair products of w[0..15] with x[0..15] into an f32.
__device__ inline float dot16(const h2 *w, const h2 *x)
{
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) s = fdot2(w[i], x[i], s);
    return s;
}

__device__ inline float dot8(const h2 *w, const h2 *x)
{
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) s = fdot2(w[i], x[i], s);
    return s;
}

// Index of this thread's wavefront in its workgroup, as a wave-uniform value.
__device__ inline int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Q8_0 (dequantQ8_0, gguf.zig:827-840): a unit is two 32-element blocks; the tile
// stores q + 128, so a pair holds 1152 + q and the block sum is corrected by
// 1152 * (sum of the block's activations).
struct DecQ8_0 {
    static constexpr int kUnit = 64, kSteps = 1;
    struct Raw {
        u32x4 q[4];
        uint32_t s;
    };
    struct W {
        h2 w[32];
        float d0, d1;
    };
    struct State {};
    __device__ static inline void load(Raw &r, const QMat &m, int mat, int rg, int u, int, int lane)
    {
        const Fmt f{64, 4, 4};
        const uint8_t *q = m.q + (size_t)mat * m.q_stride;
#pragma unroll
        for (int c = 0; c < 4; c++) r.q[c] = ld_stream((const u32x4 *)(q + tile_q_off(f, m.units, rg, u, c, lane)));
        r.s = ld_stream((const uint32_t *)(m.s + (size_t)mat * m.s_stride + tile_s_off(f, m.units, rg, u, lane)));
    }
    __device__ static inline void convert(const Raw &r, int, W &w, State &)
    {
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                w.w[c * 8 + 2 * i] = pair02(r.q[c][i]);
                w.w[c * 8 + 2 * i + 1] = pair13(r.q[c][i]);
            }
        w.d0 = f16_bits_to_f32((uint16_t)(r.s & 0xFFFFu));
        w.d1 = f16_bits_to_f32((uint16_t)(r.s >> 16));
    }
    template <int NT>
    __device__ static inline void dot(const W &w, const State &, int, const h2 *x, int xs,
                                      const float4 *sd, int ss, int nt, float *acc)
    {
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const h2 *xj = x + j * xs;
            const float s0 = dot16(w.w, xj), s1 = dot16(w.w + 16, xj + 16);
            const float4 g = sd[j * ss];
            acc[j] += (w.d0 * (s0 - 1152.0f * g.x) + w.d1 * (s1 - 1152.0f * g.y)) * g.z;
        }
    }
};

// Q4_0 (dequantQ4_0, gguf.zig:763-776): two 32-element blocks per unit; block
// byte j holds element j (low nibble) and j + 16 (high).  Pairs hold 1024 + n,
// corrected by 1032 * (block activation sum).
struct DecQ4_0 {
    static constexpr int kUnit = 64, kSteps = 1;
    struct Raw {
        u32x4 q[2];
        uint32_t s;
    };
    struct W {
        h2 w[32];
        float d0, d1;
    };
    struct State {};
    __device__ static inline void load(Raw &r, const QMat &m, int mat, int rg, int u, int, int lane)
    {
        const Fmt f{64, 2, 4};
        const uint8_t *q = m.q + (size_t)mat * m.q_stride;
#pragma unroll
        for (int c = 0; c < 2; c++) r.q[c] = ld_stream((const u32x4 *)(q + tile_q_off(f, m.units, rg, u, c, lane)));
        r.s = ld_stream((const uint32_t *)(m.s + (size_t)mat * m.s_stride + tile_s_off(f, m.units, rg, u, lane)));
    }
    __device__ static inline void convert(const Raw &r, int, W &w, State &)
    {
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t v = r.q[b][i];
                const uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
                w.w[(8 * b + i) * 2] = pair02(lo);
                w.w[(8 * b + i) * 2 + 1] = pair13(lo);
                w.w[(8 * b + 4 + i) * 2] = pair02(hi);
                w.w[(8 * b + 4 + i) * 2 + 1] = pair13(hi);
            }
        w.d0 = f16_bits_to_f32((uint16_t)(r.s & 0xFFFFu));
        w.d1 = f16_bits_to_f32((uint16_t)(r.s >> 16));
    }
    template <int NT>
    __device__ static inline void dot(const W &w, const State &, int, const h2 *x, int xs,
                                      const float4 *sd, int ss, int nt, float *acc)
    {
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const h2 *xj = x + j * xs;
            const float s0 = dot16(w.w, xj), s1 = dot16(w.w + 16, xj + 16);
            const float4 g = sd[j * ss];
            acc[j] += (w.d0 * (s0 - 1032.0f * g.x) + w.d1 * (s1 - 1032.0f * g.y)) * g.z;
        }
    }
};

// Byte i (0..11) of the 12 scale bytes held in 3 dwords, i at run time.
__device__ inline int scale_byte(const uint32_t s1, const uint32_t s2, const uint32_t s3, int i)
{
    const uint32_t w = i < 4 ? s1 : i < 8 ? s2 : s3;
    return (int)((w >> (8 * (i & 3))) & 0xFFu);
}

// getScaleMinK4 (gguf.zig:948-958) over the 12 scale bytes held in 3 dwords.
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

// Q4_K (dequantQ4K, gguf.zig:960-996): a unit is one 256-element super-block; step
// g covers elements 64g..64g+63 = sub-blocks 2g (low nibbles of qs[32g..32g+31])
// and 2g+1 (high nibbles).  y = d1 * n - m1 with d1 = d * sc, m1 = dmin * m; with
// pairs holding 1024 + n:  sum y x = d1 * sum w x - (1024 d1 + m1) * sum x.
struct DecQ4_K {
    static constexpr int kUnit = 256, kSteps = 4;
    struct Raw {
        u32x4 c0;      // d, dmin, scales (step 0 only)
        u32x4 qs[2];
    };
    struct W {
        h2 w[32];      // [0..15] low nibbles (sub-block 2g), [16..31] high (2g+1)
        float d1, m1, d2, m2;
    };
    struct State {
        u32x4 c0;
    };
    __device__ static inline void load(Raw &r, const QMat &m, int mat, int rg, int u, int g, int lane)
    {
        const Fmt f{256, 9, 0};
        const uint8_t *q = m.q + (size_t)mat * m.q_stride;
        if (g == 0) r.c0 = ld_stream((const u32x4 *)(q + tile_q_off(f, m.units, rg, u, 0, lane)));
#pragma unroll
        for (int c = 0; c < 2; c++)
            r.qs[c] = ld_stream((const u32x4 *)(q + tile_q_off(f, m.units, rg, u, 1 + 2 * g + c, lane)));
    }
    __device__ static inline void convert(const Raw &r, int g, W &w, State &st)
    {
        if (g == 0) st.c0 = r.c0;
        const float d = f16_bits_to_f32((uint16_t)(st.c0[0] & 0xFFFFu));
        const float dmin = f16_bits_to_f32((uint16_t)(st.c0[0] >> 16));
        int a, b;
        scale_min_k4(2 * g, st.c0[1], st.c0[2], st.c0[3], a, b);
        w.d1 = d * (float)a;
        w.m1 = 1024.0f * w.d1 + dmin * (float)b;
        scale_min_k4(2 * g + 1, st.c0[1], st.c0[2], st.c0[3], a, b);
        w.d2 = d * (float)a;
        w.m2 = 1024.0f * w.d2 + dmin * (float)b;
#pragma unroll
        for (int cc = 0; cc < 2; cc++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t v = r.qs[cc][i];
                const uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
                const int n = (4 * cc + i) * 2;
                w.w[n] = pair02(lo);
                w.w[n + 1] = pair13(lo);
                w.w[16 + n] = pair02(hi);
                w.w[16 + n + 1] = pair13(hi);
            }
    }
    template <int NT>
    __device__ static inline void dot(const W &w, const State &, int g, const h2 *x, int xs,
                                      const float4 *sd, int ss, int nt, float *acc)
    {
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const h2 *xg = x + j * xs + 32 * g;
            const float sl = dot16(w.w, xg), sh = dot16(w.w + 16, xg + 16);
            const float4 gs = sd[j * ss + g];
            acc[j] += (w.d1 * sl - w.m1 * gs.x + w.d2 * sh - w.m2 * gs.y) * gs.z;
        }
    }
};

// Q6_K (dequantQ6K, gguf.zig:1036-1059): a unit is one 256-element super-block of
// 16-element sub-blocks with int8 scales; y = d * sc * (q - 32).  Step s = 2h + lh
// covers, for l in [16 lh, 16 lh + 16) of half h, the four quants built from
// ql[l], ql[l+32] and qh[l]: sub-blocks 8h + {lh, 2+lh, 4+lh, 6+lh}.  Pairs hold
// 1024 + q - 1056 = q - 32 exactly.
struct DecQ6_K {
    static constexpr int kUnit = 256, kSteps = 4;
    struct Raw {
        u32x4 a, b, qh;
        u32x4 sc;      // step 0 only
        uint32_t d;    // step 0 only
    };
    struct W {
        h2 w[32];      // [8i .. 8i+7] = sub-block 8h + 2i + lh, i = 0..3
        float c[4];    // d * scale of those sub-blocks
    };
    struct State {
        u32x4 sc;
        float d;
    };
    __device__ static inline void load(Raw &r, const QMat &m, int mat, int rg, int u, int s, int lane)
    {
        const Fmt f{256, 13, 2};
        const uint8_t *q = m.q + (size_t)mat * m.q_stride;
        const int h = s >> 1, lh = s & 1;
        r.a = ld_stream((const u32x4 *)(q + tile_q_off(f, m.units, rg, u, 4 * h + lh, lane)));
        r.b = ld_stream((const u32x4 *)(q + tile_q_off(f, m.units, rg, u, 4 * h + 2 + lh, lane)));
        r.qh = ld_stream((const u32x4 *)(q + tile_q_off(f, m.units, rg, u, 8 + 2 * h + lh, lane)));
        if (s == 0) {
            r.sc = ld_stream((const u32x4 *)(q + tile_q_off(f, m.units, rg, u, 12, lane)));
            r.d = *(const uint16_t *)(m.s + (size_t)mat * m.s_stride + tile_s_off(f, m.units, rg, u, lane));
        }
    }
    __device__ static inline void convert(const Raw &r, int s, W &w, State &st)
    {
        if (s == 0) {
            st.sc = r.sc;
            st.d = f16_bits_to_f32((uint16_t)r.d);
        }
        const int h = s >> 1, lh = s & 1;
        // sub-blocks 8h + 2i + lh: dword 2h (i = 0, 1) or 2h + 1 (i = 2, 3) of the scales,
        // bytes lh and 2 + lh of it
        const uint32_t s0 = h ? st.sc[2] : st.sc[0], s1 = h ? st.sc[3] : st.sc[1];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t wd = i < 2 ? s0 : s1;
            const int sh = 8 * (2 * (i & 1) + lh);
            w.c[i] = st.d * (float)(int8_t)((wd >> sh) & 0xFFu);
        }
        const h2 bias = {(half_t)1056.0f, (half_t)1056.0f};
#pragma unroll
        for (int dl = 0; dl < 4; dl++) {
            const uint32_t A = r.a[dl], B = r.b[dl], Q = r.qh[dl];
            const uint32_t q[4] = {(A & 0x0F0F0F0Fu) | ((Q & 0x03030303u) << 4),
                                   (B & 0x0F0F0F0Fu) | ((Q << 2) & 0x30303030u),
                                   ((A >> 4) & 0x0F0F0F0Fu) | (Q & 0x30303030u),
                                   ((B >> 4) & 0x0F0F0F0Fu) | ((Q >> 2) & 0x30303030u)};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                w.w[8 * i + 2 * dl] = pair02(q[i]) - bias;
                w.w[8 * i + 2 * dl + 1] = pair13(q[i]) - bias;
            }
        }
    }
    template <int NT>
    __device__ static inline void dot(const W &w, const State &, int s, const h2 *x, int xs,
                                      const float4 *sd, int ss, int nt, float *acc)
    {
        const int h = s >> 1, lh = s & 1;
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const h2 *xh = x + j * xs + 64 * h;
            const float s0 = dot8(w.w, xh + 8 * lh), s1 = dot8(w.w + 8, xh + 8 * (2 + lh));
            const float s2 = dot8(w.w + 16, xh + 8 * (4 + lh)), s3 = dot8(w.w + 24, xh + 8 * (6 + lh));
            acc[j] += (w.c[0] * s0 + w.c[1] * s1) * sd[j * ss + 2 * h].z +
                      (w.c[2] * s2 + w.c[3] * s3) * sd[j * ss + 2 * h + 1].z;
        }
    }
};

// Streams units [ub, ue) of one row group's weights through a decoder for
// exactly NT tokens, the next step's bytes in flight while the current step's
// products run.  (Straight-line code per token count: per-token conditionals
// would let the compiler speculate every token's LDS reads up front.)
// `raw` holds step 0 of unit ub, loaded by the caller before the barrier that
// publishes the staged activations.
template <class D, int NT>
__device__ inline void gemv_span(const QMat &M, int mat, int rg, int ub, int ue, int u0, int lane,
                                 const h2 *xs, int xs_h2, const float4 *ss, int ss_n, int nt,
                                 typename D::Raw &raw, float *acc)
{
    const int n = (ue - ub) * D::kSteps;
    if (n <= 0) return;
    typename D::State state;
    for (int t = 0; t < n; t++) {
        const int u = ub + t / D::kSteps, st = t % D::kSteps;
        typename D::W w;
        D::convert(raw, st, w, state);
        if (t + 1 < n) D::load(raw, M, mat, rg, ub + (t + 1) / D::kSteps, (t + 1) % D::kSteps, lane);
        D::template dot<NT>(w, state, st, xs + (u - u0) * (D::kUnit / 2), xs_h2, ss + (u - u0) * (D::kUnit / 64),
                            ss_n, nt, acc);
    }
}

// gemv_span for the pass's actual token count nt (1 <= nt <= NT), chosen once per
// pass; acc[nt..NT) stay untouched.
template <class D, int NT>
__device__ inline void gemv_tokens(const QMat &M, int mat, int rg, int ub, int ue, int u0, int lane, const h2 *xs,
                                   int xs_h2, const float4 *ss, int ss_n, int nt, typename D::Raw &raw, float *acc)
{
#define ANEDVD_NT_CASE(N)                                                                                   \
    case N:                                                                                                 \
        if constexpr (N <= NT) gemv_span<D, N>(M, mat, rg, ub, ue, u0, lane, xs, xs_h2, ss, ss_n, N, raw, acc); \
        break;
    switch (nt) {
        ANEDVD_NT_CASE(1)
        ANEDVD_NT_CASE(2)
        ANEDVD_NT_CASE(3)
        ANEDVD_NT_CASE(4)
        ANEDVD_NT_CASE(5)
        ANEDVD_NT_CASE(6)
        ANEDVD_NT_CASE(7)
        ANEDVD_NT_CASE(8)
    default: break;
    }
#undef ANEDVD_NT_CASE
}

// Copies nt activation rows (the span [k0, k0 + span) of each) and their group
// records into LDS: xs [nt][span] halves, ss [nt][span/64].
__device__ inline void stage_rows(const ActQ &src, int K, const int32_t *__restrict__ rowids, int row0, int nt, int k0,
                                  int span, half_t *xs, float4 *ss)
{
    const int n16 = span / 8, ng = span / 64, G = K / 64;
#pragma unroll 4
    for (int i = threadIdx.x; i < nt * n16; i += 256) {
        const int j = i / n16, c = i - j * n16;
        const int row = rowids ? rowids[row0 + j] : row0 + j;
        ((uint4 *)xs)[i] = ((const uint4 *)(src.q + (size_t)row * K + k0))[c];
    }
    for (int i = threadIdx.x; i < nt * ng; i += 256) {
        const int j = i / ng, g = i - j * ng;
        const int row = rowids ? rowids[row0 + j] : row0 + j;
        ss[i] = src.side[(size_t)row * G + k0 / 64 + g];
    }
}

__device__ inline float gelu_tanh(float x)
{
    const float c = 0.7978845608028654f;
    return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

// ------------------------------------------------------------ gate / up

struct GateUpArgs {
    QMat gate, up;          // tile layout, n = E
    ActQ x;                 // [T][H]
    Dispatch d;
    float *part;            // [KS][P][2][I] when KS > 1
    ActQ act;               // out: [P][I]
    int H, I, KS, P, use_gelu;
};

// SiLU(g) * u (moeExpertAccumF32's g / (1 + exp(-g)), cpu.zig:434-437) for the 64
// rows of one row group (lane = row), converted to the activation format; the 64
// rows are exactly one group of the down product's input.
__device__ inline void write_act(const GateUpArgs &a, int pos, int rg, int lane, float g, float u)
{
    const float act = a.use_gelu ? gelu_tanh(g) : g / (1.0f + __expf(-g));
    act_group(act * u, lane, a.act.q + (size_t)pos * a.I + rg * 64, a.act.side + (size_t)pos * (a.I / 64) + rg);
}

// Grid (I/64 * KS, max_u), 256 threads.  Waves 0,1 compute gate rows, 2,3 up
// rows; within a matrix the two waves split the workgroup's K span.  With KS > 1
// the K partials go to `part` and k_act_reduce finishes them.
template <class D, int NT>
__global__ __launch_bounds__(256, ANEDVD_GEMV_MIN_WAVES) void k_gateup(GateUpArgs a)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_raw[];
    __shared__ float red_s[2][NT][64];

    const int ua = blockIdx.y;
    if (ua >= a.d.meta[0]) return;  // uniform over the workgroup
    const int e = a.d.active[ua];
    const int p0 = a.d.offsets[e], ne = a.d.offsets[e + 1] - p0;
    const int rg = blockIdx.x / a.KS, ks = blockIdx.x % a.KS;
    const int units = a.H / D::kUnit, upw = units / a.KS, u0 = ks * upw;
    const int span = upw * D::kUnit, k0 = u0 * D::kUnit;
    const int wv = wave_id(), lane = threadIdx.x & 63;
    const int mat = wv >> 1, half = wv & 1;
    const int hu = (upw + 1) / 2;
    const int ub = u0 + half * hu, ue = min(u0 + upw, ub + hu);
    const QMat &M = mat ? a.up : a.gate;
    half_t *xs = (half_t *)lds_raw;
    float4 *ss = (float4 *)(lds_raw + (size_t)NT * span * sizeof(half_t));

    for (int c0 = 0; c0 < ne; c0 += NT) {
        const int nt = min(NT, ne - c0);
        stage_rows(a.x, a.H, a.d.rows, p0 + c0, nt, k0, span, xs, ss);
        typename D::Raw raw;  // first weight bytes in flight across the barrier
        if (ub < ue) D::load(raw, M, e, rg, ub, 0, lane);
        __syncthreads();
        float acc[NT];
#pragma unroll
        for (int j = 0; j < NT; j++) acc[j] = 0.0f;
        gemv_tokens<D, NT>(M, e, rg, ub, ue, u0, lane, (const h2 *)xs, span / 2, ss, span / 64, nt, raw, acc);
        if (half) {
#pragma unroll
            for (int j = 0; j < NT; j++) red_s[mat][j][lane] = acc[j];
        }
        __syncthreads();
        if (!half) {
#pragma unroll
            for (int j = 0; j < NT; j++) acc[j] += red_s[mat][j][lane];
        }
        __syncthreads();
        if (a.KS == 1) {
            if (wv == 2) {  // the up sums, to the gate wavefront
#pragma unroll
                for (int j = 0; j < NT; j++) red_s[1][j][lane] = acc[j];
            }
            __syncthreads();
            if (wv == 0) {
#pragma unroll
                for (int j = 0; j < NT; j++)
                    if (j < nt) write_act(a, p0 + c0 + j, rg, lane, acc[j], red_s[1][j][lane]);
            }
        } else if (!half) {
#pragma unroll
            for (int j = 0; j < NT; j++)
                if (j < nt) a.part[(((size_t)ks * a.P + p0 + c0 + j) * 2 + mat) * a.I + rg * 64 + lane] = acc[j];
        }
        __syncthreads();
    }
}

// Finishes a K-split gate/up: one wavefront per (position, 64-row group) adds the
// KS partials in ks order, applies SiLU(g) * u and writes the activations.  Grid:
// P * I/64 wavefronts, 4 per workgroup.
__global__ __launch_bounds__(256) void k_act_reduce(GateUpArgs a, int n_pos)
{
    const size_t w = (size_t)blockIdx.x * 4 + wave_id();
    const int G = a.I / 64, lane = threadIdx.x & 63;
    if (w >= (size_t)n_pos * G) return;
    const int pos = (int)(w / G), rg = (int)(w % G);
    float g = 0.0f, u = 0.0f;
    for (int s = 0; s < a.KS; s++) {
        const float *pp = a.part + ((size_t)s * a.P + pos) * 2 * a.I + rg * 64 + lane;
        g += pp[0];
        u += pp[a.I];
    }
    write_act(a, pos, rg, lane, g, u);
}

// ---------------------------------------------------------------- down

struct DownArgs {
    QMat down;              // tile layout [E][H][I]
    ActQ act;               // [P][I]
    Dispatch d;
    float *ypart;           // [KS][P][H]
    int H, I, KS, P;
};

// Grid (H/64/WR * KS, max_u), 256 threads; WR = 4/WK row groups per workgroup,
// WK wavefronts splitting each row group's K span, summed in wave order.
template <class D, int NT, int WK>
__global__ __launch_bounds__(256, ANEDVD_GEMV_MIN_WAVES) void k_down(DownArgs a)
{
    constexpr int WR = kWaves / WK;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_raw[];
    __shared__ float red_s[kWaves][NT][64];

    const int ua = blockIdx.y;
    if (ua >= a.d.meta[0]) return;
    const int e = a.d.active[ua];
    const int p0 = a.d.offsets[e], ne = a.d.offsets[e + 1] - p0;
    const int rb = blockIdx.x / a.KS, ks = blockIdx.x % a.KS;
    const int units = a.I / D::kUnit, upw = units / a.KS, u0 = ks * upw;
    const int span = upw * D::kUnit, k0 = u0 * D::kUnit;
    const int wv = wave_id(), lane = threadIdx.x & 63;
    const int wr = wv / WK, wk = wv % WK;
    const int rg = rb * WR + wr;
    const int ub = u0 + (upw * wk) / WK, ue = u0 + (upw * (wk + 1)) / WK;
    half_t *xs = (half_t *)lds_raw;
    float4 *ss = (float4 *)(lds_raw + (size_t)NT * span * sizeof(half_t));

    for (int c0 = 0; c0 < ne; c0 += NT) {
        const int nt = min(NT, ne - c0);
        stage_rows(a.act, a.I, nullptr, p0 + c0, nt, k0, span, xs, ss);
        typename D::Raw raw;  // first weight bytes in flight across the barrier
        if (ub < ue) D::load(raw, a.down, e, rg, ub, 0, lane);
        __syncthreads();
        float acc[NT];
#pragma unroll
        for (int j = 0; j < NT; j++) acc[j] = 0.0f;
        gemv_tokens<D, NT>(a.down, e, rg, ub, ue, u0, lane, (const h2 *)xs, span / 2, ss, span / 64, nt, raw, acc);
        if (WK > 1) {
#pragma unroll
            for (int j = 0; j < NT; j++) red_s[wv][j][lane] = acc[j];
            __syncthreads();
            if (wk == 0) {
#pragma unroll
                for (int j = 0; j < NT; j++)
                    for (int q = 1; q < WK; q++) acc[j] += red_s[wv + q][j][lane];
            }
        }
        if (wk == 0) {
#pragma unroll
            for (int j = 0; j < NT; j++)
                if (j < nt) a.ypart[((size_t)ks * a.P + p0 + c0 + j) * a.H + rg * 64 + lane] = acc[j];
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------- combine

// out[t][h] = sum over slots s (in slot order) of p[t][s] * y[pos(t,s)][h], the
// KS down partials of a position added in fixed order; a deterministic gather,
// no atomics (main.zig:495-509 / engine.zig:725-777).  Then + scale * shared.
__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ ypart, const int32_t *__restrict__ inv,
                                                 const float *__restrict__ probs, int T, int k, int H, int KS, int P,
                                                 const float *__restrict__ shared, const float *__restrict__ shared_scale,
                                                 int sKS, float *__restrict__ out)
{
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int H4 = H / 4;
    if (id >= (size_t)T * H4) return;
    const int t = (int)(id / H4), h = (int)(id % H4) * 4;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < k; s++) {
        const int pos = inv[(size_t)t * k + s];
        if (pos < 0) continue;
        const float p = probs[(size_t)t * k + s];
        float4 y = *(const float4 *)(ypart + (size_t)pos * H + h);
        for (int q = 1; q < KS; q++) {
            const float4 z = *(const float4 *)(ypart + ((size_t)q * P + pos) * H + h);
            y.x += z.x; y.y += z.y; y.z += z.z; y.w += z.w;
        }
        acc.x += p * y.x; acc.y += p * y.y; acc.z += p * y.z; acc.w += p * y.w;
    }
    if (shared) {  // the shared expert's down partials [sKS][T][H], then its scale
        const float sc = shared_scale ? shared_scale[t] : 1.0f;
        float4 y = *(const float4 *)(shared + (size_t)t * H + h);
        for (int q = 1; q < sKS; q++) {
            const float4 z = *(const float4 *)(shared + ((size_t)q * T + t) * H + h);
            y.x += z.x; y.y += z.y; y.z += z.z; y.w += z.w;
        }
        acc.x += sc * y.x; acc.y += sc * y.y; acc.z += sc * y.z; acc.w += sc * y.w;
    }
    *(float4 *)(out + (size_t)t * H + h) = acc;
}

// ------------------------------------------------------------- planning

static int unit_elems(int type)
{
    switch (type) {
    case ANEDVD_Q8_0: return DecQ8_0::kUnit;
    case ANEDVD_Q4_0: return DecQ4_0::kUnit;
    case ANEDVD_Q4_K: return DecQ4_K::kUnit;
    case ANEDVD_Q6_K: return DecQ6_K::kUnit;
    default: return 0;
    }
}

// Smallest K span a wavefront should stream: 2 units of 64 or 1 super-block.
static int min_units_per_wave(int type) { return unit_elems(type) == 64 ? 2 : 1; }

bool gemv_supported(int type) { return unit_elems(type) != 0; }

constexpr size_t kMaxStageLds = 65536;

static size_t stage_lds(int nt, int span) { return (size_t)nt * span * sizeof(half_t) + (size_t)nt * (span / 64) * 16; }

GemvPlan plan_gemv(int gate_type, int down_type, int H, int I, int max_u, int max_group)
{
    GemvPlan p{};
    // tokens per pass: up to 8 (ANEDVD_GEMV_MAX_NT = 1, 2 or 4 lowers it, for tuning)
    static const int max_nt = [] {
        const char *v = getenv("ANEDVD_GEMV_MAX_NT");
        const int n = v ? atoi(v) : 8;
        return n == 1 || n == 2 || n == 4 ? n : 8;
    }();
    p.nt = 1;
    while (p.nt < max_nt && p.nt < max_group) p.nt *= 2;
    const long target = 1024;  // workgroups: 4 per CU
    // gate/up: 2 wavefronts split each matrix's K span
    {
        const int units = H / unit_elems(gate_type), mu = min_units_per_wave(gate_type), rgs = I / 64;
        p.ks_gu = 1;
        for (int ks = 1; ks <= 16; ks++) {
            if (units % ks || units / ks < 2 * mu) continue;
            p.ks_gu = ks;
            if ((long)max_u * rgs * ks >= target) break;
        }
        while (p.nt > 1 && stage_lds(p.nt, H / p.ks_gu) > kMaxStageLds) p.nt /= 2;
    }
    // down: WK wavefronts split one row group's K, ks workgroups split it further
    {
        const int units = I / unit_elems(down_type), mu = min_units_per_wave(down_type);
        long best_wg = -1;
        int best_units = 0;
        p.ks_dn = 1;
        p.wk_dn = 1;
        for (int wk = 1; wk <= 4; wk *= 2)
            for (int ks = 1; ks <= 16; ks++) {
                if (units % ks || (H / 64) % (4 / wk)) continue;
                const int upw = units / ks;
                if (upw / wk < mu) continue;
                const long wg = (long)max_u * (H / 64 / (4 / wk)) * ks;
                const int per_wave = upw / wk;
                // prefer reaching the target with the longest streams, else the most workgroups
                const bool better = best_wg < 0 ||
                                    (wg >= target && (best_wg < target || per_wave > best_units)) ||
                                    (wg < target && best_wg < target && wg > best_wg);
                if (better) {
                    best_wg = wg;
                    best_units = per_wave;
                    p.ks_dn = ks;
                    p.wk_dn = wk;
                }
            }
    }
    return p;
}

// ------------------------------------------------------------- launchers

template <class D, int NT>
static void launch_gateup_nt(const GateUpArgs &a, int max_u, hipStream_t st)
{
    const int span = a.H / a.KS;
    hipLaunchKernelGGL((k_gateup<D, NT>), dim3(a.I / 64 * a.KS, max_u), dim3(256), stage_lds(NT, span), st, a);
}

template <class D>
static int launch_gateup_t(const GateUpArgs &a, int nt, int max_u, hipStream_t st)
{
    switch (nt) {
    case 1: launch_gateup_nt<D, 1>(a, max_u, st); break;
    case 2: launch_gateup_nt<D, 2>(a, max_u, st); break;
    case 4: launch_gateup_nt<D, 4>(a, max_u, st); break;
    default: launch_gateup_nt<D, 8>(a, max_u, st); break;
    }
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

template <class D, int NT, int WK>
static void launch_down_nt(const DownArgs &a, int max_u, hipStream_t st)
{
    const int span = a.I / a.KS;
    hipLaunchKernelGGL((k_down<D, NT, WK>), dim3(a.H / 64 / (kWaves / WK) * a.KS, max_u), dim3(256),
                       stage_lds(NT, span), st, a);
}

template <class D, int WK>
static void launch_down_wk(const DownArgs &a, int nt, int max_u, hipStream_t st)
{
    switch (nt) {
    case 1: launch_down_nt<D, 1, WK>(a, max_u, st); break;
    case 2: launch_down_nt<D, 2, WK>(a, max_u, st); break;
    case 4: launch_down_nt<D, 4, WK>(a, max_u, st); break;
    default: launch_down_nt<D, 8, WK>(a, max_u, st); break;
    }
}

template <class D>
static int launch_down_t(const DownArgs &a, const GemvPlan &p, int max_u, hipStream_t st)
{
    switch (p.wk_dn) {
    case 1: launch_down_wk<D, 1>(a, p.nt, max_u, st); break;
    case 2: launch_down_wk<D, 2>(a, p.nt, max_u, st); break;
    default: launch_down_wk<D, 4>(a, p.nt, max_u, st); break;
    }
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

int launch_expert_gateup(const QMat &gate, const QMat &up, const ActQ &x, int H, int I, const Dispatch &d, int P,
                         int max_u, const GemvPlan &plan, float *part, const ActQ &act, int use_gelu, hipStream_t st)
{
    if (gate.type != up.type) {
        set_error("expert gate/up: gate type %d and up type %d differ", gate.type, up.type);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
    GateUpArgs a{gate, up, x, d, part, act, H, I, plan.ks_gu, P, use_gelu};
    int rc;
    switch (gate.type) {
    case ANEDVD_Q8_0: rc = launch_gateup_t<DecQ8_0>(a, plan.nt, max_u, st); break;
    case ANEDVD_Q4_0: rc = launch_gateup_t<DecQ4_0>(a, plan.nt, max_u, st); break;
    case ANEDVD_Q4_K: rc = launch_gateup_t<DecQ4_K>(a, plan.nt, max_u, st); break;
    case ANEDVD_Q6_K: rc = launch_gateup_t<DecQ6_K>(a, plan.nt, max_u, st); break;
    default:
        set_error("expert gate/up: ggml type %d has no decode kernel", gate.type);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
    if (rc != ANEDVD_OK || plan.ks_gu == 1) return rc;
    // positions past the dispatched ones are never read; reducing all P keeps the
    // launch free of a device-side count
    const size_t waves = (size_t)P * (I / 64);
    hipLaunchKernelGGL(k_act_reduce, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, a, P);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

int launch_expert_down(const QMat &down, const ActQ &act, int H, int I, const Dispatch &d, int P, int max_u,
                       const GemvPlan &plan, float *ypart, hipStream_t st)
{
    DownArgs a{down, act, d, ypart, H, I, plan.ks_dn, P};
    switch (down.type) {
    case ANEDVD_Q8_0: return launch_down_t<DecQ8_0>(a, plan, max_u, st);
    case ANEDVD_Q4_0: return launch_down_t<DecQ4_0>(a, plan, max_u, st);
    case ANEDVD_Q4_K: return launch_down_t<DecQ4_K>(a, plan, max_u, st);
    case ANEDVD_Q6_K: return launch_down_t<DecQ6_K>(a, plan, max_u, st);
    default:
        set_error("expert down: ggml type %d has no decode kernel", down.type);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
}

int launch_combine(const float *ypart, const int32_t *inv, const float *probs, int T, int k, int H, int KS, int P,
                   const float *shared, const float *shared_scale, int sKS, float *out, hipStream_t st)
{
    const size_t n = (size_t)T * (H / 4);
    if (n == 0) return ANEDVD_OK;
    hipLaunchKernelGGL(k_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, ypart, inv, probs, T, k, H, KS, P,
                       shared, shared_scale, sKS, out);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

}  // namespace anedvd
