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

namespace anedvd {

constexpr int kWaves = 4;
constexpr int kMTile = 16;  // tokens per MFMA pass

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

template <class T>
__device__ inline T ld_stream(const T *p)
{
    return __builtin_nontemporal_load(p);
}

__device__ inline uint32_t pick4(u32x4 v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

// ------------------------------------------------------------------ decoders
//
// A decoder loads one step of its wavefront's four tiles (load), takes what
// stays valid for a whole scale unit (begin), and yields the B operand of (tile
// t, block j) with the block's scale d and min coefficient mn (operand); the
// MFMA result r then contributes d * r - mn * (activation block sum).

struct MQ8_0 {
    static constexpr int kSpu = 1;
    static constexpr bool kMin = false;
    struct Raw {
        u32x4 q[4];
        uint32_t s[4];
    };
    struct State {};
    __device__ static inline void load(Raw &r, const QMat &m, int mat, int rb, int s, int lane)
    {
        const Fmt f = tile_fmt(ANEDVD_Q8_0);
        const uint8_t *q = m.q + (size_t)mat * m.q_stride, *sp = m.s + (size_t)mat * m.s_stride;
#pragma unroll
        for (int t = 0; t < 4; t++) r.q[t] = ld_stream((const u32x4 *)(q + tile_q_off(f, m.steps, rb, s, t, lane)));
#pragma unroll
        for (int t = 0; t < 4; t++)
            r.s[t] = ld_stream((const uint32_t *)(sp + tile_s_off(f, m.units, rb, s, t, lane & 15)));
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
    __device__ static inline void load(Raw &r, const QMat &m, int mat, int rb, int s, int lane)
    {
        const Fmt f = tile_fmt(ANEDVD_Q4_0);
        const uint8_t *q = m.q + (size_t)mat * m.q_stride, *sp = m.s + (size_t)mat * m.s_stride;
#pragma unroll
        for (int t = 0; t < 4; t++) r.q[t] = ld_stream((const u32x2 *)(q + tile_q_off(f, m.steps, rb, s, t, lane)));
#pragma unroll
        for (int t = 0; t < 4; t++)
            r.s[t] = ld_stream((const uint32_t *)(sp + tile_s_off(f, m.units, rb, s, t, lane & 15)));
    }
    __device__ static inline void begin(const Raw &, State &, int) {}
    __device__ static inline void operand(const Raw &r, const State &, int, int, int t, int j, half8 &b, float &d,
                                          float &mn)
    {
        const uint32_t v = r.q[t][j];
        b = bytes_h8(v & 0x0F0F0F0Fu, (v >> 4) & 0x0F0F0F0Fu) - (half_t)1032.0f;  // n - 8
        d = f16_bits_to_f32((uint16_t)(r.s[t] >> (16 * j)));
        mn = 0.0f;
    }
};

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
    __device__ static inline void load(Raw &r, const QMat &m, int mat, int rb, int s, int lane)
    {
        const Fmt f = tile_fmt(ANEDVD_Q4_K);
        const uint8_t *q = m.q + (size_t)mat * m.q_stride, *sp = m.s + (size_t)mat * m.s_stride;
#pragma unroll
        for (int t = 0; t < 4; t++) r.q[t] = ld_stream((const u32x2 *)(q + tile_q_off(f, m.steps, rb, s, t, lane)));
        if ((s & 3) == 0) {
#pragma unroll
            for (int t = 0; t < 4; t++)
                r.sc[t] = ld_stream((const u32x4 *)(sp + tile_s_off(f, m.units, rb, s >> 2, t, lane & 15)));
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
        b = bytes_h8(v & 0x0F0F0F0Fu, (v >> 4) & 0x0F0F0F0Fu) - (half_t)1024.0f;  // n
        const u32x4 sc = st.sc[t];
        int a, m;
        scale_min_k4(2 * (s & 3) + j, sc.y, sc.z, sc.w, a, m);
        d = f16_bits_to_f32((uint16_t)(sc.x & 0xFFFFu)) * (float)a;
        mn = f16_bits_to_f32((uint16_t)(sc.x >> 16)) * (float)m;
    }
};

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
    __device__ static inline void load(Raw &r, const QMat &m, int mat, int rb, int s, int lane)
    {
        const Fmt f = tile_fmt(ANEDVD_Q6_K);
        const uint8_t *q = m.q + (size_t)mat * m.q_stride, *hp = m.h + (size_t)mat * m.h_stride;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            r.q[t] = ld_stream((const u32x2 *)(q + tile_q_off(f, m.steps, rb, s, t, lane)));
            r.h[t] = ld_stream((const uint32_t *)(hp + tile_h_off(m.steps, rb, s, t, lane)));
        }
        if ((s & 3) == 0) {
            const uint8_t *sp = m.s + (size_t)mat * m.s_stride, *dp = m.d + (size_t)mat * m.d_stride;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                r.sc[t] = ld_stream((const u32x4 *)(sp + tile_s_off(f, m.units, rb, s >> 2, t, lane & 15)));
                r.d[t] = *(const uint16_t *)(dp + tile_d_off(m.units, rb, s >> 2, t, lane & 15));
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

// Streams steps [s0, s1) of the wavefront's four tiles (row block rb of matrix
// `mat`) against 16 tokens: lane l feeds A rows from `arow` (its token l % 16, the
// row's column 0) and accumulates acc[t][i] = sum_k W[64 rb + 16 t + l % 16][k] *
// x[token 4 (l / 16) + i][k], the tokens' descales taken from ds[step * ld +
// dsrow[i]].  The next step's weights, activations and descales are in flight
// while the current step's MFMAs run.
template <class D>
__device__ inline void mm_steps(const QMat &W, int mat, int rb, int s0, int s1, int lane, const half_t *arow,
                                const float *ds, int ld, const int *dsrow, f32x4 *acc)
{
    if (s0 >= s1) return;
    const int g = lane >> 4;
    typename D::Raw cur, nxt;
    typename D::State st;
    D::load(cur, W, mat, rb, s0, lane);
    const half8 *ap = (const half8 *)(arow + (size_t)kStep * s0 + 16 * g);
    half8 a0 = ap[0], a1 = ap[1];
    float dv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) dv[i] = ds[(size_t)s0 * ld + dsrow[i]];
    const half8 ones = (half8)(half_t)1.0f;
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = s0; s < s1; s++) {
        half8 na0 = a0, na1 = a1;
        float ndv[4] = {dv[0], dv[1], dv[2], dv[3]};
        if (s + 1 < s1) {
            D::load(nxt, W, mat, rb, s + 1, lane);
            const half8 *np = (const half8 *)(arow + (size_t)kStep * (s + 1) + 16 * g);
            na0 = np[0];
            na1 = np[1];
#pragma unroll
            for (int i = 0; i < 4; i++) ndv[i] = ds[(size_t)(s + 1) * ld + dsrow[i]];
        }
        D::begin(cur, st, s);
        f32x4 sum0 = zero, sum1 = zero;
        if (D::kMin) {
            sum0 = mfma(a0, ones, zero);
            sum1 = mfma(a1, ones, zero);
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                half8 b;
                float d, mn;
                D::operand(cur, st, s, lane, t, j, b, d, mn);
                const f32x4 r = mfma(j ? a1 : a0, b, zero);
                const f32x4 sm = j ? sum1 : sum0;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float v = D::kMin ? d * r[i] - mn * sm[i] : d * r[i];
                    acc[t][i] += dv[i] * v;
                }
            }
        }
        cur = nxt;
        a0 = na0;
        a1 = na1;
#pragma unroll
        for (int i = 0; i < 4; i++) dv[i] = ndv[i];
    }
}

__device__ inline float gelu_tanh(float x)
{
    const float c = 0.7978845608028654f;
    return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

// moeExpertAccumF32's activation: g / (1 + exp(-g)) (cpu.zig:434-437), or gelu.
__device__ inline float gate_act(float g, int use_gelu) { return use_gelu ? gelu_tanh(g) : g / (1.0f + __expf(-g)); }

struct MmArgs {
    QMat w0, w1;     // gate and up (gate/up), or down (w0)
    ActQ x;          // input activations: tokens (gate/up) or positions (down)
    Dispatch d;
    float *part;     // gate/up K partials [KS][P][2][I] when KS > 1
    ActQ act;        // gate/up output [P][I]
    float *ypart;    // down output [KS][P][H]
    int H, I, KS, P, use_gelu;
};

// ------------------------------------------------------------ gate / up

// Grid (I/64 * KS, max_u), 256 threads.  Wave w: matrix w >> 1 (gate, up), half
// w & 1 of the workgroup's K units; the four are summed through LDS and wave 0
// applies SiLU(g) * u to its 64 rows x 16 tokens.
template <class D>
__global__ __launch_bounds__(256) void k_mm_gateup(MmArgs a)
{
    __shared__ f32x4 xch[3][4][64];
    const int ua = blockIdx.y;
    if (ua >= a.d.meta[0]) return;  // uniform over the workgroup
    const int e = a.d.active[ua];
    const int p0 = a.d.offsets[e], ne = a.d.offsets[e + 1] - p0;
    const int rb = blockIdx.x / a.KS, ks = blockIdx.x % a.KS;
    const int units = a.H / kStep / D::kSpu, upw = units / a.KS, u0 = ks * upw;
    const int wv = wave_id(), lane = threadIdx.x & 63;
    const int mat = wv >> 1, half = wv & 1;
    const int hu = (upw + 1) / 2;
    const int ub = u0 + half * hu, ue = min(u0 + upw, ub + hu);
    const QMat &W = mat ? a.w1 : a.w0;
    const int n = lane & 15, gq = lane >> 4;

    for (int c0 = 0; c0 < ne; c0 += kMTile) {
        const int nt = min(kMTile, ne - c0);
        const int tok = a.d.rows[p0 + c0 + min(n, nt - 1)];
        int dsrow[4];
#pragma unroll
        for (int i = 0; i < 4; i++) dsrow[i] = a.d.rows[p0 + c0 + min(4 * gq + i, nt - 1)];
        f32x4 acc[4];
#pragma unroll
        for (int t = 0; t < 4; t++) acc[t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        mm_steps<D>(W, e, rb, ub * D::kSpu, ue * D::kSpu, lane, a.x.q + (size_t)tok * a.H, a.x.ds, a.x.ld, dsrow,
                    acc);
        if (wv) {
#pragma unroll
            for (int t = 0; t < 4; t++) xch[wv - 1][t][lane] = acc[t];
        }
        __syncthreads();
        if (wv == 0) {
            f32x4 gs[4], us[4];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                gs[t] = acc[t] + xch[0][t][lane];
                us[t] = xch[1][t][lane] + xch[2][t][lane];
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
                    const int m = 4 * gq + i;
                    const float sc = pow2_scale(row_max_f32(mx[i]));
                    if (m < nt) {
                        const size_t pos = (size_t)p0 + c0 + m;
                        half_t *dst = a.act.q + pos * a.I + (size_t)kStep * rb;
#pragma unroll
                        for (int t = 0; t < 4; t++) dst[mma_pos(16 * t + n)] = (half_t)(v[t][i] * sc);
                        if (n == 0) a.act.ds[(size_t)rb * a.act.ld + pos] = 1.0f / sc;
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int m = 4 * gq + i;
                    if (m < nt) {
                        float *pp = a.part + (((size_t)ks * a.P + p0 + c0 + m) * 2) * a.I + (size_t)kStep * rb + n;
#pragma unroll
                        for (int t = 0; t < 4; t++) {
                            pp[16 * t] = gs[t][i];
                            pp[a.I + 16 * t] = us[t][i];
                        }
                    }
                }
            }
        }
        __syncthreads();
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

// Grid (ceil(H/256) * KS, max_u), 256 threads; wave w owns row block 4 x + w of
// the output and the workgroup's K units.
template <class D>
__global__ __launch_bounds__(256) void k_mm_down(MmArgs a)
{
    const int ua = blockIdx.y;
    if (ua >= a.d.meta[0]) return;
    const int e = a.d.active[ua];
    const int p0 = a.d.offsets[e], ne = a.d.offsets[e + 1] - p0;
    const int wv = wave_id(), lane = threadIdx.x & 63;
    const int rb = kWaves * (blockIdx.x / a.KS) + wv, ks = blockIdx.x % a.KS;
    if (rb >= a.H / kRowBlock) return;  // no barriers in this kernel
    const int units = a.I / kStep / D::kSpu, upw = units / a.KS, u0 = ks * upw;
    const int n = lane & 15, gq = lane >> 4;

    for (int c0 = 0; c0 < ne; c0 += kMTile) {
        const int nt = min(kMTile, ne - c0);
        const int pos = p0 + c0 + min(n, nt - 1);
        int dsrow[4];
#pragma unroll
        for (int i = 0; i < 4; i++) dsrow[i] = p0 + c0 + min(4 * gq + i, nt - 1);
        f32x4 acc[4];
#pragma unroll
        for (int t = 0; t < 4; t++) acc[t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        mm_steps<D>(a.w0, e, rb, u0 * D::kSpu, (u0 + upw) * D::kSpu, lane, a.x.q + (size_t)pos * a.I, a.x.ds, a.x.ld,
                    dsrow, acc);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = 4 * gq + i;
            if (m < nt) {
                float *yp = a.ypart + ((size_t)ks * a.P + p0 + c0 + m) * a.H + (size_t)kRowBlock * rb + n;
#pragma unroll
                for (int t = 0; t < 4; t++) yp[16 * t] = acc[t][i];
            }
        }
    }
}

// ------------------------------------------------------------- combine

// out[t][h] = sum over slots s (in slot order) of p[t][s] * y[pos(t,s)][h], the
// KS down partials of a position added in fixed order; a deterministic gather,
// no atomics (main.zig:495-509 / engine.zig:725-777).  Then + scale * shared.
// Slots are taken 8 at a time with their loads issued together (indices clamped
// rather than branched on, so nothing waits on the previous slot).
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
    for (int s0 = 0; s0 < k; s0 += 8) {
        int pos[8];
        float p[8];
        bool ok[8];
        float4 y[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int s = min(s0 + i, k - 1);
            pos[i] = inv[(size_t)t * k + s];
            p[i] = probs[(size_t)t * k + s];
            ok[i] = s0 + i < k && pos[i] >= 0;
            pos[i] = max(pos[i], 0);
            y[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        for (int q = 0; q < KS; q++) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 z = *(const float4 *)(ypart + ((size_t)q * P + pos[i]) * H + h);
                y[i].x += z.x; y[i].y += z.y; y[i].z += z.z; y[i].w += z.w;
            }
        }
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (ok[i]) {
                acc.x += p[i] * y[i].x; acc.y += p[i] * y[i].y; acc.z += p[i] * y[i].z; acc.w += p[i] * y[i].w;
            }
    }
    if (shared) {  // the shared expert's down partials [sKS][T][H], then its scale
        const float sc = shared_scale ? shared_scale[t] : 1.0f;
        float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int q = 0; q < sKS; q++) {
            const float4 z = *(const float4 *)(shared + ((size_t)q * T + t) * H + h);
            y.x += z.x; y.y += z.y; y.z += z.z; y.w += z.w;
        }
        acc.x += sc * y.x; acc.y += sc * y.y; acc.z += sc * y.z; acc.w += sc * y.w;
    }
    *(float4 *)(out + (size_t)t * H + h) = acc;
}

// ------------------------------------------------------------- planning

static int steps_per_unit(int type) { return tile_fmt(type).spu; }

bool mm_supported(int type) { return tile_fmt(type).qb != 0; }

// Splits a K axis of `units` scale units over ks workgroups, ks dividing units:
// the smallest ks that gives `wg_per_ks * ks` >= 1024 workgroups (4 per CU) while
// every wavefront keeps >= `min_steps` steps of `waves_per_k` shares, else the
// largest ks keeping them.
static int choose_ks(int units, int spu, long wg_per_ks, int waves_per_k, int min_steps)
{
    int best = 1;
    for (int ks = 1; ks <= units; ks++) {
        if (units % ks) continue;
        const int steps = (units / ks) * spu / waves_per_k;
        if (ks > 1 && steps < min_steps) break;
        best = ks;
        if (wg_per_ks * ks >= 1024) break;
    }
    return best;
}

MmPlan plan_mm(int gate_type, int down_type, int H, int I, int max_u)
{
    MmPlan p{};
    p.ks_gu = choose_ks(H / kStep / steps_per_unit(gate_type), steps_per_unit(gate_type), (long)max_u * (I / kRowBlock),
                        2, 2);
    p.ks_dn = choose_ks(I / kStep / steps_per_unit(down_type), steps_per_unit(down_type),
                        (long)max_u * ((H / kRowBlock + kWaves - 1) / kWaves), 1, 2);
    return p;
}

// ------------------------------------------------------------- launchers

template <class D>
static int launch_gateup_t(const MmArgs &a, int max_u, hipStream_t st)
{
    hipLaunchKernelGGL(k_mm_gateup<D>, dim3(a.I / kRowBlock * a.KS, max_u), dim3(256), 0, st, a);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

template <class D>
static int launch_down_t(const MmArgs &a, int max_u, hipStream_t st)
{
    const int rbb = (a.H / kRowBlock + kWaves - 1) / kWaves;
    hipLaunchKernelGGL(k_mm_down<D>, dim3(rbb * a.KS, max_u), dim3(256), 0, st, a);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

int launch_expert_gateup(const QMat &gate, const QMat &up, const ActQ &x, int H, int I, const Dispatch &d, int P,
                         int max_u, const MmPlan &plan, float *part, const ActQ &act, int use_gelu, hipStream_t st)
{
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
    int rc;
    switch (gate.type) {
    case ANEDVD_Q8_0: rc = launch_gateup_t<MQ8_0>(a, max_u, st); break;
    case ANEDVD_Q4_0: rc = launch_gateup_t<MQ4_0>(a, max_u, st); break;
    case ANEDVD_Q4_K: rc = launch_gateup_t<MQ4_K>(a, max_u, st); break;
    case ANEDVD_Q6_K: rc = launch_gateup_t<MQ6_K>(a, max_u, st); break;
    default:
        set_error("expert gate/up: ggml type %d has no kernel", gate.type);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
    if (rc != ANEDVD_OK || plan.ks_gu == 1) return rc;
    const size_t waves = (size_t)P * (I / kStep);
    hipLaunchKernelGGL(k_act_reduce, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, a);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

int launch_expert_down(const QMat &down, const ActQ &act, int H, int I, const Dispatch &d, int P, int max_u,
                       const MmPlan &plan, float *ypart, hipStream_t st)
{
    MmArgs a{};
    a.w0 = down;
    a.x = act;
    a.d = d;
    a.ypart = ypart;
    a.H = H;
    a.I = I;
    a.KS = plan.ks_dn;
    a.P = P;
    switch (down.type) {
    case ANEDVD_Q8_0: return launch_down_t<MQ8_0>(a, max_u, st);
    case ANEDVD_Q4_0: return launch_down_t<MQ4_0>(a, max_u, st);
    case ANEDVD_Q4_K: return launch_down_t<MQ4_K>(a, max_u, st);
    case ANEDVD_Q6_K: return launch_down_t<MQ6_K>(a, max_u, st);
    default:
        set_error("expert down: ggml type %d has no kernel", down.type);
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
