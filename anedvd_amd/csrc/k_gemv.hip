// k_gemv.hip -- decode-regime expert kernels: GGUF dequant fused into the
// SwiGLU gate/up and down products, for the token groups the dispatch built.
//
// Semantics follow cpu.moeExpertAccumF32 (cpu.zig:416-452): g = W_g h,
// u = W_u h, a = silu(g) * u, y = W_d a; the combine adds p * y per slot.
//
// Bandwidth design (HBM-bound GEMV, no MFMA): one weight row per lane, 64 rows
// per wavefront, weights in the tile layout of common.h so every
// global_load_dwordx4 of a wavefront reads 1 KiB contiguous.  A lane converts its
// quants to exact f16 integers once per unit and reuses them for every token of
// the group; activations are staged in LDS as f16 scaled by a per-token power of
// two (exact, and keeps any activation range inside f16), read back as
// wave-uniform broadcasts, and multiplied with v_dot2_f32_f16 into f32 sums; the
// per-block scale is applied to the f32 block sum.  The K axis is split over KS
// workgroups when a call has too few rows to fill 256 CUs; the KS partial sums
// are added in a fixed order by the next kernel, so results are deterministic.
#include "common.h"
#include "kernels.h"

namespace anedvd {

constexpr int kNT = 8;      // tokens per pass over the weights
constexpr int kWaves = 4;   // wavefronts per workgroup

__device__ inline float fdot2(h2 a, h2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }

__device__ inline h2 as_h2(uint32_t u)
{
    h2 r;
    __builtin_memcpy(&r, &u, 4);
    return r;
}

// ----------------------------------------------------------- unit decoders
//
// A unit decoder loads one lane's unit of one row (raw), converts it to f16
// (exact small integers), and dots it with a token's staged activations.  The
// activation order in LDS is the decoder's `perm` of the unit's elements.

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Q8_0: 4 chunks = 64 int8 quants (two blocks), 2 f16 scales.  A dword of four
// quants q0..q3 becomes the f16 pairs (q0, q2) and (q1, q3): byte-permute each
// biased quant (q ^ 0x80 = q + 128) under 0x64 to form 1024 + q + 128 exactly,
// then subtract 1152.  Activations are staged in the same pairing.
struct UnitQ8_0 {
    static constexpr int kType = ANEDVD_Q8_0;
    static constexpr int kUnit = 64;
    struct Raw {
        u32x4 q[4];
        uint32_t s;
    };
    h2 w[32];
    float d[2];

    __device__ static inline void load(Raw &r, const QMat &m, int mat, int rg, int u, int lane)
    {
        const Fmt f{64, 4, 4};
        const uint8_t *q = m.q + (size_t)mat * m.q_stride;
#pragma unroll
        for (int c = 0; c < 4; c++)
            r.q[c] = __builtin_nontemporal_load((const u32x4 *)(q + tile_q_off(f, m.units, rg, u, c, lane)));
        r.s = __builtin_nontemporal_load((const uint32_t *)(m.s + (size_t)mat * m.s_stride + tile_s_off(f, m.units, rg, u, lane)));
    }

    __device__ inline void convert(const Raw &r)
    {
        const h2 bias = {(half_t)1152.0f, (half_t)1152.0f};
#pragma unroll
        for (int c = 0; c < 4; c++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t b = r.q[c][i] ^ 0x80808080u;
                w[c * 8 + 2 * i] = as_h2(__builtin_amdgcn_perm(0x64646464u, b, 0x04020400u)) - bias;
                w[c * 8 + 2 * i + 1] = as_h2(__builtin_amdgcn_perm(0x64646464u, b, 0x04030401u)) - bias;
            }
        }
        d[0] = f16_bits_to_f32((uint16_t)(r.s & 0xFFFFu));
        d[1] = f16_bits_to_f32((uint16_t)(r.s >> 16));
    }

    // Staged position of unit element i (0..63): quants 4m..4m+3 pair as
    // (4m, 4m+2), (4m+1, 4m+3).
    __device__ static inline int perm(int i)
    {
        const int m = i >> 2, r = i & 3;
        return m * 4 + (r & 1) * 2 + (r >> 1);
    }

    // x: the 64 staged halves of this unit (LDS), as 32 h2.
    __device__ inline float dot(const h2 *x) const
    {
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) s0 = fdot2(w[i], x[i], s0);
#pragma unroll
        for (int i = 16; i < 32; i++) s1 = fdot2(w[i], x[i], s1);
        return d[0] * s0 + d[1] * s1;
    }
};

// ------------------------------------------------------------- staging

// Power-of-two scale bringing max|v| into [2^14, 2^15): exact, and the f16
// products and f32 sums of the dot stay far from overflow.
__device__ inline float pow2_scale(float maxabs)
{
    if (!(maxabs > 0.0f) || !(maxabs < __builtin_inff())) return 1.0f;
    int e;
    frexpf(maxabs, &e);  // maxabs = m * 2^e, m in [0.5, 1)
    return ldexpf(1.0f, min(15 - e, 126));
}

__device__ inline float block_max(float v, float *red)
{
    // wave max, then across the 4 wavefronts through LDS
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    const int wv = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wv] = v;
    __syncthreads();
    v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    return v;
}

// ------------------------------------------------------------ gate / up

struct GateUpArgs {
    QMat gate, up;               // tile layout, n = E
    const float *x;              // [T][H]
    const int32_t *offsets;      // [E+1]
    const int32_t *rows;         // [P] token of each position
    const int32_t *active;       // [E] experts with tokens
    const int32_t *meta;         // [0] = number of active experts
    float *part;                 // [KS][P][2][I]
    int H, I, KS, P;
};

// Grid (I/64 * KS, maxU), 256 threads.  Waves 0,1 compute gate rows, 2,3 up
// rows; within a matrix the two waves split the workgroup's K span.
template <class U>
__global__ __launch_bounds__(256) void k_gateup(GateUpArgs a)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_raw[];
    __shared__ float red_s[2][kNT][64];
    __shared__ float sc_s[kNT];
    __shared__ float mx_s[kWaves];

    const int ua = blockIdx.y;
    if (ua >= a.meta[0]) return;  // uniform over the workgroup
    const int e = a.active[ua];
    const int p0 = a.offsets[e], ne = a.offsets[e + 1] - p0;
    const int rg = blockIdx.x / a.KS, ks = blockIdx.x % a.KS;
    const int units = a.H / U::kUnit, upw = units / a.KS, u0 = ks * upw;
    const int span = upw * U::kUnit, k0 = u0 * U::kUnit;
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int mat = wv >> 1, half = wv & 1;
    const int hu = (upw + 1) / 2;
    const int ub = u0 + half * hu, ue = min(u0 + upw, ub + hu);
    const QMat &M = mat ? a.up : a.gate;
    half_t *xh = (half_t *)lds_raw;  // [kNT][span]

    for (int c0 = 0; c0 < ne; c0 += kNT) {
        const int nt = min(kNT, ne - c0);
        // stage the group's activations: per-token max, then scaled f16
        for (int j = 0; j < nt; j++) {
            const float *xr = a.x + (size_t)a.rows[p0 + c0 + j] * a.H + k0;
            float m = 0.0f;
            for (int i = threadIdx.x; i < span; i += 256) m = fmaxf(m, fabsf(xr[i]));
            m = block_max(m, mx_s);
            if (threadIdx.x == 0) sc_s[j] = pow2_scale(m);
        }
        __syncthreads();
        for (int j = 0; j < nt; j++) {
            const float *xr = a.x + (size_t)a.rows[p0 + c0 + j] * a.H + k0;
            const float sc = sc_s[j];
            for (int i = threadIdx.x; i < span; i += 256) {
                const int uo = (i / U::kUnit) * U::kUnit;
                xh[j * span + uo + U::perm(i - uo)] = (half_t)(xr[i] * sc);
            }
        }
        __syncthreads();

        float acc[kNT];
#pragma unroll
        for (int j = 0; j < kNT; j++) acc[j] = 0.0f;
        typename U::Raw raw;
        if (ub < ue) U::load(raw, M, e, rg, ub, lane);
        for (int u = ub; u < ue; u++) {
            U w;
            w.convert(raw);
            if (u + 1 < ue) U::load(raw, M, e, rg, u + 1, lane);  // next unit in flight
            const h2 *xu = (const h2 *)(xh + (u - u0) * U::kUnit);
#pragma unroll
            for (int j = 0; j < kNT; j++)
                if (j < nt) acc[j] += w.dot(xu + (size_t)j * span / 2);
        }
        if (half) {
#pragma unroll
            for (int j = 0; j < kNT; j++) red_s[mat][j][lane] = acc[j];
        }
        __syncthreads();
        if (!half) {
            for (int j = 0; j < nt; j++) {
                const float v = (acc[j] + red_s[mat][j][lane]) / sc_s[j];
                a.part[(((size_t)ks * a.P + p0 + c0 + j) * 2 + mat) * a.I + rg * 64 + lane] = v;
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------- down

struct DownArgs {
    QMat down;                   // tile layout [E][H][I]
    const float *part;           // gate/up partials [KSg][P][2][I]
    const int32_t *offsets, *active, *meta;
    float *ypart;                // [KS][P][H]
    int H, I, KS, KSg, P, use_gelu;
};

__device__ inline float gelu_tanh(float x)
{
    const float c = 0.7978845608028654f;
    return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

__device__ inline float swiglu_at(const DownArgs &a, int p, int i)
{
    float g = 0.0f, u = 0.0f;
    for (int s = 0; s < a.KSg; s++) {  // fixed order over the K split
        const float *pp = a.part + ((size_t)s * a.P + p) * 2 * a.I;
        g += pp[i];
        u += pp[a.I + i];
    }
    // moeExpertAccumF32's activation: g / (1 + exp(-g)), times up (cpu.zig:434-437)
    const float act = a.use_gelu ? gelu_tanh(g) : g / (1.0f + __expf(-g));
    return act * u;
}

// Grid (H/64 * KS, maxU), 256 threads; the 4 wavefronts split the workgroup's
// K span of the same 64 output rows and are summed in wave order.
template <class U>
__global__ __launch_bounds__(256) void k_down(DownArgs a)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_raw[];
    __shared__ float red_s[kWaves][kNT][64];
    __shared__ float sc_s[kNT];
    __shared__ float mx_s[kWaves];

    const int ua = blockIdx.y;
    if (ua >= a.meta[0]) return;
    const int e = a.active[ua];
    const int p0 = a.offsets[e], ne = a.offsets[e + 1] - p0;
    const int rg = blockIdx.x / a.KS, ks = blockIdx.x % a.KS;
    const int units = a.I / U::kUnit, upw = units / a.KS, u0 = ks * upw;
    const int span = upw * U::kUnit, k0 = u0 * U::kUnit;
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ub = u0 + (upw * wv) / kWaves, ue = u0 + (upw * (wv + 1)) / kWaves;
    half_t *xh = (half_t *)lds_raw;

    for (int c0 = 0; c0 < ne; c0 += kNT) {
        const int nt = min(kNT, ne - c0);
        for (int j = 0; j < nt; j++) {
            float m = 0.0f;
            for (int i = threadIdx.x; i < span; i += 256) m = fmaxf(m, fabsf(swiglu_at(a, p0 + c0 + j, k0 + i)));
            m = block_max(m, mx_s);
            if (threadIdx.x == 0) sc_s[j] = pow2_scale(m);
        }
        __syncthreads();
        for (int j = 0; j < nt; j++) {
            const float sc = sc_s[j];
            for (int i = threadIdx.x; i < span; i += 256) {
                const int uo = (i / U::kUnit) * U::kUnit;
                xh[j * span + uo + U::perm(i - uo)] = (half_t)(swiglu_at(a, p0 + c0 + j, k0 + i) * sc);
            }
        }
        __syncthreads();

        float acc[kNT];
#pragma unroll
        for (int j = 0; j < kNT; j++) acc[j] = 0.0f;
        typename U::Raw raw;
        if (ub < ue) U::load(raw, a.down, e, rg, ub, lane);
        for (int u = ub; u < ue; u++) {
            U w;
            w.convert(raw);
            if (u + 1 < ue) U::load(raw, a.down, e, rg, u + 1, lane);
            const h2 *xu = (const h2 *)(xh + (u - u0) * U::kUnit);
#pragma unroll
            for (int j = 0; j < kNT; j++)
                if (j < nt) acc[j] += w.dot(xu + (size_t)j * span / 2);
        }
#pragma unroll
        for (int j = 0; j < kNT; j++) red_s[wv][j][lane] = acc[j];
        __syncthreads();
        if (wv == 0) {
            for (int j = 0; j < nt; j++) {
                const float v = (((red_s[0][j][lane] + red_s[1][j][lane]) + red_s[2][j][lane]) + red_s[3][j][lane]) / sc_s[j];
                a.ypart[((size_t)ks * a.P + p0 + c0 + j) * a.H + rg * 64 + lane] = v;
            }
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

// ------------------------------------------------------------- launchers

template <class U>
static int launch_gateup_t(const GateUpArgs &a, int max_u, hipStream_t st)
{
    const int units = a.H / U::kUnit;
    const size_t lds = (size_t)kNT * (units / a.KS) * U::kUnit * sizeof(half_t);
    hipLaunchKernelGGL(k_gateup<U>, dim3(a.I / 64 * a.KS, max_u), dim3(256), lds, st, a);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

template <class U>
static int launch_down_t(const DownArgs &a, int max_u, hipStream_t st)
{
    const int units = a.I / U::kUnit;
    const size_t lds = (size_t)kNT * (units / a.KS) * U::kUnit * sizeof(half_t);
    hipLaunchKernelGGL(k_down<U>, dim3(a.H / 64 * a.KS, max_u), dim3(256), lds, st, a);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

int gemv_unit_elems(int type)
{
    switch (type) {
    case ANEDVD_Q8_0: return UnitQ8_0::kUnit;
    default: return 0;
    }
}

int launch_expert_gateup(const QMat &gate, const QMat &up, const float *x, const int32_t *offsets,
                         const int32_t *rows, const int32_t *active, const int32_t *meta, float *part, int H, int I,
                         int KS, int P, int max_u, hipStream_t st)
{
    GateUpArgs a{gate, up, x, offsets, rows, active, meta, part, H, I, KS, P};
    switch (gate.type) {
    case ANEDVD_Q8_0: return launch_gateup_t<UnitQ8_0>(a, max_u, st);
    default:
        set_error("expert gate/up: ggml type %d has no decode kernel yet", gate.type);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
}

int launch_expert_down(const QMat &down, const float *part, const int32_t *offsets, const int32_t *active,
                       const int32_t *meta, float *ypart, int H, int I, int KS, int KSg, int P, int use_gelu,
                       int max_u, hipStream_t st)
{
    DownArgs a{down, part, offsets, active, meta, ypart, H, I, KS, KSg, P, use_gelu};
    switch (down.type) {
    case ANEDVD_Q8_0: return launch_down_t<UnitQ8_0>(a, max_u, st);
    default:
        set_error("expert down: ggml type %d has no decode kernel yet", down.type);
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
