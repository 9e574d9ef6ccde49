// k_route.hip -- router logits, softmax/top-k/renormalisation and token-to-expert
// dispatch.  All three are bit-exact against the reference on the CPU:
//   router   cpu.matmulF16 (cpu.zig:461-475): 8 strided lane accumulators,
//            multiply and add rounded separately, lanes summed in order;
//   route    cpu.moeRoute (cpu.zig:1236-1288): exp via expf_exact (== libm),
//            sequential sum, one IEEE division, strict-max top-k (ties to the
//            lowest expert), optional renormalisation by the slot-order sum;
//   dispatch engine.zig:1204-1216: a stable counting sort of (token, slot) by
//            expert, tokens ascending within an expert.
#pragma clang fp contract(off)

#include "common.h"
#include "expf_exact.h"
#include "kernels.h"

namespace anedvd {

__constant__ uint64_t c_exp2_tab[32] = ANEDVD_EXP2_TABLE;

// ------------------------------------------------------------------ router

// Block: 256 threads = 32 experts x 8 lanes.  Grid: (ceil(E/32), ceil(T/TT)).
// Thread (e, l) accumulates x[t][8j+l] * f32(w[e][8j+l]) for j ascending, for TT
// tokens at once; the 8 lane sums of an expert are then added lane 0..7 in order.
template <int TT>
__global__ __launch_bounds__(256) void k_router(const uint16_t *__restrict__ w, const float *__restrict__ x,
                                                int T, int E, int H, float *__restrict__ logits)
{
    extern __shared__ float xs[];  // [TT][H]
    const int t0 = blockIdx.y * TT;
    const int nt = min(TT, T - t0);
    for (int i = threadIdx.x; i < nt * H; i += blockDim.x) xs[i] = x[(size_t)t0 * H + i];
    __syncthreads();

    const int l = threadIdx.x & 7;
    const int e = blockIdx.x * 32 + (threadIdx.x >> 3);
    const bool live = e < E;
    const uint16_t *row = w + (size_t)(live ? e : 0) * H;
    float acc[TT];
#pragma unroll
    for (int t = 0; t < TT; t++) acc[t] = 0.0f;
    const int H8 = H & ~7;
    for (int i = l; i < H8; i += 8) {
        const float wv = f16_bits_to_f32(row[i]);
#pragma unroll
        for (int t = 0; t < TT; t++)
            if (t < nt) acc[t] = __fadd_rn(acc[t], __fmul_rn(xs[t * H + i], wv));
    }
    // Ordered lane sum: lane 0 + lane 1 + ... + lane 7, then the scalar tail.
#pragma unroll
    for (int t = 0; t < TT; t++) {
        float sum = __shfl(acc[t], (threadIdx.x & ~7), 64);
        for (int j = 1; j < 8; j++) sum = __fadd_rn(sum, __shfl(acc[t], (threadIdx.x & ~7) + j, 64));
        for (int i = H8; i < H; i++) sum = __fadd_rn(sum, __fmul_rn(f16_bits_to_f32(row[i]), xs[t * H + i]));
        if (live && l == 0 && t < nt) logits[(size_t)(t0 + t) * E + e] = sum;
    }
}

int launch_router(const uint16_t *d_w, const float *d_x, int T, int E, int H, float *d_logits, hipStream_t st)
{
    if (T <= 0) return ANEDVD_OK;
    // Tokens per block sized so the staged activations fit in 64 KiB of LDS.
    const dim3 block(256);
    if ((size_t)8 * H * 4 <= 65536) {
        const dim3 grid((E + 31) / 32, (T + 7) / 8);
        hipLaunchKernelGGL(k_router<8>, grid, block, (size_t)8 * H * 4, st, d_w, d_x, T, E, H, d_logits);
    } else if ((size_t)2 * H * 4 <= 65536) {
        const dim3 grid((E + 31) / 32, (T + 1) / 2);
        hipLaunchKernelGGL(k_router<2>, grid, block, (size_t)2 * H * 4, st, d_w, d_x, T, E, H, d_logits);
    } else {
        set_error("router: hidden size %d too large for the staged router", H);
        return ANEDVD_E_INVALID_ARG;
    }
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

// ------------------------------------------------------------------- route

__device__ inline float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ inline uint64_t wave_max_u64(uint64_t v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint64_t w = __shfl_xor(v, o, 64);
        v = w > v ? w : v;
    }
    return v;
}

constexpr int kRouteWaves = 4;
constexpr int kMaxExperts = 256;
constexpr int kMaxK = 32;

// One wavefront per token; lane j holds experts j, j+64, j+128, j+192.
// Selection key = (p bits << 32) | ~e: p >= 0, so its bits order like the value,
// and among equal p the lowest expert has the largest key -- the reference's
// strict `p > best_p` scan in ascending e.
__global__ __launch_bounds__(256) void k_route(const float *__restrict__ logits, int T, int E, int k, int norm,
                                               float *__restrict__ probs, uint32_t *__restrict__ idx)
{
    __shared__ float ex_s[kRouteWaves][kMaxExperts];
    __shared__ float p_s[kRouteWaves][kMaxK];
    __shared__ uint32_t i_s[kRouteWaves][kMaxK];
    __shared__ float inv_s[kRouteWaves];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = blockIdx.x * kRouteWaves + wv;
    const bool live = t < T;  // every thread reaches every barrier
    const float *lg = logits + (size_t)(live ? t : 0) * E;

    float v[4];
    float mx = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int e = lane + 64 * j;
        v[j] = (live && e < E) ? lg[e] : -__builtin_inff();
        if (e < E) mx = fmaxf(mx, v[j]);
    }
    mx = wave_max(mx);

    float ex[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int e = lane + 64 * j;
        ex[j] = expf_exact(v[j] - mx, c_exp2_tab);
        if (e < E) ex_s[wv][e] = ex[j];
    }
    __syncthreads();
    if (lane == 0) {  // the reference's sum is sequential in e
        float s = 0.0f;
        for (int e = 0; e < E; e++) s = __fadd_rn(s, ex_s[wv][e]);
        inv_s[wv] = s > 0.0f ? __fdiv_rn(1.0f, s) : 0.0f;
    }
    __syncthreads();
    const float inv_sum = inv_s[wv];

    uint64_t key[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int e = lane + 64 * j;
        const float p = __fmul_rn(ex[j], inv_sum);
        const bool ok = e < E && !(p != p);
        key[j] = ok ? ((uint64_t)__float_as_uint(p) << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e) : 0ull;
    }
    for (int slot = 0; slot < k; slot++) {
        uint64_t best = key[0];
#pragma unroll
        for (int j = 1; j < 4; j++) best = key[j] > best ? key[j] : best;
        best = wave_max_u64(best);
        float bp = 0.0f;
        uint32_t be = 0;
        if (best != 0ull) {
            be = 0xFFFFFFFFu - (uint32_t)best;
            bp = __uint_as_float((uint32_t)(best >> 32));
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (lane + 64 * j == (int)be) key[j] = 0ull;
        }
        if (lane == 0) {
            p_s[wv][slot] = bp;
            i_s[wv][slot] = be;
        }
    }
    __syncthreads();
    if (lane == 0 && norm) {
        float s = 0.0f;
        for (int j = 0; j < k; j++) s = __fadd_rn(s, p_s[wv][j]);
        if (s > 0.0f)
            for (int j = 0; j < k; j++) p_s[wv][j] = __fdiv_rn(p_s[wv][j], s);
    }
    __syncthreads();
    if (live && lane < k) {
        probs[(size_t)t * k + lane] = p_s[wv][lane];
        idx[(size_t)t * k + lane] = i_s[wv][lane];
    }
}

int launch_route(const float *d_logits, int T, int E, int k, int norm, float *d_probs, uint32_t *d_idx,
                 hipStream_t st)
{
    if (T <= 0) return ANEDVD_OK;
    if (E > kMaxExperts || k > kMaxK || k > E || k <= 0 || k > 64) {
        set_error("route: unsupported E=%d k=%d (E <= %d, 0 < k <= min(E, %d))", E, k, kMaxExperts, kMaxK);
        return ANEDVD_E_INVALID_ARG;
    }
    hipLaunchKernelGGL(k_route, dim3((T + kRouteWaves - 1) / kRouteWaves), dim3(256), 0, st, d_logits, T, E, k,
                       norm, d_probs, d_idx);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

// ---------------------------------------------------------------- dispatch

// A single workgroup of NTH threads.  Thread i owns the contiguous token range
// [i*P, (i+1)*P), P = ceil(T/NTH), and counts its (token, slot) entries per
// expert in column i of lc[E][NTH].  A scan down each expert's column, then
// across experts, gives every thread the first position it writes for each
// expert; walking its tokens in order then places entries stably.
//
// Outputs: offsets[E+1]; rows/slots[T*k] in expert-major order; inv[t*k+s] =
// the position of (t, s); active[0..n_active) = experts with tokens, ascending;
// meta[0] = n_active, meta[1] = largest group, meta[2] = entries dropped because
// idx >= E (they are never written out of bounds).
template <int NTH>
__global__ __launch_bounds__(NTH) void k_dispatch(const uint32_t *__restrict__ idx, int T, int k, int E,
                                                  int32_t *__restrict__ offsets, int32_t *__restrict__ rows,
                                                  int32_t *__restrict__ slots, int32_t *__restrict__ inv,
                                                  int32_t *__restrict__ active, int32_t *__restrict__ meta)
{
    extern __shared__ uint16_t lc[];  // [E][NTH]
    __shared__ int32_t base_s[kMaxExperts + 1];
    __shared__ int32_t bad_s;
    const int tid = threadIdx.x;
    const int P = (T + NTH - 1) / NTH;
    const int t_begin = min(T, tid * P), t_end = min(T, t_begin + P);
    for (int i = tid; i < E * NTH; i += NTH) lc[i] = 0;
    if (tid == 0) bad_s = 0;
    __syncthreads();
    int bad = 0;
    for (int t = t_begin; t < t_end; t++)
        for (int s = 0; s < k; s++) {
            const uint32_t e = idx[(size_t)t * k + s];
            if (e < (uint32_t)E) lc[e * NTH + tid]++;
            else bad++;
        }
    if (bad) atomicAdd(&bad_s, bad);
    __syncthreads();
    for (int e = tid; e < E; e += NTH) {  // exclusive scan down column e
        int run = 0;
        for (int i = 0; i < NTH; i++) {
            const int c = lc[e * NTH + i];
            lc[e * NTH + i] = (uint16_t)run;
            run += c;
        }
        base_s[e] = run;  // the expert's count, for now
    }
    __syncthreads();
    if (tid == 0) {
        int pos = 0, n_active = 0, biggest = 0;
        for (int e = 0; e < E; e++) {
            const int c = base_s[e];
            offsets[e] = pos;
            base_s[e] = pos;
            if (c > 0) active[n_active++] = e;
            biggest = c > biggest ? c : biggest;
            pos += c;
        }
        offsets[E] = pos;
        meta[0] = n_active;
        meta[1] = biggest;
        meta[2] = bad_s;
    }
    __syncthreads();
    for (int t = t_begin; t < t_end; t++)
        for (int s = 0; s < k; s++) {
            const uint32_t e = idx[(size_t)t * k + s];
            if (e >= (uint32_t)E) {
                inv[(size_t)t * k + s] = -1;
                continue;
            }
            const int pos = base_s[e] + lc[e * NTH + tid]++;
            rows[pos] = t;
            slots[pos] = s;
            inv[(size_t)t * k + s] = pos;
        }
}

int launch_dispatch(const uint32_t *d_idx, int T, int k, int E, int32_t *d_offsets, int32_t *d_rows, int32_t *d_slots,
                    int32_t *d_inv, int32_t *d_active, int32_t *d_meta, hipStream_t st)
{
    if (E > kMaxExperts || E <= 0 || T <= 0 || k <= 0) {
        set_error("dispatch: unsupported shape T=%d k=%d E=%d (E <= %d)", T, k, E, kMaxExperts);
        return ANEDVD_E_INVALID_ARG;
    }
    // lc[E][nth] u16 kept within 32 KiB of LDS
    const int nth = E <= 64 ? 256 : E <= 128 ? 128 : 64;
    const int P = (T + nth - 1) / nth;
    if ((long)P * k > 65535) {
        set_error("dispatch: %d tokens x top-%d exceeds the per-thread counter range", T, k);
        return ANEDVD_E_INVALID_ARG;
    }
    const size_t lds = (size_t)E * nth * sizeof(uint16_t);
    if (nth == 256)
        hipLaunchKernelGGL(k_dispatch<256>, dim3(1), dim3(256), lds, st, d_idx, T, k, E, d_offsets, d_rows, d_slots,
                           d_inv, d_active, d_meta);
    else if (nth == 128)
        hipLaunchKernelGGL(k_dispatch<128>, dim3(1), dim3(128), lds, st, d_idx, T, k, E, d_offsets, d_rows, d_slots,
                           d_inv, d_active, d_meta);
    else
        hipLaunchKernelGGL(k_dispatch<64>, dim3(1), dim3(64), lds, st, d_idx, T, k, E, d_offsets, d_rows, d_slots,
                           d_inv, d_active, d_meta);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

}  // namespace anedvd
