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

#include <type_traits>

#include "common.h"
#include "expf_exact.h"
#include "kernels.h"
#include "mma.h"

namespace anedvd {

__constant__ uint64_t c_exp2_tab[32] = ANEDVD_EXP2_TABLE;

// The exp table is read per lane with data-dependent indices straight from
// constant memory.  Each routing wavefront touches the whole table while its
// logits load (exp_table_warm, one load per lane beside theirs), so the lookups
// that follow hit the L1 instead of making a second trip to memory; no LDS copy
// and no barrier.
__device__ inline uint64_t exp_table_warm(int lane) { return c_exp2_tab[lane & 31]; }
__device__ inline void exp_table_ready(uint64_t warm) { asm volatile("" ::"v"(warm)); }

// ------------------------------------------------------------------ router

// cpu.matmulF16's order fixes, for each (token, expert), eight sequential chains:
// chain l adds x[8j+l] * f32(w[8j+l]) for j = 0, 1, ... (multiply and add rounded
// separately); the eight chain sums are then added l = 0..7 in order, then the
// scalar tail i >= H8 = H & ~7.  The chains cannot be split, so every chain runs
// in one lane: lane (g, l) of a block runs chain l of EX experts (g, g + 32) for
// TT tokens, the eight lanes of an expert in one DPP row for the ordered sum.
//
// The router is stored once per layer as f32 (f16 -> f32 is exact, so the products
// are the reference's, and the kernel converts nothing), interleaved so that a
// wavefront's loads of one 8-j block are one contiguous run: experts in groups of
// 64, and wt[((grp NB + jb) 64 + ei) 64 + 8 l + q] = w[64 grp + ei][8 (8 jb + q) + l]
// (NB = ceil(J / 8) blocks of eight j's, J = H / 8; zero past E and past J).  A lane
// reads its 8 j's of one block in two 16-byte loads through a buffer descriptor
// with a scalar per-block offset.  The token's x is staged in LDS as xs[l JP + j]
// = x[8 j + l], the row stride JP (>= J, four times an odd number) putting the
// eight chains' 16-byte reads on distinct banks.
//
// What bounds it (Qwen3 512 and DeepSeek-V2-Lite 1024 tokens, 134 M products):
// at TT = EX = 1 the 16-byte weight loads cost 4 bytes per product through the
// L1 and the staged x 4 bytes of LDS; TT = 2 halves the first, EX = 2 the second,
// leaving the multiply and add (2 VALU per product) as the largest term.
__host__ __device__ inline int router_stride(int J) { return ((J + 3) / 4 | 1) * 4; }
constexpr int kRouterGroup = 64;  // experts per layout group

__host__ __device__ inline size_t router_blocks(int H) { return (size_t)(((H >> 3) + 7) / 8); }

size_t router_layout_floats(int E, int H)
{
    return (size_t)((E + kRouterGroup - 1) / kRouterGroup) * router_blocks(H) * kRouterGroup * 64;
}

__global__ void k_router_layout(const uint16_t *__restrict__ w, int E, int H, float *__restrict__ wt, size_t n)
{
    const int J = H >> 3, NB = (int)router_blocks(H);
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int q = (int)(i & 7), l = (int)(i >> 3) & 7;
    const size_t r = i >> 6;  // (grp NB + jb) 64 + ei
    const int ei = (int)(r % kRouterGroup);
    const size_t r2 = r / kRouterGroup;
    const int jb = (int)(r2 % NB), grp = (int)(r2 / NB);
    const int e = kRouterGroup * grp + ei, j = 8 * jb + q;
    wt[i] = (e < E && j < J) ? f16_bits_to_f32(w[(size_t)e * H + 8 * (size_t)j + l]) : 0.0f;
}

// Block: 256 threads = 32 lane groups x 8 chains, 32 EX experts.  Grid:
// (ceil(E / (32 EX)), ceil(T / TT)), or the two swapped (`tx`, tokens on x) when the
// token blocks pass the 65536 limit of the grid's y.
template <int TT, int EX>
__global__ __launch_bounds__(256) void k_router(const float *__restrict__ wt, const uint16_t *__restrict__ w,
                                                const float *__restrict__ x, int T, int E, int H,
                                                float *__restrict__ logits, int tx)
{
    const int tb = tx ? blockIdx.x : blockIdx.y, eb = tx ? blockIdx.y : blockIdx.x;
    static_assert(EX == 1 || EX == 2, "a block's experts lie in one layout group");
    extern __shared__ float xs[];  // [TT][8][JP]
    const int J = H >> 3, H8 = J * 8, JP = router_stride(J), NB = (int)router_blocks(H), NBF = J / 8;
    const int t0 = tb * TT;
    const int nt = min(TT, T - t0);
    const int e0 = eb * 32 * EX;  // the block's first expert
    // The block's experts: layout group e0 / 64, from expert e0 % 64 of it (0, or 32
    // when EX = 1); a block of the group is 64 x 256 bytes.
    const rsrc_t rs = make_rsrc(wt + ((size_t)(e0 / kRouterGroup) * NB * kRouterGroup + e0 % kRouterGroup) * 64,
                                (size_t)NB * kRouterGroup * 256);
    // The first 8 kWarmBlocks blocks (kWarmBlocks per XCD, workgroup b on XCD b mod 8)
    // pull the router slice of their experts into their XCD's L2 before staging x,
    // each a kWarmBlocks-th of it: a layer's router is cold when its call starts, and
    // otherwise every block waits on the same misses at each 8-j block.  One dword per
    // 128-byte line, up to kWarm lines per thread, folded after the staging (whose
    // waits cover them) so they hold no register in the main loop.
    constexpr int kWarm = 4, kWarmBlocks = 16;
    uint32_t warm = 0;
    const int lin = blockIdx.x + blockIdx.y * gridDim.x;
    if (lin < 8 * kWarmBlocks) {
        const int lpb = 2 * min(32 * EX, E - e0);  // lines per 8-j block
        const int L = NB * lpb, per = (L + kWarmBlocks - 1) / kWarmBlocks, i0 = (lin / 8) * per;
        uint32_t wv[kWarm];
#pragma unroll
        for (int k = 0; k < kWarm; k++) {
            const int d = (int)threadIdx.x + 256 * k, i = i0 + d, jb = i / lpb;
            wv[k] = d < per && i < L ? __builtin_amdgcn_raw_buffer_load_b32(rs, (i % lpb) * 128, jb * kRouterGroup * 256, 0)
                                     : 0u;
        }
#pragma unroll
        for (int k = 0; k < kWarm; k++) warm ^= wv[k];
    }
    // Staging: kB loads per token in flight per thread before their LDS writes (one
    // load, wait and write per element measured 37 us for Mixtral's 2048 tokens).
    constexpr int kB = 8;
    for (int i0 = threadIdx.x; i0 < H8; i0 += kB * blockDim.x) {
        float v[TT][kB];
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int b = 0; b < kB; b++) {
                const int i = i0 + b * blockDim.x;
                v[t][b] = (t < nt && i < H8) ? x[(size_t)(t0 + t) * H + i] : 0.0f;
            }
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int b = 0; b < kB; b++) {
                const int i = i0 + b * blockDim.x;
                if (t < nt && i < H8) xs[(t * 8 + (i & 7)) * JP + (i >> 3)] = v[t][b];
            }
    }
    asm volatile("" ::"v"(warm));
    __syncthreads();

    const int l = threadIdx.x & 7, g = threadIdx.x >> 3;
    // A wavefront holds lane groups 8w .. 8w + 7; one whose first expert is past E
    // leaves (no barrier follows): with E = 8 three of the four would otherwise run
    // every chain on a stand-in expert.
    if (e0 + 8 * (int)(threadIdx.x >> 6) >= E) return;
    const int vo = threadIdx.x * 32;
    auto wl = [&](int jb, int m, int h) {
        return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, vo + 16 * h,
                                                                                 jb * kRouterGroup * 256 + m * 8192, 0));
    };
    float acc[TT][EX];
#pragma unroll
    for (int t = 0; t < TT; t++)
#pragma unroll
        for (int m = 0; m < EX; m++) acc[t][m] = 0.0f;
    float xv[TT][8];
    float4 cur[EX][2];
#pragma unroll
    for (int m = 0; m < EX; m++) {
        cur[m][0] = wl(0, m, 0);
        cur[m][1] = wl(0, m, 1);
    }
    // x of block jb (its first nq j's) from LDS
    auto ldx = [&](int jb, int nq) {
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const float *xr = &xs[(t * 8 + l) * JP + 8 * jb];
            if (nq == 8) {
                const float4 a = *(const float4 *)xr, b = *(const float4 *)(xr + 4);
                xv[t][0] = a.x; xv[t][1] = a.y; xv[t][2] = a.z; xv[t][3] = a.w;
                xv[t][4] = b.x; xv[t][5] = b.y; xv[t][6] = b.z; xv[t][7] = b.w;
            } else {
#pragma unroll
                for (int q = 0; q < 8; q++) xv[t][q] = q < nq ? xr[q] : 0.0f;
            }
        }
    };
    // the first nq j's of the block in `cur` against xv
    auto step = [&](int nq) {
#pragma unroll
        for (int q = 0; q < 8; q++) {
            if (q >= nq) break;
#pragma unroll
            for (int m = 0; m < EX; m++) {
                const float4 h = cur[m][q >> 2];
                const float wf = (q & 3) == 0 ? h.x : (q & 3) == 1 ? h.y : (q & 3) == 2 ? h.z : h.w;
#pragma unroll
                for (int t = 0; t < TT; t++) acc[t][m] = __fadd_rn(acc[t][m], __fmul_rn(xv[t][q], wf));
            }
        }
    };
    // Full blocks, the next block's weights loaded before this one's adds (past the
    // last block they lie outside the descriptor's range and read 0, no request).
    for (int jb = 0; jb < NBF; jb++) {
        float4 nxt[EX][2];
#pragma unroll
        for (int m = 0; m < EX; m++) {
            nxt[m][0] = wl(jb + 1, m, 0);
            nxt[m][1] = wl(jb + 1, m, 1);
        }
        ldx(jb, 8);
        step(8);
#pragma unroll
        for (int m = 0; m < EX; m++) {
            cur[m][0] = nxt[m][0];
            cur[m][1] = nxt[m][1];
        }
    }
    if (NB > NBF) {  // the last block's first J - 8 NBF j's
        ldx(NBF, J - 8 * NBF);
        step(J - 8 * NBF);
    }
    // Ordered lane sum: lane 0 + lane 1 + ... + lane 7, then the scalar tail.
#pragma unroll
    for (int m = 0; m < EX; m++) {
        const int e = e0 + 32 * m + g;
        const bool live = e < E;
        const uint16_t *row = w + (size_t)(live ? e : 0) * H;
#pragma unroll
        for (int t = 0; t < TT; t++) {
            float sum = __shfl(acc[t][m], (threadIdx.x & ~7), 64);
            for (int q = 1; q < 8; q++) sum = __fadd_rn(sum, __shfl(acc[t][m], (threadIdx.x & ~7) + q, 64));
            if (live && l == 0 && t < nt) {
                for (int i = H8; i < H; i++)
                    sum = __fadd_rn(sum, __fmul_rn(f16_bits_to_f32(row[i]), x[(size_t)(t0 + t) * H + i]));
                logits[(size_t)(t0 + t) * E + e] = sum;
            }
        }
    }
}

int launch_router_layout(const uint16_t *d_w, int E, int H, float *d_wt, hipStream_t st)
{
    const size_t n = router_layout_floats(E, H);
    if (!n) return ANEDVD_OK;
    hipLaunchKernelGGL(k_router_layout, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, d_w, E, H, d_wt, n);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

int launch_router(const float *d_wt, const uint16_t *d_w, const float *d_x, int T, int E, int H, float *d_logits,
                  hipStream_t st)
{
    if (T <= 0) return ANEDVD_OK;
    if (router_blocks(H) * kRouterGroup * 256 > (size_t)INT32_MAX) {
        set_error("router: hidden size %d too large", H);
        return ANEDVD_E_INVALID_ARG;
    }
    // Two tokens and two experts per lane once the grid still has about two
    // wavefronts per SIMD that way (Qwen3 512 tokens, DeepSeek-V2-Lite 1024: 11.5
    // and 11.8 us against 13.1 and 13.4 at one expert, 19.9 and 20.6 at one token
    // and one expert); one of each below (64 tokens of 128 experts: 5.1 against
    // 6.3 us at two tokens), and one expert for E < 64 (Mixtral's E = 8).
    const bool big = E >= 64 && (long)T * E >= 65536;
    auto go = [&](auto tt, auto ex) -> int {
        constexpr int TT = decltype(tt)::value, EX = decltype(ex)::value;
        const size_t lds = (size_t)TT * 8 * router_stride(H >> 3) * 4;
        if (lds > 65536) return -1;
        const unsigned nt = (unsigned)((T + TT - 1) / TT), ne = (unsigned)((E + 32 * EX - 1) / (32 * EX));
        if (ne > 65536u && nt > 65536u) return -2;
        const int tx = nt > 65536u;
        hipLaunchKernelGGL((k_router<TT, EX>), tx ? dim3(nt, ne) : dim3(ne, nt), dim3(256), lds, st, d_wt, d_w, d_x, T, E,
                           H, d_logits, tx);
        return 0;
    };
    int rc = -1;
    if (big) rc = go(std::integral_constant<int, 2>{}, std::integral_constant<int, 2>{});
    if (rc) rc = go(std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
    if (rc == -2) {
        set_error("router: %d tokens x %d experts is too many for one launch", T, E);
        return ANEDVD_E_INVALID_ARG;
    }
    if (rc) {
        set_error("router: hidden size %d too large for the staged router", H);
        return ANEDVD_E_INVALID_ARG;
    }
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

// ------------------------------------------------------------------- route

constexpr int kMaxExperts = kMaxRouteExperts;
constexpr int kMaxK = kMaxRouteSlots;

// -------------------------------------------------- one token per wavefront
//
// Lane l holds experts [VPL l, VPL l + VPL) (VPL = 1, 2, 4 for E <= 64, 128, 256).
// Maxima go through DPP within each row of 16 lanes and readlane across the four
// rows, so every lane ends with the wavefront's value.  The softmax denominator is
// the reference's sequential sum in ascending expert order: the lanes put their exps
// in an LDS row, lane 0 adds them one at a time.  A top-k slot takes the largest key,
// then the lowest expert holding it (one ballot per register), and clears it.

template <int CTRL>
__device__ inline uint32_t dpp_u32(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, 0xF, 0xF, false);
}

__device__ inline uint32_t row_max_u32(uint32_t v)
{
    v = max(v, dpp_u32<0xB1>(v));
    v = max(v, dpp_u32<0x4E>(v));
    v = max(v, dpp_u32<0x141>(v));
    v = max(v, dpp_u32<0x140>(v));
    return v;
}

__device__ inline uint32_t lane_u32(uint32_t v, int l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, l); }
__device__ inline float lane_f32(float v, int l) { return __uint_as_float(lane_u32(__float_as_uint(v), l)); }

// Wavefront-wide maxima (every lane gets the result).
__device__ inline uint32_t wave_max_u32(uint32_t v)
{
    v = row_max_u32(v);
    return max(max(lane_u32(v, 0), lane_u32(v, 16)), max(lane_u32(v, 32), lane_u32(v, 48)));
}


// cpu.moeRoute (cpu.zig:1236-1288) for the token whose E logits start at `lg`.
// Each unchosen expert with a non-NaN probability p carries key = bits(p) + 1 (p is
// in [0, 1], so its bits order like its value and +0 still beats an empty slot);
// chosen experts, NaNs and lanes past E carry 0.  A slot takes the largest key, then
// the lowest expert holding it -- the reference's strict `p > best_p` scan in
// ascending e.  A slot with nothing left gets (0, expert 0), as in the reference.
// `v` holds the row's logits as route_logits loaded them; `row` is this
// wavefront's LDS row of 64 VPL floats; `idx2`, when given, gets a second copy of
// the ids (the fused dispatch's LDS).
template <int VPL>
__device__ __forceinline__ void route_wave(const float *v, int E, int k, int norm, float *__restrict__ probs,
                           uint32_t *__restrict__ idx, int lane, const uint64_t *tab, float *row, uint32_t *idx2)
{
    float mx = v[0];
#pragma unroll
    for (int j = 1; j < VPL; j++) mx = fmaxf(mx, v[j]);
    mx = wave_max(mx);  // @max over the row: NaN only if every logit is NaN
    float ex[VPL];
#pragma unroll
    for (int j = 0; j < VPL; j++) {
        ex[j] = VPL * lane + j < E ? expf_exact(v[j] - mx, tab) : 0.0f;
        row[VPL * lane + j] = ex[j];  // the padding past E is +0, which leaves the sum as it is
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    float t = 0.0f;
    if (lane == 0) {  // the sum in ascending e, by one lane
        const float4 *r4 = reinterpret_cast<const float4 *>(row);
        for (int q = 0; q < (E + 3) / 4; q++) {
            const float4 c = r4[q];
            t = __fadd_rn(__fadd_rn(__fadd_rn(__fadd_rn(t, c.x), c.y), c.z), c.w);
        }
    }
    const float sum = lane_f32(t, 0);
    const float inv_sum = sum > 0.0f ? __fdiv_rn(1.0f, sum) : 0.0f;

    uint32_t key[VPL];
#pragma unroll
    for (int j = 0; j < VPL; j++) {
        const float p = __fmul_rn(ex[j], inv_sum);
        key[j] = (VPL * lane + j < E && !(p != p)) ? __float_as_uint(p) + 1u : 0u;
    }
    float my_p = 0.0f, rsum = 0.0f;
    uint32_t my_i = 0;
    for (int slot = 0; slot < k; slot++) {
        uint32_t m = key[0];
#pragma unroll
        for (int j = 1; j < VPL; j++) m = max(m, key[j]);
        const uint32_t best = wave_max_u32(m);
        float bp = 0.0f;
        uint32_t be = 0;
        if (best != 0u) {
            uint32_t first = 0xFFFFFFFFu;
#pragma unroll
            for (int j = 0; j < VPL; j++) {
                const uint64_t mk = __ballot(key[j] == best);
                if (mk) first = min(first, (uint32_t)(VPL * __builtin_ctzll(mk) + j));
            }
            be = first;
            bp = __uint_as_float(best - 1u);
#pragma unroll
            for (int j = 0; j < VPL; j++)
                if ((uint32_t)(VPL * lane + j) == be) key[j] = 0u;
        }
        rsum = __fadd_rn(rsum, bp);  // the renormalisation sum, in slot order
        if (lane == slot) {
            my_p = bp;
            my_i = be;
        }
    }
    if (norm && rsum > 0.0f) my_p = __fdiv_rn(my_p, rsum);
    if (lane < k) {
        probs[lane] = my_p;
        idx[lane] = my_i;
        if (idx2) idx2[lane] = my_i;
    }
}

// Token t's logits into v (VPL = 1, 2 or 4 per lane as E needs; lanes past E get
// -inf), issued ahead of the exp table's barrier.  The loads are unconditional
// (addresses clamped into the row, t clamped to a valid token) so the compiler
// counts them exactly and waits for the table alone.
__device__ inline void route_logits(const float *__restrict__ logits, int t, int T, int E, int lane, float (&v)[4])
{
    const float *lg = logits + (size_t)min(t, T - 1) * E;
    auto load = [&](auto vpl_c) {
        constexpr int VPL = decltype(vpl_c)::value;
#pragma unroll
        for (int j = 0; j < VPL; j++) {
            const int e = VPL * lane + j;
            const float x = lg[min(e, E - 1)];
            v[j] = e < E ? x : -__builtin_inff();
        }
    };
    if (E <= 64) load(std::integral_constant<int, 1>{});
    else if (E <= 128) load(std::integral_constant<int, 2>{});
    else load(std::integral_constant<int, 4>{});
}

// Routes token t on this wavefront (t < T) from its logits in v; its k slots start
// at row t of kk (of probs, idx and, when given, ids).
__device__ inline void route_token(const float (&v)[4], int t, int E, int k, int kk, int norm,
                                   float *__restrict__ probs, uint32_t *__restrict__ idx, int lane,
                                   const uint64_t *tab, float *row, uint32_t *ids = nullptr)
{
    float *pr = probs + (size_t)t * kk;
    uint32_t *ix = idx + (size_t)t * kk;
    uint32_t *i2 = ids ? ids + (size_t)t * kk : nullptr;
    if (E <= 64) route_wave<1>(v, E, k, norm, pr, ix, lane, tab, row, i2);
    else if (E <= 128) route_wave<2>(v, E, k, norm, pr, ix, lane, tab, row, i2);
    else route_wave<4>(v, E, k, norm, pr, ix, lane, tab, row, i2);
}

// ---------------------------------------------------------------- dispatch
//
// Stable counting sort of the T*k (token, slot) entries by expert, done by one
// workgroup of NTH threads:
//   1. per-expert counts (LDS atomics; order-free), then an exclusive scan over
//      experts gives offsets[E+1] and the ascending list of active experts;
//   2. entries are ranked within their expert.  When E rows of ceil(P/32) bitmap
//      words fit in LDS, through the bitmap: each entry sets bit (entry) of its
//      expert's row; the count of earlier entries of the same expert before a
//      word, plus the popcount of the lower bits of the entry's own word, is its
//      rank, and one pass does it all (row prefixes per expert, three barriers).
//      Otherwise (more than 128 experts and more than 512 entries) by segments
//      (dispatch_segments: no atomics, the ids loaded once).  A workgroup takes at
//      most NTH = kDispBlock entries: launch_dispatch sends larger calls to
//      k_dispatch_multi, one workgroup per block of entries, and the routed-and-
//      dispatched launch takes at most 16 tokens.
// Outputs: offsets[E+1]; rows/slots[T*k] grouped by expert, tokens ascending;
// inv[t*k+s] = position of (t, s) or -1 for an expert id >= E; active[0..n) =
// experts with tokens, ascending; meta[0] = n, meta[1] = largest group,
// meta[2] = entries with expert id >= E (never written out of bounds); and, when
// `chunks` is given, the expert kernels' work list: chunks[c] = chunk_entry(e, p0,
// nt) for each `chunk`-token slice of expert e's group (first position p0, nt
// tokens), experts ascending, meta[3] = their count.  With `small` > 0, groups of
// 1..small tokens go instead to a second list, chunks_s[c] = chunk_entry(e, p0,
// n), one entry per group, experts ascending, and meta[7] = its count.
constexpr int kDispWords = 4096;

struct DispLds {
    int32_t cnt[kMaxExperts];
    int32_t off[kMaxExperts];
    int32_t base[kMaxExperts];
    union {
        struct {
            uint32_t bits[kDispWords];
            int32_t pre[kDispWords + 1];
        };
        int32_t perm[2 * kDispWords + 1];  // dispatch_segments: the entry at each position
    };
    int32_t bad;
};

template <int CTRL, int ROW_MASK = 0xF>
__device__ inline int dpp_or_zero(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xF, false);
}

// Inclusive prefix sum over the wavefront: row_shr 1, 2, 4, 8 within each row of
// 16 lanes, then the row totals carried up with row_bcast 15 and 31.
__device__ inline int wave_incl_scan(int v, int)
{
    v += dpp_or_zero<0x111>(v);
    v += dpp_or_zero<0x112>(v);
    v += dpp_or_zero<0x114>(v);
    v += dpp_or_zero<0x118>(v);
    v += dpp_or_zero<0x142, 0xA>(v);
    v += dpp_or_zero<0x143, 0xC>(v);
    return v;
}

// Where the dispatch puts the work list beyond `chunks`: the small groups' list
// and the XCD ranges (Dispatch's chunks_s / small and xr / xper).
struct ListOpts {
    uint64_t *chunks_s;
    int small;
    int32_t *xr;
    int xper;
};
__device__ inline ListOpts list_opts(const Dispatch &d) { return ListOpts{d.chunks_s, d.small, d.xr, d.xper}; }

// Wavefront 0 of the dispatch: offsets[E+1], the active experts, the chunk list
// and meta from the per-expert counts in s.cnt (4 experts per lane, E <= 256);
// s.off gets the offsets.
template <class S>
__device__ __forceinline__ void dispatch_offsets(int E, int lane, int32_t *__restrict__ offsets, int32_t *__restrict__ active,
                                 int32_t *__restrict__ meta, uint64_t *__restrict__ chunks, int chunk, int n_routed,
                                 ListOpts lo, S &s, bool write = true)
{
    uint64_t *__restrict__ chunks_s = lo.chunks_s;
    const int small = lo.small;
    int c[4], tot = 0, nz = 0, mx = 0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int e = lane * 4 + q;
        c[q] = e < E ? s.cnt[e] : 0;
        tot += c[q];
        nz += c[q] > 0;
        if (n_routed <= 0 || e < n_routed) mx = max(mx, c[q]);
    }
    // groups of 1..small tokens go to the second list, one entry each
    auto is_small = [&](int n) { return n > 0 && n <= small; };
    int nch = 0, nsm = 0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        if (is_small(c[q])) nsm++;
        else nch += (c[q] + chunk - 1) / chunk;
    }
    int run = wave_incl_scan(tot, lane) - tot;
    int runa = wave_incl_scan(nz, lane) - nz;
    int runc = wave_incl_scan(nch, lane) - nch;
    int runs = wave_incl_scan(nsm, lane) - nsm;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int e = lane * 4 + q;
        if (e < E) {
            s.off[e] = run;
            if (write) {
                offsets[e] = run;
                if (c[q]) active[runa++] = e;
                if (chunks && is_small(c[q]))
                    chunks_s[runs++] = chunk_entry(e, run, c[q]);
                else if (chunks)
                    for (int j = 0; j * chunk < c[q]; j++)
                        chunks[runc++] = chunk_entry(e, run + j * chunk, min(chunk, c[q] - j * chunk));
            }
            run += c[q];
        }
    }
    if (!write) return;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = max(mx, __shfl_xor(mx, o, 64));
    if (lane == 63) {
        offsets[E] = run;
        meta[0] = runa;
        meta[3] = runc;
        if (small) meta[7] = runs;
    }
    if (lane == 0) {
        meta[1] = mx;
        meta[2] = s.bad;
    }
    // The work list cut into 8 XCD ranges of at most xper chunks, whole experts in
    // list order (next fit), so an expert's chunks share their weight slices in one
    // L2; if an expert does not fit, the even split x * xper.
    if (lo.xper > 0 && chunks && lane == 0) {
        int32_t start[9];
        int x = 0, fill = 0, pos = 0;
        bool ok = true;
        start[0] = 0;
        for (int e = 0; e < E && ok; e++) {
            const int n = s.cnt[e];
            const int nc = (n == 0 || (small && n <= small)) ? 0 : (n + chunk - 1) / chunk;
            if (nc == 0) continue;
            if (nc > lo.xper) {
                ok = false;
            } else {
                if (fill + nc > lo.xper) {
                    if (++x == 8) {
                        ok = false;
                        break;
                    }
                    start[x] = pos;
                    fill = 0;
                }
                fill += nc;
                pos += nc;
            }
        }
        for (int y = 0; y <= 8; y++) lo.xr[y] = ok ? (y <= x ? start[y] : pos) : y * lo.xper;
    }
}

// Calls of more entries than threads (or too many for the one-pass bitmap), up to
// (NTH / 64) * 64 * kSegBatches entries: wavefront w takes the w-th contiguous segment of entries, 64 at a time.
// The lanes holding the same expert id are found with nine ballots (one per bit
// of the id; padding and ids >= E share an id no expert has), so each entry's rank
// among its segment's earlier entries of the same expert is the running count of
// that expert in the wavefront's LDS row plus the lanes below it in its batch; the
// group's lowest lane then advances the count.  A scan over the wavefronts' rows
// gives each segment's base per expert: position = offset[e] + base[w][e] + rank,
// the same stable order (entries ascending within an expert) with two barriers
// after the counting.
constexpr int kSegBatches = 16;

template <int NTH>
__device__ __forceinline__ void dispatch_segments(const uint32_t *__restrict__ idx, int P, int k, int E,
                                  int32_t *__restrict__ offsets, int32_t *__restrict__ rows,
                                  int32_t *__restrict__ slots, int32_t *__restrict__ inv, int32_t *__restrict__ active,
                                  int32_t *__restrict__ meta, uint64_t *__restrict__ chunks, int chunk, int n_routed,
                                  ListOpts lo, DispLds &s)
{
    constexpr int NW = NTH / 64;
    static_assert(NW * kMaxExperts <= kDispWords, "per-wavefront counts live in the bitmap's words");
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nb = (P + NW * 64 - 1) / (NW * 64);  // batches per wavefront, <= kSegBatches
    const int seg0 = wv * nb * 64;
    int32_t *wcnt = reinterpret_cast<int32_t *>(s.bits) + wv * kMaxExperts;  // this wavefront's row
    for (int e = lane; e < E; e += 64) wcnt[e] = 0;
    if (tid == 0) s.bad = 0;
    __syncthreads();
    uint32_t key[kSegBatches];  // the id (9 bits), then the rank << 16 as well
    int bad = 0;
    const uint64_t below_mask = (1ull << lane) - 1ull;
    // every batch's ids first: one memory round trip, not one per batch
#pragma unroll
    for (int b = 0; b < kSegBatches; b++) {
        const int i = seg0 + 64 * b + lane;
        key[b] = b < nb && i < P ? idx[i] : 0x1FFu;
    }
#pragma unroll
    for (int b = 0; b < kSegBatches; b++) {
        if (b >= nb) continue;  // uniform; the loop stays fully unrolled, key and rank in registers
        const int i = seg0 + 64 * b + lane;
        uint32_t e = key[b];
        if (e >= (uint32_t)E) {
            bad += i < P;
            e = 0x1FFu;
        }
        uint64_t same = ~0ull;
#pragma unroll
        for (int bit = 0; bit < 9; bit++) {
            const bool on = (e >> bit) & 1u;
            const uint64_t bb = __ballot(on);
            same &= on ? bb : ~bb;
        }
        const int below = __popcll(same & below_mask);
        const int base = e < (uint32_t)E ? wcnt[e] : 0;
        key[b] = e | (uint32_t)(base + below) << 16;
        if (e < (uint32_t)E && below == 0) wcnt[e] = base + __popcll(same);
    }
    if (bad) atomicAdd(&s.bad, bad);
    __syncthreads();
    // per expert: the wavefronts' exclusive prefix in place, the total to cnt
    for (int e = tid; e < E; e += NTH) {
        int run = 0;
        for (int w = 0; w < NW; w++) {
            int32_t *c = reinterpret_cast<int32_t *>(s.bits) + w * kMaxExperts + e;
            const int v = *c;
            *c = run;
            run += v;
        }
        s.cnt[e] = run;
    }
    __syncthreads();
    if (wv == 0) dispatch_offsets(E, lane, offsets, active, meta, chunks, chunk, n_routed, lo, s);
    __syncthreads();
    // Each entry's position (inv, written in entry order); the entries go to LDS by
    // position, so rows and slots are written in position order (coalesced) rather
    // than scattered, when P positions fit in the bitmap's words.
    int pos[kSegBatches];
#pragma unroll
    for (int b = 0; b < kSegBatches; b++) {
        const int i = seg0 + 64 * b + lane;
        pos[b] = -1;
        if (b >= nb || i >= P) continue;
        const uint32_t e = key[b] & 0xFFFFu;
        if (e < (uint32_t)E) pos[b] = s.off[e] + wcnt[e] + (int)(key[b] >> 16);
        inv[i] = pos[b];
    }
    const bool staged = P <= 2 * kDispWords + 1;
    if (staged) __syncthreads();  // uniform: every wavefront is done with the counts
#pragma unroll
    for (int b = 0; b < kSegBatches; b++) {
        const int i = seg0 + 64 * b + lane;
        if (b >= nb || pos[b] < 0) continue;
        if (staged) {
            s.perm[pos[b]] = i;
        } else {
            rows[pos[b]] = i / k;
            slots[pos[b]] = i % k;
        }
    }
    if (!staged) return;
    __syncthreads();
    const int n = P - s.bad;  // positions filled
    for (int p = tid; p < n; p += NTH) {
        const int i = s.perm[p];
        rows[p] = i / k;
        slots[p] = i % k;
    }
}

template <int NTH>
__device__ __forceinline__ void dispatch_block(const uint32_t *__restrict__ idx, int T, int k, int E, int32_t *__restrict__ offsets,
                               int32_t *__restrict__ rows, int32_t *__restrict__ slots, int32_t *__restrict__ inv,
                               int32_t *__restrict__ active, int32_t *__restrict__ meta, uint64_t *__restrict__ chunks,
                               int chunk, int n_routed, ListOpts lo, DispLds &s)
{
    static_assert(NTH >= 128, "wavefront 0 computes the offsets while the others prefix the bitmap");
    const int P = T * k, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int W1 = (P + 31) / 32;  // bitmap words per expert if every entry fits at once
    if (P <= NTH && E * W1 <= kDispWords) {
        // One pass: the counts and the bitmap in the same sweep; then wavefront 0
        // takes the offsets while the others prefix each expert's row of the bitmap
        // (pre[e W + w] = entries of e before word w); an entry's rank is its row
        // prefix plus the popcount of the lower bits of its own word.
        for (int e = tid; e < E; e += NTH) s.cnt[e] = 0;
        for (int w = tid; w < E * W1; w += NTH) s.bits[w] = 0;
        if (tid == 0) s.bad = 0;
        __syncthreads();
        int bad = 0;
        for (int i = tid; i < P; i += NTH) {
            const uint32_t e = idx[i];
            if (e < (uint32_t)E) {
                atomicAdd(&s.cnt[e], 1);
                atomicOr(&s.bits[e * W1 + (i >> 5)], 1u << (i & 31));
            } else {
                bad++;
            }
        }
        if (bad) atomicAdd(&s.bad, bad);
        __syncthreads();
        if (wv == 0) {
            dispatch_offsets(E, lane, offsets, active, meta, chunks, chunk, n_routed, lo, s);
        } else {
            for (int e = tid - 64; e < E; e += NTH - 64) {
                int run = 0;
                for (int w = 0; w < W1; w++) {
                    s.pre[e * W1 + w] = run;
                    run += __popc(s.bits[e * W1 + w]);
                }
            }
        }
        __syncthreads();
        for (int i = tid; i < P; i += NTH) {
            const uint32_t e = idx[i];
            if (e >= (uint32_t)E) {
                inv[i] = -1;
                continue;
            }
            const int w = e * W1 + (i >> 5);
            const int pos = s.off[e] + s.pre[w] + __popc(s.bits[w] & ((1u << (i & 31)) - 1u));
            rows[pos] = i / k;
            slots[pos] = i % k;
            inv[i] = pos;
        }
        return;
    }
    // larger workgroup calls (P <= kDispBlock entries: launch_dispatch sends more to
    // k_dispatch_multi; the fused route + dispatch takes at most 16 tokens) rank by segments
    static_assert((NTH / 64) * 64 * kSegBatches >= NTH, "the segments take every entry a workgroup is given");
    dispatch_segments<NTH>(idx, P, k, E, offsets, rows, slots, inv, active, meta, chunks, chunk, n_routed, lo, s);
}

// --------------------------------------------------- activation conversion

// x f32 [rows][K] -> the MFMA activation format (common.h) with one power of two
// per row: wavefront w takes row w, finds its largest magnitude, then converts
// it; every group's descale ds[g * ld + row] holds the row's, so the grouped GEMM
// can accumulate a whole row's K in the MFMA.
__device__ __forceinline__ void act_prep_wave(const float *__restrict__ x, int rows, int K, const ActQ &xq, size_t w, int lane)
{
    if (w >= (size_t)rows) return;
    const float *xr = x + w * K;
    const int G = K / 64, R = K / 8;  // 64-column groups, 8-element runs
    half_t *q = xq.q + w * K;
    // Run r (elements 8r .. 8r + 7) of group r / 8 lands at 16 (a & 3) + 8 (a >> 2),
    // a = r % 8, within its group in mma_pos order: eight contiguous halves.  Lane l
    // takes runs l, l + 64, ...: two 16-byte loads and one 16-byte store each, the
    // whole row in registers for K <= 64 kB 8 (one memory round trip).
    constexpr int kB = 8;
    if (R <= 64 * kB) {
        float4 v[kB][2];
        float m = 0.0f;
#pragma unroll
        for (int b = 0; b < kB; b++) {
            const int r = lane + 64 * b;
            if (r < R) {
                v[b][0] = *(const float4 *)(xr + 8 * r);
                v[b][1] = *(const float4 *)(xr + 8 * r + 4);
            } else {
                v[b][0] = v[b][1] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
#pragma unroll
        for (int b = 0; b < kB; b++)
#pragma unroll
            for (int h = 0; h < 2; h++)
                m = fmaxf(m, fmaxf(fmaxf(fabsf(v[b][h].x), fabsf(v[b][h].y)), fmaxf(fabsf(v[b][h].z), fabsf(v[b][h].w))));
        const float sc = pow2_scale(wave_max(m)), inv = 1.0f / sc;
#pragma unroll
        for (int b = 0; b < kB; b++) {
            const int r = lane + 64 * b;
            if (r < R) {
                const int a = r & 7;
                half8 o;
                o[0] = (_Float16)(v[b][0].x * sc); o[1] = (_Float16)(v[b][0].y * sc);
                o[2] = (_Float16)(v[b][0].z * sc); o[3] = (_Float16)(v[b][0].w * sc);
                o[4] = (_Float16)(v[b][1].x * sc); o[5] = (_Float16)(v[b][1].y * sc);
                o[6] = (_Float16)(v[b][1].z * sc); o[7] = (_Float16)(v[b][1].w * sc);
                *(half8 *)(q + 64 * (r >> 3) + 16 * (a & 3) + 8 * (a >> 2)) = o;
            }
        }
        for (int g = lane; g < G; g += 64) xq.ds[(size_t)g * xq.ld + w] = inv;
        return;
    }
    float m = 0.0f;
    for (int g = 0; g < G; g++) m = fmaxf(m, fabsf(xr[64 * g + lane]));
    const float sc = pow2_scale(wave_max(m)), inv = 1.0f / sc;
    for (int g = 0; g < G; g++) {
        q[64 * g + mma_pos(lane)] = (half_t)(xr[64 * g + lane] * sc);
        if (lane == 0) xq.ds[(size_t)g * xq.ld + w] = inv;
    }
}

// ------------------------------------------------------- route launches

struct RouteArgs {
    const float *logits;
    int T, E, k, norm;
    float *probs;
    uint32_t *idx;
    const float *x;  // activations to convert in the same launch (null = none)
    int H;
    ActQ xq;
    int n_route_blocks;
    int kk;              // slots per token row of probs/idx: k routed + n_sh shared pieces
    int n_sh;            // shared expert pieces (experts E .. E+n_sh-1), written by the conversion
    const uint16_t *sh_lin;  // shared gate vector [H] f16, or null (scale 1)
    // With `rwt` (fused route and dispatch only) the routing workgroup forms the
    // logits itself from x: the router in the router kernel's layout (rwt) and as
    // stored (rw).
    const float *rwt;
    const uint16_t *rw;
};

constexpr int kRouteWaves = 4;      // tokens per routing workgroup, one per wavefront
constexpr int kDispThreads = 1024;  // threads of the dispatch workgroup

// Activation row w of the launch's conversion blocks, and the token's shared
// slots: experts E .. E+n_sh-1 with its shared scale, sigmoid(shared_gate_lin . h)
// (main.zig:512-515) or 1 (engine.zig:1170).
__device__ inline void act_row_wave(const RouteArgs &a, size_t w, int lane)
{
    act_prep_wave(a.x, a.T, a.H, a.xq, w, lane);
    if (a.n_sh && w < (size_t)a.T) {
        float s = 1.0f;
        if (a.sh_lin) {
            const float *xr = a.x + w * a.H;
            float g = 0.0f;
            for (int i = lane; i < a.H; i += 64) g += f16_bits_to_f32(a.sh_lin[i]) * xr[i];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) g += __shfl_xor(g, o, 64);
            s = shared_sigmoid(g);
        }
        if (lane < a.n_sh) {
            a.probs[w * a.kk + a.k + lane] = s;
            a.idx[w * a.kk + a.k + lane] = (uint32_t)(a.E + lane);
        }
    }
}

// Blocks [0, n_route_blocks) route kRouteWaves tokens each (one wavefront per
// token, so no SIMD holds more than one routing wavefront of a workgroup); the
// blocks after them convert the activations, one row per wavefront.  The dispatch
// is a launch of its own: handing the ids to one workgroup inside this launch
// (release fence, arrival counter, acquire fence) measured 3.3 us at 64 tokens,
// against 1.3 us for an empty launch.
__global__ __launch_bounds__(256) void k_route(RouteArgs a)
{
    __shared__ __attribute__((aligned(16))) float rows[kRouteWaves][kMaxExperts];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if ((int)blockIdx.x >= a.n_route_blocks) {
        act_row_wave(a, (size_t)(blockIdx.x - a.n_route_blocks) * kRouteWaves + wv, lane);
        return;
    }
    const int t = (int)blockIdx.x * kRouteWaves + wv;
    if (t >= a.T) return;  // no barriers in this kernel
    float v[4];
    route_logits(a.logits, t, a.T, a.E, lane, v);
    exp_table_ready(exp_table_warm(lane));
    route_token(v, t, a.E, a.k, a.kk, a.norm, a.probs, a.idx, lane, c_exp2_tab, rows[wv]);
}

// The router logits of a few tokens inside the routing workgroup (T E 8 <= its
// threads): the tokens' x staged in LDS as k_router stages them (in xs, the
// dispatch's LDS, idle until the routing is done), thread (t, e, l) runs chain l of
// (token t, expert e) -- the same adds in the same order as k_router, so the same
// bits -- and lane 0 of each eight adds the chains in order, then the scalar tail,
// into lg[t][e].  No second launch and no trip of the logits through memory.
__device__ inline void router_chains(const RouteArgs &a, float (*lg)[kMaxExperts], float *xs)
{
    const int J = a.H >> 3, H8 = J * 8, JP = router_stride(J);  // xs: [T][8][JP]
    const int NB = (int)router_blocks(a.H), NBF = J / 8;
    for (int i = threadIdx.x; i < a.T * H8; i += kDispThreads) {
        const int t = i / H8, c = i - t * H8;
        xs[(t * 8 + (c & 7)) * JP + (c >> 3)] = a.x[(size_t)t * a.H + c];
    }
    __syncthreads();
    const int n = a.T * a.E * 8;
    if ((int)(threadIdx.x & ~63u) >= n) return;  // a wavefront with no chain (uniform; the caller's barrier follows)
    const int ch = min((int)threadIdx.x, n - 1);  // lanes past the chains repeat the last (not stored)
    const int t = ch / (a.E * 8), e = (ch >> 3) % a.E, l = ch & 7;
    // chain l of expert e in the router layout: block jb's 8 j's at wr + jb 64 64
    const float *wr = a.rwt + ((size_t)(e / kRouterGroup) * NB * kRouterGroup + e % kRouterGroup) * 64 + 8 * l;
    const size_t bstride = (size_t)kRouterGroup * 64;
    const float *xr = xs + (t * 8 + l) * JP;
    float acc = 0.0f;
    if (NB > 0) {
        // 8 j's per two 16-byte loads, the next block's issued before this one's adds
        float4 c0 = *(const float4 *)wr, c1 = *(const float4 *)(wr + 4);
        auto add = [&](int jb, int nq) {
            const float wf[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
            for (int q = 0; q < 8; q++)
                if (q < nq) acc = __fadd_rn(acc, __fmul_rn(xr[8 * jb + q], wf[q]));
        };
        for (int jb = 0; jb < NBF; jb++) {
            const float *nw = wr + (size_t)min(jb + 1, NB - 1) * bstride;
            const float4 n0 = *(const float4 *)nw, n1 = *(const float4 *)(nw + 4);
            add(jb, 8);
            c0 = n0;
            c1 = n1;
        }
        if (NB > NBF) add(NBF, J - 8 * NBF);
    }
    float sum = __shfl(acc, (threadIdx.x & ~7), 64);
    for (int q = 1; q < 8; q++) sum = __fadd_rn(sum, __shfl(acc, (threadIdx.x & ~7) + q, 64));
    if ((int)threadIdx.x < n && l == 0) {
        const uint16_t *row = a.rw + (size_t)e * a.H;
        for (int i = H8; i < a.H; i++) sum = __fadd_rn(sum, __fmul_rn(f16_bits_to_f32(row[i]), a.x[(size_t)t * a.H + i]));
        lg[t][e] = sum;
    }
}

// Up to kFusedTokens tokens routed and dispatched in one launch.  Block 0's
// wavefront w routes token w; the ids also go to LDS (the shared
// slots' ids are fixed: E + j), and after a barrier the same workgroup dispatches
// them from there, with no trip through memory and no second launch.  The blocks
// after it convert the activations, one row per wavefront.
constexpr int kFusedTokens = 16;
constexpr int kFusedIds = kFusedTokens * (kMaxK + 64);
static_assert(kFusedTokens <= kDispThreads / 64, "one token per wavefront of the fused workgroup");

__global__ __launch_bounds__(kDispThreads) void k_route_dispatch(RouteArgs a, Dispatch d)
{
    constexpr int kW = kDispThreads / 64;
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (blockIdx.x > 0) {
        act_row_wave(a, (size_t)(blockIdx.x - 1) * kW + wv, lane);
        return;
    }
    __shared__ __attribute__((aligned(16))) float rows[kW][kMaxExperts];
    __shared__ uint32_t ids[kFusedIds];
    __shared__ DispLds s;
    if (a.rwt) {
        static_assert(sizeof(DispLds) % 4 == 0 && alignof(DispLds) >= 4, "x staged in the dispatch's LDS");
        router_chains(a, rows, reinterpret_cast<float *>(&s));
        __syncthreads();
    }
    if (wv < a.T) {  // T <= kW: one token per wavefront
        float v[4];
        if (a.rwt) route_logits(rows[wv], 0, 1, a.E, lane, v);
        else route_logits(a.logits, wv, a.T, a.E, lane, v);
        exp_table_ready(exp_table_warm(lane));
        route_token(v, wv, a.E, a.k, a.kk, a.norm, a.probs, a.idx, lane, c_exp2_tab, rows[wv], ids);
    }
    for (int i = threadIdx.x; i < a.T * a.n_sh; i += kDispThreads)
        ids[(i / a.n_sh) * a.kk + a.k + i % a.n_sh] = (uint32_t)(a.E + i % a.n_sh);
    __syncthreads();
    dispatch_block<kDispThreads>(ids, a.T, a.kk, a.E + a.n_sh, d.offsets, d.rows, d.slots, d.inv, d.active, d.meta,
                                 d.chunks, d.chunk, d.n_routed, list_opts(d), s);
}

__global__ __launch_bounds__(kDispThreads) void k_dispatch(const uint32_t *__restrict__ idx, int T, int k, int E,
                                                           Dispatch d)
{
    __shared__ DispLds s;
    dispatch_block<kDispThreads>(idx, T, k, E, d.offsets, d.rows, d.slots, d.inv, d.active, d.meta, d.chunks, d.chunk,
                                 d.n_routed, list_opts(d), s);
}

// Dispatch of more entries than one workgroup ranks at once, by kDispBlock-entry
// blocks, one workgroup each and no communication between them.  Every workgroup
// counts all P entries per expert (the totals give the offsets), apart those of
// the blocks before its own (their sum is its base per expert), and ranks its own
// block's entries the way dispatch_segments does (each wavefront 64 entries,
// same-id lanes found with nine ballots, a prefix over the wavefronts): position =
// offset[e] + entries of e in earlier blocks + earlier in this block.  Workgroup 0
// also writes the offsets, the active experts, the chunk list and meta.  The order
// is the single-workgroup dispatch's: entries ascending within an expert.
//
// The counting: wavefront w takes the batches of 64 entries at 1024 q + 64 w (so
// its batch of this block is the one it ranks), every batch's ids loaded before the
// first barrier (one memory round trip); each entry adds one to its expert in the
// wavefront's own LDS row (before / this / after the block) with one LDS atomic per
// batch, no contention between wavefronts, and the rows are summed per expert
// once.  The nine-ballot match runs on the block's own batch only: on every batch
// it took 6.7 us of the 10.6 us DeepSeek-V2-Lite 1024-token dispatch (8192 entries,
// each workgroup's VALU on one CU).
constexpr int kDispBlock = kDispThreads;  // entries per workgroup: one per thread
constexpr int kDispWaves = kDispThreads / 64;

struct MultiLds {
    int32_t cnt[kMaxExperts];   // all entries of e
    int32_t off[kMaxExperts];   // offsets (dispatch_offsets)
    int32_t base[kMaxExperts];  // entries of e in blocks before this one
    int32_t bef[kDispWaves][kMaxExperts], own[kDispWaves][kMaxExperts], aft[kDispWaves][kMaxExperts];
    int32_t bad;
};

// Lanes of the wavefront holding the same 9-bit id as this lane (ids >= E and
// padding all share 0x1FF, which no expert has).
__device__ inline uint64_t same_id_lanes(uint32_t e)
{
    uint64_t same = ~0ull;
#pragma unroll
    for (int bit = 0; bit < 9; bit++) {
        const bool on = (e >> bit) & 1u;
        const uint64_t bb = __ballot(on);
        same &= on ? bb : ~bb;
    }
    return same;
}

__global__ __launch_bounds__(kDispThreads) void k_dispatch_multi(const uint32_t *__restrict__ idx, int P, int k, int E,
                                                                 Dispatch d)
{
    constexpr int NW = kDispWaves, kB = 8;
    constexpr int kIt = 64 * NW * kB;  // entries per round of batches
    __shared__ MultiLds s;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int blk = blockIdx.x, i0 = blk * kDispBlock;  // this block's first entry
    const uint64_t below_mask = (1ull << lane) - 1ull;
    uint32_t ids[kB];
    auto load = [&](int r) {
#pragma unroll
        for (int q = 0; q < kB; q++) {
            const int j = r + 1024 * q + 64 * wv + lane;
            ids[q] = j < P ? idx[j] : 0x1FFu;
        }
    };
    load(0);
    for (int i = tid; i < NW * kMaxExperts; i += kDispThreads) {
        (&s.bef[0][0])[i] = 0;
        (&s.own[0][0])[i] = 0;
        (&s.aft[0][0])[i] = 0;
    }
    if (tid == 0) s.bad = 0;
    __syncthreads();
    int bad = 0, below = 0;
    uint32_t mine = 0x1FFu;  // this thread's entry of the block (0x1FF: none or id >= E)
    for (int r = 0; r < P; r += kIt) {
        if (r) load(r);
#pragma unroll
        for (int q = 0; q < kB; q++) {
            const int b0 = r + 1024 * q + 64 * wv, bq = b0 >> 10;  // the batch's first entry and its block
            if (b0 >= P) break;  // uniform
            uint32_t x = ids[q];
            if (x >= (uint32_t)E) {
                bad += b0 + lane < P;
                x = 0x1FFu;
            }
            if (bq == blk) {  // this block's batch: ranks within the wavefront
                mine = x;
                below = __popcll(same_id_lanes(x) & below_mask);
            }
            int32_t *row = bq < blk ? s.bef[wv] : bq == blk ? s.own[wv] : s.aft[wv];
            if (x < (uint32_t)E) atomicAdd(&row[x], 1);  // the wavefront's own row
        }
    }
    if (bad) atomicAdd(&s.bad, bad);
    __syncthreads();
    // per expert: the totals, the base, and the wavefronts' exclusive prefix of this
    // block's counts in place
    for (int x = tid; x < E; x += kDispThreads) {
        int b = 0, a = 0, run = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            b += s.bef[w][x];
            a += s.aft[w][x];
            const int v = s.own[w][x];
            s.own[w][x] = run;
            run += v;
        }
        s.base[x] = b;
        s.cnt[x] = b + run + a;
    }
    __syncthreads();
    if (wv == NW - 1) dispatch_offsets(E, lane, d.offsets, d.active, d.meta, d.chunks, d.chunk, d.n_routed, list_opts(d),
                                      s, blk == 0);
    __syncthreads();
    // positions of this block's entries
    const int i = i0 + 64 * wv + lane;
    if (i < P) {
        int pos = -1;
        if (mine < (uint32_t)E) {
            pos = s.off[mine] + s.base[mine] + s.own[wv][mine] + below;
            d.rows[pos] = i / k;
            d.slots[pos] = i % k;
        }
        d.inv[i] = pos;
    }
}

__global__ __launch_bounds__(256) void k_act_prep(const float *__restrict__ x, int rows, int K, ActQ xq)
{
    act_prep_wave(x, rows, K, xq, (size_t)blockIdx.x * 4 + (threadIdx.x >> 6), threadIdx.x & 63);
}

static int check_route_shape(int T, int E, int k)
{
    if (E > kMaxExperts || E <= 0 || k > kMaxK || k > E || k <= 0) {
        set_error("route: unsupported E=%d k=%d (E <= %d, 0 < k <= min(E, %d))", E, k, kMaxExperts, kMaxK);
        return ANEDVD_E_INVALID_ARG;
    }
    if ((long)T * k > (1l << 30)) {
        set_error("route: %d tokens x top-%d is too many entries", T, k);
        return ANEDVD_E_INVALID_ARG;
    }
    return ANEDVD_OK;
}

int launch_route(const float *d_logits, int T, int E, int k, int norm, float *d_probs, uint32_t *d_idx,
                 const float *d_x, int H, const ActQ &xq, hipStream_t st, const SharedSlots &sh)
{
    if (T <= 0) return ANEDVD_OK;
    ANEDVD_TRY(check_route_shape(T, E, k));
    if (d_x && H % 64) {
        set_error("route: hidden %d is not a multiple of 64", H);
        return ANEDVD_E_INVALID_SHAPE;
    }
    if (sh.n && (!d_x || sh.n > 64 || E + sh.n > kMaxExperts)) {
        set_error("route: %d shared pieces need the activations and E + pieces <= %d", sh.n, kMaxExperts);
        return ANEDVD_E_INVALID_ARG;
    }
    RouteArgs a{d_logits, T, E, k, norm, d_probs, d_idx, d_x, H, xq, (T + kRouteWaves - 1) / kRouteWaves,
                k + sh.n, sh.n, sh.lin};
    const size_t waves = d_x ? (size_t)T : 0;  // activation conversion: one wavefront per token
    const unsigned blocks = (unsigned)(a.n_route_blocks + (waves + kRouteWaves - 1) / kRouteWaves);
    hipLaunchKernelGGL(k_route, dim3(blocks), dim3(256), 0, st, a);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

int launch_dispatch(const uint32_t *d_idx, int T, int k, int E, const Dispatch &d, hipStream_t st)
{
    if (T <= 0) return ANEDVD_OK;
    ANEDVD_TRY(check_route_shape(T, E, k));
    const long P = (long)T * k;
    if (P > kDispBlock)
        hipLaunchKernelGGL(k_dispatch_multi, dim3((unsigned)((P + kDispBlock - 1) / kDispBlock)), dim3(kDispThreads), 0,
                           st, d_idx, (int)P, k, E, d);
    else
        hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(kDispThreads), 0, st, d_idx, T, k, E, d);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

bool route_fusable(int T, int)
{
    return T > 0 && T <= kFusedTokens;
}

bool route_router_fusable(int T, int E, int H)
{
    return route_fusable(T, E) && T * E * 8 <= kDispThreads && E <= kMaxExperts &&
           (size_t)T * 8 * router_stride(H >> 3) * 4 <= sizeof(DispLds);
}

int launch_route_and_dispatch(const float *d_logits, int T, int E, int k, int norm, float *d_probs, uint32_t *d_idx,
                              const float *d_x, int H, const ActQ &xq, const Dispatch &d, hipStream_t st,
                              const SharedSlots &sh, const float *d_rwt, const uint16_t *d_rw)
{
    if (!d_logits && (!d_rwt || !d_rw || !d_x || !route_router_fusable(T, E, H))) {
        set_error("route: no logits, and the router cannot be fused into this call (%d tokens, %d experts)", T, E);
        return ANEDVD_E_INVALID_ARG;
    }
    if (!route_fusable(T, E)) {
        ANEDVD_TRY(launch_route(d_logits, T, E, k, norm, d_probs, d_idx, d_x, H, xq, st, sh));
        return launch_dispatch(d_idx, T, k + sh.n, E + sh.n, d, st);
    }
    ANEDVD_TRY(check_route_shape(T, E, k));
    ANEDVD_TRY(check_route_shape(T, E + sh.n, k + sh.n));
    if (d_x && H % 64) {
        set_error("route: hidden %d is not a multiple of 64", H);
        return ANEDVD_E_INVALID_SHAPE;
    }
    if (sh.n && (!d_x || sh.n > 64)) {
        set_error("route: %d shared pieces need the activations and at most 64 pieces", sh.n);
        return ANEDVD_E_INVALID_ARG;
    }
    RouteArgs a{d_logits, T, E, k, norm, d_probs, d_idx, d_x, H, xq, 1, k + sh.n, sh.n, sh.lin, nullptr, nullptr};
    if (!d_logits) {
        a.rwt = d_rwt;
        a.rw = d_rw;
    }
    const unsigned blocks = 1 + (d_x ? (unsigned)((T + kDispThreads / 64 - 1) / (kDispThreads / 64)) : 0u);
    hipLaunchKernelGGL(k_route_dispatch, dim3(blocks), dim3(kDispThreads), 0, st, a, d);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

int launch_act_prep(const float *d_x, int rows, int K, const ActQ &xq, hipStream_t st)
{
    if (rows <= 0) return ANEDVD_OK;
    if (K % 64) {
        set_error("activation conversion: %d columns is not a multiple of 64", K);
        return ANEDVD_E_INVALID_SHAPE;
    }
    hipLaunchKernelGGL(k_act_prep, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, d_x, rows, K, xq);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

}  // namespace anedvd
