// k_pf.hip -- the grouped GEMM for prefill-sized expert groups.
//
// Same math as the decode kernels (cpu.moeExpertAccumF32, cpu.zig:416-452, over
// the gguf.zig block formats), organised for groups of tens to hundreds of tokens:
//   - a workgroup takes 64 or 128 tokens of one expert's group (part of a chunk
//     of the dispatch's work list) and 128 weight rows of both gate and up, or 256
//     rows of down (all of K, or one of two K shares);
//   - the tokens' activations go from memory straight into a four-slot LDS ring
//     (direct-to-LDS loads, three steps ahead), shared by the four wavefronts;
//   - each wavefront dequantises its four 16-row tiles once per 64-column step to
//     f16 (Q8_0, Q4_0: d * q rounded once; Q4_K, Q6_K: the quant exact, the
//     sub-block scale and min as f16, one rounding in the FMA) and runs them
//     against the 16-token tiles, accumulating the whole K inside the MFMA;
//   - activations carry one power of two per row: x as converted, and the SwiGLU
//     activations (a power of two per 64-column group) rescaled in LDS to their
//     row's largest descale before use, so nothing is rescaled inside the K loop;
//   - gate/up: a wavefront holds gate and up of the same 32 rows, so SiLU(g) * u
//     and the activation format's scale form in registers;
//   - groups of at most 16 tokens (skewed routing) run in the same launches, one
//     16-token tile per workgroup, their activations read straight from memory.
#include <type_traits>

#include "common.h"
#include "fq.h"
#include "kernels.h"
#include "mma.h"

namespace anedvd {

// ------------------------------------------------------------ direct-to-LDS staging

// The gate/up activations (x rows gathered through the dispatch, one power of two
// per row, so they need no rescaling) go from memory straight to LDS with
// buffer_load_dwordx4 ... lds: no register ring, so a step's activations are
// requested kXDepth steps ahead.  Four ring slots, one per unrolled step, each its
// own LDS array; a slot holds 16 MT token rows of 128 bytes (the step's 64
// columns), row r's 16-byte piece p at physical piece p ^ x_sw(r), so the MFMA
// operand reads of 8 or 16 consecutive rows hit distinct banks.  The hardware
// writes lane l of such a load at byte 16 l of its 1 KiB destination: a
// wavefront's load fills 8 rows, lane l the physical piece l % 8 of row l / 8.
constexpr int kXDepth = 3;

__device__ inline int x_sw(int r) { return (r & 7) ^ ((r >> 3) & 1); }

typedef __attribute__((address_space(3))) void lds_void;

// A stager issues one step's loads into a ring slot (issue: kIssue vector-memory
// instructions) and, once they are done, fixes up the bytes its own wavefront's
// loads wrote before the barrier that publishes the slot (fix).

// gate/up: x rows (one power of two per row) need no fix.
template <int MT>
struct DmaX {
    static constexpr int kInst = MT / 2;  // loads per wavefront per step: 16 MT rows x 128 B / 4 wavefronts / 1 KiB
    static constexpr int kIssue = kInst;
    static constexpr int kRawCap = 80;  // weight slots up to this size go two steps ahead
    rsrc_t q;
    int off[kInst];  // load i: the lane's token row base + its logical piece (bytes)
    int dst;         // this wavefront's first destination byte in a slot
    __device__ inline void issue(half_t *slot, int s, int)
    {
#if __HIP_DEVICE_COMPILE__  // the compiler's host pass has no LDS-pointer builtins
#pragma unroll
        for (int i = 0; i < kInst; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(q, (lds_void *)((char *)slot + dst + 1024 * i), 16, off[i],
                                                     s * 2 * kStep, 0, 0);
#endif
    }
    __device__ inline void fix(half_t *, int) {}
};

// down: the SwiGLU activations carry a power of two per (position, 64-column
// group) -- one per step.  With the pieces, each wavefront loads its rows'
// descales for the step into its own 64 floats of LDS (lane j the row of piece
// load j / 8, lane j / 8 % ... as the pieces' lanes l / 8), and fix() rescales its
// own 16-byte pieces in place to the row's reference: a power of two <= 1, exact,
// as the register staging did.
template <int MT>
struct DmaAct {
    static constexpr int kInst = MT / 2;
    static constexpr int kIssue = kInst + 1;  // the pieces, then the descales
    // The 80-byte slots (Q8_0, Q5_0, Q5_1) stay one step ahead: two waves per SIMD
    // at 128 tokens, three at 64 (the Q8_0 kernel at 64 tokens: 166 VGPRs against
    // 202 with its weights two steps ahead).
    static constexpr int kRawCap = 72;
    rsrc_t q, ds;
    int off[kInst];     // load i: the lane's position's piece (bytes)
    int doff;           // the descale of row 8 (w kInst + j / 8) + j % 8, j = min(lane, 8 kInst - 1) (bytes)
    int dst, ld4, wv;
    float *dgs;         // LDS [4 slots][4 wavefronts][64]: the loaded descales
    const float *rinv;  // LDS [16 MT]: 1 / each row's reference
    __device__ inline void issue(half_t *slot, int s, int b)
    {
#if __HIP_DEVICE_COMPILE__
#pragma unroll
        for (int i = 0; i < kInst; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(q, (lds_void *)((char *)slot + dst + 1024 * i), 16, off[i],
                                                     s * 2 * kStep, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ds, (lds_void *)(dgs + (b * 4 + wv) * 64), 4, doff, s * ld4, 0, 0);
#endif
    }
    __device__ inline void fix(half_t *slot, int b)
    {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int i = 0; i < kInst; i++) {
            const int j = 8 * i + (lane >> 3);
            const half_t f = (half_t)(dgs[(b * 4 + wv) * 64 + j] * rinv[8 * wv * kInst + j]);
            half8 *p = (half8 *)((char *)slot + dst + 1024 * i + 16 * lane);
            *p = *p * f;
        }
    }
};

// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt at their maxima: no wait).
template <int N>
__device__ inline void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// s_waitcnt lgkmcnt(0) alone.
__device__ inline void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14)); }

// Waits until the activation loads of the next step are done, given what this
// wavefront issued after them: two weight load() calls of at least F::kMinLoads
// instructions each, and c activation steps of X::kIssue loads.  (VMEM loads
// complete in order; counting fewer than were issued only waits longer.)
template <class F, class X>
__device__ inline void x_wait(int c)
{
    constexpr int kI = X::kIssue, kW = F::kMinLoads;
    if (c == 2) wait_vm<2 * kW + 2 * kI>();
    else if (c == 1) wait_vm<2 * kW + kI>();
    else wait_vm<2 * kW>();
}

// The workgroup barrier of the direct-to-LDS loop.  __syncthreads() would wait
// for every load into LDS in flight (its release fence covers them); the loop's
// own vmcnt wait has covered the next step's, and the stager's fix-up writes are
// waited for here.  The acquire fence after it keeps the next step's LDS reads
// below it.
__device__ inline void x_barrier()
{
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    __builtin_amdgcn_sched_barrier(0);
}

// Weight steps in flight ahead in the direct-to-LDS loop.  The compiler's own
// waits for a weight load do not count the activation loads issued after it (it
// treats them as no vector-memory result), so they also wait for whatever of
// those is older than the loads it does count: with the weights two steps ahead
// and issued before each step's activation loads, that is the next step's
// activations, which the barrier needs anyway.
#ifndef ANEDVD_PF_DMA_WD
#define ANEDVD_PF_DMA_WD 2
#endif

// B operands one half-step ahead (decoders whose scales change every step, kSpu
// 1): a step's MFMAs of block j = 0 run while the wavefront dequantises block 1,
// and those of block 1 while it dequantises the next step's block 0, so the
// dequantising VALU work issues in the shadow of the wavefront's own MFMAs
// instead of before them.  Weights then go three steps ahead: the compiler's wait
// for the next step's weights (issued three steps earlier) only covers loads at
// least a step old.
//
// Taken for Q4_0 at 128-token workgroups (Mixtral 2048 tokens, one box, A/B:
// gate/up 910-928 -> 883-887 us, down 622-642 -> 602-609 us; 244 and 256 VGPRs,
// still two wavefronts per SIMD).  Q8_0's larger weight slots would take its
// 128-token down kernel to 289 VGPRs (one wavefront per SIMD) and its gate/up
// kernel is at 256 already.
#ifndef ANEDVD_PF_PIPE
#define ANEDVD_PF_PIPE 1
#endif
template <class F, int MT>
constexpr bool pf_pipe()
{
    return ANEDVD_PF_PIPE && MT == 8 && std::is_same<F, FQ4_0>::value;
}

// The decoder's kUnit for the step at offset v of a four-step block: whether it
// starts a scale unit (kCt), or -1 to leave it to the decoder.
template <class F, bool kCt>
constexpr int pf_unit(int v)
{
    return kCt ? (int)(v % F::kSpu == 0) : -1;
}

// pf_loop with the activations in the direct-to-LDS ring (steps [s0w, s0w + steps)
// of the weights; the stager's offsets already point at step s0w).  Per step s the
// wavefront issues the weight loads of step s + D, then the activation loads of
// step s + 3; before the barrier that ends step s it waits for step s + 1's
// activation loads, issued two steps earlier: younger than them are the weight
// loads issued at steps s - 1 and s and the activation loads of steps s + 2 and
// s + 3 that exist.  The slot step s + 4 will fill is the one step s reads, free
// after that barrier.
template <class F, int MT, int MTL, bool kPeel, class TS, class X>
__device__ inline void pf_loop_dma(const TS &W, int rb, int s0w, int steps, int lane, X &x, half_t *xs0,
                                   half_t *xs1, half_t *xs2, half_t *xs3, f32x4 (*acc)[MT])
{
    constexpr int U = 4, DA = kXDepth;
    static_assert(U % F::kSpu == 0, "a scale unit must fit an unrolled block");
    // (larger weight slots stay one step ahead: two more of them would not fit)
    constexpr bool kP = pf_pipe<F, MT>();
    // Whether a step starts a scale unit is known here at compile time (blocks of
    // four steps from a multiple of four).  The down kernels pass it to the decoder,
    // so only the slot that holds a unit's first step carries its scales: the Q6_K
    // kernel's 52-byte-per-lane spill went, and the Qwen3 Q4_K_M 512-token down
    // launch took 53-56 us against 63.  The gate/up kernels leave it to the decoder
    // (the Q4_K kernel spilled more with it: 77 against 69 us).
    constexpr bool kCtUnit = !std::is_same<X, DmaX<MT>>::value;
    static_assert(!kP || F::kSpu == 1, "B operands ahead only where every step has its own scales");
    constexpr int DW = sizeof(typename F::Raw) <= X::kRawCap ? ANEDVD_PF_DMA_WD : 1;
    constexpr int D = kP ? 3 : F::kDepth > DW ? F::kDepth : DW;
    constexpr int R = D == 1 ? 2 : 4;
    static_assert(D >= 1 && D <= 3, "at most three steps ahead");
    const int n = lane & 15, g = lane >> 4;
    const int so = (W.src(0).nrb - rb) * W.src(0).steps;
    auto ws = [&](int v) { return v < steps ? s0w + v : so; };  // weights of step v of this K share
    auto slot = [&](int b) { return b == 0 ? xs0 : b == 1 ? xs1 : b == 2 ? xs2 : xs3; };  // b a constant
    typename F::Raw w[R];
    typename F::State st;
    // the steady state's order: weights of v + D, activations of v + DA (v = -DA .. -1)
    if constexpr (kCtUnit) {
        auto pro = [&](auto ic) {
            constexpr int v = decltype(ic)::value - DA;
            if constexpr (v + D >= 0) F::template load<pf_unit<F, true>(v + D)>(w[(v + D) % R], W, rb, ws(v + D), lane);
            if (v + DA < steps) x.issue(slot((v + DA) & 3), v + DA, (v + DA) & 3);
        };
        static_assert(DA == 3, "the prologue issues three steps");
        pro(std::integral_constant<int, 0>{});
        pro(std::integral_constant<int, 1>{});
        pro(std::integral_constant<int, 2>{});
    } else {
#pragma unroll
        for (int v = -DA; v < 0; v++) {
            if (v + D >= 0) F::load(w[(v + D) % R], W, rb, ws(v + D), lane);
            if (v + DA < steps) x.issue(slot((v + DA) & 3), v + DA, (v + DA) & 3);
        }
    }
    // step 0's activations: younger than them are the weight loads of the
    // virtual steps -2 and -1 that exist (min(D, 2) calls) and the activation
    // loads of steps 1 and 2 (not counted: only stricter)
    wait_vm<(D >= 2 ? 2 : 1) * F::kMinLoads>();
    x.fix(slot(0), 0);
    x_barrier();
    // the lane's operand offsets in a slot (halves): row n of a token tile, piece 2 g + j
    const int ao0 = n * 64 + (((2 * g) ^ x_sw(n)) << 3), ao1 = n * 64 + (((2 * g + 1) ^ x_sw(n)) << 3);
    half8 bc[kPfTiles], bn[kPfTiles];  // with kP: block 0 of the current step, block 1
    if constexpr (kP) {
#pragma unroll
        for (int tt = 0; tt < kPfTiles; tt++) bc[tt] = F::bop(w[0], st, 0, tt, 0, lane);
    }
    // Step s = s0 + k of an unrolled block (k a constant).  With kPeel, the blocks
    // whose steps all lie DA or more before the end (kTail false) issue every
    // prefetch unguarded with constant wait counts, and only the remaining blocks
    // keep the guards.  (The gate/up kernels peel: Qwen3 Q4_K_M 512-token gate/up
    // 74 -> 69 us.  The down kernels do not: their register pressure rose with it,
    // the Q6_K kernel's spill from 36 to 112 bytes per lane and the 128-token Q8_0
    // kernel's registers from 226 to 274, and they ran slower.)
    auto step = [&](auto kc, auto tailc, int s0) {
        constexpr int k = decltype(kc)::value;
        constexpr bool kTail = decltype(tailc)::value;
        const int s = s0 + k;
        F::template load<pf_unit<F, kCtUnit>(k + D)>(w[(k + D) % R], W, rb, kTail ? ws(s + D) : s0w + s + D, lane);
        if (!kTail || s + DA < steps) x.issue(slot((k + DA) & 3), s + DA, (k + DA) & 3);
        __builtin_amdgcn_sched_barrier(0);
        const int ss = k % F::kSpu;
        const half_t *a = slot(k);
        F::begin(w[k % R], st, ss, lane);
        if constexpr (kP) {
            // block 0 against bc while block 1 is dequantised into bn, then block 1
            // against bn while the next step's block 0 is dequantised into bc
            // (tile t's operand after token tile group mt = (t + 1) G - 1, G = max(MTL / 4, 1))
            constexpr int G = MTL >= 2 * kPfTiles ? MTL / kPfTiles : 1;
            const bool nxt = !kTail || s + 1 < steps;  // uniform
            // Each token tile's A fragment is read two groups ahead of its MFMAs
            // (fragment i: tile i % MTL of block i / MTL); scheduling barriers keep
            // every group's reads, MFMAs and dequantisation in their own region, so
            // the reads stay ahead and the VALU work shares a region with MFMAs.
            auto afrag = [&](int i) { return *(const half8 *)(a + (i % MTL) * 16 * 64 + (i < MTL ? ao0 : ao1)); };
            half8 p0 = afrag(0), p1 = afrag(1);
#pragma unroll
            for (int i = 0; i < 2 * MTL; i++) {
                const int j = i / MTL, mt = i % MTL;
                const half8 cur = p0;
                p0 = p1;
                if (i + 2 < 2 * MTL) p1 = afrag(i + 2);
#pragma unroll
                for (int tt = 0; tt < kPfTiles; tt++)
                    acc[tt][mt] = mfma(cur, j ? bn[tt] : bc[tt], acc[tt][mt]);
                if (mt % G == G - 1 && mt / G < kPfTiles) {
                    if (j == 0) bn[mt / G] = F::bop(w[k % R], st, ss, mt / G, 1, lane);
                    else if (nxt) bc[mt / G] = F::bop(w[(k + 1) % R], st, 0, mt / G, 0, lane);
                }
                if (mt == MTL - 1) {  // operands the groups did not reach (MTL < 4)
#pragma unroll
                    for (int tt = MTL / G; tt < kPfTiles; tt++) {
                        if (j == 0) bn[tt] = F::bop(w[k % R], st, ss, tt, 1, lane);
                        else if (nxt) bc[tt] = F::bop(w[(k + 1) % R], st, 0, tt, 0, lane);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
        half8 av[2][MT];
        if constexpr (F::kHoistA) {
#pragma unroll
            for (int mt = 0; mt < MTL; mt++) {
                av[0][mt] = *(const half8 *)(a + mt * 16 * 64 + ao0);
                av[1][mt] = *(const half8 *)(a + mt * 16 * 64 + ao1);
            }
        }
#pragma unroll
        for (int j = 0; j < 2; j++) {
            half8 b[kPfTiles];
#pragma unroll
            for (int tt = 0; tt < kPfTiles; tt++) b[tt] = F::bop(w[k % R], st, ss, tt, j, lane);
#pragma unroll
            for (int mt = 0; mt < MTL; mt++) {
                if constexpr (!F::kHoistA) av[j][mt] = *(const half8 *)(a + mt * 16 * 64 + (j ? ao1 : ao0));
#pragma unroll
                for (int tt = 0; tt < kPfTiles; tt++) acc[tt][mt] = mfma(av[j][mt], b[tt], acc[tt][mt]);
            }
        }
        }
        if constexpr (!kTail) {
            x_wait<F, X>(2);
            x.fix(slot((k + 1) & 3), (k + 1) & 3);
            x_barrier();
        } else if (s + 1 < steps) {
            x_wait<F, X>((s + 2 < steps) + (s + 3 < steps));
            x.fix(slot((k + 1) & 3), (k + 1) & 3);
            x_barrier();
        }
    };
    using C0 = std::integral_constant<int, 0>;
    using C1 = std::integral_constant<int, 1>;
    using C2 = std::integral_constant<int, 2>;
    using C3 = std::integral_constant<int, 3>;
    static_assert(U == 4, "the blocks below unroll four steps");
    int s0 = 0;
    if constexpr (kPeel)
        for (; s0 + U + DA - 1 < steps; s0 += U) {
            step(C0{}, std::false_type{}, s0);
            step(C1{}, std::false_type{}, s0);
            step(C2{}, std::false_type{}, s0);
            step(C3{}, std::false_type{}, s0);
        }
    for (; s0 < steps; s0 += U) {
        step(C0{}, std::true_type{}, s0);
        if (s0 + 1 < steps) step(C1{}, std::true_type{}, s0);  // uniform
        if (s0 + 2 < steps) step(C2{}, std::true_type{}, s0);
        if (s0 + 3 < steps) step(C3{}, std::true_type{}, s0);
    }
}

// ------------------------------------------------------------ small groups
//
// A group of at most 16 tokens is one 16-token tile: its workgroup would stage a
// mostly empty ring and wait at a barrier every step for it.  Its wavefronts read
// their activation fragments straight from memory instead (L2 hits: the rows are
// shared by the workgroups of every row group), like the weights, two steps ahead
// in registers, with no LDS and no barrier in the K loop.  The weights go through
// the same decoders as the grouped GEMM (each step dequantised once, scales folded
// into the f16 weights), so a small group costs the same dequantisation as one
// grouped chunk and none of the decode kernels' per-block f32 rescaling.

// gate/up: the lane's token row of x (one power of two per row, no rescale).
struct DirX {
    struct Frag {
        u32x4 v[2];
    };
    rsrc_t q;
    int off;  // the lane's token row + its 32-byte piece of a 64-column step (bytes)
    __device__ inline void load(Frag &f, int s) const
    {
        f.v[0] = __builtin_amdgcn_raw_buffer_load_b128(q, off, s * 2 * kStep, 0);
        f.v[1] = __builtin_amdgcn_raw_buffer_load_b128(q, off + 16, s * 2 * kStep, 0);
    }
    __device__ inline void prep(const Frag &f, half8 *av) const
    {
        av[0] = as_h8(f.v[0]);
        av[1] = as_h8(f.v[1]);
    }
};

// down: the SwiGLU activations of the lane's position carry a power of two per
// 64-column group (one per step); each step's fragments are rescaled to the row's
// reference (the largest descale, so the factor is a power of two <= 1, exact) and
// the result is multiplied by the reference once at the end, as the ring does.
struct DirAct {
    struct Frag {
        u32x4 v[2];
        float d;
    };
    rsrc_t q, ds;
    int off, doff, ld4;
    float rinv;
    __device__ inline void load(Frag &f, int s) const
    {
        f.v[0] = __builtin_amdgcn_raw_buffer_load_b128(q, off, s * 2 * kStep, 0);
        f.v[1] = __builtin_amdgcn_raw_buffer_load_b128(q, off + 16, s * 2 * kStep, 0);
        f.d = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ds, doff, s * ld4, 0));
    }
    __device__ inline void prep(const Frag &f, half8 *av) const
    {
        const half_t k = (half_t)(f.d * rinv);
        av[0] = as_h8(f.v[0]) * k;
        av[1] = as_h8(f.v[1]) * k;
    }
};

// Steps [0, steps) of the wavefront's four tiles against one 16-token tile whose
// activation fragments come from `as`: weights and activations two steps ahead in
// a four-register ring (the same unconditional loads as pf_loop_dma: weights past
// the last step read 0 out of range, activations repeat the last step).
template <class F, class TS, class AS>
__device__ inline void pf_loop_direct(const TS &W, int rb, int steps, int lane, const AS &as, f32x4 (*acc)[1])
{
    constexpr int U = 4, D = 2, R = 4;
    static_assert(U % F::kSpu == 0, "a scale unit must fit an unrolled block");
    const int so = (W.src(0).nrb - rb) * W.src(0).steps;
    auto ws = [&](int v) { return v < steps ? v : so; };
    typename F::Raw w[R];
    typename F::State st;
    typename AS::Frag xa[R];
#pragma unroll
    for (int v = 0; v < D; v++) {
        F::load(w[v], W, rb, ws(v), lane);
        as.load(xa[v], min(v, steps - 1));
    }
    for (int s0 = 0; s0 < steps; s0 += U) {
#pragma unroll
        for (int k = 0; k < U; k++) {
            const int s = s0 + k;
            if (s >= steps) break;  // uniform
            F::load(w[(k + D) % R], W, rb, ws(s + D), lane);
            as.load(xa[(k + D) % R], min(s + D, steps - 1));
            __builtin_amdgcn_sched_barrier(0);
            const int ss = k % F::kSpu;
            F::begin(w[k % R], st, ss, lane);
            half8 av[2];
            as.prep(xa[k % R], av);
#pragma unroll
            for (int j = 0; j < 2; j++) {
                half8 b[kPfTiles];
#pragma unroll
                for (int tt = 0; tt < kPfTiles; tt++) b[tt] = F::bop(w[k % R], st, ss, tt, j, lane);
#pragma unroll
                for (int tt = 0; tt < kPfTiles; tt++) acc[tt][0] = mfma(av[j], b[tt], acc[tt][0]);
            }
        }
    }
}

template <class F, int MT, bool kPeel, int L = MT, class TS, class X>
__device__ inline void pf_loop_dma_live(const TS &W, int rb, int s0w, int steps, int lane, X &x, half_t *xs0,
                                        half_t *xs1, half_t *xs2, half_t *xs3, int mt_live, f32x4 (*acc)[MT])
{
    if constexpr (L > 1) {
        if (mt_live < L) {
            pf_loop_dma_live<F, MT, kPeel, L - 1>(W, rb, s0w, steps, lane, x, xs0, xs1, xs2, xs3, mt_live, acc);
            return;
        }
    }
    pf_loop_dma<F, MT, L, kPeel>(W, rb, s0w, steps, lane, x, xs0, xs1, xs2, xs3, acc);
}

struct PfArgs {
    QMat w0, w1;  // gate, up (or down in w0)
    ActQ x;       // gate/up input (tokens) or down input (positions)
    Dispatch d;
    ActQ act;     // gate/up output
    float *ypart; // down output [P][H], rows in (token, slot) order
    int H, I, P, nchunk, use_gelu;
    int kk;       // slots per token row of ypart
    int sub;      // workgroups per work-list chunk: d.chunk / (16 MT)
    int ks;       // down: K shares (planes of ypart)
    int contig;   // pf_item's order: 0 round robin, 1 contiguous XCD ranges, 2 rows split over the XCDs
    int nsmall;   // capacity of the small groups' list (d.chunks_s): workgroups per row group after the grouped ones
};

// Workgroup order.  The hardware deals workgroups to the 8 XCDs round robin
// (workgroup b to XCD b % 8), each with its own L2; the nw work items (chunk
// parts) are padded to nw8, a multiple of 8, so a work item's row groups all run
// on one XCD and share its activations there.  With `contig` (experts averaging
// two or more chunks) each XCD takes a contiguous range of work items, so the
// consecutive chunks of one expert also share its weight slices in one L2
// (Mixtral 2048 tokens: fabric reads of the gate/up launch 2.58 -> 2.24 GB,
// 1197 -> 1121 us).  With one work item per chunk, the ranges are the dispatch's
// (xr): whole experts per XCD where each fits a range, so no expert's slices are
// read by two L2s (gate/up fabric reads 2.13 -> 1.63 GB, 984 -> 946 us).
// Otherwise work items go round robin, which spreads unequal groups evenly over
// the XCDs (contiguous ranges measured 23 % slower on the Zipf-routed Qwen3
// 512-token prefill); with two work items per chunk (sub 2, nw8 then a multiple of
// 16) the round robin deals chunks, so both halves of a chunk run on one XCD and
// read the expert's slice through one L2.
// With contig 2 (contiguous order whose R row groups -- times K shares -- divide
// by 8) the rows are split over the XCDs instead: XCD x takes rest values
// [x R/8, (x + 1) R/8) of every work item, item-major, so every XCD gets the same
// work however unequal the experts' groups are, each weight row is still read by
// one XCD (the chunks of an expert, consecutive in the list, share it in that L2),
// and each chunk's activations are read by all 8 at about the same time.
__device__ inline void pf_item(const Dispatch &d, int sub, int b, int nw8, int contig, int R, int &w, int &rest)
{
    if (contig == 2) {
        const int rx = R >> 3, x = b & 7, j = b >> 3;
        w = j / rx;
        rest = x * rx + j % rx;
    } else if (contig) {
        const int per = nw8 >> 3, x = b & 7, j = b >> 3;
        rest = j / per;
        if (sub == 1 && d.xper == per) {  // the dispatch's XCD ranges: whole experts where they fit
            const int lo = d.xr[x], hi = d.xr[x + 1];
            w = lo + j % per;
            if (w >= hi) w = 1 << 30;  // past this range: nothing
        } else {
            w = x * per + j % per;
        }
    } else if (sub == 2) {
        const int i = b % nw8, x = i & 7, q = i >> 3;
        w = 16 * (q >> 1) + 2 * x + (q & 1);
        rest = b / nw8;
    } else {
        w = b % nw8;
        rest = b / nw8;
    }
}

// Work items nw padded for pf_item: a multiple of 8, of 16 with two per chunk.
__host__ __device__ inline int pf_nw8(int nw, int sub) { return sub == 2 ? (nw + 15) & ~15 : (nw + 7) & ~7; }

// Split the rows over the XCDs (pf_item's contig 2) where a contiguous order's
// row groups allow it.
#ifndef ANEDVD_PF_RSPLIT
#define ANEDVD_PF_RSPLIT 1
#endif

// Work item w of the grid's nchunk * sub: part w % sub (16 MT tokens) of the
// work-list chunk w / sub.  False past the list's end or the chunk's tokens.
template <int MT>
__device__ inline bool pf_chunk(const Dispatch &d, int w, int sub, int &e, int &p0, int &nt)
{
    const int ci = w / sub, part = w - ci * sub;
    const int n = d.meta[3];
    const uint64_t c = d.chunks[ci];  // ci < the list's capacity: loaded beside the count
    if (ci >= n) return false;
    e = (int)(c & 0xFFu);
    nt = (int)((c >> 8) & 0xFFu) - 16 * MT * part;
    p0 = (int)(c >> 16) + 16 * MT * part;
    if (nt <= 0) return false;
    nt = min(nt, 16 * MT);
    return true;
}

// ------------------------------------------------------------ gate / up

// The gate/up epilogue of a workgroup's 16 MT tokens (positions p0 .. p0 + nt - 1):
// act = SiLU(g dv) * (u dv) over the gate accumulators (token tiles past the
// chunk's live ones hold zeros, and stay zero), a power of two per (token,
// 64-column group) from the wavefront pair's largest magnitudes (met in LDS:
// gmax[wv][m], 16 MT floats per wavefront), f16 pairs stored.  tdv: thread m's
// token descale (m < 16 MT); dvs: LDS [16 MT].
template <int MT>
__device__ inline void pf_gu_epilogue(const PfArgs &a, f32x4 (*acc)[MT], int p0, int nt, int rb, int t0, int wv,
                                      int lane, float tdv, float *dvs, float *gmax)
{
    const int n = lane & 15, g = lane >> 4;
    if ((int)threadIdx.x < 16 * MT) dvs[threadIdx.x] = tdv;
    __syncthreads();
    // the activation choice is uniform, taken once outside the unrolled loops
    auto act_pass = [&](auto gelu) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = 16 * mt + 4 * g + i;
                const float dv = dvs[m];
                float mx = 0.0f;
#pragma unroll
                for (int tp = 0; tp < 2; tp++) {
                    const float v = gate_act(acc[tp][mt][i] * dv, decltype(gelu)::value) * (acc[2 + tp][mt][i] * dv);
                    acc[tp][mt][i] = v;
                    mx = fmaxf(mx, fabsf(v));
                }
                mx = row_max_f32(mx);
                if (n == 0) gmax[wv * 16 * MT + m] = mx;
            }
    };
    if (a.use_gelu) act_pass(std::true_type{});
    else act_pass(std::false_type{});
    __syncthreads();
    // Lane n even stores the f16 pair of columns (n, n + 1), adjacent in the
    // activation format, through a buffer descriptor: the token row's offset is
    // scalar, the lane's row and column offset fixed.
    const bool even = (n & 1) == 0;
    const rsrc_t aq = make_rsrc(a.act.q, (size_t)a.P * a.I * 2);
    const rsrc_t ads = make_rsrc(a.act.ds, (size_t)(a.I / kStep) * a.act.ld * 4);
    const int lrow = 4 * g * a.I * 2;
    const int col[2] = {2 * (kStep * rb + mma_pos(16 * t0 + n)), 2 * (kStep * rb + mma_pos(16 * (t0 + 1) + n))};
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = 16 * mt + 4 * g + i;
            const float sc = pow2_scale(fmaxf(gmax[wv * 16 * MT + m], gmax[(wv ^ 1) * 16 * MT + m]));
            const int srow = (p0 + 16 * mt + i) * a.I * 2;  // uniform
#pragma unroll
            for (int tp = 0; tp < 2; tp++) {
                const float v = acc[tp][mt][i] * sc;
                const float vn = dpp_f32<0xB1>(v);  // quad_perm [1,0,3,2]: lane n ^ 1's value
                if (m < nt && even) {
                    const h2 pr = {(half_t)v, (half_t)vn};
                    __builtin_amdgcn_raw_buffer_store_b32(h2_bits(pr), aq, lrow + col[tp], srow, 0);
                }
            }
            if (m < nt && t0 == 0 && n == 0)
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(pow2_recip(sc)), ads, 16 * g,
                                                      (rb * a.act.ld + p0 + 16 * mt + i) * 4, 0);
        }
}

// Workgroup b of a small group's part of the gate/up grid: group b % nsmall of
// the small list, row-block pair b / nsmall, the grouped kernel's wavefront
// mapping (gate and up of the same 32 rows per wavefront) on one 16-token tile.
template <class F>
__device__ inline void pf_small_gateup(const PfArgs &a, int b, float *dvs, float *gmax)
{
    const int item = b % a.nsmall, rbg = b / a.nsmall;
    const uint64_t c = a.d.chunks_s[item];  // item < the list's capacity: loaded beside the count
    if (item >= a.d.meta[7]) return;        // uniform over the workgroup
    const int e = (int)(c & 0xFFu), nt = (int)((c >> 8) & 0xFFu), p0 = (int)(c >> 16);
    const int wv = wave_id(), lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const int t0 = 2 * (wv & 1), rb = 2 * rbg + (wv >> 1);
    const Tiles2 W{planes(a.w0, e), planes(a.w1, e), t0};
    f32x4 acc[kPfTiles][1];
#pragma unroll
    for (int tt = 0; tt < kPfTiles; tt++) acc[tt][0] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    const float tdv = (int)threadIdx.x < 16 ? a.x.ds[a.d.rows[p0 + min((int)threadIdx.x, nt - 1)]] : 0.0f;
    DirX xs;
    xs.q = make_rsrc(a.x.q, (size_t)a.x.ld * a.H * 2);
    xs.off = a.d.rows[p0 + min(n, nt - 1)] * a.H * 2 + 32 * g;
    pf_loop_direct<F>(W, rb, a.H / kStep, lane, xs, acc);
    pf_gu_epilogue<1>(a, acc, p0, nt, rb, t0, wv, lane, tdv, dvs, gmax);
}

// Grid nw8 * I/128 workgroups of 256 threads (pf_item's order), then nsmall * I/128
// for the small groups.  Wave w: tiles t0 = 2 (w & 1) and t0 + 1 of both gate and
// up of row block 2 x + (w >> 1), x the workgroup's row-block pair, so SiLU(g) * u
// forms in registers.  A token's 64-column activation group (one row block) is
// split over the wavefront pair (w, w ^ 1): each takes its 32 columns' largest
// magnitude (in-lane over two tiles, DPP over the 16 lanes of a row), the pair
// meets in LDS, and each writes its 32 columns scaled by the group's power of two.
// Three wavefronts per SIMD where the decoder fits them without spilling (Q4_K at
// 64-token workgroups: 170 -> 168 VGPRs), else the compiler's choice.
template <class F, int MT>
constexpr int pf_gu_waves()
{
    return std::is_same<F, FQ4_K>::value && MT == 4 ? 3 : 1;
}

template <class F, int MT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(pf_gu_waves<F, MT>()))) void k_pf_gateup(PfArgs a)
{
    __shared__ float dvs[16 * MT];
    __shared__ float gmax[4][16 * MT];  // per wavefront: its 32 columns' largest |act| per token
    int e, p0, nt, w, rbg;
    const int nw = a.nchunk * a.sub;
    if constexpr (MT == 4) {
        const int nbig = pf_nw8(nw, a.sub) * (a.I / (2 * kRowBlock));
        if ((int)blockIdx.x >= nbig) {
            pf_small_gateup<F>(a, (int)blockIdx.x - nbig, dvs, &gmax[0][0]);
            return;
        }
    }
    pf_item(a.d, a.sub, (int)blockIdx.x, pf_nw8(nw, a.sub), a.contig, a.I / (2 * kRowBlock), w, rbg);
    if (w >= nw || !pf_chunk<MT>(a.d, w, a.sub, e, p0, nt)) return;  // uniform over the workgroup
    const int wv = wave_id(), lane = threadIdx.x & 63;
    const int t0 = 2 * (wv & 1), rb = 2 * rbg + (wv >> 1);
    const Tiles2 W{planes(a.w0, e), planes(a.w1, e), t0};
    f32x4 acc[kPfTiles][MT];  // [0, 1]: gate tiles t0, t0 + 1; [2, 3]: up
#pragma unroll
    for (int tt = 0; tt < kPfTiles; tt++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[tt][mt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    // token m's descale for the epilogue, loaded by thread m before the K loop
    const float tdv = (int)threadIdx.x < 16 * MT ? a.x.ds[a.d.rows[p0 + min((int)threadIdx.x, nt - 1)]] : 0.0f;
    const int mt_live = __builtin_amdgcn_readfirstlane((nt + 15) / 16);
    __shared__ __attribute__((aligned(1024))) half_t xs0[16 * MT * 64], xs1[16 * MT * 64], xs2[16 * MT * 64],
        xs3[16 * MT * 64];
    DmaX<MT> xd;
    xd.q = make_rsrc(a.x.q, (size_t)a.x.ld * a.H * 2);
    xd.dst = wv * DmaX<MT>::kInst * 1024;
#pragma unroll
    for (int i = 0; i < DmaX<MT>::kInst; i++) {
        const int row = 8 * (wv * DmaX<MT>::kInst + i) + (lane >> 3);
        xd.off[i] = a.d.rows[p0 + min(row, nt - 1)] * a.H * 2 + 16 * ((lane & 7) ^ x_sw(row));
    }
    pf_loop_dma_live<F, MT, true>(W, rb, 0, a.H / kStep, lane, xd, xs0, xs1, xs2, xs3, mt_live, acc);
    pf_gu_epilogue<MT>(a, acc, p0, nt, rb, t0, wv, lane, tdv, dvs, &gmax[0][0]);
}

// ---------------------------------------------------------------- down

// Three wavefronts per SIMD for the down decoder built for them (FQ6_KDown),
// else the compiler's choice.
template <class F, int MT>
constexpr int pf_dn_waves()
{
    return std::is_same<F, FQ6_KDown>::value ? 3 : 1;
}

// Workgroup b of a small group's part of the down grid (K not split): group
// b % nsmall of the small list, row-block group b / nsmall (wave w: row block
// 4 (b / nsmall) + w), one 16-position tile; the positions' row references found
// as the grouped kernel does (ref, orow, red: LDS of 16, 16 and 256 entries).
template <class F>
__device__ inline void pf_small_down(const PfArgs &a, int b, float *ref, int *orow, float *red)
{
    const int item = b % a.nsmall, rbg = b / a.nsmall;
    const uint64_t c = a.d.chunks_s[item];  // item < the list's capacity: loaded beside the count
    if (item >= a.d.meta[7]) return;        // uniform over the workgroup
    const int e = (int)(c & 0xFFu), nt = (int)((c >> 8) & 0xFFu), p0 = (int)(c >> 16);
    const int wv = wave_id(), lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const int rb = 4 * rbg + wv;
    const int G = a.I / kStep, ld = a.x.ld;
    {
        // thread (part, m): every 16th group of position m; the 16 partial maxima meet in LDS
        const int m = threadIdx.x & 15, part = threadIdx.x >> 4;
        const int pr = min(p0 + m, a.P - 1);
        if (part == 0) orow[m] = a.d.rows[pr] * a.kk + a.d.slots[pr];
        float mx = 0.0f;
        for (int g0 = part; g0 < G; g0 += 16) mx = fmaxf(mx, a.x.ds[(size_t)g0 * ld + pr]);
        red[part * 16 + m] = mx;
        __syncthreads();
        if (part == 0) {
            float r = red[m];
#pragma unroll
            for (int i = 1; i < 16; i++) r = fmaxf(r, red[i * 16 + m]);
            ref[m] = r;
        }
        __syncthreads();
    }
    f32x4 acc[kPfTiles][1];
#pragma unroll
    for (int tt = 0; tt < kPfTiles; tt++) acc[tt][0] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    const int pn = min(p0 + n, a.P - 1);  // the lane's position
    DirAct xs;
    xs.q = make_rsrc(a.x.q, (size_t)a.P * a.I * 2);
    xs.ds = make_rsrc(a.x.ds, (size_t)G * ld * 4);
    xs.off = pn * a.I * 2 + 32 * g;
    xs.doff = pn * 4;
    xs.ld4 = ld * 4;
    xs.rinv = 1.0f / ref[n];
    pf_loop_direct<F>(Tiles1{planes(a.w0, e)}, rb, G, lane, xs, acc);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int m = 4 * g + i;
        if (m < nt) {
            float *yp = a.ypart + (size_t)orow[m] * a.H + (size_t)kRowBlock * rb + n;
#pragma unroll
            for (int tt = 0; tt < kPfTiles; tt++) yp[16 * tt] = acc[tt][0][i] * ref[m];
        }
    }
}

// Grid nw8 * H/256 * ks workgroups of 256 threads (pf_item's order), then
// nsmall * H/256 for the small groups (ks = 1).  Wave w: row block 4 x + w, K share
// kq.  Before the K loop the workgroup finds each position's largest descale
// over the I/64 groups (the row reference); staging scales every group to it, and
// the results are multiplied by it once at the end.  Positions past the group's
// end are computed on the next group's (or, past the last position, the last
// position's) activations and not stored.
template <class F, int MT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(pf_dn_waves<F, MT>()))) void k_pf_down(PfArgs a)
{
    __shared__ float ref[16 * MT];
    __shared__ int orow[16 * MT];  // output rows of the chunk's positions, (token, slot) order
    __shared__ float ref4[256 / (16 * MT)][16 * MT];
    int e, p0, nt, w, rest;
    const int nw = a.nchunk * a.sub;
    if constexpr (MT == 4) {
        const int nbig = pf_nw8(nw, a.sub) * (a.H / (4 * kRowBlock)) * a.ks;
        if ((int)blockIdx.x >= nbig) {
            pf_small_down<F>(a, (int)blockIdx.x - nbig, ref, orow, &ref4[0][0]);
            return;
        }
    }
    pf_item(a.d, a.sub, (int)blockIdx.x, pf_nw8(nw, a.sub), a.contig, a.H / (4 * kRowBlock) * a.ks, w, rest);
    if (w >= nw || !pf_chunk<MT>(a.d, w, a.sub, e, p0, nt)) return;
    const int rbg = rest / a.ks, kq = rest - rbg * a.ks;
    const int wv = wave_id(), lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const int rb = 4 * rbg + wv;
    const int ksteps = a.I / kStep / a.ks, s0 = kq * ksteps;  // this workgroup's K share
    const Tiles1 W{planes(a.w0, e)};
    const int G = a.I / kStep, ld = a.x.ld;
    {
        // the row references: thread (part, m) takes every NP-th group of position m,
        // eight loads in flight at a time, and the NP partial maxima meet in LDS
        constexpr int NP = 256 / (16 * MT);
        static_assert(NP * 16 * MT == 256, "a whole number of threads per chunk position");
        const int m = threadIdx.x % (16 * MT), part = threadIdx.x / (16 * MT);
        const int pr = min(p0 + m, a.P - 1);
        if (part == 0) orow[m] = a.d.rows[pr] * a.kk + a.d.slots[pr];
        float mx = 0.0f;
        for (int g0 = part; g0 < G; g0 += NP * 8) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = g0 + NP * i < G ? a.x.ds[(size_t)(g0 + NP * i) * ld + pr] : 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) mx = fmaxf(mx, v[i]);
        }
        ref4[part][m] = mx;
        __syncthreads();
        if (part == 0) {
            float r = ref4[0][m];
#pragma unroll
            for (int i = 1; i < NP; i++) r = fmaxf(r, ref4[i][m]);
            ref[m] = r;
        }
        __syncthreads();
    }
    f32x4 acc[kPfTiles][MT];
#pragma unroll
    for (int tt = 0; tt < kPfTiles; tt++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[tt][mt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    const int mt_live = __builtin_amdgcn_readfirstlane((nt + 15) / 16);
    __shared__ __attribute__((aligned(1024))) half_t ys0[16 * MT * 64], ys1[16 * MT * 64], ys2[16 * MT * 64],
        ys3[16 * MT * 64];
    __shared__ float dgs[4 * 4 * 64], rinv[16 * MT];
    if ((int)threadIdx.x < 16 * MT) rinv[threadIdx.x] = 1.0f / ref[threadIdx.x];
    __syncthreads();
    constexpr int kI = DmaAct<MT>::kInst;
    DmaAct<MT> xd;
    xd.q = make_rsrc(a.x.q, (size_t)a.P * a.I * 2);
    xd.ds = make_rsrc(a.x.ds, (size_t)G * ld * 4);
    xd.ld4 = ld * 4;
    xd.wv = wv;
    xd.dst = wv * kI * 1024;
    xd.dgs = dgs;
    xd.rinv = rinv;
#pragma unroll
    for (int i = 0; i < kI; i++) {
        const int row = 8 * (wv * kI + i) + (lane >> 3);
        xd.off[i] = min(p0 + row, a.P - 1) * a.I * 2 + 16 * ((lane & 7) ^ x_sw(row)) + s0 * 2 * kStep;
    }
    {
        const int j = min(lane, 8 * kI - 1), row = 8 * (wv * kI + j / 8) + j % 8;
        xd.doff = min(p0 + row, a.P - 1) * 4 + s0 * xd.ld4;
    }
    pf_loop_dma_live<F, MT, false>(W, rb, s0, ksteps, lane, xd, ys0, ys1, ys2, ys3, mt_live, acc);
    float *ypk = a.ypart + (size_t)kq * a.P * a.H;
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = 16 * mt + 4 * g + i;
            if (m < nt) {
                float *yp = ypk + (size_t)orow[m] * a.H + (size_t)kRowBlock * rb + n;
#pragma unroll
                for (int tt = 0; tt < kPfTiles; tt++) yp[16 * tt] = acc[tt][mt][i] * ref[m];
            }
        }
}

// ------------------------------------------------------------- launchers

bool grouped_supported(int H, int I) { return H % 256 == 0 && I % 128 == 0; }

bool grouped_down_ks_ok(int, int I, int ks)
{
    const int steps = I / kStep;  // a share past the first starts on a whole block of four steps
    return ks == 1 || (ks > 1 && steps % ks == 0 && (steps / ks) % 4 == 0);
}

// The chunk list's d.chunk tokens in workgroups of 16 mt.
static int pf_sub(const Dispatch &d, int mt)
{
    if (mt < 1 || d.chunk % (16 * mt) || d.chunk / (16 * mt) > 2) {
        set_error("grouped GEMM: %d-token workgroups do not divide the %d-token chunks", 16 * mt, d.chunk);
        return 0;
    }
    return d.chunk / (16 * mt);
}

// G decodes the gate/up weights, D the down weights (the same format, read the
// way each kernel holds it).
template <class G, class D, int MT>
static int launch_pf(const PfArgs &a, bool gateup, hipStream_t st)
{
    if (a.nsmall && (MT != 4 || a.ks != 1 || !a.d.chunks_s)) {
        set_error("grouped GEMM: small groups need 64-token workgroups, an unsplit K and the dispatch's list");
        return ANEDVD_E_INVALID_ARG;
    }
    if (gateup) {
        const size_t wgs = ((size_t)pf_nw8(a.nchunk * a.sub, a.sub) + a.nsmall) * (a.I / (2 * kRowBlock));
        hipLaunchKernelGGL((k_pf_gateup<G, MT>), dim3((unsigned)wgs), dim3(256), 0, st, a);
    } else {
        const size_t wgs = ((size_t)pf_nw8(a.nchunk * a.sub, a.sub) * a.ks + a.nsmall) * (a.H / (4 * kRowBlock));
        hipLaunchKernelGGL((k_pf_down<D, MT>), dim3((unsigned)wgs), dim3(256), 0, st, a);
    }
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

// 64-token chunks (mt = 4), or 128-token ones (mt = 8) for the decoders that keep
// two wavefronts per SIMD with twice the accumulators: Q8_0, Q4_0, F16 and the
// other 32-element formats (the super-block formats would drop to one).
template <class G, class D, bool WIDE>
static int launch_pf_mt(const PfArgs &a, int mt, bool gateup, hipStream_t st)
{
    if (mt == 4) return launch_pf<G, D, 4>(a, gateup, st);
    if constexpr (WIDE)
        if (mt == 8) return launch_pf<G, D, 8>(a, gateup, st);
    set_error("grouped GEMM: no %d-token chunk kernel for this type", 16 * mt);
    return ANEDVD_E_INVALID_ARG;
}

bool grouped_wide(int type)
{
    switch (type) {
    case ANEDVD_Q8_0: case ANEDVD_Q8_1: case ANEDVD_F16: case ANEDVD_Q4_0: case ANEDVD_Q4_1: case ANEDVD_Q5_0:
    case ANEDVD_Q5_1: return true;
    default: return false;
    }
}

// The down kernel keeps 64-token workgroups for Q8_0 even where gate/up takes 128:
// at three wavefronts per SIMD (weights one step ahead) DeepSeek-V2-Lite's
// 1024-token down launch measured 99 us against 109-110 us at 128 tokens and two
// (one box, A/B).
bool grouped_wide_down(int type) { return grouped_wide(type) && type != ANEDVD_Q8_0 && type != ANEDVD_Q8_1; }

static int launch_pf_type(int type, const PfArgs &a, int mt, bool gateup, hipStream_t st)
{
    switch (type) {
    case ANEDVD_Q8_0:
    case ANEDVD_Q8_1: return launch_pf_mt<FQ8_0, FQ8_0, true>(a, mt, gateup, st);  // one tile layout
    case ANEDVD_F16: return launch_pf_mt<FF16, FF16, true>(a, mt, gateup, st);
    case ANEDVD_Q4_0: return launch_pf_mt<FQ4_0, FQ4_0, true>(a, mt, gateup, st);
    case ANEDVD_Q4_1: return launch_pf_mt<FQ4_1, FQ4_1, true>(a, mt, gateup, st);
    case ANEDVD_Q5_0: return launch_pf_mt<FQ5_0, FQ5_0, true>(a, mt, gateup, st);
    case ANEDVD_Q5_1: return launch_pf_mt<FQ5_1, FQ5_1, true>(a, mt, gateup, st);
    case ANEDVD_Q2_K: return launch_pf_mt<FQ2_K, FQ2_K, false>(a, mt, gateup, st);
    case ANEDVD_Q3_K: return launch_pf_mt<FQ3_K, FQ3_K, false>(a, mt, gateup, st);
    case ANEDVD_Q4_K: return launch_pf_mt<FQ4_K, FQ4_K, false>(a, mt, gateup, st);
    case ANEDVD_Q5_K: return launch_pf_mt<FQ5_K, FQ5_K, false>(a, mt, gateup, st);
    case ANEDVD_Q6_K: return launch_pf_mt<FQ6_K, FQ6_KDown, false>(a, mt, gateup, st);
    default:
        set_error("grouped GEMM: ggml type %d has no kernel", type);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
}

int launch_grouped_gateup(const QMat &gate, const QMat &up, const ActQ &x, int H, int I, const Dispatch &d, int P,
                          int mt, int nchunk, int contig, int nsmall, const ActQ &act, int use_gelu, hipStream_t st)
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
    a.ks = 1;
    // rows split over the XCDs: Mixtral 2048 tokens' gate/up 928-950 -> 906-917 us
    a.contig = contig && ANEDVD_PF_RSPLIT && (I / (2 * kRowBlock)) % 8 == 0 ? 2 : contig;
    a.nsmall = nsmall;
    if (!(a.sub = pf_sub(d, mt))) return ANEDVD_E_INVALID_ARG;
    return launch_pf_type(gate.type, a, mt, true, st);
}

int launch_grouped_down(const QMat &down, const ActQ &act, int H, int I, const Dispatch &d, int P, int mt,
                        int nchunk, int contig, int nsmall, int ks, float *ypart, int kk, hipStream_t st)
{
    if (!grouped_down_ks_ok(down.type, I, ks)) {
        set_error("grouped down: %d K shares do not split %d steps into whole blocks of four", ks, I / kStep);
        return ANEDVD_E_INVALID_ARG;
    }
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
    a.ks = ks;
    a.contig = contig;  // (split rows: Mixtral 2048 tokens' down 605-609 -> 629-633 us)
    a.nsmall = nsmall;
    if (!(a.sub = pf_sub(d, mt))) return ANEDVD_E_INVALID_ARG;
    return launch_pf_type(down.type, a, mt, false, st);
}

}  // namespace anedvd
