// kernels.h -- host-side launchers of the gfx950 kernels (stream-ordered, no sync).
#pragma once

#include "common.h"

namespace anedvd {

// MFMA activation format (common.h): f16 values q[rows][K] in mma_pos order within
// each 64-column group, and the descale of each (group, row) in ds[g * ld + row].
struct ActQ {
    half_t *q;
    float *ds;
    int ld;
};

// Token-to-expert dispatch of T*k (token, slot) entries (engine.zig:1204-1216):
// offsets[E+1]; rows/slots[T*k] grouped by expert, tokens ascending; inv[T*k] =
// position of (t, s); active[] = experts with tokens, ascending; meta[0] = number
// of active experts, meta[1] = largest group, meta[2] = ids >= E, meta[3] = number
// of chunks; chunks[] (optional) = chunk_entry(e, p0, nt) for each `chunk`-token
// slice of expert e's group, experts ascending -- the expert kernels' work list.
// With small > 0, groups of 1..small tokens are listed in chunks_s instead (one
// entry per group, experts ascending; meta[7] = their count, meta holding 8 ints).
// With xper > 0, xr[9] gives each XCD's range of the work list (see below).
struct Dispatch {
    int32_t *offsets, *rows, *slots, *inv, *active, *meta;
    uint64_t *chunks;  // the work list: chunk_entry(e, first position, tokens) per chunk
    int chunk;
    int n_routed;  // meta[1] counts experts below this one only (0 = all): merged shared pieces are not groups
    uint64_t *chunks_s;  // the small groups' list (small > 0)
    int small;
    // With xper > 0: xr[0..8], the work list cut into 8 XCD ranges of at most xper
    // chunks, whole experts per range where they fit (else xr[x] = x * xper).
    int32_t *xr;
    int xper;

};

// A work-list entry: expert e (< 256), the chunk's first position p0 and its
// tokens nt (<= 255), one 8-byte load for the kernels that take it.
__host__ __device__ inline uint64_t chunk_entry(int e, int p0, int nt)
{
    return (uint64_t)(uint32_t)e | (uint64_t)(uint32_t)nt << 8 | (uint64_t)(uint32_t)p0 << 16;
}


// k_dequant.hip
int launch_dequant_gguf(int type, const uint8_t *d_src, size_t n_blocks, float *d_out, hipStream_t st);
int launch_repack(const QMat &m, const uint8_t *d_src, hipStream_t st);
int launch_dequant_tiles(const QMat &m, int mat, float *d_out, hipStream_t st);
int launch_f32_to_f16(const float *d_src, uint16_t *d_dst, size_t n, hipStream_t st);
int launch_f16_to_f32(const uint16_t *d_src, float *d_dst, size_t n, hipStream_t st);

// k_route.hip
constexpr int kMaxRouteExperts = 256;  // experts the route and dispatch kernels take (ids fit a byte)
constexpr int kMaxRouteSlots = 32;     // slots per token
// cpu.matmulF16 of T rows of x against the [E][H] f16 router: d_wt is the router
// in the kernel's layout (launch_router_layout: f32, interleaved for the chains,
// router_layout_floats(E, H) floats), d_w the [E][H] matrix itself (read only for
// a tail of H % 8 columns).
size_t router_layout_floats(int E, int H);
int launch_router_layout(const uint16_t *d_w, int E, int H, float *d_wt, hipStream_t st);
int launch_router(const float *d_wt, const uint16_t *d_w, const float *d_x, int T, int E, int H, float *d_logits,
                  hipStream_t st);
// cpu.moeRoute for T rows of logits; with d_x non-null the same launch also
// converts x [T][H] to the GEMV activation format `xq`.
// Shared-expert pieces merged into the routed experts: n pieces, experts E..E+n-1,
// every token's slots k..k+n-1, scale sigmoid(lin . h) or 1 when lin is null.
struct SharedSlots {
    int n = 0;
    const uint16_t *lin = nullptr;
};
int launch_route(const float *d_logits, int T, int E, int k, int norm, float *d_probs, uint32_t *d_idx,
                 const float *d_x, int H, const ActQ &xq, hipStream_t st, const SharedSlots &sh = {});
int launch_dispatch(const uint32_t *d_idx, int T, int k, int E, const Dispatch &d, hipStream_t st);
// Route, dispatch and (d_x non-null) activation conversion of one forward call.
// route_fusable(T, E): one launch does it all (up to 16 tokens); otherwise the route
// launch (one wavefront per token, the conversion beside it), then the
// one-workgroup dispatch launch.
bool route_fusable(int T, int E);
// route_router_fusable(T, E, H): the fused launch can also form the router logits
// (a chain per thread); then d_logits is null and d_rwt / d_rw the router (in
// launch_router_layout's layout, as stored), and d_x the call's activations.
bool route_router_fusable(int T, int E, int H);
int launch_route_and_dispatch(const float *d_logits, int T, int E, int k, int norm, float *d_probs, uint32_t *d_idx,
                              const float *d_x, int H, const ActQ &xq, const Dispatch &d, hipStream_t st,
                              const SharedSlots &sh = {}, const float *d_rwt = nullptr,
                              const uint16_t *d_rw = nullptr);
int launch_act_prep(const float *d_x, int rows, int K, const ActQ &xq, hipStream_t st);

// k_mm.hip -- expert products on MFMA
enum MmKind {
    kMmDecode = 0,   // k_mm_gateup / k_mm_down: 16-token tiles, per-block f32 scales, K split
    kMmStaged = 1    // k_pf_gateup / k_pf_down: 64-token chunks, activations staged in LDS
};
struct MmPlan {
    int kind;     // MmKind
    int ks_gu;    // K split of gate/up (workgroups per 64-row block)
    int ks_dn;    // K split of down
    int mt;       // 16-token tiles per chunk: 1 (decode), 4 or 8 (grouped GEMM)
    int mt_gu;    // grouped GEMM: 16-token tiles per gate/up workgroup (4 or 8, at most mt)
    int mt_dn;    // grouped GEMM: 16-token tiles per down workgroup (4 or 8, at most mt)
    int contig;   // grouped GEMM: XCD-contiguous workgroup order
    int chunk;    // tokens per work-list chunk (16 mt), the dispatch's `chunk`
    int nchunk;   // bound on the work list's length: P / chunk + max_u
    int small;    // grouped GEMM: groups of at most this many tokens run on one 16-token tile each (0 = none)
    int nsmall;   // grouped GEMM with small: capacity of the small groups' list (max_u)
    int xper;     // grouped GEMM with contig: chunks per XCD range of the work list (0 = none)
    int fuse;     // decode, ks_gu > 1: the down kernel finishes gate/up's K partials (no k_act_reduce)
};
bool mm_supported(int type);
// P (token, slot) entries of T tokens over at most max_u experts.
MmPlan plan_mm(int gate_type, int down_type, int H, int I, int P, int max_u, int T);
// gate/up + SiLU(gate)*up for every dispatched (token, expert) position, written
// to `act` [P][I] in the activation format.  With plan.ks_gu > 1 the K partials
// go to `part` [ks][P][2][I] and a second launch finishes them, or, with
// plan.fuse, the down launch does (act is then not written).
int launch_expert_gateup(const QMat &gate, const QMat &up, const ActQ &x, int H, int I, const Dispatch &d, int P,
                         const MmPlan &plan, float *part, const ActQ &act, int use_gelu, hipStream_t st);
// down for every position: ypart [ks_dn][T * kk][H] in (token, slot) order --
// position p's output row is rows[p] * kk + slots[p] -- so the combine reads a
// token's slots without going through `inv` (the combine adds the K partials).
// With plan.fuse its input is gate/up's partials `part` (SiLU or geluTanh by
// use_gelu), not `act`.
int launch_expert_down(const QMat &down, const ActQ &act, int H, int I, const Dispatch &d, int P,
                       const MmPlan &plan, const float *part, int use_gelu, float *ypart, int kk, hipStream_t st);
// k_pf.hip -- the grouped GEMM for prefill-sized groups (chunks of 16 mt tokens)
bool grouped_supported(int H, int I);
bool grouped_wide(int type);  // the type has a 128-token-chunk grouped kernel
bool grouped_wide_down(int type);  // ... and its down product takes it
// A workgroup takes 16 mt tokens of a work-list chunk of d.chunk tokens.
// contig: XCD-contiguous workgroup order (experts averaging two or more chunks).
// nsmall > 0 (mt 4, K not split): the same launch also runs the groups of the
// dispatch's small list (d.chunks_s, capacity nsmall), a 16-token tile each.
int launch_grouped_gateup(const QMat &gate, const QMat &up, const ActQ &x, int H, int I, const Dispatch &d, int P,
                          int mt, int nchunk, int contig, int nsmall, const ActQ &act, int use_gelu, hipStream_t st);
// With ks > 1 the K axis is split over ks workgroups, each writing plane ks of ypart.
int launch_grouped_down(const QMat &down, const ActQ &act, int H, int I, const Dispatch &d, int P, int mt,
                        int nchunk, int contig, int nsmall, int ks, float *ypart, int kk, hipStream_t st);
bool grouped_down_ks_ok(int type, int I, int ks);  // I/64 steps split into ks whole scale-unit blocks

// k_ops.hip -- cpu.moeExpertAccumF32 / moeExpertAccum on caller weight slices
// ([inter][hidden] gate and up, [hidden][inter] down; f32, or f16 bits when f16):
// act[inter] = act(gate . h) * (up . h), then out[hidden] += weight * down . act.
int launch_expert_accum_ops(bool f16, const void *gate, const void *up, const void *down, const float *h, int inter,
                            int hidden, float weight, int use_gelu, float *act, float *out, hipStream_t st);

// out = sum over slots of p * y (+ s * shared) [+ resid: the engine's x += proj].
int launch_combine(const float *ypart, const int32_t *inv, const float *probs, int T, int k, int H, int KS, int P,
                   const float *shared, const float *shared_scale, int sKS, float *out, hipStream_t st,
                   const float *resid = nullptr);

}  // namespace anedvd
