// moe_api.hip -- the extern "C" boundary (include/anedvd_moe.h): contexts,
// resident layers, and the forward pass as a stream-ordered chain of kernels
//   router -> route -> dispatch -> expert gate/up -> expert down
//   [-> shared gate/up -> shared down] -> combine
// with no host synchronisation inside a forward.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

#include "common.h"
#include "kernels.h"

namespace anedvd {

static thread_local char g_err[512] = "";

void set_error(const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

}  // namespace anedvd

using namespace anedvd;

// Device workspace of one context, carved from one allocation and grown on demand.
struct Workspace {
    void *base = nullptr;
    size_t cap = 0;
};

struct anedvd_moe_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipStream_t aux = nullptr;            // the shared expert runs here beside the routed experts
    hipEvent_t fork = nullptr, join = nullptr;
    Workspace ws;
    Workspace io;  // staging for the host-pointer entry points
    // The last forward call on this context (route counts read its dispatch).
    const anedvd_moe_layer *last_layer = nullptr;
    const int32_t *last_offsets = nullptr;
    int last_tokens = 0;
};

struct anedvd_moe_layer {
    anedvd_moe_ctx *ctx = nullptr;
    uint32_t H = 0, I = 0, E = 0, k = 0;
    int norm = 0, gelu = 0;
    QMat gate{}, up{}, down{};
    uint16_t *router = nullptr;    // [E][H] f16
    float *router_t = nullptr;  // the router kernel's f32 interleaved copy (launch_router_layout)
    uint32_t Is = 0;
    uint32_t n_sh = 0;  // shared expert merged as n_sh expert-width pieces after the E routed experts
    QMat sgate{}, sup{}, sdown{};  // the shared expert when it is not merged
    uint16_t *sgate_lin = nullptr;
    uint64_t device_bytes = 0;
    double expert_bytes = 0, shared_bytes = 0;
};

// ------------------------------------------------- the no-allocation forward
//
// anedvd_moe_layer_forward_device_noalloc carves its per-call scratch (routing,
// dispatch, f16 activations, partial sums: fwd_layout) from this file-scope device
// array instead of the context's growable workspace.  Every GPU the library runs
// on holds its own copy, at its own address, until the process ends.  In host code
// `scratch` names a host-side stand-in, not device memory: host code uses only the
// address hipGetSymbolAddress returns, looked up once per device (with that device
// current) when a context opens it, and kept in g_scratch.  Nothing in it needs to
// start at zero: every call writes each scratch word it later reads.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
static std::mutex g_scratch_mu;
static void *g_scratch[kMaxDevices];

namespace {

// Looks up this device's copy of `scratch` (the device is current).
int scratch_setup(int device)
{
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device < 0 || device >= kMaxDevices) {
        set_error("no-allocation scratch: device %d is beyond the %d this build tracks", device, kMaxDevices);
        return ANEDVD_E_NO_DEVICE;
    }
    if (g_scratch[device]) return ANEDVD_OK;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        set_error("hipGetSymbolAddress(scratch) on device %d failed: %s", device, hipGetErrorString(e));
        return ANEDVD_E_HIP;
    }
    g_scratch[device] = p;
    return ANEDVD_OK;
}

void *scratch_of(int device)
{
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return device >= 0 && device < kMaxDevices ? g_scratch[device] : nullptr;
}

struct Carve {
    uint8_t *p;
    template <class T>
    T *take(size_t n)
    {
        T *r = (T *)p;
        p += (n * sizeof(T) + 255) & ~(size_t)255;
        return r;
    }
};

int ensure(Workspace &w, size_t bytes, hipStream_t st)
{
    if (w.cap >= bytes) return ANEDVD_OK;
    if (w.base) {
        ANEDVD_HIP(hipStreamSynchronize(st));
        ANEDVD_HIP(hipFree(w.base));
        w.base = nullptr;
        w.cap = 0;
    }
    const size_t want = std::max(bytes, (size_t)1 << 20);
    ANEDVD_HIP(hipMalloc(&w.base, want));
    w.cap = want;
    return ANEDVD_OK;
}

// A host block copied into the upload staging buffer after the previous ones:
// `height` rows of `width` bytes, `pitch` bytes apart in host memory.
struct Seg {
    const void *src;
    size_t width, height, pitch;
};

int make_qmat(QMat &m, int type, int rows, int cols, int n, const void *host, size_t bytes, hipStream_t st,
              uint64_t &dev_bytes, const char *what, const std::vector<Seg> &extra = {}, int n_extra = 0)
{
    const Fmt f = tile_fmt(type);
    if (!mm_supported(type)) {
        set_error("%s: ggml type %d is not supported by the GPU layout (f16, q8_0, q8_1, q4_0, q4_1, q5_0, q5_1, q2_k, q3_k, q4_k, q5_k, q6_k)", what, type);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
    const int unit_cols = kStep * f.spu;
    if (rows % kRowBlock || cols % unit_cols) {
        set_error("%s: %d x %d is not a multiple of %d rows x %d columns", what, rows, cols, kRowBlock, unit_cols);
        return ANEDVD_E_INVALID_SHAPE;
    }
    const size_t per = (size_t)rows * cols / block_elems(type) * block_bytes(type);
    if (bytes != per * n) {
        set_error("%s: %zu bytes given, %d x %d x %d of type %d needs %zu", what, bytes, n, rows, cols, type, per * n);
        return ANEDVD_E_DIMENSION;
    }
    // `extra` holds n_extra more matrices of the same shape (a shared expert cut
    // into expert-width pieces), appended after the n given ones.
    n += n_extra;
    m.type = type;
    m.rows = rows;
    m.cols = cols;
    m.n = n;
    m.steps = cols / kStep;
    m.units = m.steps / f.spu;
    // per matrix: rows/64 row blocks x steps x 4 tiles x 64 lanes x qb bytes, ...
    m.q_stride = (size_t)rows * m.steps * 4 * f.qb;
    m.s_stride = (size_t)rows * m.units * f.sb;
    m.h_stride = (size_t)rows * m.steps * 4 * tile_hb(type);
    m.d_stride = (size_t)rows * m.units * tile_db(type);
    // The kernels address one matrix's planes with 32-bit buffer offsets.
    if (m.q_stride > ((size_t)1 << 30)) {
        set_error("%s: one %d x %d matrix is %zu bytes; at most 1 GiB per expert matrix", what, rows, cols, m.q_stride);
        return ANEDVD_E_INVALID_SHAPE;
    }
    ANEDVD_HIP(hipMalloc(&m.q, m.q_stride * n));
    ANEDVD_HIP(hipMalloc(&m.s, m.s_stride * n));
    if (m.h_stride) ANEDVD_HIP(hipMalloc(&m.h, m.h_stride * n));
    if (m.d_stride) ANEDVD_HIP(hipMalloc(&m.d, m.d_stride * n));
    dev_bytes += (m.q_stride + m.s_stride + m.h_stride + m.d_stride) * n;
    uint8_t *staging = nullptr;
    ANEDVD_HIP(hipMalloc(&staging, per * n));
    hipError_t e = hipMemcpyAsync(staging, host, bytes, hipMemcpyHostToDevice, st);
    size_t off = bytes;
    for (const Seg &g : extra) {
        if (e != hipSuccess) break;
        e = hipMemcpy2DAsync(staging + off, g.width, g.src, g.pitch, g.width, g.height, hipMemcpyHostToDevice, st);
        off += g.width * g.height;
    }
    if (e == hipSuccess && off != per * n) {
        (void)hipStreamSynchronize(st);
        (void)hipFree(staging);
        set_error("%s: %zu bytes staged, %zu expected", what, off, per * n);
        return ANEDVD_E_DIMENSION;
    }
    int rc = e == hipSuccess ? launch_repack(m, staging, st) : ANEDVD_E_HIP;
    if (e != hipSuccess) set_error("%s: upload failed: %s", what, hipGetErrorString(e));
    hipError_t e2 = hipStreamSynchronize(st);
    (void)hipFree(staging);
    if (rc != ANEDVD_OK) return rc;
    if (e2 != hipSuccess) {
        set_error("%s: repack failed: %s", what, hipGetErrorString(e2));
        return ANEDVD_E_HIP;
    }
    return ANEDVD_OK;
}

void free_qmat(QMat &m)
{
    for (uint8_t **p : {&m.q, &m.s, &m.h, &m.d}) {
        if (*p) (void)hipFree(*p);
        *p = nullptr;
    }
}

// All device scratch of one forward call of T tokens with k slots each.
struct Fwd {
    float *logits, *probs;
    uint32_t *idx;
    Dispatch d;
    ActQ xq;            // [T][H]
    ActQ act;           // [P][I]
    float *part, *ypart;
    // shared expert
    Dispatch sd;
    ActQ sact;          // [T][Is]
    float *sh_part, *sh_ypart, *sh_scale;
    float *h_in, *l_in, *out;  // staging for host-pointer calls
    MmPlan plan, splan;
    int max_u, P;
};

// k: slots per token (the routed top-k plus the merged shared pieces for a
// forward call).  Dispatch arrays cover the E routed experts and the pieces.
size_t fwd_layout(const anedvd_moe_layer *L, int T, int k, Fwd *f, uint8_t *base, bool with_io)
{
    const int H = L->H, I = L->I, E = L->E + L->n_sh, P = T * k;
    Fwd x{};
    x.P = P;
    x.max_u = std::min(E, P);
    x.plan = plan_mm(L->gate.type, L->down.type, H, I, P, x.max_u, T);
    Carve c{base};
    x.logits = c.take<float>((size_t)T * L->E);
    x.probs = c.take<float>(P);
    x.idx = c.take<uint32_t>(P);
    x.d.offsets = c.take<int32_t>(E + 1);
    x.d.rows = c.take<int32_t>(P);
    x.d.slots = c.take<int32_t>(P);
    x.d.inv = c.take<int32_t>(P);
    x.d.active = c.take<int32_t>(E);
    x.d.meta = c.take<int32_t>(8);
    x.d.chunks = c.take<uint64_t>((size_t)x.plan.nchunk);
    x.d.chunk = x.plan.chunk;
    x.d.n_routed = L->E;
    if (x.plan.small) {
        x.d.chunks_s = c.take<uint64_t>((size_t)x.max_u);
        x.d.small = x.plan.small;
    }
    if (x.plan.xper) {
        x.d.xr = c.take<int32_t>(9);
        x.d.xper = x.plan.xper;
    }
    x.xq = ActQ{c.take<half_t>((size_t)T * H), c.take<float>((size_t)T * (H / kStep)), T};
    x.act = ActQ{c.take<half_t>((size_t)P * I), c.take<float>((size_t)P * (I / kStep)), P};
    x.part = x.plan.ks_gu > 1 ? c.take<float>((size_t)x.plan.ks_gu * P * 2 * I) : nullptr;
    x.ypart = c.take<float>((size_t)x.plan.ks_dn * P * H);
    if (L->Is && !L->n_sh) {
        const int Is = (int)L->Is;
        x.splan = plan_mm(L->sgate.type, L->sdown.type, H, Is, T, 1, T);
        x.sd.offsets = c.take<int32_t>(2);
        x.sd.rows = c.take<int32_t>(T);
        x.sd.slots = c.take<int32_t>(T);
        x.sd.active = c.take<int32_t>(1);
        x.sd.meta = c.take<int32_t>(4);
        x.sd.chunks = c.take<uint64_t>((size_t)x.splan.nchunk);
        x.sd.chunk = x.splan.chunk;
        x.sact = ActQ{c.take<half_t>((size_t)T * Is), c.take<float>((size_t)T * (Is / kStep)), T};
        x.sh_part = x.splan.ks_gu > 1 ? c.take<float>((size_t)x.splan.ks_gu * T * 2 * Is) : nullptr;
        x.sh_ypart = c.take<float>((size_t)x.splan.ks_dn * T * H);
        x.sh_scale = c.take<float>(T);
    }
    if (with_io) {
        x.h_in = c.take<float>((size_t)T * H);
        x.l_in = c.take<float>((size_t)T * L->E);
        x.out = c.take<float>((size_t)T * H);
    }
    if (f) *f = x;
    return (size_t)(c.p - base);
}

// Fills the shared expert's one-expert dispatch (all T tokens, in order, and its
// chunk list) and, if it is gated, its per-token scale sigmoid(shared_gate_lin . h).
__global__ void k_shared_prep(const float *__restrict__ h, const uint16_t *__restrict__ lin, int T, int H, Dispatch d,
                              float *scale)
{
    const int t = blockIdx.x;
    if (t == 0 && threadIdx.x == 0) {
        d.offsets[0] = 0;
        d.offsets[1] = T;
        d.active[0] = 0;
        d.meta[0] = 1;
        d.meta[1] = T;
        d.meta[2] = 0;
        d.meta[3] = (T + d.chunk - 1) / d.chunk;
    }
    if (threadIdx.x == 0) {
        d.rows[t] = t;
        d.slots[t] = 0;
        if (t % d.chunk == 0) d.chunks[t / d.chunk] = chunk_entry(0, t, min(d.chunk, T - t));  // expert 0
    }
    if (!lin) return;
    // one wavefront per token; sigmoid as cpu.sigmoid (cpu.zig:1223-1230)
    float g = 0.0f;
    for (int i = threadIdx.x; i < H; i += 64) g += f16_bits_to_f32(lin[i]) * h[(size_t)t * H + i];
    for (int o = 32; o > 0; o >>= 1) g += __shfl_xor(g, o);
    if (threadIdx.x == 0) scale[t] = shared_sigmoid(g);
}

// One forward call on stream st.  With `resid` the output is resid + the block's
// output (the engine's x += proj, main.zig:519), as a stack of layers chains it.
int forward_device(anedvd_moe_layer *L, const float *d_h, int T, const float *d_logits, float *d_out, const Fwd &f,
                   hipStream_t st, hipEvent_t *ev, const float *resid = nullptr)
{
    const int H = L->H, I = L->I, E = L->E, k = L->k, kk = k + (int)L->n_sh, P = T * kk;
    L->ctx->last_layer = L;
    L->ctx->last_offsets = f.d.offsets;
    L->ctx->last_tokens = T;
    auto mark = [&](int i) {
        if (ev) (void)hipEventRecord(ev[i], st);
    };
    mark(0);
    // The router GEMV runs in the routing launch itself when the call is a few
    // tokens (a chain per thread of the routing workgroup), else in its own launch.
    const float *logits = d_logits;
    const bool fuse_router = !logits && route_router_fusable(T, E, H);
    if (!logits && !fuse_router) {
        ANEDVD_TRY(launch_router(L->router_t, L->router, d_h, T, E, H, f.logits, st));
        logits = f.logits;
    }
    SharedSlots sh;
    sh.n = (int)L->n_sh;
    sh.lin = L->sgate_lin;
    ANEDVD_TRY(launch_route_and_dispatch(logits, T, E, k, L->norm, f.probs, f.idx, d_h, H, f.xq, f.d, st, sh,
                                         fuse_router ? L->router_t : nullptr, fuse_router ? L->router : nullptr));
    mark(1);
    // A shared expert that is not merged into the routed launches needs only x
    // (converted by the route launch): it runs on the context's second stream beside
    // the routed experts, joined before the combine.  With stage events everything
    // stays on `st`, so the stages time one at a time.  (Groups of a few tokens,
    // plan.small, run inside the grouped launches.)
    const bool separate = L->Is && !L->n_sh;
    const bool fork = separate && !ev;
    hipStream_t ss = fork ? L->ctx->aux : st;
    auto shared = [&]() -> int {
        const int Is = (int)L->Is;
        hipLaunchKernelGGL(k_shared_prep, dim3(T), dim3(64), 0, ss, d_h, L->sgate_lin, T, H, f.sd, f.sh_scale);
        ANEDVD_HIP(hipGetLastError());
        ANEDVD_TRY(launch_expert_gateup(L->sgate, L->sup, f.xq, H, Is, f.sd, T, f.splan, f.sh_part, f.sact,
                                        L->gelu, ss));
        return launch_expert_down(L->sdown, f.sact, H, Is, f.sd, T, f.splan, f.sh_part, L->gelu, f.sh_ypart, 1, ss);
    };
    auto routed = [&]() -> int {
        ANEDVD_TRY(launch_expert_gateup(L->gate, L->up, f.xq, H, I, f.d, P, f.plan, f.part, f.act, L->gelu, st));
        mark(2);
        ANEDVD_TRY(launch_expert_down(L->down, f.act, H, I, f.d, P, f.plan, f.part, L->gelu, f.ypart, kk, st));
        mark(3);
        return ANEDVD_OK;
    };
    if (fork) {
        ANEDVD_HIP(hipEventRecord(L->ctx->fork, st));
        ANEDVD_HIP(hipStreamWaitEvent(ss, L->ctx->fork, 0));
        // Once forked, the main stream waits for the second one on every path, so an
        // error never leaves its kernels writing the workspace into the next call.
        int rc = shared();
        const int jrc = hipEventRecord(L->ctx->join, ss) == hipSuccess ? ANEDVD_OK : ANEDVD_E_HIP;
        if (rc == ANEDVD_OK) rc = jrc;
        if (rc == ANEDVD_OK) rc = routed();
        if (jrc == ANEDVD_OK) {
            if (hipStreamWaitEvent(st, L->ctx->join, 0) != hipSuccess && rc == ANEDVD_OK) {
                set_error("forward: joining the second stream failed");
                rc = ANEDVD_E_HIP;
            }
        } else if (hipStreamSynchronize(ss) != hipSuccess && rc == ANEDVD_OK) {
            rc = ANEDVD_E_HIP;
        }
        if (jrc != ANEDVD_OK && rc == ANEDVD_E_HIP) set_error("forward: recording the second stream's join failed");
        ANEDVD_TRY(rc);
    } else {
        ANEDVD_TRY(routed());
        if (separate) ANEDVD_TRY(shared());
    }
    mark(4);
    ANEDVD_TRY(launch_combine(f.ypart, f.d.inv, f.probs, T, kk, H, f.plan.ks_dn, P, separate ? f.sh_ypart : nullptr,
                              (separate && L->sgate_lin) ? f.sh_scale : nullptr, separate ? f.splan.ks_dn : 0, d_out,
                              st, resid));
    mark(5);
    return ANEDVD_OK;
}

int check_layer(const anedvd_moe_layer *L)
{
    if (!L || !L->ctx) {
        set_error("null layer");
        return ANEDVD_E_INVALID_ARG;
    }
    return ANEDVD_OK;
}

// The most tokens one forward call takes.  The expert kernels address the
// activations through 32-bit buffer descriptors with int offsets: x [T][H] f16, the
// SwiGLU activations [T*kk][I] f16 (plus a 64-row tile of look-ahead past the last
// position) and a separate shared expert's [T][Is] f16 must each stay below 2^31
// bytes.
size_t max_tokens(const anedvd_moe_layer *L)
{
    const uint64_t lim = (1ull << 31) - 1, kk = L->k + L->n_sh;
    uint64_t t = lim / (2ull * L->H);
    t = std::min<uint64_t>(t, lim / (2ull * L->I) / kk - 64);
    if (L->Is && !L->n_sh) t = std::min<uint64_t>(t, lim / (2ull * L->Is) - 64);
    return (size_t)std::min<uint64_t>(t, 1u << 20);
}

}  // namespace

extern "C" {

const char *anedvd_moe_last_error(void) { return g_err; }

int anedvd_moe_abi_version(void) { return ANEDVD_MOE_ABI_VERSION; }

int anedvd_moe_open(int device, anedvd_moe_ctx **out)
{
    if (!out) {
        set_error("anedvd_moe_open: out is null");
        return ANEDVD_E_INVALID_ARG;
    }
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= device || device < 0) {
        set_error("anedvd_moe_open: device %d not present (%d HIP devices)", device, n);
        return ANEDVD_E_NO_DEVICE;
    }
    hipDeviceProp_t prop;
    ANEDVD_HIP(hipGetDeviceProperties(&prop, device));
    if (!strstr(prop.gcnArchName, "gfx950")) {
        set_error("anedvd_moe_open: device %d is %s; this library is built for gfx950 only", device, prop.gcnArchName);
        return ANEDVD_E_NO_DEVICE;
    }
    ANEDVD_HIP(hipSetDevice(device));
    // This device's no-allocation scratch, looked up once per device.  A failure
    // here only concerns anedvd_moe_layer_forward_device_noalloc, which looks again
    // and reports it; every other entry point works without the array.
    (void)scratch_setup(device);
    anedvd_moe_ctx *c = new anedvd_moe_ctx();
    c->device = device;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&c->aux, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&c->fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&c->join, hipEventDisableTiming) != hipSuccess) {
        if (c->fork) (void)hipEventDestroy(c->fork);
        if (c->aux) (void)hipStreamDestroy(c->aux);
        if (c->stream) (void)hipStreamDestroy(c->stream);
        delete c;
        set_error("anedvd_moe_open: stream or event creation failed");
        return ANEDVD_E_HIP;
    }
    *out = c;
    return ANEDVD_OK;
}

void anedvd_moe_close(anedvd_moe_ctx *ctx)
{
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipStreamSynchronize(ctx->aux);
    if (ctx->ws.base) (void)hipFree(ctx->ws.base);
    if (ctx->io.base) (void)hipFree(ctx->io.base);
    (void)hipEventDestroy(ctx->fork);
    (void)hipEventDestroy(ctx->join);
    (void)hipStreamDestroy(ctx->aux);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

int anedvd_moe_layer_create(anedvd_moe_ctx *ctx, const anedvd_moe_layer_desc *d, anedvd_moe_layer **out)
{
    if (!ctx || !d || !out) {
        set_error("anedvd_moe_layer_create: null argument");
        return ANEDVD_E_INVALID_ARG;
    }
    *out = nullptr;
    if (!d->hidden || !d->inter || !d->n_experts || !d->k || d->k > d->n_experts || d->n_experts > 256 || d->k > 32 ||
        !d->gate || !d->up || !d->down || !d->router) {
        set_error("anedvd_moe_layer_create: bad shape H=%u I=%u E=%u k=%u (need 0 < k <= E <= 256, k <= 32) or missing tensor",
                  d->hidden, d->inter, d->n_experts, d->k);
        return ANEDVD_E_INVALID_ARG;
    }
    if (d->hidden % 64) {
        set_error("anedvd_moe_layer_create: hidden %u is not a multiple of 64", d->hidden);
        return ANEDVD_E_INVALID_SHAPE;
    }
    ANEDVD_HIP(hipSetDevice(ctx->device));
    anedvd_moe_layer *L = new anedvd_moe_layer();
    L->ctx = ctx;
    L->H = d->hidden;
    L->I = d->inter;
    L->E = d->n_experts;
    L->k = d->k;
    L->norm = d->norm_topk_prob != 0;
    L->gelu = d->use_gelu != 0;
    const int H = (int)d->hidden, I = (int)d->inter, E = (int)d->n_experts, Is = (int)d->shared_inter;
    // A shared expert of the routed experts' type whose width is a multiple of
    // theirs is cut into Is / I expert-width pieces appended to the routed experts:
    // every token takes them as extra slots with its shared scale, in the same
    // launches (SwiGLU is separable over the intermediate width, so the pieces sum
    // to the whole).  Otherwise it keeps matrices of its own and a launch sequence
    // on the context's second stream.
    // The pieces are extra experts and extra slots of every token: the route and
    // dispatch take at most kMaxRouteExperts experts and kMaxRouteSlots slots, so a
    // shared expert that would exceed either keeps its own matrices instead.
    const int st_ = d->shared_type, bl = block_elems(st_), bb = block_bytes(st_);
    const bool merge = Is > 0 && I > 0 && st_ == d->gate_type && st_ == d->up_type && st_ == d->down_type && bl &&
                       Is % I == 0 && I % bl == 0 && H % bl == 0 &&
                       E + Is / I <= kMaxRouteExperts && (int)d->k + Is / I <= kMaxRouteSlots &&
                       d->shared_gate_bytes == (size_t)Is * H / bl * bb && d->shared_up_bytes == d->shared_gate_bytes &&
                       d->shared_down_bytes == d->shared_gate_bytes;
    const int nsh = merge ? Is / I : 0;
    std::vector<Seg> sg, su, sdn;
    if (merge) {
        sg.push_back({d->shared_gate, d->shared_gate_bytes, 1, d->shared_gate_bytes});
        su.push_back({d->shared_up, d->shared_up_bytes, 1, d->shared_up_bytes});
        const size_t piece = (size_t)I / bl * bb, row = (size_t)Is / bl * bb;  // down [H][Is]: column slices
        for (int j = 0; j < nsh; j++)
            sdn.push_back({(const uint8_t *)d->shared_down + j * piece, piece, (size_t)H, row});
    }
    L->n_sh = (uint32_t)nsh;
    int rc = make_qmat(L->gate, d->gate_type, I, H, E, d->gate, d->gate_bytes, ctx->stream, L->device_bytes, "gate",
                       sg, nsh);
    if (!rc)
        rc = make_qmat(L->up, d->up_type, I, H, E, d->up, d->up_bytes, ctx->stream, L->device_bytes, "up", su, nsh);
    if (!rc)
        rc = make_qmat(L->down, d->down_type, H, I, E, d->down, d->down_bytes, ctx->stream, L->device_bytes, "down",
                       sdn, nsh);
    if (!rc) {
        // the router as given ([E][H], for a tail of H % 8 columns) and in the router
        // kernel's layout (f32, interleaved for its chains)
        const size_t rb = (size_t)E * H * 2, rtb = router_layout_floats(E, H) * 4;
        if (hipMalloc(&L->router, rb) != hipSuccess || hipMalloc(&L->router_t, rtb) != hipSuccess ||
            hipMemcpy(L->router, d->router, rb, hipMemcpyHostToDevice) != hipSuccess) {
            set_error("router upload failed");
            rc = ANEDVD_E_HIP;
        }
        if (!rc) rc = launch_router_layout(L->router, E, H, L->router_t, ctx->stream);
        if (!rc && hipStreamSynchronize(ctx->stream) != hipSuccess) {
            set_error("router layout failed");
            rc = ANEDVD_E_HIP;
        }
        L->device_bytes += rb + rtb;
    }
    if (!rc && d->shared_inter) {
        L->Is = d->shared_inter;
        if (!merge) {
            rc = make_qmat(L->sgate, d->shared_type, Is, H, 1, d->shared_gate, d->shared_gate_bytes, ctx->stream,
                           L->device_bytes, "shared gate");
            if (!rc) rc = make_qmat(L->sup, d->shared_type, Is, H, 1, d->shared_up, d->shared_up_bytes, ctx->stream,
                                    L->device_bytes, "shared up");
            if (!rc)
                rc = make_qmat(L->sdown, d->shared_type, H, Is, 1, d->shared_down, d->shared_down_bytes, ctx->stream,
                               L->device_bytes, "shared down");
        }
        if (!rc && d->shared_gate_lin) {
            if (hipMalloc(&L->sgate_lin, (size_t)H * 2) != hipSuccess ||
                hipMemcpy(L->sgate_lin, d->shared_gate_lin, (size_t)H * 2, hipMemcpyHostToDevice) != hipSuccess) {
                set_error("shared_gate_lin upload failed");
                rc = ANEDVD_E_HIP;
            }
        }
    }
    if (rc) {
        anedvd_moe_layer_free(L);
        return rc;
    }
    auto bpw = [](int t) { return (double)block_bytes(t) / block_elems(t); };
    L->expert_bytes = (double)I * H * (bpw(L->gate.type) + bpw(L->up.type) + bpw(L->down.type));
    L->shared_bytes = L->Is ? 3.0 * H * L->Is * bpw(d->shared_type) : 0.0;
    *out = L;
    return ANEDVD_OK;
}

void anedvd_moe_layer_free(anedvd_moe_layer *L)
{
    if (!L) return;
    if (L->ctx) {
        (void)hipSetDevice(L->ctx->device);
        (void)hipStreamSynchronize(L->ctx->stream);
        if (L->ctx->last_layer == L) L->ctx->last_layer = nullptr;
    }
    free_qmat(L->gate);
    free_qmat(L->up);
    free_qmat(L->down);
    free_qmat(L->sgate);
    free_qmat(L->sup);
    free_qmat(L->sdown);
    if (L->router) (void)hipFree(L->router);
    if (L->router_t) (void)hipFree(L->router_t);
    if (L->sgate_lin) (void)hipFree(L->sgate_lin);
    delete L;
}

uint64_t anedvd_moe_layer_device_bytes(const anedvd_moe_layer *L) { return L ? L->device_bytes : 0; }

size_t anedvd_moe_layer_max_tokens(const anedvd_moe_layer *L) { return L ? max_tokens(L) : 0; }

// ------------------------------------------------------------ op mirrors

int anedvd_dequantize_range(anedvd_moe_ctx *ctx, int t, const void *src, size_t src_len, uint64_t elem_offset,
                            float *out, size_t n)
{
    // The checks of dequantizeRange (gguf.zig:694-728), in its order.
    const int epb = block_elems(t), bpb = block_bytes(t);
    if (!epb || !bpb) {
        set_error("dequantize_range: unsupported ggml type %d", t);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
    if (n == 0) return ANEDVD_OK;
    if (n % epb || elem_offset % epb) {
        set_error("dequantize_range: %zu elements at offset %llu are not whole blocks of %d", n,
                  (unsigned long long)elem_offset, epb);
        return ANEDVD_E_INVALID_SHAPE;
    }
    const uint64_t blocks_before = elem_offset / epb;
    if (blocks_before > UINT64_MAX / bpb || blocks_before * bpb > src_len) {
        set_error("dequantize_range: offset past the end of the data");
        return ANEDVD_E_TRUNCATED;
    }
    const size_t start = (size_t)(blocks_before * bpb), blocks = n / epb;
    if (src_len - start < blocks * (size_t)bpb) {
        set_error("dequantize_range: %zu blocks need %zu bytes, %zu available", blocks, blocks * (size_t)bpb, src_len - start);
        return ANEDVD_E_TRUNCATED;
    }
    if (!ctx || !src || !out) {
        set_error("dequantize_range: null argument");
        return ANEDVD_E_INVALID_ARG;
    }
    ANEDVD_HIP(hipSetDevice(ctx->device));
    const size_t in_b = blocks * bpb, out_b = n * sizeof(float);
    ANEDVD_TRY(ensure(ctx->io, in_b + out_b + 512, ctx->stream));
    uint8_t *d_in = (uint8_t *)ctx->io.base;
    float *d_out = (float *)((uint8_t *)ctx->io.base + ((in_b + 255) & ~(size_t)255));
    ANEDVD_HIP(hipMemcpyAsync(d_in, (const uint8_t *)src + start, in_b, hipMemcpyHostToDevice, ctx->stream));
    ANEDVD_TRY(launch_dequant_gguf(t, d_in, blocks, d_out, ctx->stream));
    ANEDVD_HIP(hipMemcpyAsync(out, d_out, out_b, hipMemcpyDeviceToHost, ctx->stream));
    ANEDVD_HIP(hipStreamSynchronize(ctx->stream));
    return ANEDVD_OK;
}

int anedvd_moe_load_expert_f32(anedvd_moe_layer *L, int which, uint32_t expert, float *out, size_t n)
{
    ANEDVD_TRY(check_layer(L));
    const QMat *m = which == 0 ? &L->gate : which == 1 ? &L->up : which == 2 ? &L->down : nullptr;
    if (!m || !out) {
        set_error("load_expert_f32: which must be 0 (gate), 1 (up) or 2 (down)");
        return ANEDVD_E_INVALID_ARG;
    }
    if (expert >= L->E) {
        set_error("load_expert_f32: expert %u of %u", expert, L->E);
        return ANEDVD_E_OUT_OF_RANGE;
    }
    if (n != (size_t)m->rows * m->cols) {
        set_error("load_expert_f32: out holds %zu, expert has %d x %d", n, m->rows, m->cols);
        return ANEDVD_E_DIMENSION;
    }
    anedvd_moe_ctx *ctx = L->ctx;
    ANEDVD_HIP(hipSetDevice(ctx->device));
    ANEDVD_TRY(ensure(ctx->io, n * sizeof(float), ctx->stream));
    ANEDVD_TRY(launch_dequant_tiles(*m, (int)expert, (float *)ctx->io.base, ctx->stream));
    ANEDVD_HIP(hipMemcpyAsync(out, ctx->io.base, n * sizeof(float), hipMemcpyDeviceToHost, ctx->stream));
    ANEDVD_HIP(hipStreamSynchronize(ctx->stream));
    return ANEDVD_OK;
}

int anedvd_moe_load_expert_f16(anedvd_moe_layer *L, int which, uint32_t expert, uint16_t *out, size_t n)
{
    ANEDVD_TRY(check_layer(L));
    const QMat *m = which == 0 ? &L->gate : which == 1 ? &L->up : which == 2 ? &L->down : nullptr;
    if (!m || !out) {
        set_error("load_expert_f16: which must be 0 (gate), 1 (up) or 2 (down)");
        return ANEDVD_E_INVALID_ARG;
    }
    if (expert >= L->E) {
        set_error("load_expert_f16: expert %u of %u", expert, L->E);
        return ANEDVD_E_OUT_OF_RANGE;
    }
    if (n != (size_t)m->rows * m->cols) {
        set_error("load_expert_f16: out holds %zu, expert has %d x %d", n, m->rows, m->cols);
        return ANEDVD_E_DIMENSION;
    }
    // readExpertF16 dequantises 2048-element chunks and rounds each (gguf.zig:521-530);
    // the chunks are whole blocks, so dequantising the expert at once and rounding
    // every value gives the same f16 values.
    anedvd_moe_ctx *ctx = L->ctx;
    ANEDVD_HIP(hipSetDevice(ctx->device));
    const size_t f32b = (n * sizeof(float) + 255) & ~(size_t)255;
    ANEDVD_TRY(ensure(ctx->io, f32b + n * sizeof(uint16_t), ctx->stream));
    float *d32 = (float *)ctx->io.base;
    uint16_t *d16 = (uint16_t *)((uint8_t *)ctx->io.base + f32b);
    ANEDVD_TRY(launch_dequant_tiles(*m, (int)expert, d32, ctx->stream));
    ANEDVD_TRY(launch_f32_to_f16(d32, d16, n, ctx->stream));
    ANEDVD_HIP(hipMemcpyAsync(out, d16, n * sizeof(uint16_t), hipMemcpyDeviceToHost, ctx->stream));
    ANEDVD_HIP(hipStreamSynchronize(ctx->stream));
    return ANEDVD_OK;
}

int anedvd_matmul_f16(anedvd_moe_ctx *ctx, float *out, const uint16_t *w, const float *x, size_t out_dim,
                      size_t in_dim, size_t n_vec)
{
    if (!ctx || !out || !w || !x || !out_dim || !in_dim || out_dim > (1u << 30) || in_dim > (1u << 20)) {
        set_error("matmul_f16: bad arguments");
        return ANEDVD_E_INVALID_ARG;
    }
    if (!n_vec) return ANEDVD_OK;
    ANEDVD_HIP(hipSetDevice(ctx->device));
    const size_t wb = out_dim * in_dim * 2, xb = n_vec * in_dim * 4, ob = n_vec * out_dim * 4;
    const size_t nwt = router_layout_floats((int)out_dim, (int)in_dim);
    ANEDVD_TRY(ensure(ctx->io, wb + nwt * 4 + xb + ob + 1024, ctx->stream));
    Carve c{(uint8_t *)ctx->io.base};
    uint16_t *dw = c.take<uint16_t>(out_dim * in_dim);
    float *dwt = c.take<float>(nwt);
    float *dx = c.take<float>(n_vec * in_dim);
    float *dout = c.take<float>(n_vec * out_dim);
    ANEDVD_HIP(hipMemcpyAsync(dw, w, wb, hipMemcpyHostToDevice, ctx->stream));
    ANEDVD_HIP(hipMemcpyAsync(dx, x, xb, hipMemcpyHostToDevice, ctx->stream));
    ANEDVD_TRY(launch_router_layout(dw, (int)out_dim, (int)in_dim, dwt, ctx->stream));
    ANEDVD_TRY(launch_router(dwt, dw, dx, (int)n_vec, (int)out_dim, (int)in_dim, dout, ctx->stream));
    ANEDVD_HIP(hipMemcpyAsync(out, dout, ob, hipMemcpyDeviceToHost, ctx->stream));
    ANEDVD_HIP(hipStreamSynchronize(ctx->stream));
    return ANEDVD_OK;
}

int anedvd_moe_route(anedvd_moe_ctx *ctx, const float *logits, size_t T, size_t E, size_t k, int norm, float *probs,
                     uint32_t *idx)
{
    if (!ctx || !logits || !probs || !idx || T > (1u << 24)) {
        set_error("moe_route: bad arguments");
        return ANEDVD_E_INVALID_ARG;
    }
    if (!T) return ANEDVD_OK;
    ANEDVD_HIP(hipSetDevice(ctx->device));
    ANEDVD_TRY(ensure(ctx->io, T * E * 4 + T * k * 20 + E * 8 + 8192, ctx->stream));
    Carve c{(uint8_t *)ctx->io.base};
    float *dl = c.take<float>(T * E);
    float *dp = c.take<float>(T * k);
    uint32_t *di = c.take<uint32_t>(T * k);
    ANEDVD_HIP(hipMemcpyAsync(dl, logits, T * E * 4, hipMemcpyHostToDevice, ctx->stream));
    if (route_fusable((int)T, (int)E)) {
        // the layer forward's small-call kernel (routing and dispatch in one launch),
        // so this entry point checks the routing it does; the dispatch is discarded
        Dispatch d{};
        d.offsets = c.take<int32_t>(E + 1);
        d.rows = c.take<int32_t>(T * k);
        d.slots = c.take<int32_t>(T * k);
        d.inv = c.take<int32_t>(T * k);
        d.active = c.take<int32_t>(E);
        d.meta = c.take<int32_t>(4);
        d.chunk = 16;
        d.n_routed = (int)E;
        ANEDVD_TRY(launch_route_and_dispatch(dl, (int)T, (int)E, (int)k, norm, dp, di, nullptr, 0, ActQ{}, d,
                                             ctx->stream, SharedSlots{}));
    } else {
        ANEDVD_TRY(launch_route(dl, (int)T, (int)E, (int)k, norm, dp, di, nullptr, 0, ActQ{}, ctx->stream));
    }
    ANEDVD_HIP(hipMemcpyAsync(probs, dp, T * k * 4, hipMemcpyDeviceToHost, ctx->stream));
    ANEDVD_HIP(hipMemcpyAsync(idx, di, T * k * 4, hipMemcpyDeviceToHost, ctx->stream));
    ANEDVD_HIP(hipStreamSynchronize(ctx->stream));
    return ANEDVD_OK;
}

int anedvd_moe_dispatch(anedvd_moe_ctx *ctx, const uint32_t *idx, size_t T, size_t k, size_t E, int32_t *offsets,
                        int32_t *rows, int32_t *slots)
{
    if (!ctx || !idx || !offsets || !rows || !slots || T > (1u << 24) || k > 64) {
        set_error("moe_dispatch: bad arguments");
        return ANEDVD_E_INVALID_ARG;
    }
    if (!T) {
        for (size_t e = 0; e <= E; e++) offsets[e] = 0;
        return ANEDVD_OK;
    }
    ANEDVD_HIP(hipSetDevice(ctx->device));
    const size_t P = T * k;
    ANEDVD_TRY(ensure(ctx->io, P * 16 + E * 8 + 4096, ctx->stream));
    Carve c{(uint8_t *)ctx->io.base};
    uint32_t *di = c.take<uint32_t>(P);
    int32_t *doff = c.take<int32_t>(E + 1);
    int32_t *drows = c.take<int32_t>(P);
    int32_t *dslots = c.take<int32_t>(P);
    int32_t *dinv = c.take<int32_t>(P);
    int32_t *dact = c.take<int32_t>(E);
    int32_t *dmeta = c.take<int32_t>(4);
    ANEDVD_HIP(hipMemcpyAsync(di, idx, P * 4, hipMemcpyHostToDevice, ctx->stream));
    const Dispatch dd{doff, drows, dslots, dinv, dact, dmeta, nullptr, 16};
    ANEDVD_TRY(launch_dispatch(di, (int)T, (int)k, (int)E, dd, ctx->stream));
    int32_t meta[4];
    ANEDVD_HIP(hipMemcpyAsync(offsets, doff, (E + 1) * 4, hipMemcpyDeviceToHost, ctx->stream));
    ANEDVD_HIP(hipMemcpyAsync(rows, drows, P * 4, hipMemcpyDeviceToHost, ctx->stream));
    ANEDVD_HIP(hipMemcpyAsync(slots, dslots, P * 4, hipMemcpyDeviceToHost, ctx->stream));
    ANEDVD_HIP(hipMemcpyAsync(meta, dmeta, 16, hipMemcpyDeviceToHost, ctx->stream));
    ANEDVD_HIP(hipStreamSynchronize(ctx->stream));
    if (meta[2]) {
        set_error("moe_dispatch: %d expert ids >= %zu", meta[2], E);
        return ANEDVD_E_OUT_OF_RANGE;
    }
    return ANEDVD_OK;
}

static int expert_accum_ops(anedvd_moe_ctx *ctx, bool f16, float *out, const float *h, const void *gate,
                            const void *up, const void *down, size_t inter, size_t hidden, float weight, int use_gelu)
{
    if (!ctx || !out || !h || !gate || !up || !down || !inter || !hidden || inter > (1u << 24) ||
        hidden > (1u << 24) || inter * hidden > ((size_t)1 << 31)) {
        set_error("expert_accum: bad arguments (inter %zu, hidden %zu)", inter, hidden);
        return ANEDVD_E_INVALID_ARG;
    }
    ANEDVD_HIP(hipSetDevice(ctx->device));
    const size_t wb = inter * hidden * (f16 ? 2 : 4);
    ANEDVD_TRY(ensure(ctx->io, 3 * (wb + 256) + (hidden + inter + hidden) * 4 + 1024, ctx->stream));
    Carve c{(uint8_t *)ctx->io.base};
    uint8_t *dg = c.take<uint8_t>(wb), *du = c.take<uint8_t>(wb), *dd = c.take<uint8_t>(wb);
    float *dh = c.take<float>(hidden), *dact = c.take<float>(inter), *dout = c.take<float>(hidden);
    hipStream_t st = ctx->stream;
    ANEDVD_HIP(hipMemcpyAsync(dg, gate, wb, hipMemcpyHostToDevice, st));
    ANEDVD_HIP(hipMemcpyAsync(du, up, wb, hipMemcpyHostToDevice, st));
    ANEDVD_HIP(hipMemcpyAsync(dd, down, wb, hipMemcpyHostToDevice, st));
    ANEDVD_HIP(hipMemcpyAsync(dh, h, hidden * 4, hipMemcpyHostToDevice, st));
    ANEDVD_HIP(hipMemcpyAsync(dout, out, hidden * 4, hipMemcpyHostToDevice, st));
    ANEDVD_TRY(launch_expert_accum_ops(f16, dg, du, dd, dh, (int)inter, (int)hidden, weight, use_gelu != 0, dact, dout,
                                       st));
    ANEDVD_HIP(hipMemcpyAsync(out, dout, hidden * 4, hipMemcpyDeviceToHost, st));
    ANEDVD_HIP(hipStreamSynchronize(st));
    return ANEDVD_OK;
}

int anedvd_moe_expert_accum_f32(anedvd_moe_ctx *ctx, float *out, const float *h, const float *gate, const float *up,
                                const float *down, size_t inter, size_t hidden, float weight, int use_gelu)
{
    return expert_accum_ops(ctx, false, out, h, gate, up, down, inter, hidden, weight, use_gelu);
}

int anedvd_moe_expert_accum_f16(anedvd_moe_ctx *ctx, float *out, const float *h, const uint16_t *gate,
                                const uint16_t *up, const uint16_t *down, size_t inter, size_t hidden, float weight,
                                int use_gelu)
{
    return expert_accum_ops(ctx, true, out, h, gate, up, down, inter, hidden, weight, use_gelu);
}

int anedvd_moe_expert_accum(anedvd_moe_layer *L, uint32_t expert, const float *h, float weight, float *out)
{
    ANEDVD_TRY(check_layer(L));
    if (!h || !out || expert >= L->E) {
        set_error("expert_accum: bad arguments (expert %u of %u)", expert, L->E);
        return ANEDVD_E_INVALID_ARG;
    }
    if (!mm_supported(L->gate.type) || !mm_supported(L->down.type)) {
        set_error("expert_accum: no expert kernel for types %d/%d", L->gate.type, L->down.type);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
    anedvd_moe_ctx *ctx = L->ctx;
    ANEDVD_HIP(hipSetDevice(ctx->device));
    // One token routed to `expert` with probability `weight`: the forward's
    // kernels on a one-entry dispatch; then out += the combined row
    // (`out[o] += weight * total`, cpu.zig:450).
    const int H = (int)L->H, I = (int)L->I, E = (int)L->E;
    Fwd f;
    const size_t bytes = fwd_layout(L, 1, 1, nullptr, (uint8_t *)0, true);
    ANEDVD_TRY(ensure(ctx->ws, bytes + 4096, ctx->stream));
    fwd_layout(L, 1, 1, &f, (uint8_t *)ctx->ws.base, true);
    std::vector<int32_t> off(E + 1);
    for (int e = 0; e <= E; e++) off[e] = e > (int)expert ? 1 : 0;
    const int32_t zero = 0, act = (int32_t)expert, meta[4] = {1, 1, 0, 1};
    const uint64_t chunk0 = chunk_entry((int)expert, 0, 1);
    hipStream_t st = ctx->stream;
    ANEDVD_HIP(hipMemcpyAsync(f.h_in, h, (size_t)H * 4, hipMemcpyHostToDevice, st));
    ANEDVD_HIP(hipMemcpyAsync(f.d.offsets, off.data(), (size_t)(E + 1) * 4, hipMemcpyHostToDevice, st));
    ANEDVD_HIP(hipMemcpyAsync(f.d.rows, &zero, 4, hipMemcpyHostToDevice, st));
    ANEDVD_HIP(hipMemcpyAsync(f.d.slots, &zero, 4, hipMemcpyHostToDevice, st));
    ANEDVD_HIP(hipMemcpyAsync(f.d.inv, &zero, 4, hipMemcpyHostToDevice, st));
    ANEDVD_HIP(hipMemcpyAsync(f.d.active, &act, 4, hipMemcpyHostToDevice, st));
    ANEDVD_HIP(hipMemcpyAsync(f.d.meta, meta, sizeof meta, hipMemcpyHostToDevice, st));
    ANEDVD_HIP(hipMemcpyAsync(f.d.chunks, &chunk0, sizeof chunk0, hipMemcpyHostToDevice, st));
    ANEDVD_HIP(hipMemcpyAsync(f.probs, &weight, 4, hipMemcpyHostToDevice, st));
    ANEDVD_TRY(launch_act_prep(f.h_in, 1, H, f.xq, st));
    ANEDVD_TRY(launch_expert_gateup(L->gate, L->up, f.xq, H, I, f.d, 1, f.plan, f.part, f.act, L->gelu, st));
    ANEDVD_TRY(launch_expert_down(L->down, f.act, H, I, f.d, 1, f.plan, f.part, L->gelu, f.ypart, 1, st));
    ANEDVD_TRY(launch_combine(f.ypart, f.d.inv, f.probs, 1, 1, H, f.plan.ks_dn, 1, nullptr, nullptr, 0, f.out, st));
    std::vector<float> y(H);
    ANEDVD_HIP(hipMemcpyAsync(y.data(), f.out, (size_t)H * 4, hipMemcpyDeviceToHost, st));
    ANEDVD_HIP(hipStreamSynchronize(st));
    for (int o = 0; o < H; o++) out[o] += y[o];
    return ANEDVD_OK;
}

// ------------------------------------------------------------------ layer

int anedvd_moe_layer_route(anedvd_moe_layer *L, const float *h, size_t T, float *logits, float *probs, uint32_t *idx)
{
    ANEDVD_TRY(check_layer(L));
    if (!h || !probs || !idx || T > (1u << 20)) {
        set_error("layer_route: bad arguments");
        return ANEDVD_E_INVALID_ARG;
    }
    if (!T) return ANEDVD_OK;
    anedvd_moe_ctx *ctx = L->ctx;
    ANEDVD_HIP(hipSetDevice(ctx->device));
    const size_t H = L->H, E = L->E, k = L->k;
    ANEDVD_TRY(ensure(ctx->io, T * H * 4 + T * E * 4 + T * k * 8 + 1024, ctx->stream));
    Carve c{(uint8_t *)ctx->io.base};
    float *dh = c.take<float>(T * H);
    float *dl = c.take<float>(T * E);
    float *dp = c.take<float>(T * k);
    uint32_t *di = c.take<uint32_t>(T * k);
    ANEDVD_HIP(hipMemcpyAsync(dh, h, T * H * 4, hipMemcpyHostToDevice, ctx->stream));
    ANEDVD_TRY(launch_router(L->router_t, L->router, dh, (int)T, (int)E, (int)H, dl, ctx->stream));
    ANEDVD_TRY(launch_route(dl, (int)T, (int)E, (int)k, L->norm, dp, di, nullptr, 0, ActQ{}, ctx->stream));
    if (logits) ANEDVD_HIP(hipMemcpyAsync(logits, dl, T * E * 4, hipMemcpyDeviceToHost, ctx->stream));
    ANEDVD_HIP(hipMemcpyAsync(probs, dp, T * k * 4, hipMemcpyDeviceToHost, ctx->stream));
    ANEDVD_HIP(hipMemcpyAsync(idx, di, T * k * 4, hipMemcpyDeviceToHost, ctx->stream));
    ANEDVD_HIP(hipStreamSynchronize(ctx->stream));
    return ANEDVD_OK;
}

// The checks every forward entry point makes before it touches memory; makes the
// layer's device current.
static int check_forward(anedvd_moe_layer *L, size_t T)
{
    ANEDVD_TRY(check_layer(L));
    if (T > max_tokens(L)) {
        set_error("forward: %zu tokens is more than one call takes at this shape (%zu; "
                  "anedvd_moe_layer_max_tokens): split the call", T, max_tokens(L));
        return ANEDVD_E_INVALID_ARG;
    }
    ANEDVD_HIP(hipSetDevice(L->ctx->device));
    if (!mm_supported(L->gate.type) || !mm_supported(L->down.type) || L->gate.type != L->up.type ||
        (L->Is && !L->n_sh && (!mm_supported(L->sgate.type) || !mm_supported(L->sdown.type)))) {
        set_error("forward: no expert kernel for ggml types gate=%d up=%d down=%d", L->gate.type, L->up.type,
                  L->down.type);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
    return ANEDVD_OK;
}

static int prepare(anedvd_moe_layer *L, size_t T, bool io, Fwd &f)
{
    ANEDVD_TRY(check_forward(L, T));
    anedvd_moe_ctx *ctx = L->ctx;
    const int ks = (int)(L->k + L->n_sh);
    const size_t bytes = fwd_layout(L, (int)T, ks, nullptr, (uint8_t *)0, io);
    ANEDVD_TRY(ensure(ctx->ws, bytes + 4096, ctx->stream));
    fwd_layout(L, (int)T, ks, &f, (uint8_t *)ctx->ws.base, io);
    return ANEDVD_OK;
}

int anedvd_moe_layer_forward(anedvd_moe_layer *L, const float *h, size_t T, const float *logits, float *out,
                             anedvd_moe_stats *stats)
{
    if (!h || !out) {
        set_error("layer_forward: null h or out");
        return ANEDVD_E_INVALID_ARG;
    }
    Fwd f;
    ANEDVD_TRY(prepare(L, T, true, f));
    if (!T) return ANEDVD_OK;
    hipStream_t st = L->ctx->stream;
    ANEDVD_HIP(hipMemcpyAsync(f.h_in, h, T * L->H * 4, hipMemcpyHostToDevice, st));
    if (logits) ANEDVD_HIP(hipMemcpyAsync(f.l_in, logits, T * L->E * 4, hipMemcpyHostToDevice, st));
    ANEDVD_TRY(forward_device(L, f.h_in, (int)T, logits ? f.l_in : nullptr, f.out, f, st, nullptr));
    int32_t meta[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    ANEDVD_HIP(hipMemcpyAsync(out, f.out, T * L->H * 4, hipMemcpyDeviceToHost, st));
    ANEDVD_HIP(hipMemcpyAsync(meta, f.d.meta, sizeof(meta), hipMemcpyDeviceToHost, st));
    ANEDVD_HIP(hipStreamSynchronize(st));
    if (stats) {
        stats->n_tokens = (uint32_t)T;
        const int touched = meta[0] - (T ? (int)L->n_sh : 0);  // the merged shared pieces are always active
        stats->touched_experts = (uint32_t)touched;
        stats->max_group = (uint32_t)meta[1];
        stats->weight_bytes = (uint64_t)(touched * L->expert_bytes + L->shared_bytes + (logits ? 0.0 : 2.0 * L->E * L->H));
        stats->path = f.plan.kind == kMmStaged ? 1 : 0;
        stats->chunk = (uint32_t)f.plan.chunk;
        stats->down_ks = (uint32_t)f.plan.ks_dn;
        stats->small_groups = f.plan.small ? (uint32_t)meta[7] : 0u;
    }
    return ANEDVD_OK;
}

int anedvd_moe_layer_route_counts(anedvd_moe_layer *L, uint32_t *counts, uint32_t *n_tokens)
{
    if (!L || !counts) {
        set_error("layer_route_counts: null layer or counts");
        return ANEDVD_E_INVALID_ARG;
    }
    anedvd_moe_ctx *ctx = L->ctx;
    if (ctx->last_layer != L || !ctx->last_offsets) {
        set_error("layer_route_counts: the last forward call on this context was not this layer's");
        return ANEDVD_E_INVALID_ARG;
    }
    std::vector<int32_t> off(L->E + 1);
    ANEDVD_HIP(hipMemcpyAsync(off.data(), ctx->last_offsets, off.size() * 4, hipMemcpyDeviceToHost, ctx->stream));
    ANEDVD_HIP(hipStreamSynchronize(ctx->stream));
    for (uint32_t e = 0; e < L->E; e++) counts[e] += (uint32_t)(off[e + 1] - off[e]);
    if (n_tokens) *n_tokens += (uint32_t)ctx->last_tokens;
    return ANEDVD_OK;
}

int anedvd_moe_layer_forward_device(anedvd_moe_layer *L, const float *d_h, size_t T, const float *d_logits, float *d_out)
{
    if (!d_h || !d_out) {
        set_error("layer_forward_device: null pointer");
        return ANEDVD_E_INVALID_ARG;
    }
    Fwd f;
    ANEDVD_TRY(prepare(L, T, false, f));
    if (!T) return ANEDVD_OK;
    return forward_device(L, d_h, (int)T, d_logits, d_out, f, L->ctx->stream, nullptr);
}

int anedvd_moe_layer_forward_device_f16(anedvd_moe_layer *L, const uint16_t *d_h, size_t T, const float *d_logits,
                                        float *d_out)
{
    if (!d_h || !d_out) {
        set_error("layer_forward_device_f16: null pointer");
        return ANEDVD_E_INVALID_ARG;
    }
    Fwd f;
    ANEDVD_TRY(prepare(L, T, true, f));
    if (!T) return ANEDVD_OK;
    hipStream_t st = L->ctx->stream;
    ANEDVD_TRY(launch_f16_to_f32(d_h, f.h_in, T * L->H, st));
    return forward_device(L, f.h_in, (int)T, d_logits, d_out, f, st, nullptr);
}

int anedvd_moe_layer_forward_device_noalloc(anedvd_moe_layer *L, const float *d_h, size_t T, const float *d_logits,
                                            float *d_out)
{
    if (!d_h || !d_out) {
        set_error("layer_forward_device_noalloc: null pointer");
        return ANEDVD_E_INVALID_ARG;
    }
    ANEDVD_TRY(check_forward(L, T));
    if (!T) return ANEDVD_OK;
    const int ks = (int)(L->k + L->n_sh);
    const size_t need = fwd_layout(L, (int)T, ks, nullptr, (uint8_t *)0, false);
    if (need > kNoAllocScratchBytes) {
        size_t lo = 0, hi = T;  // the largest call that fits, for the message
        while (hi - lo > 1) {
            const size_t mid = (lo + hi) / 2;
            (fwd_layout(L, (int)mid, ks, nullptr, (uint8_t *)0, false) <= kNoAllocScratchBytes ? lo : hi) = mid;
        }
        set_error("layer_forward_device_noalloc: %zu tokens need %zu bytes of scratch, more than its %zu; "
                  "at most %zu tokens per call at this shape",
                  T, need, kNoAllocScratchBytes, lo);
        return ANEDVD_E_INVALID_ARG;
    }
    uint8_t *base = (uint8_t *)scratch_of(L->ctx->device);
    if (!base) {  // the lookup at open failed: once more here (no allocation), reporting why
        ANEDVD_HIP(hipSetDevice(L->ctx->device));
        const int rc = scratch_setup(L->ctx->device);
        if (rc != ANEDVD_OK) return rc == ANEDVD_E_HIP ? ANEDVD_E_NO_DEVICE : rc;
        base = (uint8_t *)scratch_of(L->ctx->device);
    }
    Fwd f;
    fwd_layout(L, (int)T, ks, &f, base, false);
    return forward_device(L, d_h, (int)T, d_logits, d_out, f, L->ctx->stream, nullptr);
}

// ------------------------------------------------------------ memory, timing

int anedvd_moe_device_alloc(anedvd_moe_ctx *ctx, size_t bytes, void **p)
{
    if (!ctx || !p) return ANEDVD_E_INVALID_ARG;
    ANEDVD_HIP(hipSetDevice(ctx->device));
    ANEDVD_HIP(hipMalloc(p, bytes));
    return ANEDVD_OK;
}

int anedvd_moe_device_free(anedvd_moe_ctx *ctx, void *p)
{
    if (!ctx) return ANEDVD_E_INVALID_ARG;
    ANEDVD_HIP(hipSetDevice(ctx->device));
    ANEDVD_HIP(hipStreamSynchronize(ctx->stream));
    ANEDVD_HIP(hipFree(p));
    return ANEDVD_OK;
}

int anedvd_moe_memcpy_h2d(anedvd_moe_ctx *ctx, void *d, const void *s, size_t n)
{
    if (!ctx) return ANEDVD_E_INVALID_ARG;
    ANEDVD_HIP(hipMemcpyAsync(d, s, n, hipMemcpyHostToDevice, ctx->stream));
    ANEDVD_HIP(hipStreamSynchronize(ctx->stream));
    return ANEDVD_OK;
}

int anedvd_moe_memcpy_d2h(anedvd_moe_ctx *ctx, void *d, const void *s, size_t n)
{
    if (!ctx) return ANEDVD_E_INVALID_ARG;
    ANEDVD_HIP(hipMemcpyAsync(d, s, n, hipMemcpyDeviceToHost, ctx->stream));
    ANEDVD_HIP(hipStreamSynchronize(ctx->stream));
    return ANEDVD_OK;
}

int anedvd_moe_synchronize(anedvd_moe_ctx *ctx)
{
    if (!ctx) return ANEDVD_E_INVALID_ARG;
    ANEDVD_HIP(hipStreamSynchronize(ctx->stream));
    return ANEDVD_OK;
}

int anedvd_moe_time_forward(anedvd_moe_layer *const *layers, size_t n_layers, const float *d_h, size_t T,
                            const float *d_logits, float *d_out, int warmup, int iters, int flags, float *ms,
                            float *kernel_ms)
{
    if (!layers || !n_layers || !ms || iters <= 0 || warmup < 0) {
        set_error("time_forward: bad arguments");
        return ANEDVD_E_INVALID_ARG;
    }
    anedvd_moe_ctx *ctx = layers[0]->ctx;
    for (size_t i = 0; i < n_layers; i++)
        if (!layers[i] || layers[i]->ctx != ctx || layers[i]->H != layers[0]->H || layers[i]->E != layers[0]->E ||
            layers[i]->I != layers[0]->I || layers[i]->k != layers[0]->k || layers[i]->Is != layers[0]->Is ||
            layers[i]->n_sh != layers[0]->n_sh) {
            set_error("time_forward: layers must share a context and a shape");
            return ANEDVD_E_INVALID_ARG;
        }
    const bool chain = (flags & ANEDVD_TIME_CHAIN) != 0;
    if (chain && (flags & (ANEDVD_TIME_GRAPH | ANEDVD_TIME_EXPERT_SOLO))) {
        set_error("time_forward: a chained stack is timed with directly launched calls and stage events only");
        return ANEDVD_E_INVALID_ARG;
    }
    hipStream_t st = ctx->stream;
    Fwd f;
    ANEDVD_TRY(prepare(layers[0], T, false, f));
    // Call i: layer i mod n.  Chained, the layers form a stack: each pass over it
    // starts from d_h, layer j reads the previous layer's x (two ping-pong buffers)
    // and writes x + its block output, layer j routes logits row block j of
    // d_logits, and the last layer writes d_out.
    const size_t H = layers[0]->H, E = layers[0]->E;
    float *pp[2] = {nullptr, nullptr};
    struct PpFree {
        float **p;
        ~PpFree()
        {
            for (int i = 0; i < 2; i++)
                if (p[i]) (void)hipFree(p[i]);
        }
    } pp_free{pp};
    if (chain && n_layers > 1)
        for (int i = 0; i < 2; i++) ANEDVD_HIP(hipMalloc(&pp[i], T * H * sizeof(float)));
    struct Call {
        anedvd_moe_layer *L;
        const float *in, *logits, *resid;
        float *out;
    };
    auto call_of = [&](int i) -> Call {
        const size_t j = (size_t)i % n_layers;
        if (!chain) return Call{layers[j], d_h, d_logits, nullptr, d_out};
        const float *in = j == 0 ? d_h : pp[(j - 1) % 2];
        float *out = j + 1 == n_layers ? d_out : pp[j % 2];
        return Call{layers[j], in, d_logits ? d_logits + j * T * E : nullptr, in, out};
    };
    auto run_call = [&](int i, hipEvent_t *ev) -> int {
        const Call c = call_of(i);
        return forward_device(c.L, c.in, (int)T, c.logits, c.out, f, st, ev, c.resid);
    };
    // With ANEDVD_TIME_GRAPH each layer's forward is captured once into a HIP graph
    // and the timed loop replays the graphs (one submission per call).
    std::vector<hipGraphExec_t> execs;
    auto destroy = [&]() {
        for (auto &e : execs) (void)hipGraphExecDestroy(e);
        execs.clear();
    };
    if (flags & ANEDVD_TIME_GRAPH) {
        for (size_t i = 0; i < n_layers; i++) {
            ANEDVD_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
            const int rc = run_call((int)i, nullptr);
            hipGraph_t g = nullptr;
            const hipError_t e = hipStreamEndCapture(st, &g);
            if (rc != ANEDVD_OK || e != hipSuccess) {
                if (g) (void)hipGraphDestroy(g);
                destroy();
                if (rc == ANEDVD_OK) set_error("time_forward: graph capture failed: %s", hipGetErrorString(e));
                return rc != ANEDVD_OK ? rc : ANEDVD_E_HIP;
            }
            hipGraphExec_t x = nullptr;
            const hipError_t e2 = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            if (e2 != hipSuccess) {
                destroy();
                set_error("time_forward: graph instantiation failed: %s", hipGetErrorString(e2));
                return ANEDVD_E_HIP;
            }
            execs.push_back(x);
        }
    }
    auto step = [&](int i) -> int {
        if (!execs.empty()) {
            const hipError_t e = hipGraphLaunch(execs[(size_t)i % n_layers], st);
            if (e != hipSuccess) {
                set_error("time_forward: graph launch failed: %s", hipGetErrorString(e));
                return ANEDVD_E_HIP;
            }
            return ANEDVD_OK;
        }
        return run_call(i, nullptr);
    };
    int rc = ANEDVD_OK;
    for (int i = 0; i < warmup && rc == ANEDVD_OK; i++) rc = step(i);
    hipEvent_t t0 = nullptr, t1 = nullptr;
    if (rc == ANEDVD_OK && (hipEventCreate(&t0) != hipSuccess || hipEventCreate(&t1) != hipSuccess)) {
        set_error("time_forward: event creation failed");
        rc = ANEDVD_E_HIP;
    }
    if (rc == ANEDVD_OK && (hipStreamSynchronize(st) != hipSuccess || hipEventRecord(t0, st) != hipSuccess)) {
        set_error("time_forward: synchronisation failed");
        rc = ANEDVD_E_HIP;
    }
    for (int i = 0; i < iters && rc == ANEDVD_OK; i++) rc = step(i);
    if (rc == ANEDVD_OK && (hipEventRecord(t1, st) != hipSuccess || hipEventSynchronize(t1) != hipSuccess ||
                            hipEventElapsedTime(ms, t0, t1) != hipSuccess)) {
        set_error("time_forward: timing failed");
        rc = ANEDVD_E_HIP;
    }
    if (t0) (void)hipEventDestroy(t0);
    if (t1) (void)hipEventDestroy(t1);
    destroy();
    if (rc != ANEDVD_OK) return rc;
    if (kernel_ms) {
        std::vector<hipEvent_t> ev((size_t)iters * 6);
        for (auto &e : ev) ANEDVD_HIP(hipEventCreate(&e));
        for (int i = 0; i < iters; i++) ANEDVD_TRY(run_call(i, &ev[(size_t)i * 6]));
        ANEDVD_HIP(hipStreamSynchronize(st));
        double acc[6] = {0, 0, 0, 0, 0, 0};
        for (int i = 0; i < iters; i++) {
            hipEvent_t *e = &ev[(size_t)i * 6];
            float x;
            for (int s = 0; s < 5; s++) {
                ANEDVD_HIP(hipEventElapsedTime(&x, e[s], e[s + 1]));
                acc[s] += x;
            }
            ANEDVD_HIP(hipEventElapsedTime(&x, e[0], e[5]));
            acc[5] += x;
        }
        // order: route, gate/up, down, shared, combine, total
        for (int s = 0; s < 6; s++) kernel_ms[s] = (float)(acc[s] / iters);
        for (auto &e : ev) (void)hipEventDestroy(e);
    }
    if (kernel_ms && (flags & ANEDVD_TIME_EXPERT_SOLO)) {
        // The routed expert products alone: `iters` back-to-back launches of the
        // gate/up (then the down) kernels over the rotated layers, reading the
        // dispatch, activations and gate/up output the last call left in place (the
        // calls above routed the same inputs).  Events bracket each loop only.  Then
        // the router GEMV kernel alone (a call of a few tokens forms its logits in
        // the routing launch instead; this times the separate kernel).
        const int H = layers[0]->H, I = layers[0]->I, P = (int)T * (int)(layers[0]->k + layers[0]->n_sh);
        hipEvent_t a = nullptr, b = nullptr;
        ANEDVD_HIP(hipEventCreate(&a));
        ANEDVD_HIP(hipEventCreate(&b));
        int src = ANEDVD_OK;
        for (int s = 0; s < 3 && src == ANEDVD_OK; s++) {
            auto launch = [&](int i) -> int {
                const anedvd_moe_layer *L = layers[(size_t)i % n_layers];
                if (s == 2)  // the router GEMV alone: T tokens of d_h against the layer's [E][H] f16 router
                    return launch_router(L->router_t, L->router, d_h, (int)T, (int)L->E, H, f.logits, st);
                return s == 0 ? launch_expert_gateup(L->gate, L->up, f.xq, H, I, f.d, P, f.plan, f.part, f.act,
                                                     L->gelu, st)
                              : launch_expert_down(L->down, f.act, H, I, f.d, P, f.plan, f.part, L->gelu, f.ypart,
                                                   (int)(L->k + L->n_sh), st);
            };
            for (int i = 0; i < warmup && src == ANEDVD_OK; i++) src = launch(i);
            if (src == ANEDVD_OK && hipEventRecord(a, st) != hipSuccess) src = ANEDVD_E_HIP;
            for (int i = 0; i < iters && src == ANEDVD_OK; i++) src = launch(i);
            float x = 0.0f;
            if (src == ANEDVD_OK && (hipEventRecord(b, st) != hipSuccess || hipEventSynchronize(b) != hipSuccess ||
                                     hipEventElapsedTime(&x, a, b) != hipSuccess)) {
                set_error("time_forward: expert timing failed");
                src = ANEDVD_E_HIP;
            }
            kernel_ms[s == 2 ? 0 : 1 + s] = x / iters;
        }
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
        if (src != ANEDVD_OK) return src;
    }
    return ANEDVD_OK;
}

}  // extern "C"
