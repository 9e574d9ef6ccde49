/*
 * anedvd_moe.h -- C ABI of the MI355X (gfx950) quantised mixture-of-experts FFN.
 *
 * Replaces, for ANEDVD's MoE block, the in-process Zig calls of src/cpu.zig and
 * the expert reads of src/gguf.zig.  Conventions follow the reference's only
 * foreign ABI, src/ane/shim.h:
 *   - opaque handles;
 *   - int status, 0 = ok, < 0 = error (shim.h:49-57);
 *   - a thread-local, human-readable last error (shim.h:55-57);
 *   - caller-owned buffers; nothing returned needs freeing except handles.
 * Entry points taking `const float *h` etc. without a `_device` suffix take HOST
 * pointers and are synchronous: results are in host memory on return.
 *
 * Threading: one caller thread per context (the engine is single-threaded,
 * engine.zig:1-17); each context owns one HIP stream.
 */
#ifndef ANEDVD_MOE_H
#define ANEDVD_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ANEDVD_MOE_ABI_VERSION 5

/* ggml tensor type ids as stored in GGUF (gguf.zig:30-46). */
enum anedvd_ggml_type {
    ANEDVD_F32 = 0, ANEDVD_F16 = 1, ANEDVD_Q4_0 = 2, ANEDVD_Q4_1 = 3, ANEDVD_Q5_0 = 6,
    ANEDVD_Q5_1 = 7, ANEDVD_Q8_0 = 8, ANEDVD_Q8_1 = 9, ANEDVD_Q2_K = 10, ANEDVD_Q3_K = 11,
    ANEDVD_Q4_K = 12, ANEDVD_Q5_K = 13, ANEDVD_Q6_K = 14, ANEDVD_Q8_K = 15, ANEDVD_BF16 = 30
};

/* Status codes.  -1..-5 are the Zig errors of the replaced functions
 * (gguf.zig:694-728, 533-552); the rest are this library's. */
enum anedvd_status {
    ANEDVD_OK = 0,
    ANEDVD_E_UNSUPPORTED_TYPE = -1,  /* error.UnsupportedType */
    ANEDVD_E_INVALID_SHAPE = -2,     /* error.InvalidTensorShape */
    ANEDVD_E_TRUNCATED = -3,         /* error.TruncatedFile */
    ANEDVD_E_DIMENSION = -4,         /* error.DimensionMismatch */
    ANEDVD_E_OUT_OF_RANGE = -5,      /* error.TensorDataOutOfRange */
    ANEDVD_E_INVALID_ARG = -6,
    ANEDVD_E_HIP = -7,               /* a HIP runtime call failed; see last_error */
    ANEDVD_E_NO_DEVICE = -8,
    /* GGUF container and loader errors (gguf.zig:587-657, load_gguf.zig:109-128, 358-386) */
    ANEDVD_E_NOT_GGUF = -9,          /* error.NotGgufFile */
    ANEDVD_E_GGUF_VERSION = -10,     /* error.UnsupportedVersion */
    ANEDVD_E_INVALID_METADATA = -11, /* error.InvalidMetadata / TooMany* / UnsupportedMetadataType / no experts */
    ANEDVD_E_MISSING_TENSOR = -12    /* error.MissingTensor: a tensor or config key the layer needs */
};

typedef struct anedvd_moe_ctx anedvd_moe_ctx;
typedef struct anedvd_moe_layer anedvd_moe_layer;

/* One MoE layer, as ANEDVD's loaders hand it over (load_gguf.zig:767-826,
 * model.zig:414-470).  Expert tensors are the GGUF payloads of
 * blk.N.ffn_{gate,up,down}_exps.weight: E experts stacked on the slowest axis,
 * each expert [out][in] row-major with quant blocks along `in`.  All pointers are
 * host memory and may be freed once anedvd_moe_layer_create returns. */
typedef struct {
    uint32_t hidden;          /* H */
    uint32_t inter;           /* I, one routed expert's width (Config.moe_inter) */
    uint32_t n_experts;       /* E */
    uint32_t k;               /* experts per token */
    int32_t norm_topk_prob;   /* renormalise the top-k weights (Config.norm_topk_prob) */
    int32_t use_gelu;         /* geluTanh(gate)*up instead of silu(gate)*up (cpu.zig:78-81, 434-437) */
    int32_t gate_type, up_type, down_type;
    const void *gate; size_t gate_bytes;   /* [E][I][H] */
    const void *up;   size_t up_bytes;     /* [E][I][H] */
    const void *down; size_t down_bytes;   /* [E][H][I] */
    const uint16_t *router;                /* [E][H] f16 bits (MoeWeights.router) */
    uint32_t shared_inter;                 /* 0 = no shared expert */
    int32_t shared_type;                   /* one type for the three shared tensors */
    const void *shared_gate; size_t shared_gate_bytes;  /* [Is][H] */
    const void *shared_up;   size_t shared_up_bytes;    /* [Is][H] */
    const void *shared_down; size_t shared_down_bytes;  /* [H][Is] */
    const uint16_t *shared_gate_lin;       /* [H] f16 bits, or NULL: shared scale 1.0 */
} anedvd_moe_layer_desc;

/* Filled by the forward calls when non-NULL. */
typedef struct {
    uint32_t n_tokens;
    uint32_t touched_experts;      /* experts with >= 1 routed token in this call */
    uint64_t weight_bytes;         /* expert + shared + router bytes the call had to read */
    uint32_t max_group;            /* largest tokens-per-expert group */
    uint32_t path;                 /* expert kernels: 0 = decode (16-token tiles), 1 = grouped GEMM */
    uint32_t chunk;                /* tokens per expert-kernel work item: 16, 64 or 128 */
    uint32_t down_ks;              /* K shares of the down product (partial planes the combine adds) */
    uint32_t small_groups;         /* grouped GEMM calls: groups of <= 16 tokens run on the decode kernels */
} anedvd_moe_stats;

/* ------------------------------------------------------------------ lifetime */

/* Human-readable description of the last failure on this thread (shim.h:55-57). */
const char *anedvd_moe_last_error(void);
int anedvd_moe_abi_version(void);

/* Opens `device` and creates the context's stream (ane_shim_init, shim.h:49-53). */
int anedvd_moe_open(int device, anedvd_moe_ctx **out);
void anedvd_moe_close(anedvd_moe_ctx *ctx);

/* Uploads one layer to HBM and repacks its quant blocks into the GPU tile layout,
 * keeping every weight's bytes and dequantised value (loadMoeLayerStreaming,
 * load_gguf.zig:767-826; MoeWeights, model.zig:414-470). */
int anedvd_moe_layer_create(anedvd_moe_ctx *ctx, const anedvd_moe_layer_desc *desc,
                            anedvd_moe_layer **out);
void anedvd_moe_layer_free(anedvd_moe_layer *layer);
/* Device bytes held by the layer's weights. */
uint64_t anedvd_moe_layer_device_bytes(const anedvd_moe_layer *layer);
/* The most tokens one forward call of this layer takes (the kernels address the
 * per-call activations with 32-bit offsets: T*H*2, T*(k + merged shared pieces)*I*2
 * and a separate shared expert's T*Is*2 bytes stay below 2^31).  Larger calls
 * return ANEDVD_E_INVALID_ARG; the engine's prefill chunks (Options.chunk = 128,
 * engine.zig:45) are far below it. */
size_t anedvd_moe_layer_max_tokens(const anedvd_moe_layer *layer);

/* ----------------------------------------------------- op-level mirrors of cpu.zig */

/* gguf.dequantizeRange (gguf.zig:694-728): dequantise `n` elements of GGUF blocks
 * starting at element `elem_offset`, bit-exact f32.  Same checks, same errors. */
int anedvd_dequantize_range(anedvd_moe_ctx *ctx, int ggml_type, const void *src, size_t src_len,
                            uint64_t elem_offset, float *out, size_t n);

/* MoeWeights.loadExpertF32 / Gguf.readExpertF32 (model.zig:519-541, gguf.zig:533-552)
 * from the resident layer: which 0 = gate, 1 = up, 2 = down; `out` holds
 * rows*cols f32, bit-exact. */
int anedvd_moe_load_expert_f32(anedvd_moe_layer *layer, int which, uint32_t expert, float *out, size_t n);

/* Gguf.readExpertF16 / MoeWeights.loadExpert (gguf.zig:499-531, model.zig:486-511)
 * from the resident layer: the expert dequantised and each value rounded to the
 * nearest f16, ties to even (f32ToF16Slice, gguf.zig:682-692); `out` holds
 * rows*cols f16 bits, bit-exact. */
int anedvd_moe_load_expert_f16(anedvd_moe_layer *layer, int which, uint32_t expert, uint16_t *out, size_t n);

/* cpu.matmulF16 (cpu.zig:461-475) over `n_vec` input vectors:
 * out[v][o] = sum_i f32(w[o][i]) * x[v][i], in the reference's 8-lane order,
 * bit-exact. */
int anedvd_matmul_f16(anedvd_moe_ctx *ctx, float *out, const uint16_t *w, const float *x,
                      size_t out_dim, size_t in_dim, size_t n_vec);

/* cpu.moeRoute (cpu.zig:1236-1288) for `n_tokens` rows of logits:
 * probs[t][k], idx[t][k].  Indices and probabilities are bit-exact. */
int anedvd_moe_route(anedvd_moe_ctx *ctx, const float *logits, size_t n_tokens, size_t n_experts,
                     size_t k, int norm_topk_prob, float *probs, uint32_t *idx);

/* Token-to-expert dispatch (engine.zig:1204-1216, expertWeightFor engine.zig:825-830):
 * offsets[E+1]; rows[T*k] = tokens grouped by expert, ascending within an expert;
 * slots[T*k] = which of the token's k slots chose that expert. */
int anedvd_moe_dispatch(anedvd_moe_ctx *ctx, const uint32_t *idx, size_t n_tokens, size_t k,
                        size_t n_experts, int32_t *offsets, int32_t *rows, int32_t *slots);

/* cpu.moeExpertAccumF32 (cpu.zig:416-452), the op-level drop-in: one token through
 * one expert handed over as f32 weight slices (host memory; gate and up
 * [inter][hidden], down [hidden][inter], as loadExpertF32 returns them):
 * out[hidden] += weight * down . (act(gate . h) * (up . h)), act = silu, or
 * geluTanh when use_gelu.  The reference's two scratch slices are the library's. */
int anedvd_moe_expert_accum_f32(anedvd_moe_ctx *ctx, float *out, const float *h, const float *gate,
                                const float *up, const float *down, size_t inter, size_t hidden,
                                float weight, int use_gelu);

/* cpu.moeExpertAccum (cpu.zig:1141-1185): the same with f16 weight slices (the
 * eager loader's MoeWeights.expertGate/Up/Down, model.zig:549-561). */
int anedvd_moe_expert_accum_f16(anedvd_moe_ctx *ctx, float *out, const float *h, const uint16_t *gate,
                                const uint16_t *up, const uint16_t *down, size_t inter, size_t hidden,
                                float weight, int use_gelu);

/* The same product for a resident expert of a layer (the layer's fused-dequant
 * kernels on a one-token dispatch; the streaming path's loadExpertF32 +
 * moeExpertAccumF32, engine.zig:743-758, without the f32 copy):
 * out[H] += weight * down(act(gate h) * up h). */
int anedvd_moe_expert_accum(anedvd_moe_layer *layer, uint32_t expert, const float *h, float weight,
                            float *out);

/* ------------------------------------------------------------ GGUF loading */

/* The MoE configuration of a GGUF file and the types of one block's tensors, as
 * load_gguf.zig:109-128 and 251-289 derive them (types are ggml type ids, -1 when
 * the tensor is absent). */
typedef struct {
    char arch[64];               /* general.architecture */
    uint32_t version;            /* GGUF version (2 or 3) */
    uint64_t n_tensors, data_offset;
    uint32_t hidden;             /* <arch>.embedding_length */
    uint32_t n_layers;           /* <arch>.block_count */
    uint32_t n_experts, k;       /* expert_count (blk.0.ffn_gate_exps wins), expert_used_count (2 if absent) */
    uint32_t inter;              /* routed expert width, from blk.0.ffn_gate_exps.weight or the metadata */
    uint32_t shared_inter;       /* 0 = no shared expert */
    int32_t gate_type, up_type, down_type, router_type, shared_type;  /* shared_type: of blk.N.ffn_gate_shexp */
    int32_t has_shared_gate_lin;
    int32_t use_gelu;            /* gelu(gate)*up: the gemma architectures (load_gguf.zig:145-158) */
    int32_t shared_as_f16;       /* the shared expert is read as f16 [out][in] (loadLinear, load_gguf.zig:358-386):
                                    a tensor stored {out, in}, three different types, or a type the
                                    expert kernels do not take; else its payloads are used as stored */
} anedvd_gguf_moe_cfg;

/* Options of anedvd_moe_layer_create_gguf; NULL or -1 fields = the reference GGUF
 * loader's values (norm_topk_prob false; use_gelu true for gemma* architectures). */
typedef struct {
    int32_t norm_topk_prob;
    int32_t use_gelu;
} anedvd_gguf_moe_opts;

/* Parses a GGUF v2/v3 image held in host memory (Gguf.parse, gguf.zig:587-657),
 * derives its MoE configuration and checks block `layer`'s tensors.  Host only:
 * no device is touched. */
int anedvd_gguf_moe_info(const void *gguf, size_t len, uint32_t layer, anedvd_gguf_moe_cfg *out);

/* loadMoeLayerStreaming (load_gguf.zig:767-826) onto the GPU: block `layer` of the
 * GGUF image (the caller maps the file; it may be unmapped on return).  The expert
 * payloads are uploaded as stored; the router and the shared gate vector are read
 * as f16 (any type, dequantised bit-exactly, rounded to nearest even); the shared
 * expert's tensors are uploaded as stored when they are {in, out} of one type the
 * expert kernels take, else read as f16 [out][in] as loadLinear does. */
int anedvd_moe_layer_create_gguf(anedvd_moe_ctx *ctx, const void *gguf, size_t len, uint32_t layer,
                                 const anedvd_gguf_moe_opts *opts, anedvd_moe_layer **out);

/* ---------------------------------------------------------------- the layer */

/* Router logits then moeRoute for T tokens (engine.zig:715-716, 1178-1179).
 * `logits` may be NULL. */
int anedvd_moe_layer_route(anedvd_moe_layer *layer, const float *h, size_t n_tokens,
                           float *logits, float *probs, uint32_t *idx);

/* The whole MoE block for T tokens (main.zig:488-520; engine.zig:705-779 decode,
 * 1158-1268 prefill): out[t] = sum over slots of p * expert(h_t) + s * shared(h_t),
 * s = sigmoid(shared_gate_lin . h_t) or 1.0.  `out` does not include the residual.
 * If `logits` is non-NULL the router GEMV is skipped and those [T][E] logits are
 * routed instead. */
int anedvd_moe_layer_forward(anedvd_moe_layer *layer, const float *h, size_t n_tokens,
                             const float *logits, float *out, anedvd_moe_stats *stats);

/* The engine's routing recorder (Engine.route_counts / route_tokens,
 * engine.zig:245-250, 726-731, 1190-1195): adds to counts[e], for the layer's
 * n_experts routed experts, how many of the last forward call's tokens chose
 * expert e (each token adds its k choices, as the engine's loop does; merged
 * shared-expert pieces are not counted), and the call's token count to
 * *n_tokens when n_tokens is non-NULL.  Pointing `counts` at route_counts +
 * layer * E keeps the engine's [layer][E] table through the drop-in.  It reads
 * the per-expert offsets the call's dispatch left on the device, so it refers to
 * the last forward call on the layer's context, whichever entry point made it;
 * if that call was another layer's, or there was none, it returns
 * ANEDVD_E_INVALID_ARG and adds nothing.  Synchronous (host memory). */
int anedvd_moe_layer_route_counts(anedvd_moe_layer *layer, uint32_t *counts, uint32_t *n_tokens);

/* Same with device pointers, stream-ordered on the context's stream, no host
 * synchronisation (stats are not filled). */
int anedvd_moe_layer_forward_device(anedvd_moe_layer *layer, const float *d_h, size_t n_tokens,
                                    const float *d_logits, float *d_out);

/* Same with f16 activations: d_h holds [T][H] IEEE binary16 bits (the fp16
 * activations of the benchmarked Mixtral-8x7B layer).  Each value is widened to
 * f32 exactly on the device and the call then equals anedvd_moe_layer_forward_device
 * on the widened rows, bit for bit (the reference's blocks take f32 h,
 * cpu.zig:1141-1185; main.zig:488-520).  Output and logits stay f32. */
int anedvd_moe_layer_forward_device_f16(anedvd_moe_layer *layer, const uint16_t *d_h, size_t n_tokens,
                                        const float *d_logits, float *d_out);

/* anedvd_moe_layer_forward_device without any allocation.  It has no counterpart
 * in the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).  The
 * per-call scratch comes from a static 64 MiB device array, one per GPU, held
 * until the process ends, instead of the context's workspace; no hipMalloc,
 * hipFree or allocating routine is called.  Calls whose scratch exceeds 64 MiB
 * return ANEDVD_E_INVALID_ARG, naming the most tokens that fit (Qwen3-30B-A3B
 * shape: 807 tokens; decode batches of 1-64 take under 6 MiB).  Every call
 * on one GPU shares that GPU's array: calls that overlap in time on one GPU (two
 * contexts' streams, or two threads) race and must be serialised by the caller. */
int anedvd_moe_layer_forward_device_noalloc(anedvd_moe_layer *layer, const float *d_h, size_t n_tokens,
                                            const float *d_logits, float *d_out);

/* ------------------------------------------------- device memory and timing */

int anedvd_moe_device_alloc(anedvd_moe_ctx *ctx, size_t bytes, void **d_ptr);
int anedvd_moe_device_free(anedvd_moe_ctx *ctx, void *d_ptr);
int anedvd_moe_memcpy_h2d(anedvd_moe_ctx *ctx, void *d_dst, const void *src, size_t bytes);
int anedvd_moe_memcpy_d2h(anedvd_moe_ctx *ctx, void *dst, const void *d_src, size_t bytes);
int anedvd_moe_synchronize(anedvd_moe_ctx *ctx);

/* Runs `warmup` untimed then `iters` timed forward calls, call j using
 * layers[j % n_layers], all inputs device-resident; the timed region is bracketed
 * by HIP events on the context's stream.  *ms = total milliseconds of the timed
 * region.  flags: ANEDVD_TIME_GRAPH captures each layer's forward once into a
 * HIP graph and replays it (one submission per call).  If `kernel_ms` is non-NULL,
 * a further pass of `iters` directly launched calls records events around every
 * stage and kernel_ms[0..5] receives the mean milliseconds per call of: route
 * (router + route + dispatch), expert gate/up, expert down, shared expert,
 * combine, and the whole call.  With ANEDVD_TIME_EXPERT_SOLO as well,
 * kernel_ms[1] and kernel_ms[2] are instead the mean milliseconds of one routed
 * gate/up (resp. down) launch, timed over `iters` back-to-back launches of that
 * stage alone (same layer rotation, the last call's dispatch and activations),
 * and kernel_ms[0] that of one router GEMV launch (cpu.matmulF16 of the T rows of
 * d_h against the layer's [E][H] f16 router, engine.zig:715).
 * ANEDVD_TIME_CHAIN: the layers are a stack, as the engine runs a model's MoE
 * blocks: each pass over it starts from d_h, layer j takes the previous layer's
 * x and writes x + its block output (x += proj, main.zig:519), routing row block
 * j of d_logits ([n_layers][T][E], when given); the last layer writes d_out.
 * Not with ANEDVD_TIME_GRAPH or ANEDVD_TIME_EXPERT_SOLO. */
#define ANEDVD_TIME_GRAPH 1
#define ANEDVD_TIME_EXPERT_SOLO 2
#define ANEDVD_TIME_CHAIN 4
int anedvd_moe_time_forward(anedvd_moe_layer *const *layers, size_t n_layers, const float *d_h,
                            size_t n_tokens, const float *d_logits, float *d_out, int warmup,
                            int iters, int flags, float *ms, float *kernel_ms);

#ifdef __cplusplus
}
#endif
#endif /* ANEDVD_MOE_H */
