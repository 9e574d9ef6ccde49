/*
 * moe_oracle.h -- CPU restatement of ANEDVD's quantised MoE FFN path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle the GPU path is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * CPU-baseline leg may load it; the product library never links it and
 * never falls back to it.
 *
 * Every function restates one function of the reference (Zig) in plain C,
 * in the same order of floating-point operations.  Build with
 * -ffp-contract=off so that `a*b + c` stays two roundings, as Zig's default
 * (strict) float mode does.
 */
#ifndef ANEDVD_MOE_ORACLE_H
#define ANEDVD_MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids as stored in GGUF (gguf.zig:30-46). */
enum {
    OR_F32 = 0, OR_F16 = 1, OR_Q4_0 = 2, OR_Q4_1 = 3, OR_Q5_0 = 6, OR_Q5_1 = 7,
    OR_Q8_0 = 8, OR_Q8_1 = 9, OR_Q2_K = 10, OR_Q3_K = 11, OR_Q4_K = 12,
    OR_Q5_K = 13, OR_Q6_K = 14, OR_Q8_K = 15, OR_BF16 = 30
};

/* Error codes, one per Zig error the restated functions can return. */
enum {
    OR_OK = 0,
    OR_ERR_UNSUPPORTED_TYPE = -1,   /* error.UnsupportedType */
    OR_ERR_INVALID_SHAPE = -2,      /* error.InvalidTensorShape */
    OR_ERR_TRUNCATED = -3,          /* error.TruncatedFile */
    OR_ERR_DIMENSION = -4,          /* error.DimensionMismatch */
    OR_ERR_OUT_OF_RANGE = -5        /* error.TensorDataOutOfRange */
};

/* GgmlType.blockElems / blockBytes (gguf.zig:49-77); 0 for unknown ids. */
size_t or_block_elems(int ggml_type);
size_t or_block_bytes(int ggml_type);

float or_f16_to_f32(uint16_t h);

/* dequantizeRange (gguf.zig:694-728) with every dequantiser it dispatches to. */
int or_dequantize_range(int ggml_type, const uint8_t *src, size_t src_len,
                        uint64_t elem_offset, float *out, size_t n);

/* Gguf.readExpertF32 (gguf.zig:533-552) over a stacked expert tensor payload
 * (expert axis slowest): dequantise expert `expert` of `n_experts`. */
int or_read_expert_f32(int ggml_type, const uint8_t *payload, size_t payload_len,
                       uint32_t expert, uint32_t n_experts, float *out, size_t per_expert);

/* f32 -> f16 bits, round to nearest even (f32ToF16Slice, gguf.zig:682-692). */
uint16_t or_f32_to_f16(float f);
void or_f32_to_f16_slice(const float *src, uint16_t *dst, size_t n);
/* Gguf.readExpertF16 (gguf.zig:499-531): readExpertF32 in 2048-element chunks,
 * each rounded to f16. */
int or_read_expert_f16(int ggml_type, const uint8_t *payload, size_t payload_len,
                       uint32_t expert, uint32_t n_experts, uint16_t *out, size_t per_expert);

/* cpu.matmulF16 (cpu.zig:461-475): 8 lane accumulators, ordered lane sum. */
void or_matmul_f16(float *out, const uint16_t *w, const float *x, size_t out_dim, size_t in_dim);
/* main.zig:320-326: the scalar sequential matmul refForward uses. */
void or_matmul_f16_scalar(float *out, const uint16_t *w, const float *x, size_t out_dim, size_t in_dim);
/* cpu.matmulF32 (cpu.zig:399-413). */
void or_matmul_f32(float *out, const float *w, const float *x, size_t out_dim, size_t in_dim);

/* cpu.moeRoute (cpu.zig:1236-1288). */
void or_moe_route(const float *logits, size_t n_experts, size_t k, int norm_topk_prob,
                  float *probs, uint32_t *idx);

/* cpu.moeExpertAccumF32 (cpu.zig:416-452). */
void or_moe_expert_accum_f32(float *out, float *hidden_scratch, float *inter_scratch,
                             const float *h, const float *gate, const float *up, const float *down,
                             size_t inter, size_t hidden, float weight, int use_gelu);
/* cpu.moeExpertAccum (cpu.zig:1141-1185), fp16 weights. */
void or_moe_expert_accum_f16(float *out, float *hidden_scratch, float *inter_scratch,
                             const float *h, const uint16_t *gate, const uint16_t *up, const uint16_t *down,
                             size_t inter, size_t hidden, float weight, int use_gelu);
/* cpu.mlpForward (cpu.zig:1189-1217); overwrites out. */
void or_mlp_forward(float *out, float *gate_scratch, const float *h,
                    const uint16_t *gate, const uint16_t *up, const uint16_t *down,
                    size_t inter, size_t hidden, int use_gelu);
/* cpu.sigmoid (cpu.zig:1223-1230) and cpu.geluTanh (cpu.zig:78-81). */
float or_sigmoid(float x);
float or_gelu_tanh(float x);
/* libm expf, the function Zig's @exp lowers to on x86-64 Linux with libc. */
float or_expf(float x);

/* Prefill grouping (engine.zig:1204-1216) + expertWeightFor (engine.zig:825-830):
 * for each expert ascending, the tokens that chose it in ascending order.
 * offsets[E+1]; rows[T*k] = token; slots[T*k] = the slot of that token that
 * holds the expert (its weight is probs[token*k + slot]). */
void or_dispatch(const uint32_t *idx, size_t n_tokens, size_t k, size_t n_experts,
                 int32_t *offsets, int32_t *rows, int32_t *slots);

/* One MoE layer as the engine and refForward compose it. */
typedef struct {
    uint32_t hidden, inter, n_experts, k;
    int32_t norm_topk_prob, use_gelu;
    int32_t gate_type, up_type, down_type;     /* ggml ids of the stacked expert tensors */
    const uint8_t *gate, *up, *down;           /* GGUF payloads, expert axis slowest */
    size_t gate_len, up_len, down_len;
    const uint16_t *router;                    /* [E][H] f16 bits */
    uint32_t shared_inter;                     /* 0 = no shared expert */
    const uint16_t *shared_gate, *shared_up, *shared_down;  /* f16 bits, [Is][H],[Is][H],[H][Is] */
    const uint16_t *shared_gate_lin;           /* [H] f16 bits, or NULL (scale 1.0) */
} or_layer;

/* Route T tokens: router logits with cpu.matmulF16 unless `logits_in` is given. */
void or_layer_route(const or_layer *L, const float *h, size_t n_tokens, const float *logits_in,
                    float *logits_out, float *probs, uint32_t *idx);

/* The whole block for T tokens (main.zig:488-520 with the f32 streaming experts of
 * engine.zig:705-779): out[t] = sum over slots of p * expert(h_t), then
 * + scale * shared(h_t).  Experts are dequantised per token and slot, as the
 * streaming engine does.  If `logits_in` is non-NULL the router GEMV is skipped. */
int or_layer_forward(const or_layer *L, const float *h, size_t n_tokens, const float *logits_in,
                     float *out);

/* The engine's streaming decode loop (engine.zig:705-779) literally: per token
 * and slot, dequantise the expert from the payload, then accumulate.  Bit-identical
 * to or_layer_forward; slower.  This is what the CPU baseline times. */
int or_layer_forward_streaming(const or_layer *L, const float *h, size_t n_tokens,
                               const float *logits_in, float *out);

/* Resident f32 experts (the CPU baseline's mode B): need[e] != 0 dequantises
 * expert e's three projections once; or_layer_forward_resident then runs the
 * decode loop of engine.zig:705-779 on them (bit-identical to the streaming loop). */
typedef struct or_resident or_resident;
or_resident *or_resident_create(const or_layer *L, const uint8_t *need);
void or_resident_free(or_resident *R);
int or_layer_forward_resident(const or_resident *R, const float *h, size_t n_tokens,
                              const float *logits_in, float *out);

#ifdef __cplusplus
}
#endif
#endif
