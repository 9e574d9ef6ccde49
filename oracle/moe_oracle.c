/*
 * moe_oracle.c -- CPU restatement of ANEDVD's quantised MoE FFN path.
 *
 * TEST INFRASTRUCTURE ONLY: the oracle for the HIP library, and the CPU
 * baseline that bench.py times beside it.  Nothing in the product links it.
 *
 * Each function follows one reference function (file:line in the comment)
 * in the same order of f32 operations.  Compiled with -ffp-contract=off
 * -fno-fast-math so that every `a*b + c` rounds twice, as Zig's strict float
 * mode does.  `@exp` on x86-64 Linux resolves to libm's expf, which is what
 * or_expf calls.
 *
 * Pinning (what checks each function, in tests/test_oracle.py):
 *   dequantisers      reference golden fixtures, bit for bit (gguf.zig:1528-1570),
 *                     hand blocks (gguf.zig:1424-1526), tiny_v3.gguf values,
 *                     closed-form exactness of every block product;
 *   matmul_f16/f32    f64 dot within 1e-6 relative; an 8-lane order that a
 *                     sequential sum cannot reproduce bit for bit;
 *   moe_route         reference KAT (cpu.zig:1290-1336) and brute-force sort;
 *   expert_accum      reference hand-computed KAT (cpu.zig:1338-1388), f64 brute force;
 *   mlp / sigmoid     sigmoid KAT (cpu.zig:1390-1400), f64 brute force;
 *   gelu_tanh         reference KAT (cpu.zig:1434-1449), closed forms (gelu(0) = 0,
 *                     saturation, odd symmetry), f64 formula over a sweep;
 *   f32_to_f16        numpy's round-to-nearest-even conversion over every f16
 *                     value, the midpoints between them and random f32 values;
 *   read_expert_f16   equals f32_to_f16 of read_expert_f32 (chunking cannot change
 *                     a whole-block dequantisation);
 *   dispatch          brute-force stable sort by expert;
 *   layer forward     f64 composition, and per-token streaming == by-expert order.
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------ block geometry */

size_t or_block_elems(int t)
{
    switch (t) {
    case OR_F32: case OR_F16: case OR_BF16: return 1;
    case OR_Q4_0: case OR_Q4_1: case OR_Q5_0: case OR_Q5_1: case OR_Q8_0: case OR_Q8_1: return 32;
    case OR_Q2_K: case OR_Q3_K: case OR_Q4_K: case OR_Q5_K: case OR_Q6_K: case OR_Q8_K: return 256;
    default: return 0;
    }
}

size_t or_block_bytes(int t)
{
    switch (t) {
    case OR_F32: return 4;
    case OR_F16: case OR_BF16: return 2;
    case OR_Q4_0: return 18;
    case OR_Q4_1: return 20;
    case OR_Q5_0: return 22;
    case OR_Q5_1: return 24;
    case OR_Q8_0: return 34;
    case OR_Q8_1: return 36;
    case OR_Q2_K: return 84;
    case OR_Q3_K: return 110;
    case OR_Q4_K: return 144;
    case OR_Q5_K: return 176;
    case OR_Q6_K: return 210;
    case OR_Q8_K: return 292;
    default: return 0;
    }
}

/* ------------------------------------------------------------ scalar helpers */

static inline uint16_t rd16(const uint8_t *b, size_t off) { return (uint16_t)(b[off] | (b[off + 1] << 8)); }
static inline uint32_t rd32(const uint8_t *b, size_t off)
{
    return (uint32_t)b[off] | ((uint32_t)b[off + 1] << 8) | ((uint32_t)b[off + 2] << 16) | ((uint32_t)b[off + 3] << 24);
}
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* IEEE binary16 -> binary32, exact for every input (gguf.zig:743-746). */
float or_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        float v = (float)m * 0x1p-24f; /* subnormal (or zero): m * 2^-24 is exact in f32 */
        return sign ? -v : v;
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

float or_expf(float x) { return expf(x); }

/* ---------------------------------------------------------- the dequantisers */

/* gguf.zig:751-757 */
static void deq_f32(const uint8_t *b, float *out, size_t n) { for (size_t i = 0; i < n; i++) out[i] = bits_f32(rd32(b, 4 * i)); }
static void deq_f16(const uint8_t *b, float *out, size_t n) { for (size_t i = 0; i < n; i++) out[i] = or_f16_to_f32(rd16(b, 2 * i)); }
/* gguf.zig:747-749, 759-761 */
static void deq_bf16(const uint8_t *b, float *out, size_t n) { for (size_t i = 0; i < n; i++) out[i] = bits_f32((uint32_t)rd16(b, 2 * i) << 16); }

/* dequantQ4_0, gguf.zig:763-776: y_j = (lo_j - 8) * d, y_{j+16} = (hi_j - 8) * d */
static void deq_q4_0(const uint8_t *b, float *out, size_t nb)
{
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *blk = b + i * 18;
        float d = or_f16_to_f32(rd16(blk, 0));
        for (int j = 0; j < 16; j++) {
            uint8_t q = blk[2 + j];
            float x0 = (float)((int)(q & 0x0F) - 8);
            float x1 = (float)((int)(q >> 4) - 8);
            out[i * 32 + j] = x0 * d;
            out[i * 32 + j + 16] = x1 * d;
        }
    }
}

/* dequantQ4_1, gguf.zig:778-793: x * d + m */
static void deq_q4_1(const uint8_t *b, float *out, size_t nb)
{
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *blk = b + i * 20;
        float d = or_f16_to_f32(rd16(blk, 0));
        float m = or_f16_to_f32(rd16(blk, 2));
        for (int j = 0; j < 16; j++) {
            uint8_t q = blk[4 + j];
            float x0 = (float)(q & 0x0F);
            float x1 = (float)(q >> 4);
            out[i * 32 + j] = x0 * d + m;
            out[i * 32 + j + 16] = x1 * d + m;
        }
    }
}

/* dequantQ5 (q5_0 / q5_1), gguf.zig:795-825.  q5_0 keeps `+ 0.0`, which turns a
 * -0.0 product into +0.0 exactly as the reference does. */
static void deq_q5(const uint8_t *b, float *out, size_t nb, size_t bb, int has_min)
{
    const size_t qh_off = has_min ? 4 : 2, qs_off = qh_off + 4;
    const int minus = has_min ? 0 : 16;
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *blk = b + i * bb;
        float d = or_f16_to_f32(rd16(blk, 0));
        float m = has_min ? or_f16_to_f32(rd16(blk, 2)) : 0.0f;
        uint32_t qh = rd32(blk, qh_off);
        for (int j = 0; j < 16; j++) {
            uint8_t q = blk[qs_off + j];
            uint32_t xh0 = ((qh >> j) << 4) & 0x10u;
            uint32_t xh1 = (qh >> (j + 12)) & 0x10u;
            float x0 = (float)((int)((q & 0x0F) | xh0) - minus);
            float x1 = (float)((int)((q >> 4) | xh1) - minus);
            out[i * 32 + j] = x0 * d + m;
            out[i * 32 + j + 16] = x1 * d + m;
        }
    }
}

/* dequantQ8_0, gguf.zig:827-840: y_j = d * q_j */
static void deq_q8_0(const uint8_t *b, float *out, size_t nb)
{
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *blk = b + i * 34;
        float d = or_f16_to_f32(rd16(blk, 0));
        for (int j = 0; j < 32; j++) out[i * 32 + j] = d * (float)(int8_t)blk[2 + j];
    }
}

/* dequantQ8_1, gguf.zig:842-853: q * d (the `s` field is unused) */
static void deq_q8_1(const uint8_t *b, float *out, size_t nb)
{
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *blk = b + i * 36;
        float d = or_f16_to_f32(rd16(blk, 0));
        for (int j = 0; j < 32; j++) out[i * 32 + j] = (float)(int8_t)blk[4 + j] * d;
    }
}

/* dequantQ2K, gguf.zig:855-890: dl * v - ml over 16-element groups */
static void deq_q2_k(const uint8_t *b, float *out, size_t nb)
{
    for (size_t ib = 0; ib < nb; ib++) {
        const uint8_t *blk = b + ib * 84;
        float d = or_f16_to_f32(rd16(blk, 80));
        float mn = or_f16_to_f32(rd16(blk, 82));
        const uint8_t *sc = blk;
        size_t q = 16, y = ib * 256, is = 0;
        for (int half = 0; half < 2; half++) {
            int shift = 0;
            for (int g = 0; g < 4; g++) {
                for (int part = 0; part < 2; part++) {
                    uint8_t s = sc[is++];
                    float dl = d * (float)(s & 0x0F);
                    float ml = mn * (float)(s >> 4);
                    for (int l = 0; l < 16; l++) {
                        float v = (float)((blk[q + l + 16 * part] >> shift) & 3);
                        out[y + l] = dl * v - ml;
                    }
                    y += 16;
                }
                shift += 2;
            }
            q += 32;
        }
    }
}

/* dequantQ3K, gguf.zig:892-946 */
static void deq_q3_k(const uint8_t *b, float *out, size_t nb)
{
    const uint32_t kmask1 = 0x03030303u, kmask2 = 0x0f0f0f0fu;
    for (size_t ib = 0; ib < nb; ib++) {
        const uint8_t *blk = b + ib * 110;
        float d_all = or_f16_to_f32(rd16(blk, 108));
        const uint8_t *hm = blk, *qs = blk + 32;
        uint32_t aux[4] = { rd32(blk, 96), rd32(blk, 100), rd32(blk, 104), 0 };
        uint32_t tmp = aux[2];
        aux[2] = ((aux[0] >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4);
        aux[3] = ((aux[1] >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4);
        aux[0] = (aux[0] & kmask2) | (((tmp >> 0) & kmask1) << 4);
        aux[1] = (aux[1] & kmask2) | (((tmp >> 2) & kmask1) << 4);
        int8_t scales[16];
        for (int k = 0; k < 4; k++)
            for (int bi = 0; bi < 4; bi++) scales[k * 4 + bi] = (int8_t)(uint8_t)(aux[k] >> (8 * bi));
        uint8_t m = 1;
        size_t is = 0, q = 0, y = ib * 256;
        for (int half = 0; half < 2; half++) {
            int shift = 0;
            for (int g = 0; g < 4; g++) {
                for (int part = 0; part < 2; part++) {
                    float dl = d_all * (float)((int)scales[is++] - 32);
                    for (int l = 0; l < 16; l++) {
                        int low = (qs[q + l + 16 * part] >> shift) & 3;
                        int v = low - ((hm[l + 16 * part] & m) ? 0 : 4);
                        out[y + l] = dl * (float)v;
                    }
                    y += 16;
                }
                shift += 2;
                m = (uint8_t)(m << 1);
            }
            q += 32;
        }
    }
}

/* getScaleMinK4, gguf.zig:948-958 */
static inline void scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m)
{
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* dequantQ4K, gguf.zig:960-996: y = d1 * q - m1 per 32-element sub-block */
static void deq_q4_k(const uint8_t *b, float *out, size_t nb)
{
    for (size_t ib = 0; ib < nb; ib++) {
        const uint8_t *blk = b + ib * 144;
        float d = or_f16_to_f32(rd16(blk, 0));
        float mn = or_f16_to_f32(rd16(blk, 2));
        const uint8_t *scales = blk + 4;
        size_t q = 16;
        for (int is = 0; is < 8; is += 2) {
            uint8_t sd, sm;
            scale_min_k4(is, scales, &sd, &sm);
            float d1 = d * (float)sd, m1 = mn * (float)sm;
            scale_min_k4(is + 1, scales, &sd, &sm);
            float d2 = d * (float)sd, m2 = mn * (float)sm;
            size_t y = ib * 256 + (size_t)(is / 2) * 64;
            for (int l = 0; l < 32; l++) {
                out[y + l] = d1 * (float)(blk[q + l] & 0x0F) - m1;
                out[y + 32 + l] = d2 * (float)(blk[q + l] >> 4) - m2;
            }
            q += 32;
        }
    }
}

/* dequantQ5K, gguf.zig:998-1034 */
static void deq_q5_k(const uint8_t *b, float *out, size_t nb)
{
    for (size_t ib = 0; ib < nb; ib++) {
        const uint8_t *blk = b + ib * 176;
        float d = or_f16_to_f32(rd16(blk, 0));
        float mn = or_f16_to_f32(rd16(blk, 2));
        const uint8_t *scales = blk + 4, *qh = blk + 16;
        size_t ql = 48;
        uint8_t mask1 = 1, mask2 = 2;
        for (int is = 0; is < 8; is += 2) {
            uint8_t sd, sm;
            scale_min_k4(is, scales, &sd, &sm);
            float d1 = d * (float)sd, m1 = mn * (float)sm;
            scale_min_k4(is + 1, scales, &sd, &sm);
            float d2 = d * (float)sd, m2 = mn * (float)sm;
            size_t y = ib * 256 + (size_t)(is / 2) * 64;
            for (int l = 0; l < 32; l++) {
                int hi = (qh[l] & mask1) ? 16 : 0;
                out[y + l] = d1 * (float)((blk[ql + l] & 0x0F) + hi) - m1;
            }
            for (int l = 0; l < 32; l++) {
                int hi = (qh[l] & mask2) ? 16 : 0;
                out[y + 32 + l] = d2 * (float)((blk[ql + l] >> 4) + hi) - m2;
            }
            ql += 32;
            mask1 = (uint8_t)(mask1 << 2);
            mask2 = (uint8_t)(mask2 << 2);
        }
    }
}

/* dequantQ6K, gguf.zig:1036-1059: y = d * sc * q, left to right */
static void deq_q6_k(const uint8_t *b, float *out, size_t nb)
{
    for (size_t ib = 0; ib < nb; ib++) {
        const uint8_t *blk = b + ib * 210;
        float d = or_f16_to_f32(rd16(blk, 208));
        for (int half = 0; half < 2; half++) {
            const uint8_t *ql = blk + half * 64, *qh = blk + 128 + half * 32, *sc = blk + 192 + half * 8;
            size_t y = ib * 256 + (size_t)half * 128;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                out[y + l + 0] = d * (float)(int8_t)sc[is + 0] * (float)q1;
                out[y + l + 32] = d * (float)(int8_t)sc[is + 2] * (float)q2;
                out[y + l + 64] = d * (float)(int8_t)sc[is + 4] * (float)q3;
                out[y + l + 96] = d * (float)(int8_t)sc[is + 6] * (float)q4;
            }
        }
    }
}

/* dequantQ8K, gguf.zig:1061-1071: f32 d, q * d */
static void deq_q8_k(const uint8_t *b, float *out, size_t nb)
{
    for (size_t ib = 0; ib < nb; ib++) {
        const uint8_t *blk = b + ib * 292;
        float d = bits_f32(rd32(blk, 0));
        for (int j = 0; j < 256; j++) out[ib * 256 + j] = (float)(int8_t)blk[4 + j] * d;
    }
}

/* dequantizeRange, gguf.zig:694-728: same checks in the same order. */
int or_dequantize_range(int t, const uint8_t *src, size_t src_len, uint64_t elem_offset, float *out, size_t n)
{
    size_t epb = or_block_elems(t), bpb = or_block_bytes(t);
    if (!epb || !bpb) return OR_ERR_UNSUPPORTED_TYPE;
    if (n == 0) return OR_OK;
    if (n % epb) return OR_ERR_INVALID_SHAPE;
    if (elem_offset % epb) return OR_ERR_INVALID_SHAPE;
    uint64_t blocks_before = elem_offset / epb;
    if (blocks_before > UINT64_MAX / bpb) return OR_ERR_TRUNCATED;
    uint64_t start = blocks_before * bpb;
    if (start > src_len) return OR_ERR_TRUNCATED;
    const uint8_t *body = src + start;
    size_t body_len = src_len - (size_t)start;
    size_t blocks = n / epb;
    if (blocks > SIZE_MAX / bpb) return OR_ERR_TRUNCATED;
    if (body_len < blocks * bpb) return OR_ERR_TRUNCATED;
    switch (t) {
    case OR_F32: deq_f32(body, out, n); break;
    case OR_F16: deq_f16(body, out, n); break;
    case OR_BF16: deq_bf16(body, out, n); break;
    case OR_Q4_0: deq_q4_0(body, out, blocks); break;
    case OR_Q4_1: deq_q4_1(body, out, blocks); break;
    case OR_Q5_0: deq_q5(body, out, blocks, 22, 0); break;
    case OR_Q5_1: deq_q5(body, out, blocks, 24, 1); break;
    case OR_Q8_0: deq_q8_0(body, out, blocks); break;
    case OR_Q8_1: deq_q8_1(body, out, blocks); break;
    case OR_Q2_K: deq_q2_k(body, out, blocks); break;
    case OR_Q3_K: deq_q3_k(body, out, blocks); break;
    case OR_Q4_K: deq_q4_k(body, out, blocks); break;
    case OR_Q5_K: deq_q5_k(body, out, blocks); break;
    case OR_Q6_K: deq_q6_k(body, out, blocks); break;
    case OR_Q8_K: deq_q8_k(body, out, blocks); break;
    default: return OR_ERR_UNSUPPORTED_TYPE;
    }
    return OR_OK;
}

/* Gguf.readExpertF32, gguf.zig:533-552, over the tensor's payload. */
int or_read_expert_f32(int t, const uint8_t *payload, size_t payload_len, uint32_t expert,
                       uint32_t n_experts, float *out, size_t per_expert)
{
    size_t epb = or_block_elems(t), bpb = or_block_bytes(t);
    if (!epb || !bpb) return OR_ERR_UNSUPPORTED_TYPE;
    if (payload_len % bpb) return OR_ERR_INVALID_SHAPE;
    uint64_t elems = (uint64_t)(payload_len / bpb) * epb;
    if (elems != (uint64_t)per_expert * n_experts) return OR_ERR_DIMENSION;
    if (per_expert % epb) return OR_ERR_INVALID_SHAPE;
    uint64_t per_bytes = (uint64_t)(per_expert / epb) * bpb;
    uint64_t start = (uint64_t)expert * per_bytes, end = start + per_bytes;
    if (end > payload_len) return OR_ERR_OUT_OF_RANGE;
    return or_dequantize_range(t, payload + start, (size_t)per_bytes, 0, out, per_expert);
}

/* IEEE binary32 -> binary16, round to nearest, ties to even, overflow to infinity
 * (the conversion Zig's @floatCast does for f32ToF16Slice, gguf.zig:682-692).
 * With E the value's unbiased exponent, the f16 grid step is 2^(E-10) for a
 * normal result and 2^-24 below 2^-14; the 24-bit significand is divided by the
 * step (a right shift) and rounded on the bits shifted out.  A significand that
 * rounds up to 2048 carries into the exponent by the addition. */
uint16_t or_f32_to_f16(float f)
{
    const uint32_t x = f32_bits(f), sign = (x >> 16) & 0x8000u, e = (x >> 23) & 0xffu, m = x & 0x7fffffu;
    if (e == 0xff) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u | (m >> 13) : 0u));
    if (e == 0) return (uint16_t)sign; /* |f| < 2^-126: below half the smallest f16 subnormal */
    const int E = (int)e - 127;
    if (E > 15) return (uint16_t)(sign | 0x7c00u);
    const uint32_t mant = m | 0x800000u;
    const int shift = E < -14 ? 126 - (int)e : 13;
    uint32_t q = 0;
    if (shift < 32) {
        q = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
    }
    const uint32_t bits = E < -14 ? q : ((uint32_t)(E + 14) << 10) + q;
    return (uint16_t)(sign | (bits > 0x7c00u ? 0x7c00u : bits));
}

void or_f32_to_f16_slice(const float *src, uint16_t *dst, size_t n)
{
    for (size_t i = 0; i < n; i++) dst[i] = or_f32_to_f16(src[i]);
}

/* Gguf.readExpertF16, gguf.zig:499-531: the checks of readExpertF32, then the
 * expert dequantised 2048 elements at a time and each chunk rounded to f16. */
int or_read_expert_f16(int t, const uint8_t *payload, size_t payload_len, uint32_t expert,
                       uint32_t n_experts, uint16_t *out, size_t per_expert)
{
    size_t epb = or_block_elems(t), bpb = or_block_bytes(t);
    if (!epb || !bpb) return OR_ERR_UNSUPPORTED_TYPE;
    if (payload_len % bpb) return OR_ERR_INVALID_SHAPE;
    uint64_t elems = (uint64_t)(payload_len / bpb) * epb;
    if (elems != (uint64_t)per_expert * n_experts) return OR_ERR_DIMENSION;
    if (per_expert % epb) return OR_ERR_INVALID_SHAPE;
    uint64_t per_bytes = (uint64_t)(per_expert / epb) * bpb;
    uint64_t start = (uint64_t)expert * per_bytes, end = start + per_bytes;
    if (end > payload_len) return OR_ERR_OUT_OF_RANGE;
    float buf[2048];
    for (size_t done = 0; done < per_expert;) {
        size_t m = per_expert - done < 2048 ? per_expert - done : 2048;
        int rc = or_dequantize_range(t, payload + start, (size_t)per_bytes, done, buf, m);
        if (rc) return rc;
        or_f32_to_f16_slice(buf, out + done, m);
        done += m;
    }
    return OR_OK;
}

/* ------------------------------------------------------------------- matmuls */

#define LANES 8

/* cpu.matmulF16, cpu.zig:461-475.  acc[l] += x[i+l] * f32(w[i+l]) for i stepping by
 * 8; then the ordered lane sum (@reduce(.Add) keeps associativity in strict mode);
 * then the scalar tail. */
void or_matmul_f16(float *out, const uint16_t *w, const float *x, size_t out_dim, size_t in_dim)
{
    for (size_t o = 0; o < out_dim; o++) {
        const uint16_t *row = w + o * in_dim;
        float acc[LANES] = { 0 };
        size_t i = 0;
        for (; i + LANES <= in_dim; i += LANES)
            for (int l = 0; l < LANES; l++) acc[l] = acc[l] + x[i + l] * or_f16_to_f32(row[i + l]);
        float sum = acc[0];
        for (int l = 1; l < LANES; l++) sum = sum + acc[l];
        for (; i < in_dim; i++) sum = sum + or_f16_to_f32(row[i]) * x[i];
        out[o] = sum;
    }
}

/* main.zig:320-326: scalar, sequential in i. */
void or_matmul_f16_scalar(float *out, const uint16_t *w, const float *x, size_t out_dim, size_t in_dim)
{
    for (size_t o = 0; o < out_dim; o++) {
        float acc = 0;
        for (size_t i = 0; i < in_dim; i++) acc = acc + or_f16_to_f32(w[o * in_dim + i]) * x[i];
        out[o] = acc;
    }
}

/* cpu.matmulF32, cpu.zig:399-413. */
void or_matmul_f32(float *out, const float *w, const float *x, size_t out_dim, size_t in_dim)
{
    for (size_t o = 0; o < out_dim; o++) {
        const float *row = w + o * in_dim;
        float acc[LANES] = { 0 };
        size_t i = 0;
        for (; i + LANES <= in_dim; i += LANES)
            for (int l = 0; l < LANES; l++) acc[l] = acc[l] + x[i + l] * row[i + l];
        float sum = acc[0];
        for (int l = 1; l < LANES; l++) sum = sum + acc[l];
        for (; i < in_dim; i++) sum = sum + row[i] * x[i];
        out[o] = sum;
    }
}

/* --------------------------------------------------------------- activations */

/* cpu.sigmoid, cpu.zig:1223-1230. */
float or_sigmoid(float x)
{
    if (x >= 0) {
        float e = expf(-fminf(x, 80.0f));
        return 1.0f / (1.0f + e);
    }
    float e = expf(fmaxf(x, -80.0f));
    return e / (1.0f + e);
}

/* cpu.geluTanh, cpu.zig:78-81 (tanh from libm; Zig's std.math.tanh may differ in
 * the last bit, so gelu is tolerance-level only). */
float or_gelu_tanh(float x)
{
    const float c = 0.7978845608028654f;
    return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

/* ------------------------------------------------------------------- routing */

/* cpu.moeRoute, cpu.zig:1236-1288. */
void or_moe_route(const float *logits, size_t n, size_t k, int norm_topk_prob, float *probs, uint32_t *idx)
{
    float max_v = -INFINITY;
    for (size_t e = 0; e < n; e++) max_v = fmaxf(max_v, logits[e]);
    float sum = 0;
    for (size_t e = 0; e < n; e++) sum = sum + expf(logits[e] - max_v);
    const float inv_sum = sum > 0 ? 1.0f / sum : 0.0f;

    for (size_t slot = 0; slot < k; slot++) {
        size_t best = SIZE_MAX;
        float best_p = -1.0f;
        for (size_t e = 0; e < n; e++) {
            int taken = 0;
            for (size_t s = 0; s < slot; s++)
                if (idx[s] == e) { taken = 1; break; }
            if (taken) continue;
            float p = expf(logits[e] - max_v) * inv_sum;
            if (p > best_p) { best_p = p; best = e; }
        }
        if (best == SIZE_MAX) { probs[slot] = 0; idx[slot] = 0; }
        else { probs[slot] = best_p; idx[slot] = (uint32_t)best; }
    }
    if (norm_topk_prob) {
        float s = 0;
        for (size_t i = 0; i < k; i++) s = s + probs[i];
        if (s > 0)
            for (size_t i = 0; i < k; i++) probs[i] = probs[i] / s;
    }
}

/* ------------------------------------------------------------------- experts */

static inline float gate_act(float g, int use_gelu) { return use_gelu ? or_gelu_tanh(g) : g / (1.0f + expf(-g)); }

/* cpu.moeExpertAccumF32, cpu.zig:416-452. */
void or_moe_expert_accum_f32(float *out, float *hs, float *is, const float *h, const float *gate,
                             const float *up, const float *down, size_t inter, size_t hidden,
                             float weight, int use_gelu)
{
    or_matmul_f32(hs, gate, h, inter, hidden);
    or_matmul_f32(is, up, h, inter, hidden);
    for (size_t i = 0; i < inter; i++) is[i] = gate_act(hs[i], use_gelu) * is[i];
    for (size_t o = 0; o < hidden; o++) {
        const float *row = down + o * inter;
        float acc[LANES] = { 0 };
        size_t k = 0;
        for (; k + LANES <= inter; k += LANES)
            for (int l = 0; l < LANES; l++) acc[l] = acc[l] + is[k + l] * row[k + l];
        float total = acc[0];
        for (int l = 1; l < LANES; l++) total = total + acc[l];
        for (; k < inter; k++) total = total + row[k] * is[k];
        out[o] = out[o] + weight * total;
    }
}

/* cpu.moeExpertAccum, cpu.zig:1141-1185 (fp16 weights). */
void or_moe_expert_accum_f16(float *out, float *hs, float *is, const float *h, const uint16_t *gate,
                             const uint16_t *up, const uint16_t *down, size_t inter, size_t hidden,
                             float weight, int use_gelu)
{
    or_matmul_f16(hs, gate, h, inter, hidden);
    or_matmul_f16(is, up, h, inter, hidden);
    for (size_t i = 0; i < inter; i++) {
        float s = gate_act(hs[i], use_gelu);
        is[i] = s * is[i];
    }
    for (size_t o = 0; o < hidden; o++) {
        const uint16_t *row = down + o * inter;
        float acc[LANES] = { 0 };
        size_t k = 0;
        for (; k + LANES <= inter; k += LANES)
            for (int l = 0; l < LANES; l++) acc[l] = acc[l] + is[k + l] * or_f16_to_f32(row[k + l]);
        float total = acc[0];
        for (int l = 1; l < LANES; l++) total = total + acc[l];
        for (; k < inter; k++) total = total + or_f16_to_f32(row[k]) * is[k];
        out[o] = out[o] + weight * total;
    }
}

/* cpu.mlpForward, cpu.zig:1189-1217: gate 8-lane, up and down scalar sequential. */
void or_mlp_forward(float *out, float *gs, const float *h, const uint16_t *gate, const uint16_t *up,
                    const uint16_t *down, size_t inter, size_t hidden, int use_gelu)
{
    or_matmul_f16(gs, gate, h, inter, hidden);
    for (size_t i = 0; i < inter; i++) {
        float g = gs[i], acc = 0;
        const uint16_t *row = up + i * hidden;
        for (size_t j = 0; j < hidden; j++) acc = acc + or_f16_to_f32(row[j]) * h[j];
        float s = gate_act(g, use_gelu);
        gs[i] = s * acc;
    }
    for (size_t o = 0; o < hidden; o++) {
        float acc = 0;
        const uint16_t *row = down + o * inter;
        for (size_t i = 0; i < inter; i++) acc = acc + or_f16_to_f32(row[i]) * gs[i];
        out[o] = acc;
    }
}

/* ------------------------------------------------------------------ dispatch */

/* engine.zig:1204-1216 and expertWeightFor (engine.zig:825-830). */
void or_dispatch(const uint32_t *idx, size_t n_tokens, size_t k, size_t n_experts,
                 int32_t *offsets, int32_t *rows, int32_t *slots)
{
    size_t pos = 0;
    for (size_t e = 0; e < n_experts; e++) {
        offsets[e] = (int32_t)pos;
        for (size_t j = 0; j < n_tokens; j++)
            for (size_t s = 0; s < k; s++)
                if (idx[j * k + s] == e) {
                    rows[pos] = (int32_t)j;
                    slots[pos] = (int32_t)s;
                    pos++;
                    break;
                }
    }
    offsets[n_experts] = (int32_t)pos;
}

/* -------------------------------------------------------------------- layers */

void or_layer_route(const or_layer *L, const float *h, size_t T, const float *logits_in,
                    float *logits_out, float *probs, uint32_t *idx)
{
    const size_t H = L->hidden, E = L->n_experts, k = L->k;
    float *lg = malloc(E * sizeof(float));
    for (size_t t = 0; t < T; t++) {
        if (logits_in) memcpy(lg, logits_in + t * E, E * sizeof(float));
        else or_matmul_f16(lg, L->router, h + t * H, E, H); /* engine.zig:715 / 1178 */
        if (logits_out) memcpy(logits_out + t * E, lg, E * sizeof(float));
        or_moe_route(lg, E, k, L->norm_topk_prob, probs + t * k, idx + t * k);
    }
    free(lg);
}

/* The shared expert and its gate as refForward applies them (main.zig:510-516);
 * without shared_gate_lin the scale is 1.0, as the engine does (engine.zig:687-691). */
static void shared_add(const or_layer *L, const float *h, float *proj, float *sh_out, float *sh_scr)
{
    const size_t H = L->hidden;
    or_mlp_forward(sh_out, sh_scr, h, L->shared_gate, L->shared_up, L->shared_down, L->shared_inter, H, L->use_gelu);
    float scale = 1.0f;
    if (L->shared_gate_lin) {
        float g = 0;
        for (size_t i = 0; i < H; i++) g = g + or_f16_to_f32(L->shared_gate_lin[i]) * h[i];
        scale = or_sigmoid(g);
    }
    for (size_t o = 0; o < H; o++) proj[o] = proj[o] + scale * sh_out[o];
}

/* Expert-major evaluation: every selected expert is dequantised once, its
 * per-slot contribution weight*total is stored, and the contributions are then
 * summed per token in slot order -- the same f32 values, in the same order, as
 * the per-token streaming loop (main.zig:495-509), only cheaper to compute. */
int or_layer_forward(const or_layer *L, const float *h, size_t T, const float *logits_in, float *out)
{
    const size_t H = L->hidden, I = L->inter, E = L->n_experts, k = L->k;
    int rc = OR_OK;
    float *probs = malloc(T * k * sizeof(float));
    uint32_t *idx = malloc(T * k * sizeof(uint32_t));
    int32_t *offsets = malloc((E + 1) * sizeof(int32_t));
    int32_t *rows = malloc(T * k * sizeof(int32_t)), *slots = malloc(T * k * sizeof(int32_t));
    float *contrib = calloc(T * k * H, sizeof(float));
    float *wg = malloc(I * H * sizeof(float)), *wu = malloc(I * H * sizeof(float)), *wd = malloc(I * H * sizeof(float));
    float *hs = malloc(I * sizeof(float)), *is = malloc(I * sizeof(float));
    if (!probs || !idx || !offsets || !rows || !slots || !contrib || !wg || !wu || !wd || !hs || !is) { rc = -100; goto done; }

    or_layer_route(L, h, T, logits_in, NULL, probs, idx);
    or_dispatch(idx, T, k, E, offsets, rows, slots);
    for (size_t e = 0; e < E; e++) {
        if (offsets[e + 1] == offsets[e]) continue;
        if ((rc = or_read_expert_f32(L->gate_type, L->gate, L->gate_len, (uint32_t)e, (uint32_t)E, wg, I * H))) goto done;
        if ((rc = or_read_expert_f32(L->up_type, L->up, L->up_len, (uint32_t)e, (uint32_t)E, wu, I * H))) goto done;
        if ((rc = or_read_expert_f32(L->down_type, L->down, L->down_len, (uint32_t)e, (uint32_t)E, wd, I * H))) goto done;
        for (int32_t p = offsets[e]; p < offsets[e + 1]; p++) {
            size_t t = (size_t)rows[p], s = (size_t)slots[p];
            /* contrib starts at +0.0, so `0 + weight*total` is the value the
             * reference's `out[o] += weight * total` adds for this slot. */
            or_moe_expert_accum_f32(contrib + (t * k + s) * H, hs, is, h + t * H, wg, wu, wd, I, H, probs[t * k + s], L->use_gelu);
        }
    }
    {
        float *sh_out = L->shared_inter ? malloc(H * sizeof(float)) : NULL;
        float *sh_scr = L->shared_inter ? malloc(L->shared_inter * sizeof(float)) : NULL;
        for (size_t t = 0; t < T; t++) {
            float *proj = out + t * H;
            for (size_t o = 0; o < H; o++) proj[o] = 0.0f;
            for (size_t s = 0; s < k; s++) {
                const float *c = contrib + (t * k + s) * H;
                for (size_t o = 0; o < H; o++) proj[o] = proj[o] + c[o];
            }
            if (L->shared_inter) shared_add(L, h + t * H, proj, sh_out, sh_scr);
        }
        free(sh_out);
        free(sh_scr);
    }
done:
    free(probs); free(idx); free(offsets); free(rows); free(slots); free(contrib);
    free(wg); free(wu); free(wd); free(hs); free(is);
    return rc;
}

/* Mode B of the CPU baseline: the experts dequantised to f32 once and held (as the
 * eager loader holds its experts resident, model.zig:414-470), so the per-token
 * loop below times the expert products alone.  need[e] != 0 marks the experts to
 * hold; the others stay NULL. */
struct or_resident {
    const or_layer *L;
    float **wg, **wu, **wd;
};

or_resident *or_resident_create(const or_layer *L, const uint8_t *need)
{
    const size_t E = L->n_experts, n = (size_t)L->inter * L->hidden;
    or_resident *R = calloc(1, sizeof *R);
    if (!R) return NULL;
    R->L = L;
    R->wg = calloc(E, sizeof(float *));
    R->wu = calloc(E, sizeof(float *));
    R->wd = calloc(E, sizeof(float *));
    if (!R->wg || !R->wu || !R->wd) { or_resident_free(R); return NULL; }
    for (size_t e = 0; e < E; e++) {
        if (!need[e]) continue;
        R->wg[e] = malloc(n * sizeof(float));
        R->wu[e] = malloc(n * sizeof(float));
        R->wd[e] = malloc(n * sizeof(float));
        if (!R->wg[e] || !R->wu[e] || !R->wd[e] ||
            or_read_expert_f32(L->gate_type, L->gate, L->gate_len, (uint32_t)e, (uint32_t)E, R->wg[e], n) ||
            or_read_expert_f32(L->up_type, L->up, L->up_len, (uint32_t)e, (uint32_t)E, R->wu[e], n) ||
            or_read_expert_f32(L->down_type, L->down, L->down_len, (uint32_t)e, (uint32_t)E, R->wd[e], n)) {
            or_resident_free(R);
            return NULL;
        }
    }
    return R;
}

void or_resident_free(or_resident *R)
{
    if (!R) return;
    for (size_t e = 0; R->wg && e < R->L->n_experts; e++) {
        free(R->wg[e]);
        free(R->wu[e]);
        free(R->wd[e]);
    }
    free(R->wg); free(R->wu); free(R->wd);
    free(R);
}

/* The decode loop of engine.zig:705-779 over resident experts: per token, route,
 * then moeExpertAccumF32 per slot, then the shared expert.  OR_ERR_OUT_OF_RANGE if a
 * token routes to an expert that is not held. */
int or_layer_forward_resident(const or_resident *R, const float *h, size_t T, const float *logits_in, float *out)
{
    const or_layer *L = R->L;
    const size_t H = L->hidden, I = L->inter, E = L->n_experts, k = L->k;
    int rc = OR_OK;
    float *lg = malloc(E * sizeof(float)), *probs = malloc(k * sizeof(float));
    uint32_t *idx = malloc(k * sizeof(uint32_t));
    float *hs = malloc(I * sizeof(float)), *is = malloc(I * sizeof(float));
    float *sh_out = L->shared_inter ? malloc(H * sizeof(float)) : NULL;
    float *sh_scr = L->shared_inter ? malloc(L->shared_inter * sizeof(float)) : NULL;
    for (size_t t = 0; t < T && rc == OR_OK; t++) {
        const float *ht = h + t * H;
        if (logits_in) memcpy(lg, logits_in + t * E, E * sizeof(float));
        else or_matmul_f16(lg, L->router, ht, E, H);
        or_moe_route(lg, E, k, L->norm_topk_prob, probs, idx);
        float *proj = out + t * H;
        for (size_t o = 0; o < H; o++) proj[o] = 0.0f;
        for (size_t s = 0; s < k; s++) {
            const uint32_t e = idx[s];
            if (!R->wg[e]) { rc = OR_ERR_OUT_OF_RANGE; break; }
            or_moe_expert_accum_f32(proj, hs, is, ht, R->wg[e], R->wu[e], R->wd[e], I, H, probs[s], L->use_gelu);
        }
        if (rc == OR_OK && L->shared_inter) shared_add(L, ht, proj, sh_out, sh_scr);
    }
    free(lg); free(probs); free(idx); free(hs); free(is); free(sh_out); free(sh_scr);
    return rc;
}

/* The streaming decode loop exactly as the engine runs it (engine.zig:705-779):
 * per token, per slot, dequantise the three projections from the payload and
 * accumulate.  Slow on purpose; it is the CPU baseline. */
int or_layer_forward_streaming(const or_layer *L, const float *h, size_t T, const float *logits_in, float *out)
{
    const size_t H = L->hidden, I = L->inter, E = L->n_experts, k = L->k;
    int rc = OR_OK;
    float *lg = malloc(E * sizeof(float)), *probs = malloc(k * sizeof(float));
    uint32_t *idx = malloc(k * sizeof(uint32_t));
    float *wg = malloc(I * H * sizeof(float)), *wu = malloc(I * H * sizeof(float)), *wd = malloc(I * H * sizeof(float));
    float *hs = malloc(I * sizeof(float)), *is = malloc(I * sizeof(float));
    float *sh_out = L->shared_inter ? malloc(H * sizeof(float)) : NULL;
    float *sh_scr = L->shared_inter ? malloc(L->shared_inter * sizeof(float)) : NULL;
    for (size_t t = 0; t < T && rc == OR_OK; t++) {
        const float *ht = h + t * H;
        if (logits_in) memcpy(lg, logits_in + t * E, E * sizeof(float));
        else or_matmul_f16(lg, L->router, ht, E, H);
        or_moe_route(lg, E, k, L->norm_topk_prob, probs, idx);
        float *proj = out + t * H;
        for (size_t o = 0; o < H; o++) proj[o] = 0.0f;
        for (size_t s = 0; s < k; s++) {
            uint32_t e = idx[s];
            if ((rc = or_read_expert_f32(L->gate_type, L->gate, L->gate_len, e, (uint32_t)E, wg, I * H))) break;
            if ((rc = or_read_expert_f32(L->up_type, L->up, L->up_len, e, (uint32_t)E, wu, I * H))) break;
            if ((rc = or_read_expert_f32(L->down_type, L->down, L->down_len, e, (uint32_t)E, wd, I * H))) break;
            or_moe_expert_accum_f32(proj, hs, is, ht, wg, wu, wd, I, H, probs[s], L->use_gelu);
        }
        if (rc == OR_OK && L->shared_inter) shared_add(L, ht, proj, sh_out, sh_scr);
    }
    free(lg); free(probs); free(idx); free(wg); free(wu); free(wd); free(hs); free(is);
    free(sh_out); free(sh_scr);
    return rc;
}
