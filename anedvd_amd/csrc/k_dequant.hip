// k_dequant.hip -- GGUF block dequantisation (bit-exact f32) and the repack of
// GGUF expert tensors into the HBM tile layout the GEMV/GEMM kernels read.
//
// Every block routine follows the reference dequantiser named beside it
// (gguf.zig:743-1071) in the same f32 operations.  Each product of a quant and
// its scale is exact in f32 (an f16 scale carries 11 significant bits, a
// sub-block scale at most 7 and a quant at most 7, which fit f32's 24), so
// contraction could not change a value; it is switched off anyway so the code
// says what it does.
#pragma clang fp contract(off)

#include "common.h"
#include "kernels.h"

namespace anedvd {

__device__ inline uint16_t rd16(const uint8_t *b) { return (uint16_t)(b[0] | (b[1] << 8)); }
__device__ inline uint32_t rd32(const uint8_t *b)
{
    return (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
}
__device__ inline float h2f(const uint8_t *b) { return f16_bits_to_f32(rd16(b)); }
__device__ inline float u2f(uint32_t u) { return __uint_as_float(u); }

// dequantQ4_0, gguf.zig:763-776
__device__ void deq_q4_0(const uint8_t *blk, float *y)
{
    const float d = h2f(blk);
    for (int j = 0; j < 16; j++) {
        const uint8_t q = blk[2 + j];
        y[j] = (float)((int)(q & 0x0F) - 8) * d;
        y[j + 16] = (float)((int)(q >> 4) - 8) * d;
    }
}

// dequantQ4_1, gguf.zig:778-793
__device__ void deq_q4_1(const uint8_t *blk, float *y)
{
    const float d = h2f(blk), m = h2f(blk + 2);
    for (int j = 0; j < 16; j++) {
        const uint8_t q = blk[4 + j];
        y[j] = (float)(q & 0x0F) * d + m;
        y[j + 16] = (float)(q >> 4) * d + m;
    }
}

// dequantQ5 (q5_0 / q5_1), gguf.zig:795-825
__device__ void deq_q5(const uint8_t *blk, float *y, bool has_min)
{
    const int qh_off = has_min ? 4 : 2, qs_off = qh_off + 4, minus = has_min ? 0 : 16;
    const float d = h2f(blk), m = has_min ? h2f(blk + 2) : 0.0f;
    const uint32_t qh = rd32(blk + qh_off);
    for (int j = 0; j < 16; j++) {
        const uint8_t q = blk[qs_off + j];
        const uint32_t xh0 = ((qh >> j) << 4) & 0x10u, xh1 = (qh >> (j + 12)) & 0x10u;
        y[j] = (float)((int)((q & 0x0F) | xh0) - minus) * d + m;
        y[j + 16] = (float)((int)((q >> 4) | xh1) - minus) * d + m;
    }
}

// dequantQ8_0, gguf.zig:827-840
__device__ void deq_q8_0(const uint8_t *blk, float *y)
{
    const float d = h2f(blk);
    for (int j = 0; j < 32; j++) y[j] = d * (float)(int8_t)blk[2 + j];
}

// dequantQ8_1, gguf.zig:842-853
__device__ void deq_q8_1(const uint8_t *blk, float *y)
{
    const float d = h2f(blk);
    for (int j = 0; j < 32; j++) y[j] = (float)(int8_t)blk[4 + j] * d;
}

// dequantQ2K, gguf.zig:855-890
__device__ void deq_q2_k(const uint8_t *blk, float *y)
{
    const float d = h2f(blk + 80), mn = h2f(blk + 82);
    int q = 16, is = 0, o = 0;
    for (int half = 0; half < 2; half++) {
        int shift = 0;
        for (int g = 0; g < 4; g++) {
            for (int part = 0; part < 2; part++) {
                const uint8_t sc = blk[is++];
                const float dl = d * (float)(sc & 0x0F), ml = mn * (float)(sc >> 4);
                for (int l = 0; l < 16; l++) y[o + l] = dl * (float)((blk[q + l + 16 * part] >> shift) & 3) - ml;
                o += 16;
            }
            shift += 2;
        }
        q += 32;
    }
}

// dequantQ3K, gguf.zig:892-946
__device__ void deq_q3_k(const uint8_t *blk, float *y)
{
    const uint32_t kmask1 = 0x03030303u, kmask2 = 0x0f0f0f0fu;
    const float d_all = h2f(blk + 108);
    const uint8_t *hm = blk, *qs = blk + 32;
    uint32_t aux[4] = { rd32(blk + 96), rd32(blk + 100), rd32(blk + 104), 0 };
    const uint32_t tmp = aux[2];
    aux[2] = ((aux[0] >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4);
    aux[3] = ((aux[1] >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4);
    aux[0] = (aux[0] & kmask2) | (((tmp >> 0) & kmask1) << 4);
    aux[1] = (aux[1] & kmask2) | (((tmp >> 2) & kmask1) << 4);
    uint8_t m = 1;
    int is = 0, q = 0, o = 0;
    for (int half = 0; half < 2; half++) {
        int shift = 0;
        for (int g = 0; g < 4; g++) {
            for (int part = 0; part < 2; part++) {
                const int8_t sc = (int8_t)(uint8_t)(aux[is >> 2] >> (8 * (is & 3)));
                is++;
                const float dl = d_all * (float)((int)sc - 32);
                for (int l = 0; l < 16; l++) {
                    const int low = (qs[q + l + 16 * part] >> shift) & 3;
                    y[o + l] = dl * (float)(low - ((hm[l + 16 * part] & m) ? 0 : 4));
                }
                o += 16;
            }
            shift += 2;
            m = (uint8_t)(m << 1);
        }
        q += 32;
    }
}

// getScaleMinK4, gguf.zig:948-958
__device__ inline void scale_min_k4(int j, const uint8_t *q, int &d, int &m)
{
    if (j < 4) {
        d = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// dequantQ4K, gguf.zig:960-996
__device__ void deq_q4_k(const uint8_t *blk, float *y)
{
    const float d = h2f(blk), mn = h2f(blk + 2);
    const uint8_t *scales = blk + 4;
    int q = 16;
    for (int is = 0; is < 8; is += 2) {
        int sd, sm;
        scale_min_k4(is, scales, sd, sm);
        const float d1 = d * (float)sd, m1 = mn * (float)sm;
        scale_min_k4(is + 1, scales, sd, sm);
        const float d2 = d * (float)sd, m2 = mn * (float)sm;
        float *yy = y + (is / 2) * 64;
        for (int l = 0; l < 32; l++) {
            yy[l] = d1 * (float)(blk[q + l] & 0x0F) - m1;
            yy[l + 32] = d2 * (float)(blk[q + l] >> 4) - m2;
        }
        q += 32;
    }
}

// dequantQ5K, gguf.zig:998-1034
__device__ void deq_q5_k(const uint8_t *blk, float *y)
{
    const float d = h2f(blk), mn = h2f(blk + 2);
    const uint8_t *scales = blk + 4, *qh = blk + 16;
    int ql = 48;
    uint8_t mask1 = 1, mask2 = 2;
    for (int is = 0; is < 8; is += 2) {
        int sd, sm;
        scale_min_k4(is, scales, sd, sm);
        const float d1 = d * (float)sd, m1 = mn * (float)sm;
        scale_min_k4(is + 1, scales, sd, sm);
        const float d2 = d * (float)sd, m2 = mn * (float)sm;
        float *yy = y + (is / 2) * 64;
        for (int l = 0; l < 32; l++) yy[l] = d1 * (float)((blk[ql + l] & 0x0F) + ((qh[l] & mask1) ? 16 : 0)) - m1;
        for (int l = 0; l < 32; l++) yy[l + 32] = d2 * (float)((blk[ql + l] >> 4) + ((qh[l] & mask2) ? 16 : 0)) - m2;
        ql += 32;
        mask1 = (uint8_t)(mask1 << 2);
        mask2 = (uint8_t)(mask2 << 2);
    }
}

// dequantQ6K, gguf.zig:1036-1059
__device__ void deq_q6_k(const uint8_t *blk, float *y)
{
    const float d = h2f(blk + 208);
    for (int half = 0; half < 2; half++) {
        const uint8_t *ql = blk + half * 64, *qh = blk + 128 + half * 32, *sc = blk + 192 + half * 8;
        float *yy = y + half * 128;
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
            const int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            yy[l] = d * (float)(int8_t)sc[is] * (float)q1;
            yy[l + 32] = d * (float)(int8_t)sc[is + 2] * (float)q2;
            yy[l + 64] = d * (float)(int8_t)sc[is + 4] * (float)q3;
            yy[l + 96] = d * (float)(int8_t)sc[is + 6] * (float)q4;
        }
    }
}

// dequantQ8K, gguf.zig:1061-1071
__device__ void deq_q8_k(const uint8_t *blk, float *y)
{
    const float d = u2f(rd32(blk));
    for (int j = 0; j < 256; j++) y[j] = (float)(int8_t)blk[4 + j] * d;
}

__device__ void deq_block(int t, const uint8_t *blk, float *y)
{
    switch (t) {
    case ANEDVD_F32: y[0] = u2f(rd32(blk)); break;
    case ANEDVD_F16: y[0] = h2f(blk); break;
    case ANEDVD_BF16: y[0] = u2f((uint32_t)rd16(blk) << 16); break;
    case ANEDVD_Q4_0: deq_q4_0(blk, y); break;
    case ANEDVD_Q4_1: deq_q4_1(blk, y); break;
    case ANEDVD_Q5_0: deq_q5(blk, y, false); break;
    case ANEDVD_Q5_1: deq_q5(blk, y, true); break;
    case ANEDVD_Q8_0: deq_q8_0(blk, y); break;
    case ANEDVD_Q8_1: deq_q8_1(blk, y); break;
    case ANEDVD_Q2_K: deq_q2_k(blk, y); break;
    case ANEDVD_Q3_K: deq_q3_k(blk, y); break;
    case ANEDVD_Q4_K: deq_q4_k(blk, y); break;
    case ANEDVD_Q5_K: deq_q5_k(blk, y); break;
    case ANEDVD_Q6_K: deq_q6_k(blk, y); break;
    case ANEDVD_Q8_K: deq_q8_k(blk, y); break;
    default: break;
    }
}

// One thread per GGUF block: src holds n_blocks whole blocks.
__global__ void k_dequant_gguf(int t, const uint8_t *__restrict__ src, size_t n_blocks, float *__restrict__ out)
{
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_blocks) return;
    const int epb = block_elems(t), bpb = block_bytes(t);
    deq_block(t, src + b * bpb, out + b * epb);
}

// ------------------------------------------------------------------ repack
//
// The MMA tile layout (common.h) moves the bits of the GGUF blocks; gguf_quant()
// and set_gguf_quant() read and write one element's raw quant in GGUF block
// bytes, so the repack and its inverse share one statement of each format.

// Raw 6-bit scale k (0..15) of a Q3_K block from its 12 packed bytes (the unpacking
// of dequantQ3K, gguf.zig:899-906, one scale at a time).
__device__ inline int q3k_scale(const uint8_t *s12, int k)
{
    const int b = k & 3, g = k >> 2;  // g: which of the four unpacked words
    const int lo = g == 0 ? s12[b] & 0xF : g == 1 ? s12[4 + b] & 0xF : g == 2 ? s12[b] >> 4 : s12[4 + b] >> 4;
    return lo | (((s12[8 + b] >> (2 * g)) & 3) << 4);
}

// Raw quant of element e of a GGUF block: Q8_0 / Q8_1 the int8, Q4_0 / Q4_1 / Q4_K
// the nibble, Q5_0 / Q5_1 / Q5_K the 5-bit value (before Q5_0's -16 offset), Q6_K
// the 6-bit value (before the -32 offset).
__device__ inline int gguf_quant(int t, const uint8_t *blk, int e)
{
    switch (t) {
    case ANEDVD_F16: return rd16(blk + 2 * e);  // the value's 16 bits
    case ANEDVD_Q8_0: return (int)(int8_t)blk[2 + e];
    case ANEDVD_Q8_1: return (int)(int8_t)blk[4 + e];  // dequantQ8_1: qs after d and s
    case ANEDVD_Q4_0: return e < 16 ? blk[2 + e] & 0xF : blk[2 + e - 16] >> 4;  // dequantQ4_0
    case ANEDVD_Q4_1: return e < 16 ? blk[4 + e] & 0xF : blk[4 + e - 16] >> 4;  // dequantQ4_1
    case ANEDVD_Q5_0:
    case ANEDVD_Q5_1: {  // dequantQ5 (gguf.zig:795-822): nibble of qs[e % 16], bit e of qh
        const int o = t == ANEDVD_Q5_1 ? 4 : 2;
        const uint32_t qh = blk[o] | (blk[o + 1] << 8) | (blk[o + 2] << 16) | ((uint32_t)blk[o + 3] << 24);
        const int nib = e < 16 ? blk[o + 4 + e] & 0xF : blk[o + 4 + e - 16] >> 4;
        return nib | (int)(((qh >> e) & 1) << 4);
    }
    case ANEDVD_Q2_K: {  // dequantQ2K (gguf.zig:855-889): half e/128, shift 2 (e%128)/32
        const int h = e >> 7, j = (e & 127) >> 5, l = e & 31;
        return (blk[16 + 32 * h + l] >> (2 * j)) & 3;
    }
    case ANEDVD_Q3_K: {  // dequantQ3K (gguf.zig:891-946): low 2 bits + hmask bit 4 h + j; value u - 4
        const int h = e >> 7, j = (e & 127) >> 5, l = e & 31;
        return ((blk[32 + 32 * h + l] >> (2 * j)) & 3) | (((blk[l] >> (4 * h + j)) & 1) << 2);
    }
    case ANEDVD_Q4_K: {  // dequantQ4K: group e/64, low nibbles first, then high
        const int g = e >> 6, l = e & 63;
        const uint8_t q = blk[16 + 32 * g + (l & 31)];
        return l < 32 ? q & 0xF : q >> 4;
    }
    case ANEDVD_Q5_K: {  // dequantQ5K (gguf.zig:998-1034): group e/64, nibble + qh bit 2 g + (l >= 32)
        const int g = e >> 6, l = e & 63;
        const uint8_t q = blk[48 + 32 * g + (l & 31)], qh = blk[16 + (l & 31)];
        return (l < 32 ? q & 0xF : q >> 4) | (((qh >> (2 * g + (l >> 5))) & 1) << 4);
    }
    case ANEDVD_Q6_K: {  // dequantQ6K: half e/128, quarter (e%128)/32
        const int h = e >> 7, qd = (e & 127) >> 5, l = e & 31;
        const uint8_t ql = blk[64 * h + l + (qd & 1) * 32], qh = blk[128 + 32 * h + l];
        return ((qd & 2) ? ql >> 4 : ql & 0xF) | (((qh >> (2 * qd)) & 3) << 4);
    }
    default: return 0;
    }
}

__device__ inline void set_gguf_quant(int t, uint8_t *blk, int e, int v)
{
    switch (t) {
    case ANEDVD_F16:
        blk[2 * e] = (uint8_t)(v & 0xFF);
        blk[2 * e + 1] = (uint8_t)((v >> 8) & 0xFF);
        break;
    case ANEDVD_Q8_0: blk[2 + e] = (uint8_t)v; break;
    case ANEDVD_Q8_1: blk[4 + e] = (uint8_t)v; break;
    case ANEDVD_Q4_0:
    case ANEDVD_Q4_1: {
        const int o = t == ANEDVD_Q4_1 ? 4 : 2;
        if (e < 16) blk[o + e] = (uint8_t)((blk[o + e] & 0xF0) | v);
        else blk[o + e - 16] = (uint8_t)((blk[o + e - 16] & 0x0F) | (v << 4));
        break;
    }
    case ANEDVD_Q5_0:
    case ANEDVD_Q5_1: {
        const int o = t == ANEDVD_Q5_1 ? 4 : 2;
        uint8_t &q = e < 16 ? blk[o + 4 + e] : blk[o + 4 + e - 16];
        q = e < 16 ? (uint8_t)((q & 0xF0) | (v & 0xF)) : (uint8_t)((q & 0x0F) | ((v & 0xF) << 4));
        uint8_t &h = blk[o + (e >> 3)];
        h = (uint8_t)((h & ~(1 << (e & 7))) | (((v >> 4) & 1) << (e & 7)));
        break;
    }
    case ANEDVD_Q2_K:
    case ANEDVD_Q3_K: {
        const int h = e >> 7, j = (e & 127) >> 5, l = e & 31;
        uint8_t &q = blk[(t == ANEDVD_Q3_K ? 32 : 16) + 32 * h + l];
        q = (uint8_t)((q & ~(3 << (2 * j))) | ((v & 3) << (2 * j)));
        if (t == ANEDVD_Q3_K) {
            const int sh = 4 * h + j;
            blk[l] = (uint8_t)((blk[l] & ~(1 << sh)) | (((v >> 2) & 1) << sh));
        }
        break;
    }
    case ANEDVD_Q4_K: {
        const int g = e >> 6, l = e & 63;
        uint8_t &q = blk[16 + 32 * g + (l & 31)];
        q = l < 32 ? (uint8_t)((q & 0xF0) | v) : (uint8_t)((q & 0x0F) | (v << 4));
        break;
    }
    case ANEDVD_Q5_K: {
        const int g = e >> 6, l = e & 63, sh = 2 * g + (l >> 5);
        uint8_t &q = blk[48 + 32 * g + (l & 31)], &qh = blk[16 + (l & 31)];
        q = l < 32 ? (uint8_t)((q & 0xF0) | (v & 0xF)) : (uint8_t)((q & 0x0F) | ((v & 0xF) << 4));
        qh = (uint8_t)((qh & ~(1 << sh)) | (((v >> 4) & 1) << sh));
        break;
    }
    case ANEDVD_Q6_K: {
        const int h = e >> 7, qd = (e & 127) >> 5, l = e & 31;
        uint8_t &ql = blk[64 * h + l + (qd & 1) * 32], &qh = blk[128 + 32 * h + l];
        ql = (qd & 2) ? (uint8_t)((ql & 0x0F) | ((v & 0xF) << 4)) : (uint8_t)((ql & 0xF0) | (v & 0xF));
        qh = (uint8_t)((qh & ~(3 << (2 * qd))) | (((v >> 4) & 3) << (2 * qd)));
        break;
    }
    default: break;
    }
}

// Lane bytes of one (step, tile) from the lane's 16 raw quants v[8j + i].
__device__ inline void pack_lane(int t, const int *v, uint8_t *out)
{
    switch (t) {
    case ANEDVD_F16:  // the 16 values in order, 2 bytes each: block j in bytes 16 j .. 16 j + 15
        for (int k = 0; k < 16; k++) {
            out[2 * k] = (uint8_t)(v[k] & 0xFF);
            out[2 * k + 1] = (uint8_t)((v[k] >> 8) & 0xFF);
        }
        break;
    case ANEDVD_Q8_0:
    case ANEDVD_Q8_1:
        for (int k = 0; k < 16; k++) out[k] = (uint8_t)((v[k] + 128) & 0xFF);
        break;
    case ANEDVD_Q2_K:
    case ANEDVD_Q3_K:  // bits 2 k of byte b: value 8 (k / 2) + 4 (k % 2) + b; Q3_K's third bits as the 5-bit h plane
        for (int b = 0; b < 4; b++) {
            int w = 0;
            for (int k = 0; k < 4; k++) w |= (v[8 * (k >> 1) + 4 * (k & 1) + b] & 3) << (2 * k);
            out[b] = (uint8_t)w;
        }
        if (t == ANEDVD_Q3_K) {
            int h = 0;
            for (int k = 0; k < 4; k++)
                for (int b = 0; b < 4; b++) h |= ((v[8 * (k >> 1) + 4 * (k & 1) + b] >> 2) & 1) << (4 * k + b);
            out[8] = (uint8_t)(h & 0xFF);
            out[9] = (uint8_t)(h >> 8);
        }
        break;
    case ANEDVD_Q4_0:
    case ANEDVD_Q4_1:
    case ANEDVD_Q5_0:
    case ANEDVD_Q5_1:
    case ANEDVD_Q4_K:
    case ANEDVD_Q5_K:
    case ANEDVD_Q6_K:
        for (int j = 0; j < 2; j++)
            for (int b = 0; b < 4; b++) out[4 * j + b] = (uint8_t)((v[8 * j + b] & 0xF) | ((v[8 * j + b + 4] & 0xF) << 4));
        if (tile_hb(t) == 2) {  // bit 4 (2 j + hh) + b: the fifth bit of value 8 j + 4 hh + b
            int h = 0;
            for (int j = 0; j < 2; j++)
                for (int hh = 0; hh < 2; hh++)
                    for (int b = 0; b < 4; b++) h |= ((v[8 * j + 4 * hh + b] >> 4) & 1) << (4 * (2 * j + hh) + b);
            out[8] = (uint8_t)(h & 0xFF);
            out[9] = (uint8_t)(h >> 8);
        }
        if (t == ANEDVD_Q6_K)
            for (int b = 0; b < 4; b++) {
                int h = 0;
                for (int j = 0; j < 2; j++)
                    for (int hh = 0; hh < 2; hh++) h |= ((v[8 * j + b + 4 * hh] >> 4) & 3) << (4 * j + 2 * hh);
                out[8 + b] = (uint8_t)h;
            }
        break;
    default: break;
    }
}

__device__ inline int unpack_lane(int t, const uint8_t *in, int k)
{
    switch (t) {
    case ANEDVD_F16: return in[2 * k] | (in[2 * k + 1] << 8);
    case ANEDVD_Q8_0:
    case ANEDVD_Q8_1: return (int)in[k] - 128;
    case ANEDVD_Q2_K:
    case ANEDVD_Q3_K: {
        const int j = k >> 3, i = k & 7, kk = 2 * j + (i >> 2), b = i & 3;
        const int lo = (in[b] >> (2 * kk)) & 3;
        if (t == ANEDVD_Q2_K) return lo;
        const int bit = 4 * kk + b;
        return lo | (((in[8 + (bit >> 3)] >> (bit & 7)) & 1) << 2);
    }
    case ANEDVD_Q4_0:
    case ANEDVD_Q4_1:
    case ANEDVD_Q4_K: {
        const int j = k >> 3, i = k & 7;
        return (in[4 * j + (i & 3)] >> (4 * (i >> 2))) & 0xF;
    }
    case ANEDVD_Q5_0:
    case ANEDVD_Q5_1:
    case ANEDVD_Q5_K: {
        const int j = k >> 3, i = k & 7;
        const int lo = (in[4 * j + (i & 3)] >> (4 * (i >> 2))) & 0xF;
        const int bit = 4 * (2 * j + (i >> 2)) + (i & 3);
        return lo | (((in[8 + (bit >> 3)] >> (bit & 7)) & 1) << 4);
    }
    case ANEDVD_Q6_K: {
        const int j = k >> 3, i = k & 7;
        const int lo = (in[4 * j + (i & 3)] >> (4 * (i >> 2))) & 0xF;
        const int hi = (in[8 + (i & 3)] >> (4 * j + 2 * (i >> 2))) & 3;
        return lo | (hi << 4);
    }
    default: return 0;
    }
}

// One thread per (matrix, row, scale unit): moves the unit's quants and scales
// from the stacked GGUF payload `src` (matrices slowest) into the tile layout.
template <int TYPE>
__global__ void k_repack(QMat m, const uint8_t *__restrict__ src)
{
    m.type = TYPE;  // one instantiation per format: every format switch below folds
    const Fmt f = tile_fmt(TYPE);
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t per_mat = (size_t)m.rows * m.units;
    if (id >= per_mat * m.n) return;
    const int mat = (int)(id / per_mat);
    const int r = (int)((id % per_mat) / m.units), u = (int)(id % m.units);
    const int rb = r / kRowBlock, t = (r % kRowBlock) / 16, n = r % 16;
    const int bpb = block_bytes(m.type), epb = block_elems(m.type);
    const size_t row_bytes = (size_t)m.cols / epb * bpb;
    const uint8_t *row = src + ((size_t)mat * m.rows + r) * row_bytes;
    uint8_t *q = m.q + (size_t)mat * m.q_stride;
    for (int s = u * f.spu; s < (u + 1) * f.spu; s++)
        for (int g = 0; g < 4; g++) {
            int v[16];
            for (int k = 0; k < 16; k++) {
                const int c = kStep * s + mma_col(g, k >> 3, k & 7);
                v[k] = gguf_quant(m.type, row + (size_t)(c / epb) * bpb, c % epb);
            }
            uint8_t lb[32];  // F16: 32 value bytes; Q8_0: 16 quant bytes; Q5_K / Q6_K: 8 quant + 2 / 4 high-bit bytes
            pack_lane(m.type, v, lb);
            uint8_t *dst = q + tile_q_off(f, m.steps, rb, s, t, 16 * g + n);
            for (int k = 0; k < f.qb; k++) dst[k] = lb[k];
            if (const int hb = tile_hb(m.type)) {
                uint8_t *hd = m.h + (size_t)mat * m.h_stride + tile_h_off(m.steps, rb, s, t, 16 * g + n, hb);
                for (int k = 0; k < hb; k++) hd[k] = lb[8 + k];
            }
        }
    uint8_t *sc = m.s + (size_t)mat * m.s_stride + tile_s_off(f, m.units, rb, u, t, n);
    const int c0 = u * f.spu * kStep;
    const uint8_t *b0 = row + (size_t)(c0 / epb) * bpb;
    switch (m.type) {
    case ANEDVD_Q8_0:
    case ANEDVD_Q8_1:
    case ANEDVD_Q4_0:
    case ANEDVD_Q5_0:  // the f16 d of the step's two blocks
        sc[0] = b0[0];
        sc[1] = b0[1];
        sc[2] = b0[bpb];
        sc[3] = b0[bpb + 1];
        break;
    case ANEDVD_Q4_1:
    case ANEDVD_Q5_1:  // d, m of the step's two blocks
        for (int k = 0; k < 4; k++) {
            sc[k] = b0[k];
            sc[4 + k] = b0[bpb + k];
        }
        break;
    case ANEDVD_Q2_K: {  // 16 scale|min bytes; d, dmin to the d plane
        for (int k = 0; k < 16; k++) sc[k] = b0[k];
        uint8_t *dp = m.d + (size_t)mat * m.d_stride + tile_d_off(m.units, rb, u, t, n, 4);
        for (int k = 0; k < 4; k++) dp[k] = b0[80 + k];
        break;
    }
    case ANEDVD_Q3_K: {  // the 12 packed 6-bit scales unpacked to int8 (scale - 32); d to the d plane
        for (int k = 0; k < 16; k++) sc[k] = (uint8_t)(q3k_scale(b0 + 96, k) - 32);
        uint8_t *dp = m.d + (size_t)mat * m.d_stride + tile_d_off(m.units, rb, u, t, n, 2);
        dp[0] = b0[108];
        dp[1] = b0[109];
        break;
    }
    case ANEDVD_Q4_K:  // d, dmin, 12 scale bytes
    case ANEDVD_Q5_K:
        for (int k = 0; k < 16; k++) sc[k] = b0[k];
        break;
    case ANEDVD_Q6_K: {  // 16 int8 scales; d to the d plane
        for (int k = 0; k < 16; k++) sc[k] = b0[192 + k];
        uint8_t *dp = m.d + (size_t)mat * m.d_stride + tile_d_off(m.units, rb, u, t, n, 2);
        dp[0] = b0[208];
        dp[1] = b0[209];
        break;
    }
    default: break;
    }
}

// One thread per GGUF block of matrix `mat`: rebuilds the block's bytes from the
// tile layout and dequantises them (out[rows][cols] f32, bit-exact).
template <int TYPE>
__global__ void k_dequant_tiles(QMat m, int mat, float *__restrict__ out)
{
    m.type = TYPE;  // one instantiation per format: every format switch below folds
    const Fmt f = tile_fmt(TYPE);
    const int bpb = block_bytes(m.type), epb = block_elems(m.type);
    const int bpr = m.cols / epb;
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= (size_t)m.rows * bpr) return;
    const int r = (int)(id / bpr), b = (int)(id % bpr);
    const int rb = r / kRowBlock, t = (r % kRowBlock) / 16, n = r % 16;
    const uint8_t *q = m.q + (size_t)mat * m.q_stride;
    uint8_t blk[292];
    for (int k = 0; k < bpb; k++) blk[k] = 0;
    for (int e = 0; e < epb; e++) {
        const int c = b * epb + e, s = c / kStep, w = c % kStep;
        const int j = w >> 5, g = (w & 31) >> 3, i = w & 7;
        uint8_t lb[32];  // F16: 32 value bytes; Q8_0: 16 quant bytes; Q5_K / Q6_K: 8 quant + 2 / 4 high-bit bytes
        const uint8_t *src = q + tile_q_off(f, m.steps, rb, s, t, 16 * g + n);
        for (int k = 0; k < f.qb; k++) lb[k] = src[k];
        if (const int hb = tile_hb(m.type)) {
            const uint8_t *hs = m.h + (size_t)mat * m.h_stride + tile_h_off(m.steps, rb, s, t, 16 * g + n, hb);
            for (int k = 0; k < hb; k++) lb[8 + k] = hs[k];
        }
        set_gguf_quant(m.type, blk, e, unpack_lane(m.type, lb, 8 * j + i));
    }
    const int u = (b * epb) / (f.spu * kStep);
    const uint8_t *sc = m.s + (size_t)mat * m.s_stride + tile_s_off(f, m.units, rb, u, t, n);
    switch (m.type) {
    case ANEDVD_Q8_0:
    case ANEDVD_Q8_1:  // (Q8_1's s is not read by its dequantisation; it stays 0)
    case ANEDVD_Q4_0:
    case ANEDVD_Q5_0: {
        const int j = (b * epb / 32) & 1;  // which of the step's two blocks
        blk[0] = sc[2 * j];
        blk[1] = sc[2 * j + 1];
        break;
    }
    case ANEDVD_Q4_1:
    case ANEDVD_Q5_1: {
        const int j = (b * epb / 32) & 1;
        for (int k = 0; k < 4; k++) blk[k] = sc[4 * j + k];
        break;
    }
    case ANEDVD_Q4_K:
    case ANEDVD_Q5_K:
        for (int k = 0; k < 16; k++) blk[k] = sc[k];
        break;
    case ANEDVD_Q2_K: {
        for (int k = 0; k < 16; k++) blk[k] = sc[k];
        const uint8_t *dp = m.d + (size_t)mat * m.d_stride + tile_d_off(m.units, rb, u, t, n, 4);
        for (int k = 0; k < 4; k++) blk[80 + k] = dp[k];
        break;
    }
    case ANEDVD_Q3_K: {
        int raw[16];
        for (int k = 0; k < 16; k++) raw[k] = ((int)(int8_t)sc[k] + 32) & 63;
        for (int b = 0; b < 4; b++) {  // the packing dequantQ3K unpacks (gguf.zig:899-906)
            blk[96 + b] = (uint8_t)((raw[b] & 0xF) | ((raw[8 + b] & 0xF) << 4));
            blk[100 + b] = (uint8_t)((raw[4 + b] & 0xF) | ((raw[12 + b] & 0xF) << 4));
            blk[104 + b] = (uint8_t)((raw[b] >> 4) | ((raw[4 + b] >> 4) << 2) | ((raw[8 + b] >> 4) << 4) |
                                     ((raw[12 + b] >> 4) << 6));
        }
        const uint8_t *dp = m.d + (size_t)mat * m.d_stride + tile_d_off(m.units, rb, u, t, n, 2);
        blk[108] = dp[0];
        blk[109] = dp[1];
        break;
    }
    case ANEDVD_Q6_K: {
        for (int k = 0; k < 16; k++) blk[192 + k] = sc[k];
        const uint8_t *dp = m.d + (size_t)mat * m.d_stride + tile_d_off(m.units, rb, u, t, n, 2);
        blk[208] = dp[0];
        blk[209] = dp[1];
        break;
    }
    default: break;
    }
    deq_block(m.type, blk, out + (size_t)r * m.cols + (size_t)b * epb);
}

// ------------------------------------------------------------------ launchers

int launch_dequant_gguf(int t, const uint8_t *d_src, size_t n_blocks, float *d_out, hipStream_t st)
{
    if (n_blocks == 0) return ANEDVD_OK;
    const unsigned grid = (unsigned)((n_blocks + 255) / 256);
    hipLaunchKernelGGL(k_dequant_gguf, dim3(grid), dim3(256), 0, st, t, d_src, n_blocks, d_out);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

// The formats with a tile layout, for the per-format kernel instantiations.
#define ANEDVD_TILE_TYPES(X) X(ANEDVD_Q8_0) X(ANEDVD_Q8_1) X(ANEDVD_Q4_0) X(ANEDVD_Q4_1) X(ANEDVD_Q5_0) \
    X(ANEDVD_Q5_1) X(ANEDVD_Q2_K) X(ANEDVD_Q3_K) X(ANEDVD_Q4_K) X(ANEDVD_Q5_K) X(ANEDVD_Q6_K) X(ANEDVD_F16)

int launch_repack(const QMat &m, const uint8_t *d_src, hipStream_t st)
{
    const size_t n = (size_t)m.n * m.rows * m.units;
    const dim3 grid((unsigned)((n + 255) / 256)), block(256);
    switch (m.type) {
#define ANEDVD_CASE(T) \
    case T: hipLaunchKernelGGL(k_repack<T>, grid, block, 0, st, m, d_src); break;
        ANEDVD_TILE_TYPES(ANEDVD_CASE)
#undef ANEDVD_CASE
    default:
        set_error("repack: ggml type %d has no tile layout", m.type);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

// f32ToF16Slice (gguf.zig:682-692): each value rounded to the nearest f16, ties
// to even (the hardware conversion's default rounding), overflow to infinity.
__global__ void k_f32_to_f16(const float *__restrict__ src, uint16_t *__restrict__ dst, size_t n)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const half_t h = (half_t)src[i];
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    dst[i] = b;
}

int launch_f32_to_f16(const float *d_src, uint16_t *d_dst, size_t n, hipStream_t st)
{
    if (n == 0) return ANEDVD_OK;
    hipLaunchKernelGGL(k_f32_to_f16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, d_src, d_dst, n);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

// f16 -> f32 (exact), eight values per thread: the f16-activation forward's input
// widened into the call's staging.
__global__ __launch_bounds__(256) void k_f16_to_f32(const uint16_t *__restrict__ src, float *__restrict__ dst,
                                                   size_t n)
{
    const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (i + 8 <= n && (((uintptr_t)(src + i) | (uintptr_t)(dst + i)) & 15) == 0) {
        const uint4 v = *(const uint4 *)(src + i);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        float4 lo, hi;
        lo.x = f16_bits_to_f32((uint16_t)w[0]); lo.y = f16_bits_to_f32((uint16_t)(w[0] >> 16));
        lo.z = f16_bits_to_f32((uint16_t)w[1]); lo.w = f16_bits_to_f32((uint16_t)(w[1] >> 16));
        hi.x = f16_bits_to_f32((uint16_t)w[2]); hi.y = f16_bits_to_f32((uint16_t)(w[2] >> 16));
        hi.z = f16_bits_to_f32((uint16_t)w[3]); hi.w = f16_bits_to_f32((uint16_t)(w[3] >> 16));
        *(float4 *)(dst + i) = lo;
        *(float4 *)(dst + i + 4) = hi;
    } else {
        for (size_t j = i; j < n && j < i + 8; j++) dst[j] = f16_bits_to_f32(src[j]);
    }
}

int launch_f16_to_f32(const uint16_t *d_src, float *d_dst, size_t n, hipStream_t st)
{
    if (n == 0) return ANEDVD_OK;
    const size_t threads = (n + 7) / 8;
    hipLaunchKernelGGL(k_f16_to_f32, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, d_src, d_dst, n);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

int launch_dequant_tiles(const QMat &m, int mat, float *d_out, hipStream_t st)
{
    const size_t n = (size_t)m.rows * (m.cols / block_elems(m.type));
    const dim3 grid((unsigned)((n + 255) / 256)), block(256);
    switch (m.type) {
#define ANEDVD_CASE(T) \
    case T: hipLaunchKernelGGL(k_dequant_tiles<T>, grid, block, 0, st, m, mat, d_out); break;
        ANEDVD_TILE_TYPES(ANEDVD_CASE)
#undef ANEDVD_CASE
    default:
        set_error("dequant_tiles: ggml type %d has no tile layout", m.type);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

}  // namespace anedvd
