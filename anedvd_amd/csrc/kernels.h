// kernels.h -- host-side launchers of the gfx950 kernels (stream-ordered, no sync).
#pragma once

#include "common.h"

namespace anedvd {

// k_dequant.hip
int launch_dequant_gguf(int type, const uint8_t *d_src, size_t n_blocks, float *d_out, hipStream_t st);
int launch_repack(const QMat &m, const uint8_t *d_src, hipStream_t st);
int launch_dequant_tiles(const QMat &m, int mat, float *d_out, hipStream_t st);

// k_route.hip
int launch_router(const uint16_t *d_w, const float *d_x, int T, int E, int H, float *d_logits, hipStream_t st);
int launch_route(const float *d_logits, int T, int E, int k, int norm, float *d_probs, uint32_t *d_idx, hipStream_t st);
int launch_dispatch(const uint32_t *d_idx, int T, int k, int E, int32_t *d_offsets, int32_t *d_rows, int32_t *d_slots,
                    int32_t *d_inv, int32_t *d_active, int32_t *d_meta, hipStream_t st);

// k_gemv.hip
int gemv_unit_elems(int type);
int launch_expert_gateup(const QMat &gate, const QMat &up, const float *x, const int32_t *offsets,
                         const int32_t *rows, const int32_t *active, const int32_t *meta, float *part, int H, int I,
                         int KS, int P, int max_u, hipStream_t st);
int launch_expert_down(const QMat &down, const float *part, const int32_t *offsets, const int32_t *active,
                       const int32_t *meta, float *ypart, int H, int I, int KS, int KSg, int P, int use_gelu,
                       int max_u, hipStream_t st);
int launch_combine(const float *ypart, const int32_t *inv, const float *probs, int T, int k, int H, int KS, int P,
                   const float *shared, const float *shared_scale, int sKS, float *out, hipStream_t st);

}  // namespace anedvd
