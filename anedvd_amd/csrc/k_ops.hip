// k_ops.hip -- the op-level expert product over caller-given weight slices:
// cpu.moeExpertAccumF32 (cpu.zig:416-452, f32 weights) and cpu.moeExpertAccum
// (cpu.zig:1141-1185, f16 weights) for one token.  A test and integration path,
// not the layer's: each output row is one wavefront's dot product, lanes striding
// over the input with f32 accumulation.
#include "common.h"
#include "kernels.h"
#include "mma.h"

namespace anedvd {

template <class T>
__device__ inline float wval(const T *w, size_t i);
template <>
__device__ inline float wval<float>(const float *w, size_t i) { return w[i]; }
template <>
__device__ inline float wval<uint16_t>(const uint16_t *w, size_t i) { return f16_bits_to_f32(w[i]); }

__device__ inline float wave_sum(float v)
{
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// gate and up rows for inter outputs: act[i] = act(gate_i . h) * (up_i . h)
template <class T>
__global__ __launch_bounds__(256) void k_ops_gateup(const T *__restrict__ gate, const T *__restrict__ up,
                                                    const float *__restrict__ h, int inter, int hidden,
                                                    int use_gelu, float *__restrict__ act)
{
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= inter) return;
    float g = 0.0f, u = 0.0f;
    for (int i = lane; i < hidden; i += 64) {
        g += wval(gate, (size_t)row * hidden + i) * h[i];
        u += wval(up, (size_t)row * hidden + i) * h[i];
    }
    g = wave_sum(g);
    u = wave_sum(u);
    if (lane == 0) act[row] = gate_act(g, use_gelu) * u;
}

// out[o] += weight * (down_o . act)
template <class T>
__global__ __launch_bounds__(256) void k_ops_down(const T *__restrict__ down, const float *__restrict__ act,
                                                  int inter, int hidden, float weight, float *__restrict__ out)
{
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= hidden) return;
    float s = 0.0f;
    for (int i = lane; i < inter; i += 64) s += wval(down, (size_t)row * inter + i) * act[i];
    s = wave_sum(s);
    if (lane == 0) out[row] += weight * s;
}

template <class T>
static int launch_ops(const T *g, const T *u, const T *d, const float *h, int inter, int hidden, float weight,
                      int use_gelu, float *act, float *out, hipStream_t st)
{
    hipLaunchKernelGGL(k_ops_gateup<T>, dim3((unsigned)((inter + 3) / 4)), dim3(256), 0, st, g, u, h, inter, hidden,
                       use_gelu, act);
    ANEDVD_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_ops_down<T>, dim3((unsigned)((hidden + 3) / 4)), dim3(256), 0, st, d, act, inter, hidden,
                       weight, out);
    ANEDVD_HIP(hipGetLastError());
    return ANEDVD_OK;
}

int launch_expert_accum_ops(bool f16, const void *gate, const void *up, const void *down, const float *h, int inter,
                            int hidden, float weight, int use_gelu, float *act, float *out, hipStream_t st)
{
    if (f16)
        return launch_ops((const uint16_t *)gate, (const uint16_t *)up, (const uint16_t *)down, h, inter, hidden,
                          weight, use_gelu, act, out, st);
    return launch_ops((const float *)gate, (const float *)up, (const float *)down, h, inter, hidden, weight,
                      use_gelu, act, out, st);
}

}  // namespace anedvd
