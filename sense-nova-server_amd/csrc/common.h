// Shared device helpers and launch descriptors for the MTP decode-step kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define SNL_WAVE 64

// Largest token count one decode-kernel launch handles (rows of x / proj / logits).
#define SNL_MAX_M 4

#define SNL_HIP_CHECK(expr)                                      \
    do {                                                         \
        hipError_t _e = (expr);                                  \
        if (_e != hipSuccess) return snl::device_error(_e, #expr); \
    } while (0)

namespace snl {

int device_error(hipError_t e, const char* what);

// Per-call device-side step record.  The host writes it (one small copy) before
// replaying a captured pass, so a captured graph never bakes in a position.
struct StepDev {
    int32_t pos0;   // cache position of row 0
    int32_t m;      // rows in this call
    int32_t ckpt;   // > 0: also save the recurrent state after row ckpt-1
    int32_t s_in;   // recurrent-state slot read
    int32_t s_out;  // recurrent-state slot written after the last row
    int32_t s_ck;   // recurrent-state slot written after row ckpt-1
    int32_t r0;     // MTP: first row of `hid` paired with tokens[0]
    int32_t x_off;  // LM head: first row of `hid` whose logits are produced
    uint32_t tokens[SNL_MAX_M];
    uint32_t rpos[SNL_MAX_M][4];  // rotary (t, h, w, 0) position of each row
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, SNL_WAVE);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, SNL_WAVE));
    return v;
}

// Sum over a block of NT threads (NT a multiple of 64, at most 1024); every thread gets the total.
// The order is fixed by the thread layout, so the result does not depend on anything else.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
    constexpr int NW = NT / SNL_WAVE;
    v = wave_sum(v);
    const int lane = threadIdx.x & (SNL_WAVE - 1), w = threadIdx.x / SNL_WAVE;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < NW; ++i) t += red[i];
    return t;
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }
__device__ __forceinline__ float sigmoidf_(float v) { return 1.0f / (1.0f + expf(-v)); }

}  // namespace snl
