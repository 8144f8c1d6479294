// Seeded random initialisation of a model directly in device memory.
//
// Counter-based: element i of a tensor is derived from splitmix64(key + i), and a normal
// draw is the Irwin-Hall sum of the four 16-bit lanes of that word (exact integer
// arithmetic, one int->float conversion, one multiply), so every value is bit-identical
// to the host-side generator of the tests.  Matrices are quantised per 32-block with the
// reference's rules (src/weights.rs:123-153): Q8_0 d = amax/127, q = round-half-away(v/d);
// Q4_0 d = (largest-magnitude value)/-8, n = trunc(v/d + 8.5) clamped to [0, 15].
#include "common.h"
#include "kernels.h"

// Every multiply and add below is rounded on its own (no FMA contraction), as on the host.
#pragma clang fp contract(off)

namespace snl {

namespace {

__device__ __forceinline__ uint64_t smix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

__device__ __forceinline__ float randn(uint64_t key, uint64_t i) {
    const uint64_t r = smix(key + i);
    const int32_t s = (int32_t)(r & 0xFFFF) + (int32_t)((r >> 16) & 0xFFFF) + (int32_t)((r >> 32) & 0xFFFF) +
                      (int32_t)(r >> 48);
    return (float)(s - 131070) * 0x1.bb67aep-16f;
}

__device__ __forceinline__ float randu(uint64_t key, uint64_t i) {
    const uint64_t r = smix(key + i);
    return (float)(r >> 40) * 0x1p-24f;
}

__global__ __launch_bounds__(256) void gen_matrix_kernel(uint64_t key, int64_t nblocks, float stdv, int quant,
                                                          uint8_t* q, float* sc) {
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblocks) return;
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = stdv * randn(key, (uint64_t)(b * 32 + i));
    if (quant == 0) {
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
        const float d = __fdiv_rn(amax, 127.0f);
        const float id = d > 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
        uint32_t words[8];
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            uint32_t word = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float r = roundf(v[4 * w + i] * id);
                r = fminf(fmaxf(r, -127.0f), 127.0f);
                word |= ((uint32_t)(int32_t)r & 0xFFu) << (8 * i);
            }
            words[w] = word;
        }
        uint4* dst = reinterpret_cast<uint4*>(q + b * 32);
        dst[0] = make_uint4(words[0], words[1], words[2], words[3]);
        dst[1] = make_uint4(words[4], words[5], words[6], words[7]);
        sc[b] = d;
    } else {
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i)
            if (fabsf(v[i]) > fabsf(mx)) mx = v[i];
        const float d = __fdiv_rn(mx, -8.0f);
        const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
        uint32_t words[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t word = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float t = v[w * 8 + i] * id + 8.5f;
                int32_t n = (int32_t)t;
                n = n < 0 ? 0 : (n > 15 ? 15 : n);
                word |= (uint32_t)n << (4 * i);
            }
            words[w] = word;
        }
        *reinterpret_cast<uint4*>(q + b * 16) = make_uint4(words[0], words[1], words[2], words[3]);
        sc[b] = d;
    }
}

// kind 0: std*N; 1: 1 + std*N; 2: DeltaNet vector conv w 0.25N | A_log ln16*U | dt 0.5N | norm 1+0.1N
// (aux0 = conv_dim, aux1 = n_v); 3: mHC router 0.02N for i < 16h, then N (aux0 = h).
__global__ __launch_bounds__(256) void gen_vector_kernel(uint64_t key, int64_t n, int kind, float stdv, int aux0,
                                                          int aux1, float* out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float v;
    if (kind == 0) {
        v = stdv * randn(key, i);
    } else if (kind == 1) {
        v = 1.0f + stdv * randn(key, i);
    } else if (kind == 2) {
        const int64_t cw = (int64_t)aux0 * 4;
        if (i < cw) v = 0.25f * randn(key, i);
        else if (i < cw + aux1) v = 0x1.62e43p+1f * randu(key, i);
        else if (i < cw + 2 * aux1) v = 0.5f * randn(key, i);
        else v = 1.0f + 0.1f * randn(key, i);
    } else {
        v = (i < (int64_t)16 * aux0 ? 0.02f : 1.0f) * randn(key, i);
    }
    out[i] = v;
}

}  // namespace

int launch_gen_matrix(uint64_t key, int64_t rows, int64_t cols, float stdv, int quant, void* q, float* sc,
                      hipStream_t s) {
    if (cols % 32) return -1;
    const int64_t nb = rows * cols / 32;
    hipLaunchKernelGGL(gen_matrix_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, s, key, nb, stdv, quant,
                       static_cast<uint8_t*>(q), sc);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_gen_vector(uint64_t key, int64_t n, int kind, float stdv, int aux0, int aux1, float* out, hipStream_t s) {
    hipLaunchKernelGGL(gen_vector_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, key, n, kind, stdv,
                       aux0, aux1, out);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace snl
