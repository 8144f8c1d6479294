// Streaming skinny block-quantised GEMV for decode (M = 1..4 token rows), gfx950.
//
// y[m, n] = sum_b s[n, b] * sum_{i<32} q[n, 32b + i] * x[m, 32b + i]
//
// Weights stay in the reference's row-major layout (src/weights.rs:48-55,
// src/engine.rs:84-108): quants [N, K] (Q8_0: int8; Q4_0: 16 bytes per 32-block, nibble i of
// little-endian word w = element 8w + i), then f32 scales [N, K/32].
//
// Mapping.  A block of 256 threads (4 wave64s) first stages the M token rows in LDS, then each
// wave streams its own groups of 4 weight rows over the whole K range: lane l covers elements
// [1024c + 16l, +16) of chunk c, so one load instruction reads 1 KiB (Q8, 16 B/lane) or 512 B
// (Q4, 8 B/lane) of one row contiguously.  The next (group, chunk) step's loads are issued before
// the current step is computed, so every wave keeps weight bytes in flight while it computes.
// One x slice read from LDS serves the 4 rows of the group and all M token rows are applied to
// each weight byte once: the M=2 verify pass reads each weight once.
//
// Dequantisation in registers.  Q8: the word is xor-ed with 0x80808080, which turns each int8 q
// into the unsigned byte q+128; v_cvt_f32_ubyte{0..3} converts one byte per instruction and the
// bias is removed once per lane slice, sum (q+128) x - 128 sum x.  Q4: the nibbles are masked
// into bytes and converted the same way, minus 8 sum x.  The 16-element sums of x are staged in
// LDS with x.
//
// Reduction.  Per group each lane holds 4 row partials per token row; a transposed butterfly
// (xor 32, 16 exchange halves, then xor 8..1 add) leaves lane 16r with row r.  Every token row
// takes the same instruction sequence whatever M and its index are.
//
// This vector-ALU kernel serves kernel-level calls on row-major weights that the matrix-core
// kernel (mgemv.hip, tile-order weights) does not take: K % 128 != 0, or M = 3..4 at K > 4096.
// It computes the plain product y = W x.
#include "common.h"
#include "kernels.h"

#pragma clang fp contract(off)

namespace snl {

namespace {

constexpr int kThreads = 256, kWaves = 4, kChunk = 1024;
constexpr int kLdsFloats = 32768;  // token rows staged in LDS: M * K (whole chunks) <= 32768 floats

__device__ __forceinline__ int group_row(const GemvArgs& a, int blk, int G, int wg, int r) {
    // wg = wave * G + g; returns the weight row of row r (0..3) of the group or -1
    const int row = blk * 16 * G + wg * 4 + r;
    return row < a.N ? row : -1;
}

template <int QT>
__device__ __forceinline__ void load_frag(const GemvArgs& a, int row, int k, uint32_t (&w)[4], float& sc) {
    if (row >= 0 && k < a.K) {
        if constexpr (QT == 0) {
            const uint4 t = *reinterpret_cast<const uint4*>(static_cast<const int8_t*>(a.wq) + (size_t)row * a.K + k);
            w[0] = t.x, w[1] = t.y, w[2] = t.z, w[3] = t.w;
        } else {
            const uint2 t =
                *reinterpret_cast<const uint2*>(static_cast<const uint8_t*>(a.wq) + (size_t)row * (a.K >> 1) + (k >> 1));
            w[0] = t.x, w[1] = t.y, w[2] = 0u, w[3] = 0u;
        }
        sc = a.ws[(size_t)row * (a.K >> 5) + (k >> 5)];
    } else {
        w[0] = w[1] = w[2] = w[3] = QT == 0 ? 0x80808080u : 0x88888888u;
        sc = 0.0f;
    }
}

// sum over the lane's 16 elements of (biased byte value) * x for one token row
template <int QT>
__device__ __forceinline__ float dot16(const uint32_t (&w)[4], const float (&x)[16]) {
    float p = 0.0f;
    if constexpr (QT == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t u = w[j] ^ 0x80808080u;
#pragma unroll
            for (int b = 0; b < 4; ++b) p = fmaf((float)((u >> (8 * b)) & 0xFFu), x[4 * j + b], p);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t lo = w[j] & 0x0F0F0F0Fu, hi = (w[j] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                p = fmaf((float)((lo >> (8 * b)) & 0xFFu), x[8 * j + 2 * b], p);
                p = fmaf((float)((hi >> (8 * b)) & 0xFFu), x[8 * j + 2 * b + 1], p);
            }
        }
    }
    return p;
}

// LDS layout of a staged token row: per 1024-element chunk, float4 v (0..3) of lane l sits at
// float4 index chunk*256 + v*64 + l, so the 4 ds_read_b128 of a wave hit consecutive addresses.
__device__ __forceinline__ int lds_f4(int k4) {  // k4 = k / 4
    const int c = k4 >> 8, l = (k4 >> 2) & 63, v = k4 & 3;
    return (c << 8) + (v << 6) + l;
}

template <int QT, int M>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a, int G) {
    extern __shared__ float4 lds4[];
    const int K = a.K, K4 = K >> 2, K16 = K >> 4;
    const int nchunks = (K + kChunk - 1) / kChunk;
    const int K4p = nchunks * (kChunk / 4);                         // staged row length, whole chunks
    float4* xs4 = lds4;                                             // [M][K4p] staged rows (permuted)
    float* sxs = reinterpret_cast<float*>(lds4 + (size_t)M * K4p);  // [M][K/16] 16-element sums
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int blk = blockIdx.x;
    const int steps = G * nchunks;

    // issue the first weight fragments before the prologue so HBM latency overlaps it
    uint32_t wc[4][4], wn[4][4];
    float scc[4], scn[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) load_frag<QT>(a, group_row(a, blk, G, wave * G, r), lane * 16, wc[r], scc[r]);

    // ---- prologue: stage the token rows in LDS ----
    const int row0 = a.row_base ? *a.row_base : 0;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float4* xr = reinterpret_cast<const float4*>(a.x + (size_t)(row0 + m) * a.x_stride);
        for (int k4 = tid; k4 < K4; k4 += kThreads) xs4[m * K4p + lds_f4(k4)] = xr[k4];
    }
    __syncthreads();
    // 16-element sums for the dequantisation bias
#pragma unroll
    for (int m = 0; m < M; ++m)
        for (int j = tid; j < K16; j += kThreads) {
            float s = 0.0f;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float4 t = xs4[m * K4p + lds_f4(4 * j + v)];
                s = s + t.x;
                s = s + t.y;
                s = s + t.z;
                s = s + t.w;
            }
            sxs[m * K16 + j] = s;
        }
    __syncthreads();

    // ---- streaming main loop ----
    const float bias = QT == 0 ? 128.0f : 8.0f;
    float acc[4][M];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

    for (int s = 0; s < steps; ++s) {
        const int g = s / nchunks, c = s - g * nchunks;
        if (s + 1 < steps) {
            const int g1 = (s + 1) / nchunks, c1 = (s + 1) - g1 * nchunks;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                load_frag<QT>(a, group_row(a, blk, G, wave * G + g1, r), c1 * kChunk + lane * 16, wn[r], scn[r]);
        }
        const int k = c * kChunk + lane * 16;
        if (k < K) {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                float xv[16];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float4 t = xs4[m * K4p + (c << 8) + (v << 6) + lane];
                    xv[4 * v] = t.x;
                    xv[4 * v + 1] = t.y;
                    xv[4 * v + 2] = t.z;
                    xv[4 * v + 3] = t.w;
                }
                const float sx = sxs[m * K16 + (k >> 4)];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float p = dot16<QT>(wc[r], xv);
                    acc[r][m] = fmaf(scc[r], fmaf(-bias, sx, p), acc[r][m]);
                }
            }
        }
        if (c == nchunks - 1) {
            // transposed butterfly per token row: lane 16r ends with row r of the group
            const bool b5 = lane & 32, b4 = lane & 16;
            float out[M];
#pragma unroll
            for (int m = 0; m < M; ++m) {
                float k0 = b5 ? acc[2][m] : acc[0][m], k1 = b5 ? acc[3][m] : acc[1][m];
                const float s0 = b5 ? acc[0][m] : acc[2][m], s1 = b5 ? acc[1][m] : acc[3][m];
                k0 = k0 + __shfl_xor(s0, 32, 64);
                k1 = k1 + __shfl_xor(s1, 32, 64);
                float kk = b4 ? k1 : k0;
                const float ss = b4 ? k0 : k1;
                kk = kk + __shfl_xor(ss, 16, 64);
                kk = kk + __shfl_xor(kk, 8, 64);
                kk = kk + __shfl_xor(kk, 4, 64);
                kk = kk + __shfl_xor(kk, 2, 64);
                kk = kk + __shfl_xor(kk, 1, 64);
                out[m] = kk;
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[r][m] = 0.0f;
            }
            const int r = lane >> 4;
            const int row = group_row(a, blk, G, wave * G + g, r);
            if ((lane & 15) == 0 && row >= 0)
#pragma unroll
                for (int m = 0; m < M; ++m) a.y[(size_t)m * a.y_stride + a.n_off + row] = out[m];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            scc[r] = scn[r];
#pragma unroll
            for (int j = 0; j < 4; ++j) wc[r][j] = wn[r][j];
        }
    }
}

using KernelFn = void (*)(GemvArgs, int);

KernelFn pick(int quant, int M) {
    switch (quant * 8 + M) {
        case 1: return &gemv_kernel<0, 1>;
        case 2: return &gemv_kernel<0, 2>;
        case 3: return &gemv_kernel<0, 3>;
        case 4: return &gemv_kernel<0, 4>;
        case 9: return &gemv_kernel<1, 1>;
        case 10: return &gemv_kernel<1, 2>;
        case 11: return &gemv_kernel<1, 3>;
        case 12: return &gemv_kernel<1, 4>;
    }
    return nullptr;
}

// Row groups (of 4 rows) per wave: more for tall matrices, so that fewer blocks restage x.
int groups_for(int N) {
    if (N >= 65536) return 4;
    if (N >= 16384) return 2;
    return 1;
}

}  // namespace

int gemv_init() {
    const int bytes = kLdsFloats * 4 + kLdsFloats / 16 * 4;
    for (int q = 0; q < 2; ++q)
        for (int M = 1; M <= SNL_MAX_M; ++M) {
            KernelFn f = pick(q, M);
            if (f && hipFuncSetAttribute(reinterpret_cast<const void*>(f), hipFuncAttributeMaxDynamicSharedMemorySize,
                                         bytes) != hipSuccess)
                return -2;
        }
    return mgemv_init();
}

int launch_gemv(const GemvArgs& a, int quant, int M, hipStream_t s) {
    if (M < 1 || M > SNL_MAX_M || a.K % 32 != 0 || a.K <= 0 || a.N <= 0 || (quant != 0 && quant != 1)) return -1;
    if (a.epi == GEMV_SWIGLU && a.N != 2 * a.inter) return -1;
    if (a.pro != GEMV_PLAIN && a.K % 4) return -1;
    if (a.packed) {
        const int rc = launch_mgemv(a, quant, M, s);
        return rc == 1 ? -1 : rc;
    }
    // row-major weights: the plain product only
    if (a.epi != GEMV_STORE || a.pro != GEMV_PLAIN) return -1;
    const int K4p = (a.K + kChunk - 1) / kChunk * (kChunk / 4);
    if ((size_t)M * K4p * 4 > (size_t)kLdsFloats) {
        if (a.row_base) return -1;
        return launch_gemv_ksplit(a, quant, M, s);
    }
    KernelFn f = pick(quant, M);
    if (!f) return -1;
    const int G = groups_for(a.N);
    dim3 grid((a.N + 16 * G - 1) / (16 * G));
    const size_t lds = (size_t)M * K4p * 16 + (size_t)M * (a.K / 16) * 4;
    hipLaunchKernelGGL(f, grid, dim3(kThreads), lds, s, a, G);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace snl
