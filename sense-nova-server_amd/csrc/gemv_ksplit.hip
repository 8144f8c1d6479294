// K-split skinny GEMV (fallback for shapes whose token rows do not fit the LDS of the
// streaming kernel in gemv.hip: M*K > 32768 floats), gfx950.
//
// y[m, n] = sum_b s[n, b] * sum_{i<32} q[n, 32b + i] * x[m, 32b + i]
//
// Weights stay in the reference's row-major layout (src/weights.rs:48-55,
// src/engine.rs:84-108): quants [N, K] (Q8_0: int8; Q4_0: 16 bytes per 32-block,
// nibble i of little-endian word w = element 8w + i), then f32 scales [N, K/32].
//
// Mapping.  A block of 256 threads (4 wave64s) owns R = 16 output rows and the whole
// K range.  K is cut into 1024-element chunks; wave w takes chunks w, w+4, ...  Lane l
// of a wave covers elements [chunk*1024 + 16l, +16) of every row of the block, so one
// wave-wide load reads 1 KiB (Q8, 16 B/lane) or 512 B (Q4, 8 B/lane) of one row
// contiguously.  The lane keeps its 16 x values per token row in registers and applies
// them to all 16 weight rows: the weights are read once for every token row (the M=2
// verify pass costs the weight bytes of one pass).
//
// Dequantisation in registers.  Q8: the word is xor-ed with 0x80808080, which turns
// each int8 q into the unsigned byte q+128; v_cvt_f32_ubyte{0..3} converts one byte per
// instruction and the bias is removed once per half-block, sum (q+128) x - 128 sum x.
// Q4: the nibbles n are masked into bytes and converted the same way, minus 8 sum x.
//
// Reduction.  Each lane holds 16 row partials per token row; a transposed butterfly
// (xor 32, 16, 8, 4 exchange half of the values, then xor 2, 1 add) leaves lane 4r with
// row r, then the 4 waves are summed in fixed order through LDS.  Every token row takes
// exactly the same instruction sequence whatever M is, so row m of an M=2 call is
// bitwise equal to the same row in an M=1 call (greedy output is then byte-identical
// with and without speculative drafting).
//
// It computes the plain product y = W x for kernel-level calls on row-major weights.
#include "common.h"
#include "kernels.h"

#pragma clang fp contract(off)

namespace snl {

namespace {

constexpr int kRows = 16;
constexpr int kThreads = 256;
constexpr int kChunk = 1024;

__device__ __forceinline__ int row_of(int blk, int r) { return blk * kRows + r; }

// sum over the lane's 16 products of (byte value) * x, for one token row
template <int QT>
__device__ __forceinline__ void dot16(const uint32_t (&w)[4], const float (&x)[16], float& p) {
    if constexpr (QT == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t u = w[j] ^ 0x80808080u;
#pragma unroll
            for (int b = 0; b < 4; ++b) p = fmaf((float)((u >> (8 * b)) & 0xFFu), x[4 * j + b], p);
        }
    } else {
        // two words = 16 nibbles = elements 0..15 of the lane's half block
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            uint32_t lo = w[j] & 0x0F0F0F0Fu, hi = (w[j] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                p = fmaf((float)((lo >> (8 * b)) & 0xFFu), x[8 * j + 2 * b], p);
                p = fmaf((float)((hi >> (8 * b)) & 0xFFu), x[8 * j + 2 * b + 1], p);
            }
        }
    }
}

template <int QT, int M>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int blk = blockIdx.x;
    const int K = a.K, nb = K >> 5;
    const int nchunks = (K + kChunk - 1) / kChunk;

    float acc[kRows][M];
#pragma unroll
    for (int r = 0; r < kRows; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

    for (int c = wave; c < nchunks; c += 4) {
        const int k = c * kChunk + lane * 16;
        if (k < K) {
            float xs[M][16], sx[M];
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float4* xp = reinterpret_cast<const float4*>(a.x + (size_t)m * a.x_stride + k);
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    float4 t = xp[v];
                    xs[m][4 * v] = t.x;
                    xs[m][4 * v + 1] = t.y;
                    xs[m][4 * v + 2] = t.z;
                    xs[m][4 * v + 3] = t.w;
                }
                float s = xs[m][0];
#pragma unroll
                for (int i = 1; i < 16; ++i) s = s + xs[m][i];
                sx[m] = s;
            }
            const float bias = QT == 0 ? 128.0f : 8.0f;
#pragma unroll
            for (int r0 = 0; r0 < kRows; r0 += 8) {
                uint32_t wv[8][4];
                float sc[8];
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    const int row = row_of(blk, r0 + r);
                    const bool ok = row < a.N;
                    if (ok) {
                        if constexpr (QT == 0) {
                            uint4 t = *reinterpret_cast<const uint4*>(static_cast<const int8_t*>(a.wq) +
                                                                      (size_t)row * K + k);
                            wv[r][0] = t.x, wv[r][1] = t.y, wv[r][2] = t.z, wv[r][3] = t.w;
                        } else {
                            uint2 t = *reinterpret_cast<const uint2*>(static_cast<const uint8_t*>(a.wq) +
                                                                      (size_t)row * (K >> 1) + (k >> 1));
                            wv[r][0] = t.x, wv[r][1] = t.y, wv[r][2] = 0u, wv[r][3] = 0u;
                        }
                        sc[r] = a.ws[(size_t)row * nb + (k >> 5)];
                    } else {
                        wv[r][0] = wv[r][1] = wv[r][2] = wv[r][3] = QT == 0 ? 0x80808080u : 0x88888888u;
                        sc[r] = 0.0f;
                    }
                }
#pragma unroll
                for (int r = 0; r < 8; ++r)
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        float p = 0.0f;
                        dot16<QT>(wv[r], xs[m], p);
                        acc[r0 + r][m] = fmaf(sc[r], fmaf(-bias, sx[m], p), acc[r0 + r][m]);
                    }
            }
        }
    }

    // transposed butterfly over the 64 lanes, per token row
    __shared__ float red[4][M][kRows];
    const bool b5 = lane & 32, b4 = lane & 16, b3 = lane & 8, b2 = lane & 4;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = acc[i][m];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float send = b5 ? v[i] : v[8 + i], keep = b5 ? v[8 + i] : v[i];
            v[i] = keep + __shfl_xor(send, 32, 64);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float send = b4 ? v[i] : v[4 + i], keep = b4 ? v[4 + i] : v[i];
            v[i] = keep + __shfl_xor(send, 16, 64);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            float send = b3 ? v[i] : v[2 + i], keep = b3 ? v[2 + i] : v[i];
            v[i] = keep + __shfl_xor(send, 8, 64);
        }
        {
            float send = b2 ? v[0] : v[1], keep = b2 ? v[1] : v[0];
            v[0] = keep + __shfl_xor(send, 4, 64);
        }
        v[0] = v[0] + __shfl_xor(v[0], 2, 64);
        v[0] = v[0] + __shfl_xor(v[0], 1, 64);
        if ((lane & 3) == 0) red[wave][m][lane >> 2] = v[0];
    }
    __syncthreads();

    const int t = threadIdx.x;
    if (t < kRows * M) {
        const int r = t & (kRows - 1), m = t / kRows;
        const int row = blk * kRows + r;
        if (row < a.N) {
            const float v = ((red[0][m][r] + red[1][m][r]) + red[2][m][r]) + red[3][m][r];
            a.y[(size_t)m * a.y_stride + a.n_off + row] = v;
        }
    }
}

template <int QT, int M>
int launch_q(const GemvArgs& a, hipStream_t s) {
    dim3 grid((a.N + kRows - 1) / kRows);
    hipLaunchKernelGGL((gemv_kernel<QT, M>), grid, dim3(kThreads), 0, s, a);
    return 0;
}

template <int QT>
int launch_m(const GemvArgs& a, int M, hipStream_t s) {
    switch (M) {
        case 1: return launch_q<QT, 1>(a, s);
        case 2: return launch_q<QT, 2>(a, s);
        case 3: return launch_q<QT, 3>(a, s);
        case 4: return launch_q<QT, 4>(a, s);
    }
    return -1;
}

}  // namespace

int launch_gemv_ksplit(const GemvArgs& a, int quant, int M, hipStream_t s) {
    if (M < 1 || M > SNL_MAX_M || a.K % 32 != 0 || a.K <= 0 || a.N <= 0) return -1;
    if (a.pro != GEMV_PLAIN || a.epi != GEMV_STORE) return -1;
    int rc = quant == 0 ? launch_m<0>(a, M, s) : launch_m<1>(a, M, s);
    if (rc) return rc;
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace snl
