// Matrix-core block-quantised GEMM for chunked prefill (M up to 512 token rows), gfx950.
//
// y[m, n] = sum_b s[n, b] * sum_{i<32} q[n, 32b + i] * x[m, 32b + i]
//
// The reference runs its tiled matmul for more than 8 rows (src/shaders/matmul.wgsl:200-318,
// MatKind::Tiled in src/gpu.rs:191-218).  Here every product runs on v_mfma_f32_16x16x32_f16
// with exact operands, as in the decode GEMV: quants become f16 exactly, and each token row is
// split into f16 hi + lo parts (22 significant bits) under a per-token power of two.  Unlike the
// decode GEMV, one MFMA covers exactly one quant block (its K = 32 is the block), so the 16x16
// block result of each (token tile, row tile) is scaled by its 16 block scales and accumulated
// in f32.
//
// Panel order of the weights (a second copy beside the decode GEMV's tile order, kept for the
// prefill path only):
//   row tile R    rows 16R..16R+15 (rows past N are zero, scale 0)
//   piece (R, p)  64 lanes x 16 bytes; lane l = 16g + j holds row 16R + j and, for Q8, bytes
//                 [8g, 8g+8) of blocks 2p and 2p+1; for Q4, word g of blocks 4p..4p+3
//   scales        [R][K/128][16 rows][4 blocks] f32: one float4 per (row, 4 blocks)
// Row tile R's pieces are contiguous (16 K bytes for Q8), so a wave streams its rows in 1 KiB
// loads.
//
// Token fragments (written by launch_rows_to_frags): for token tile T (16 rows) and block b, the
// hi then the lo MFMA A fragment, 64 lanes x 8 f16, lane 16g + t holding token 16T + t's
// elements 32b + 8g + (0..7) (Q4: in the order 0, 4, 1, 5, 2, 6, 3, 7 that the nibble dequant
// produces), scaled by 2^-e(token); xs[m] = 2^e(m) restores the scale.
//
// Work split: a block of 4 waves computes 64 tokens x 256 rows (128 rows when the matrix is too
// short to give every CU a block); every wave takes all 4 token tiles and its own 4 (2) row tiles.
// Blocks that share a row panel are numbered so that the 8 XCDs each take whole row panels: the
// panel is read from HBM once into one XCD's L2 and the token panels reuse it.
// Each output element's arithmetic is fixed by its row and column, whatever M or the tile it
// falls in, so a token's result does not depend on the chunk that carries it.
#include "common.h"
#include "kernels.h"

#pragma clang fp contract(off)

namespace snl {

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));


__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }

// 8 quants of one block as exact f16 (Q8: bytes of two words; Q4: the 8 nibbles of one word, in
// the order 0, 4, 1, 5, 2, 6, 3, 7).
__device__ __forceinline__ half8_t q8_to_h8(uint32_t w0, uint32_t w1) {
    const half2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
    const half2_t p0 = as_h2(__builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u)) - bias;
    const half2_t p1 = as_h2(__builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u)) - bias;
    const half2_t p2 = as_h2(__builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u)) - bias;
    const half2_t p3 = as_h2(__builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u)) - bias;
    return half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

__device__ __forceinline__ half8_t q4_to_h8(uint32_t v) {
    const half2_t bias = {(_Float16)1032.0f, (_Float16)1032.0f};
    const half2_t p0 = as_h2((v & 0x000F000Fu) | 0x64006400u) - bias;
    const half2_t p1 = as_h2(((v >> 4) & 0x000F000Fu) | 0x64006400u) - bias;
    const half2_t p2 = as_h2(((v >> 8) & 0x000F000Fu) | 0x64006400u) - bias;
    const half2_t p3 = as_h2(((v >> 12) & 0x000F000Fu) | 0x64006400u) - bias;
    return half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// ---- reference layout -> panel order ----
// one thread per (row tile, piece, lane)
__global__ __launch_bounds__(256) void panel_pack_q_kernel(int quant, int N, int K, const uint8_t* q, uint8_t* qp,
                                                           size_t n_items) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= n_items) return;
    const int lane = (int)(idx & 63);
    const size_t pc = idx >> 6;
    const int npc = quant == 0 ? K / 64 : K / 128;  // pieces per row tile
    const int R = (int)(pc / npc), p = (int)(pc % npc);
    const int j = lane & 15, g = lane >> 4;
    const int row = 16 * R + j;
    uint32_t out[4] = {0u, 0u, 0u, 0u};
    if (row < N) {
        if (quant == 0) {
            const uint8_t* src = q + (size_t)row * K;
            for (int h = 0; h < 2; ++h) {
                const uint32_t* s4 = reinterpret_cast<const uint32_t*>(src + (size_t)(2 * p + h) * 32 + 8 * g);
                out[2 * h] = s4[0];
                out[2 * h + 1] = s4[1];
            }
        } else {
            const uint8_t* src = q + (size_t)row * (K / 2);
            for (int c = 0; c < 4; ++c)
                out[c] = *reinterpret_cast<const uint32_t*>(src + (size_t)(4 * p + c) * 16 + 4 * g);
        }
    }
    uint4* dst = reinterpret_cast<uint4*>(qp) + idx;
    *dst = make_uint4(out[0], out[1], out[2], out[3]);
}

// one thread per (row tile, 4-block group, row)
__global__ __launch_bounds__(256) void panel_pack_s_kernel(int N, int K, const float* s, float* sp, size_t n_items) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= n_items) return;
    const int j = (int)(idx & 15);
    const size_t rq = idx >> 4;
    const int nq = K / 128;
    const int R = (int)(rq / nq), qd = (int)(rq % nq);
    const int row = 16 * R + j, nb = K / 32;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (row < N) {
        const float* sr = s + (size_t)row * nb + 4 * qd;
        v = make_float4(sr[0], sr[1], sr[2], sr[3]);
    }
    reinterpret_cast<float4*>(sp)[idx] = v;
}

// ---- token rows -> MFMA A fragments (hi, lo) ----
constexpr int kRowThreads = 256;

__device__ __forceinline__ float block_max256(float v, float* red) {
    v = fmaxf(v, __shfl_xor(v, 32, 64));
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    v = fmaxf(v, __shfl_xor(v, 8, 64));
    v = fmaxf(v, __shfl_xor(v, 4, 64));
    v = fmaxf(v, __shfl_xor(v, 2, 64));
    v = fmaxf(v, __shfl_xor(v, 1, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// value of element k of token m's branch input (the row the GEMM multiplies)
__device__ __forceinline__ float row_value(const RowsArgs& a, const float* xr, int m, int k, float f0, float f1,
                                           float rinv) {
    switch (a.mode) {
        case ROWS_PLAIN: return xr[k];
        case ROWS_NORM: return (xr[k] * rinv) * (1.0f + a.w[k]);
        case ROWS_NORM_MHC: return ((f0 * xr[k] + f1 * xr[a.h + k]) * rinv) * (1.0f + a.w[k]);
        default: {  // ROWS_GNORM: head factor of the gated RMS norm of 128-wide heads
            const float* ps = a.ssq + ((size_t)m * (a.K / 128) + k / 128) * kDeltaGroups;
            const float var_o = (((ps[0] + ps[1]) + ps[2]) + ps[3]) / 128.0f;
            return xr[k] * (1.0f / sqrtf(var_o + a.eps));
        }
    }
}

__global__ __launch_bounds__(kRowThreads) void rows_to_frags_kernel(RowsArgs a) {
    __shared__ float red[4];
    const int m = blockIdx.x, tid = threadIdx.x, K = a.K, nb = K / 32;
    const int T = m >> 4, t = m & 15;
    half8_t* xf = reinterpret_cast<half8_t*>(a.frags);
    if (m >= a.M) {  // padding rows of the last token tile
        const half8_t z = {};
        for (int u = tid; u < nb * 4; u += kRowThreads) {
            const int b = u >> 2, g = u & 3;
            xf[(((size_t)T * nb + b) * 2 + 0) * 64 + 16 * g + t] = z;
            xf[(((size_t)T * nb + b) * 2 + 1) * 64 + 16 * g + t] = z;
        }
        if (tid == 0) a.xs[m] = 0.0f;
        return;
    }
    const float* xr = a.x + (size_t)m * a.x_stride;
    float f0 = 1.0f, f1 = 0.0f, rinv = 1.0f;
    if (a.mode == ROWS_NORM_MHC) {
        f0 = a.coef[m * 8];
        f1 = a.coef[m * 8 + 1];
    }
    if (a.mode == ROWS_NORM || a.mode == ROWS_NORM_MHC) {
        // layers.wgsl:46-73: RMSNorm of the (pre-mixed) stream-0 row
        float ss = 0.0f;
        for (int k = tid; k < K; k += kRowThreads) {
            const float v = a.mode == ROWS_NORM ? xr[k] : f0 * xr[k] + f1 * xr[a.h + k];
            ss = fmaf(v, v, ss);
        }
        __shared__ float rs[4];
        const float tot = block_sum<kRowThreads>(ss, rs);
        rinv = 1.0f / sqrtf(tot / (float)K + a.eps);
    }
    float amax = 0.0f;
    for (int k = tid; k < K; k += kRowThreads) amax = fmaxf(amax, fabsf(row_value(a, xr, m, k, f0, f1, rinv)));
    amax = block_max256(amax, red);
    // hi = f16(v * 2^-e) with the largest magnitude in [2^14, 2^15)
    int e = 0;
    if (amax > 0.0f) e = max(ilogbf(amax) - 14, -110);
    const float down = ldexpf(1.0f, -e);
    const int q4 = a.perm4;
    for (int u = tid; u < nb * 4; u += kRowThreads) {
        const int b = u >> 2, g = u & 3;
        half8_t hi, lo;
#pragma unroll
        for (int pp = 0; pp < 8; ++pp) {
            const int off = q4 ? ((pp & 1) ? 4 + (pp >> 1) : (pp >> 1)) : pp;
            const float v = row_value(a, xr, m, 32 * b + 8 * g + off, f0, f1, rinv) * down;
            const _Float16 hv = (_Float16)v;
            hi[pp] = hv;
            lo[pp] = (_Float16)(v - (float)hv);
        }
        xf[(((size_t)T * nb + b) * 2 + 0) * 64 + 16 * g + t] = hi;
        xf[(((size_t)T * nb + b) * 2 + 1) * 64 + 16 * g + t] = lo;
    }
    if (tid == 0) a.xs[m] = ldexpf(1.0f, e);
}

// ---- the GEMM ----
// Block: 4 waves over 64 tokens (4 token tiles, shared) x 4*RT row tiles (RT per wave).  The
// token fragments of each 128-element K step go through LDS (double-buffered: the next step's
// are loaded while this one's are multiplied), the weights and scales straight into registers
// one step ahead.
constexpr int kTT = 4;                         // token tiles per block (all waves)
constexpr int kStageU4 = kTT * 4 * 2 * 64;     // uint4 per LDS stage: tiles x 4 blocks x hi/lo x lanes

template <int QT, int RT>
__global__ __launch_bounds__(256, 1) void mgemm_kernel(GemmArgs a, int rpanels, int tpanels) {
    __shared__ uint4 lds_a[2 * kStageU4];  // 64 KiB
    constexpr int BR = 4 * RT;             // row tiles per block
    constexpr int PPQ = QT == 0 ? 2 : 1;   // weight pieces per row tile per K step
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // XCD-aware numbering: block b runs on XCD b % 8; give each XCD whole row panels
    const int bid = blockIdx.x;
    const int xcd = bid & 7, idx = bid >> 3;
    const int per_xcd = (rpanels + 7) / 8;
    const int rp = xcd * per_xcd + idx / tpanels;
    const int tp = idx % tpanels;
    if (rp >= rpanels) return;
    const int K = a.K, nb = K / 32, nq = K / 128;
    const int rtiles = (a.N + 15) / 16, mtiles = (a.M + 15) / 16;
    const int j = lane & 15, g = lane >> 4;
    int R[RT];
    bool rok[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        R[r] = rp * BR + wave * RT + r;
        rok[r] = R[r] < rtiles;
        if (!rok[r]) R[r] = rtiles - 1;  // a valid address; its results are not stored
    }
    const int T0 = tp * kTT;
    const uint4* wq = reinterpret_cast<const uint4*>(a.wq);
    const float4* ws = reinterpret_cast<const float4*>(a.ws);
    const uint4* xf = reinterpret_cast<const uint4*>(a.frags);
    const int npc = QT == 0 ? K / 64 : K / 128;

    // stage qd of the token fragments: chunk i = tid + 256k of the block's 4 runs of 8 KiB
    // (token tile T0 + (i >> 9), blocks 4qd..4qd+3, hi/lo, lanes), kept in the same order in LDS
    auto load_a = [&](int qd, uint4 (&r)[8]) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int i = tid + 256 * k;
            const int T = min(T0 + (i >> 9), mtiles - 1);
            r[k] = xf[((size_t)T * nb + 4 * qd) * 128 + (i & 511)];
        }
    };
    auto store_a = [&](int buf, const uint4 (&r)[8]) {
#pragma unroll
        for (int k = 0; k < 8; ++k) lds_a[buf * kStageU4 + tid + 256 * k] = r[k];
    };
    auto load_b = [&](int qd, uint4 (&wv)[RT][PPQ], float4 (&sv)[RT]) {
#pragma unroll
        for (int r = 0; r < RT; ++r) {
#pragma unroll
            for (int pp = 0; pp < PPQ; ++pp) wv[r][pp] = wq[((size_t)R[r] * npc + qd * PPQ + pp) * 64 + lane];
            sv[r] = ws[((size_t)R[r] * nq + qd) * 16 + j];
        }
    };

    f32x4_t acc[RT][kTT];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int t = 0; t < kTT; ++t) acc[r][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    uint4 wv[RT][PPQ], wn[RT][PPQ];
    float4 sv[RT], sn[RT];
    {
        uint4 ra[8];
        load_a(0, ra);
        load_b(0, wv, sv);
        store_a(0, ra);
    }
    __syncthreads();
    for (int qd = 0; qd < nq; ++qd) {
        const int buf = qd & 1;
        const bool more = qd + 1 < nq;
        uint4 ra[8];
        if (more) {
            load_a(qd + 1, ra);
            load_b(qd + 1, wn, sn);
        }
        const uint4* la = lds_a + buf * kStageU4;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            half8_t xh[kTT], xl[kTT];
#pragma unroll
            for (int t = 0; t < kTT; ++t) {
                xh[t] = __builtin_bit_cast(half8_t, la[t * 512 + (2 * b) * 64 + lane]);
                xl[t] = __builtin_bit_cast(half8_t, la[t * 512 + (2 * b + 1) * 64 + lane]);
            }
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                half8_t wh;
                if constexpr (QT == 0) {
                    const uint4 w = wv[r][b >> 1];
                    wh = (b & 1) ? q8_to_h8(w.z, w.w) : q8_to_h8(w.x, w.y);
                } else {
                    const uint4 w = wv[r][0];
                    wh = q4_to_h8(b == 0 ? w.x : b == 1 ? w.y : b == 2 ? w.z : w.w);
                }
                const float sc = b == 0 ? sv[r].x : b == 1 ? sv[r].y : b == 2 ? sv[r].z : sv[r].w;
#pragma unroll
                for (int t = 0; t < kTT; ++t) {
                    f32x4_t d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[t], wh, f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[t], wh, d, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[r][t][i] = fmaf(sc, d[i], acc[r][t][i]);
                }
            }
        }
        if (more) {
            store_a(buf ^ 1, ra);
#pragma unroll
            for (int r = 0; r < RT; ++r) {
#pragma unroll
                for (int pp = 0; pp < PPQ; ++pp) wv[r][pp] = wn[r][pp];
                sv[r] = sn[r];
            }
        }
        __syncthreads();
    }
    // lane (n = j, g) holds tokens 4g..4g+3 of each token tile
#pragma unroll
    for (int t = 0; t < kTT; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 16 * (T0 + t) + 4 * g + i;
            if (m >= a.M) continue;
            const float xs = a.xs[m];
            float* yr = a.y + (size_t)m * a.y_stride + a.n_off;
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const int n = 16 * R[r] + j;
                if (rok[r] && n < a.N) yr[n] = acc[r][t][i] * xs;
            }
        }
    }
}

}  // namespace

size_t gemm_q_bytes(int quant, int N, int K) {
    const size_t rt = (size_t)(N + 15) / 16;
    return quant == 0 ? rt * 16 * K : rt * 8 * K;
}

size_t gemm_s_floats(int N, int K) { return (size_t)(N + 15) / 16 * 16 * (K / 32); }

int launch_panel_pack(int quant, int N, int K, const void* q, const float* s, void* qp, float* sp, hipStream_t st) {
    if (K % 128 || N <= 0 || (quant != 0 && quant != 1)) return -1;
    const size_t rt = (size_t)(N + 15) / 16;
    const size_t nq = rt * (quant == 0 ? K / 64 : K / 128) * 64;
    const size_t ns = rt * (K / 128) * 16;
    hipLaunchKernelGGL(panel_pack_q_kernel, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, st, quant, N, K,
                       (const uint8_t*)q, (uint8_t*)qp, nq);
    hipLaunchKernelGGL(panel_pack_s_kernel, dim3((unsigned)((ns + 255) / 256)), dim3(256), 0, st, N, K, s, sp, ns);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

size_t frags_bytes(int M, int K) { return (size_t)((M + 15) / 16) * 16 * K * 4; }

int launch_rows_to_frags(const RowsArgs& a, hipStream_t s) {
    if (a.M <= 0 || a.K % 128 || !a.frags || !a.xs) return -1;
    if (a.mode == ROWS_GNORM && (a.K % 128 || !a.ssq)) return -1;
    const int mpad = (a.M + 15) / 16 * 16;
    hipLaunchKernelGGL(rows_to_frags_kernel, dim3(mpad), dim3(kRowThreads), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_mgemm(const GemmArgs& a, int quant, hipStream_t s) {
    if (a.M <= 0 || a.N <= 0 || a.K % 128 || !a.wq || !a.ws || !a.frags || !a.xs || !a.y) return -1;
    const int rtiles = (a.N + 15) / 16, mtiles = (a.M + 15) / 16;
    // 16 row tiles per block for wide matrices, 8 when that leaves too few blocks for the CUs
    const bool wide = (size_t)((rtiles + 15) / 16) * ((mtiles + kTT - 1) / kTT) >= 192;
    const int br = wide ? 16 : 8;
    const int rpanels = (rtiles + br - 1) / br, tpanels = (mtiles + kTT - 1) / kTT;
    const int blocks = 8 * ((rpanels + 7) / 8) * tpanels;
    if (quant == 0) {
        if (wide) hipLaunchKernelGGL((mgemm_kernel<0, 4>), dim3(blocks), dim3(256), 0, s, a, rpanels, tpanels);
        else hipLaunchKernelGGL((mgemm_kernel<0, 2>), dim3(blocks), dim3(256), 0, s, a, rpanels, tpanels);
    } else {
        if (wide) hipLaunchKernelGGL((mgemm_kernel<1, 4>), dim3(blocks), dim3(256), 0, s, a, rpanels, tpanels);
        else hipLaunchKernelGGL((mgemm_kernel<1, 2>), dim3(blocks), dim3(256), 0, s, a, rpanels, tpanels);
    }
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace snl
