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
// Work split: a block of 8 waves computes 128 tokens x 256 rows for Q8 (64 x 256 for Q4), and
// 64 tokens x 128 rows when the matrix is too short to give every CU a block.  The block tile
// sets how often operands are re-read from L2: the token fragments once per row panel, the
// weights once per token panel, which is what bounds this kernel (halving the MFMA work or
// dropping the scale FMAs each changes its time by under 10%).  Blocks that share a row panel are
// numbered so that the 8 XCDs each take whole row panels: the panel is read from HBM once into
// one XCD's L2 and the token panels reuse it.
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
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// One block per token row: the row's 8-element groups are held in registers (GPT per thread),
// the branch input is formed (RMSNorm (1 + w) of stream 0 or of the mHC pre-mix, or the DeltaNet
// head factor, one per group), then the row's largest magnitude sets the power of two and each
// group is written as its hi and lo halves of the MFMA A fragments.
template <int GPT>
__global__ __launch_bounds__(kRowThreads) void rows_to_frags_kernel(RowsArgs a) {
    __shared__ float red[4];
    __shared__ float rs[4];
    const int m = blockIdx.x, tid = threadIdx.x, K = a.K, nb = K / 32, ngr = K / 8;
    const int T = m >> 4, t = m & 15;
    half8_t* xf = reinterpret_cast<half8_t*>(a.frags);
    if (m >= a.M) {  // padding rows of the last token tile
        const half8_t z = {};
        for (int u = tid; u < ngr; u += kRowThreads) {
            const int b = u >> 2, g = u & 3;
            xf[(((size_t)T * nb + b) * 2 + 0) * 64 + 16 * g + t] = z;
            xf[(((size_t)T * nb + b) * 2 + 1) * 64 + 16 * g + t] = z;
        }
        if (tid == 0) a.xs[m] = 0.0f;
        return;
    }
    const float* xr = a.x + (size_t)m * a.x_stride;
    float f0 = 1.0f, f1 = 0.0f;
    if (a.mode == ROWS_NORM_MHC) {
        f0 = a.coef[m * 8];
        f1 = a.coef[m * 8 + 1];
    }
    float v[GPT][8];
    float ss = 0.0f;
#pragma unroll
    for (int gi = 0; gi < GPT; ++gi) {
        const int u = tid + kRowThreads * gi;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[gi][e] = 0.0f;
        if (u < ngr) {
            const float4* p = reinterpret_cast<const float4*>(xr + 8 * u);
            const float4 p0 = p[0], p1 = p[1];
            float w8[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
            if (a.mode == ROWS_NORM_MHC) {
                const float4* q = reinterpret_cast<const float4*>(xr + a.h + 8 * u);
                const float4 q0 = q[0], q1 = q[1];
                const float u8[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) w8[e] = f0 * w8[e] + f1 * u8[e];
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                v[gi][e] = w8[e];
                ss = fmaf(w8[e], w8[e], ss);
            }
        }
    }
    if (a.mode == ROWS_NORM || a.mode == ROWS_NORM_MHC) {
        // layers.wgsl:46-73: RMSNorm of the (pre-mixed) stream-0 row
        const float tot = block_sum<kRowThreads>(ss, rs);
        const float rinv = 1.0f / sqrtf(tot / (float)K + a.eps);
#pragma unroll
        for (int gi = 0; gi < GPT; ++gi) {
            const int u = tid + kRowThreads * gi;
            if (u < ngr)
#pragma unroll
                for (int e = 0; e < 8; ++e) v[gi][e] = (v[gi][e] * rinv) * (1.0f + a.w[8 * u + e]);
        }
    } else if (a.mode == ROWS_GNORM) {  // head factor of the gated RMS norm of 128-wide heads
#pragma unroll
        for (int gi = 0; gi < GPT; ++gi) {
            const int u = tid + kRowThreads * gi;
            if (u < ngr) {
                const float* ps = a.ssq + ((size_t)m * (K / 128) + u / 16) * kDeltaPrefillGroups;
                float t = ps[0];
#pragma unroll
                for (int gi = 1; gi < kDeltaPrefillGroups; ++gi) t = t + ps[gi];
                const float var_o = t / 128.0f;
                const float f = 1.0f / sqrtf(var_o + a.eps);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[gi][e] = v[gi][e] * f;
            }
        }
    }
    float amax = 0.0f;
#pragma unroll
    for (int gi = 0; gi < GPT; ++gi)
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[gi][e]));
    amax = block_max256(amax, red);
    // hi = f16(v * 2^-e) with the largest magnitude in [2^14, 2^15)
    int ex = 0;
    if (amax > 0.0f) ex = max(ilogbf(amax) - 14, -110);
    const float down = ldexpf(1.0f, -ex);
    const int q4 = a.perm4;
#pragma unroll
    for (int gi = 0; gi < GPT; ++gi) {
        const int u = tid + kRowThreads * gi;
        if (u >= ngr) continue;
        const int b = u >> 2, g = u & 3;
        half8_t hi, lo;
#pragma unroll
        for (int pp = 0; pp < 8; ++pp) {
            // Q4 fragments take the element order 0, 4, 1, 5, 2, 6, 3, 7 of the nibble dequant
            const float x = (q4 ? v[gi][(pp & 1) ? 4 + (pp >> 1) : (pp >> 1)] : v[gi][pp]) * down;
            const _Float16 hv = (_Float16)x;
            hi[pp] = hv;
            lo[pp] = (_Float16)(x - (float)hv);
        }
        xf[(((size_t)T * nb + b) * 2 + 0) * 64 + 16 * g + t] = hi;
        xf[(((size_t)T * nb + b) * 2 + 1) * 64 + 16 * g + t] = lo;
    }
    if (tid == 0) a.xs[m] = ldexpf(1.0f, ex);
}

// ---- the GEMM ----
// Block: 8 waves, 2 along the tokens x 4 along the rows; wave (wt, wr) takes TTW token tiles x RT
// row tiles, so a block covers 2*TTW token tiles x 4*RT row tiles.  K runs in stages of one weight
// piece per row tile (2 quant blocks for Q8, 4 for Q4; TTW = 4 and 2 keep a wave's token
// fragments the same size).  Each stage's token fragments, weight pieces and scales are copied
// global -> LDS by global_load_lds (16 bytes per lane, lane i at base + 16i) into a ring of three
// buffers, two stages ahead of the one computed.  A step waits for its own stage only (the vector
// memory count may keep one stage of copies outstanding), passes a barrier, reads the stage into
// registers, issues the copies of the stage two ahead into the buffer read one step before, and
// runs the MFMAs while both later stages are in flight.
constexpr int kGemmThreads = 512;  // 8 waves

template <int QT, int RT>
struct GemmStage {
    static constexpr int TTW = QT == 0 && RT == 4 ? 4 : 2;  // token tiles per wave
    static constexpr int WT = 2, WR = 4, NW = WT * WR;      // waves along tokens, along rows
    static constexpr int TT = WT * TTW;                     // token tiles per block
    static constexpr int BR = WR * RT;                      // row tiles per block
    static constexpr int NBS = QT == 0 ? 2 : 4;   // quant blocks per stage
    static constexpr int A_U4 = TT * NBS * 2 * 64;
    static constexpr int B_U4 = BR * 64;
    static constexpr int S_U4 = BR * 16;
    static constexpr int U4 = A_U4 + B_U4 + S_U4;  // uint4 per stage
    static constexpr int NC = U4 / 64;             // 1 KiB copies per stage
    static constexpr int NC_MIN = NC / NW;         // copies per stage of the waves with the fewest
    static_assert(NW * 64 == kGemmThreads, "block size");
    static constexpr size_t BYTES = 3 * (size_t)U4 * 16;  // three stage buffers
    static_assert(BYTES <= 160 * 1024, "three stages fit the LDS");
};

// s_waitcnt immediate (gfx9 layout): vector memory count vm, LDS count 0, export count untouched
constexpr int wait_vm_lgkm0(int vm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4); }

// 1 KiB global -> LDS copy of one wave: lane i moves 16 bytes from base + voff(i) to LDS
// dst + 16 i.  Issued as inline assembly, so the compiler's wait insertion does not see it and
// does not hold every LDS read until all copies in flight have landed; the kernel orders the
// copies itself (s_waitcnt on the vector memory count before the barrier that publishes a stage).
// The compiler's own waits stay correct: loads it does not know about can only make them wait
// longer.
__device__ __forceinline__ void copy16_to_lds(const char* base, unsigned voff, unsigned dst) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(dst), "v"(voff), "s"(base)
                 : "memory", "m0");
}

template <int QT, int RT>
__global__ __launch_bounds__(kGemmThreads) void mgemm_kernel(GemmArgs a, int rpanels, int tpanels) {
    using G = GemmStage<QT, RT>;
    constexpr int TT = G::TTW, NBS = G::NBS;  // TT: this wave's token tiles
    extern __shared__ __align__(16) uint4 lds[];  // three stage buffers of G::U4
    // the wave index in a scalar register: the copy loop below then branches and forms its
    // addresses in scalar code instead of exec-masked vector code
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wt = wave / G::WR, wr = wave % G::WR;
    // XCD-aware numbering: block b runs on XCD b % 8; give each XCD whole row panels
    const int bid = blockIdx.x;
    const int xcd = bid & 7, idx = bid >> 3;
    const int per_xcd = (rpanels + 7) / 8;
    const int rp = xcd * per_xcd + idx / tpanels;
    const int tp = idx % tpanels;
    if (rp >= rpanels) return;
    const int K = a.K, nb = K / 32, nq = K / 128, nst = K / (32 * NBS);
    const int rtiles = (a.N + 15) / 16, mtiles = (a.M + 15) / 16;
    const int j = lane & 15, g = lane >> 4;
    const int R0 = rp * G::BR, T0 = tp * G::TT;
    const int npc = QT == 0 ? K / 64 : K / 128;  // pieces per row tile (= stages)

    // One stage: wave instruction c of the stage's U4/64 copies moves 1 KiB.  The panel copies and
    // the token fragments are allocated in whole block panels (gemm_q_bytes, gemm_s_floats,
    // frags_bytes), so no copy needs a clamp: each source is a scalar offset plus one of two
    // per-lane offsets.  Rows and tokens past the matrix only feed outputs that are not stored.
    const char* xf_b = reinterpret_cast<const char*>(a.frags);
    const char* wq_b = reinterpret_cast<const char*>(a.wq);
    const char* ws_b = reinterpret_cast<const char*>(a.ws);
    const unsigned lane16 = (unsigned)lane * 16u;
    // scales: lane l -> row tile + l / 16 of the copy's 4, row l % 16
    const unsigned lane_s = (unsigned)(lane >> 4) * (unsigned)nq * 256u + (unsigned)(lane & 15) * 16u;
    const unsigned lds_base = (unsigned)(uintptr_t)(__attribute__((address_space(3))) void*)lds;
    auto issue = [&](int st, int buf) {
        const unsigned dst0 = lds_base + (unsigned)(buf * G::U4) * 16u;
        constexpr int NA = G::A_U4 / 64, NB = G::B_U4 / 64, NS = G::S_U4 / 64;
        for (int c = wave; c < NA + NB + NS; c += G::NW) {
            const char* src;
            unsigned lo = lane16;
            if (c < NA) {  // token tile c / (2 NBS), block c / 2 % NBS, hi/lo c % 2
                const int t = c / (2 * NBS), bh = c % (2 * NBS);
                src = xf_b + ((((size_t)(T0 + t) * nb + st * NBS) * 2 + bh) << 10);
            } else if (c < NA + NB) {  // row tile c - NA
                src = wq_b + (((size_t)(R0 + c - NA) * npc + st) << 10);
            } else {  // scales of row tiles R0 + 4(c - NA - NB) .. + 3
                // Q8 stages take 2 of a row's 4 scales: an odd stage starts 8 bytes into the float4,
                // so the stage's scales are always .x and .y (the last 8 bytes read belong to the
                // next row, or to the padding after the last)
                src = ws_b + (((size_t)(R0 + 4 * (c - NA - NB)) * nq + st * NBS / 4) << 8) +
                      (NBS == 2 ? (st & 1) * 8 : 0);
                lo = lane_s;
            }
            copy16_to_lds(src, lo, dst0 + (unsigned)c * 1024u);
        }
    };

    f32x4_t acc[RT][TT];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[r][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // Stage st lives in buffer st % 3; two stages of copies are in flight while one is computed.
    auto step = [&](int st) {
        const uint4* la = lds + (size_t)(st % 3) * G::U4;
        // This wave's copies of stage st have landed when at most one stage's worth (the copies
        // of stage st + 1) is outstanding; every read of this wave is complete.  After the
        // barrier every wave's copies of stage st have landed and every wave has read stage
        // st - 1, whose buffer `next` then takes stage st + 2.
        // no instruction of the previous step moves past this point (its LDS reads stay ahead of
        // the wait, so they are complete before the barrier lets another wave overwrite their
        // buffer), and no LDS access of this step moves above the barrier
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        if (st + 1 < nst) __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(G::NC_MIN));
        else __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(0));
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        const uint4* lb = la + G::A_U4;
        const float4* lsc = reinterpret_cast<const float4*>(lb + G::B_U4);
        half8_t xh[NBS][TT], xl[NBS][TT];
        uint4 wv[RT];
        float4 sv[RT];
#pragma unroll
        for (int b = 0; b < NBS; ++b)
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const int tb = wt * TT + t;  // token tile in the block
                xh[b][t] = __builtin_bit_cast(half8_t, la[((tb * NBS + b) * 2) * 64 + lane]);
                xl[b][t] = __builtin_bit_cast(half8_t, la[((tb * NBS + b) * 2 + 1) * 64 + lane]);
            }
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            wv[r] = lb[(wr * RT + r) * 64 + lane];
            sv[r] = lsc[(wr * RT + r) * 16 + j];
        }
        if (st + 2 < nst) issue(st + 2, (st + 2) % 3);
#pragma unroll
        for (int b = 0; b < NBS; ++b) {
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                half8_t wh;
                if constexpr (QT == 0) wh = b ? q8_to_h8(wv[r].z, wv[r].w) : q8_to_h8(wv[r].x, wv[r].y);
                else wh = q4_to_h8(b == 0 ? wv[r].x : b == 1 ? wv[r].y : b == 2 ? wv[r].z : wv[r].w);
                const float sc = b == 0 ? sv[r].x : b == 1 ? sv[r].y : b == 2 ? sv[r].z : sv[r].w;
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    f32x4_t d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[b][t], wh, f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[b][t], wh, d, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[r][t][i] = fmaf(sc, d[i], acc[r][t][i]);
                }
            }
        }
    };
    issue(0, 0);
    if (nst > 1) issue(1, 1);
    for (int st = 0; st < nst; ++st) step(st);
    // lane (n = j, g) holds tokens 4g..4g+3 of each token tile
#pragma unroll
    for (int t = 0; t < TT; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 16 * (T0 + wt * TT + t) + 4 * g + i;
            if (m >= a.M) continue;
            const float xs = a.xs[m];
            float* yr = a.y + (size_t)m * a.y_stride + a.n_off;
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const int R = R0 + wr * RT + r;
                const int n = 16 * R + j;
                if (R < rtiles && n < a.N) yr[n] = acc[r][t][i] * xs;
            }
        }
    }
}

template <int QT, int RT>
int gemm_launch(const GemmArgs& a, int rpanels, int tpanels, hipStream_t s) {
    using G = GemmStage<QT, RT>;
    static const hipError_t attr =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&mgemm_kernel<QT, RT>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)G::BYTES);
    if (attr != hipSuccess) return -2;
    const int blocks = 8 * ((rpanels + 7) / 8) * tpanels;
    hipLaunchKernelGGL((mgemm_kernel<QT, RT>), dim3(blocks), dim3(G::NW * 64), G::BYTES, s, a, rpanels, tpanels);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace

// Row tiles of a panel copy: whole 256-row block panels, so a block's copies never run past it.
static size_t panel_tiles(int N) { return ((size_t)(N + 15) / 16 + 15) / 16 * 16; }

size_t gemm_q_bytes(int quant, int N, int K) {
    const size_t rt = panel_tiles(N);
    return quant == 0 ? rt * 16 * K : rt * 8 * K;
}

// (+ 4: the shifted scale copy of an odd Q8 stage reads 8 bytes past the last float4)
size_t gemm_s_floats(int N, int K) { return panel_tiles(N) * 16 * (K / 32) + 4; }

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

// token fragments in whole 128-token panels (8 tiles), the widest token panel of a block
size_t frags_bytes(int M, int K) { return (size_t)((M + 127) / 128) * 128 * K * 4; }

int launch_rows_to_frags(const RowsArgs& a, hipStream_t s) {
    if (a.M <= 0 || a.K % 128 || !a.frags || !a.xs) return -1;
    if (a.mode == ROWS_GNORM && (a.K % 128 || !a.ssq)) return -1;
    const int mpad = (a.M + 15) / 16 * 16;
    const int gpt = (a.K / 8 + kRowThreads - 1) / kRowThreads;
    if (gpt <= 2) hipLaunchKernelGGL(rows_to_frags_kernel<2>, dim3(mpad), dim3(kRowThreads), 0, s, a);
    else if (gpt <= 4) hipLaunchKernelGGL(rows_to_frags_kernel<4>, dim3(mpad), dim3(kRowThreads), 0, s, a);
    else if (gpt <= 6) hipLaunchKernelGGL(rows_to_frags_kernel<6>, dim3(mpad), dim3(kRowThreads), 0, s, a);
    else if (gpt <= 8) hipLaunchKernelGGL(rows_to_frags_kernel<8>, dim3(mpad), dim3(kRowThreads), 0, s, a);
    else return -1;  // rows longer than 16384
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_mgemm(const GemmArgs& a, int quant, hipStream_t s) {
    if (a.M <= 0 || a.N <= 0 || a.K % 128 || !a.wq || !a.ws || !a.frags || !a.xs || !a.y) return -1;
    const int rtiles = (a.N + 15) / 16, mtiles = (a.M + 15) / 16;
    // 16 row tiles per block for wide matrices, 8 (and 2 token tiles) when that leaves too few
    // blocks for the CUs
    const int tt_w = quant == 0 ? GemmStage<0, 4>::TT : GemmStage<1, 4>::TT;
    const int tt_n = quant == 0 ? GemmStage<0, 2>::TT : GemmStage<1, 2>::TT;
    const bool wide = (size_t)((rtiles + 15) / 16) * ((mtiles + tt_w - 1) / tt_w) >= 192;
    const int tt = wide ? tt_w : tt_n;
    const int tpanels = (mtiles + tt - 1) / tt;
    const int rpanels = wide ? (rtiles + 15) / 16 : (rtiles + 7) / 8;
    if (quant == 0) return wide ? gemm_launch<0, 4>(a, rpanels, tpanels, s) : gemm_launch<0, 2>(a, rpanels, tpanels, s);
    return wide ? gemm_launch<1, 4>(a, rpanels, tpanels, s) : gemm_launch<1, 2>(a, rpanels, tpanels, s);
}

}  // namespace snl
