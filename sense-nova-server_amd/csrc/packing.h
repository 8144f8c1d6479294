// Tile order of a block-quantised GEMV weight matrix in HBM.
//
// The reference stores a quantised matrix row-major: quants [N, K] (Q8_0: int8; Q4_0: 16 bytes
// per 32-element block) then f32 scales [N, K/32] (src/weights.rs:48-55).  The matrix-core GEMV
// feeds each MFMA B fragment from 16 weight rows at once, so in row-major order neighbouring
// lanes read different rows and a wave load touches 64 cache lines for 1 KiB.  The engine keeps
// its GEMV matrices in tile order instead, where every wave load is one contiguous KiB:
//
//   tile T        16 rows: rows 16T..16T+15, or with SwiGLU pairing (N = 2*inter) the gate rows
//                 8T..8T+7 then the matching up rows inter+8T..inter+8T+7; rows past the matrix
//                 are zero (quant 0, scale 0)
//   superstep S   128*U elements of each row (U = 4 when K % 512 == 0, else 1; K % 128 == 0)
//   load v        NI loads per superstep (Q8: 2U, Q4: U) of 16 bytes per lane
//   lane l        row j = l & 15 of the tile, lane group g = l >> 4
//
//   quants  [T][S][v][l][16 bytes] = row bytes [S*RB + g*GB + 16v, +16) with RB = 128U (Q8) or
//           64U (Q4) bytes of a row per superstep and GB = RB/4 bytes per lane group
//   scales  [T][S][l][U] = row scales [4U*S + U*g, +U)
//
// so lane (j, g) of load v holds one 16-element half block (Q8) or one whole block (Q4) of
// row j, and its U scales arrive in one load.  Sizes: tiles*16*K (Q8) or tiles*8*K (Q4) bytes
// and tiles*16*K/32 scales, the reference's sizes whenever the tile count divides the rows.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime.h>

namespace snl {

struct PackGeom {
    int quant, N, K, inter;  // inter > 0: SwiGLU pairing of gate rows [0, inter) and up rows [inter, N)
    int U, nss, NI, tiles;
    int row_bytes;           // bytes of one reference row
    int ss_bytes;            // bytes of one row per superstep
    size_t q_bytes, s_floats;
};

// false when the shape has no tile order (K % 128 != 0, or a SwiGLU matrix with N != 2*inter)
__host__ __device__ inline bool pack_geom(int quant, int N, int K, int inter, PackGeom* g) {
    if (K <= 0 || N <= 0 || K % 128 != 0 || (quant != 0 && quant != 1)) return false;
    if (inter > 0 && N != 2 * inter) return false;
    g->quant = quant;
    g->N = N;
    g->K = K;
    g->inter = inter;
    g->U = K % 512 == 0 ? 4 : 1;
    g->nss = K / (128 * g->U);
    g->NI = quant == 0 ? 2 * g->U : g->U;
    g->tiles = inter > 0 ? (inter + 7) / 8 : (N + 15) / 16;
    g->row_bytes = quant == 0 ? K : K / 2;
    g->ss_bytes = quant == 0 ? 128 * g->U : 64 * g->U;
    g->q_bytes = (size_t)g->tiles * g->nss * g->NI * 1024;
    g->s_floats = (size_t)g->tiles * g->nss * 64 * g->U;
    return true;
}

// reference row of row j (0..15) of tile T, or -1 for padding
__host__ __device__ inline int pack_row(const PackGeom& g, int T, int j) {
    if (g.inter > 0) {
        const int c = T * 8 + (j & 7);
        if (c >= g.inter) return -1;
        return j < 8 ? c : g.inter + c;
    }
    const int r = T * 16 + j;
    return r < g.N ? r : -1;
}

// byte offset inside a reference row of load v of lane group gg in superstep S
__host__ __device__ inline int pack_row_offset(const PackGeom& g, int S, int v, int gg) {
    return S * g.ss_bytes + gg * (g.ss_bytes / 4) + 16 * v;
}

// offset of the 16-byte piece (T, S, v, lane) in the packed quants
__host__ __device__ inline size_t pack_piece(const PackGeom& g, int T, int S, int v, int lane) {
    return (((size_t)T * g.nss + S) * g.NI + v) * 1024 + (size_t)lane * 16;
}

// offset of the first of the U scales of (T, S, lane) in the packed scales
__host__ __device__ inline size_t pack_scale(const PackGeom& g, int T, int S, int lane) {
    return (((size_t)T * g.nss + S) * 64 + lane) * g.U;
}

// Reference layout -> tile order on the device (q, s: reference quants and scales).
int launch_pack_matrix(const PackGeom& g, const void* q, const float* s, void* qp, float* sp, hipStream_t st);

}  // namespace snl
