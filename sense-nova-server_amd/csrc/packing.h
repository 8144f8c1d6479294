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
// Lane (j, g) of load v holds row j's bytes [S*RB + g*GB + 16v, +16) (RB = 128U (Q8) or 64U (Q4)
// bytes of a row per superstep, GB = RB/4 per lane group): one 16-element half block (Q8) or one
// whole block (Q4), and its scales are row scales [4U*S + U*g, +U).
//
// The GEMV streams each tile in KS slices of nss_w = nss/KS supersteps, one wave per (tile,
// slice) item, in chunks of CL loads (half a superstep when U == 4, else a whole one) with the
// CS = U/CPS scales of their blocks.  The order of the chunks in memory follows the launch shape:
//   tile-major (il = 0):  chunk q of item i at ((i*nch + q)*CL + vv) KiB, scales likewise
//                         (each wave streams one contiguous run; many short blocks, the
//                         vocabulary head)
//   chunk-major (il = 1): chunk q of item i at ((q*items + i)*CL + vv) KiB (one block per CU:
//                         the whole grid sweeps memory together, which streams ~5-7% faster than
//                         one contiguous run per wave)
// with vv the load inside the chunk and the scales of chunk (q, i) at ((q*items + i)*64 + l)*CS.
// Sizes: tiles*16*K (Q8) or tiles*8*K (Q4) bytes and tiles*16*K/32 scales, the reference's
// sizes whenever the tile count divides the rows.
// Q8 bytes are stored in offset binary (the int8 value plus 128, i.e. the byte xor 0x80), the
// form the GEMV turns into an exact f16 with one byte permute; padding rows hold 0x80 (zero).
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
    // streaming split (chosen from the shape alone)
    int KS, nss_w;           // K slices per tile, supersteps per slice
    int CPS, CL, CS;         // chunks per superstep, loads and scales per chunk
    int nch, items;          // chunks per item, items (tiles * KS)
    int il;                  // 1: chunk-major order (one block per CU), 0: tile-major
};

constexpr int kPackCUs = 256;       // MI355X compute units
constexpr int kPackWaves = 16;      // waves per chunk-major GEMV block

// Waves of a chunk-major block that stage the token rows: enough that a staging thread takes at
// most 3 units of 8 elements of a row, and at least 4.  The other waves stream the weights.
__host__ __device__ inline int pack_stage_waves(int K) {
    const int w = (K / 8 + 191) / 192;
    return w < 4 ? 4 : w;
}

// The K split: one block per CU holds base or base + 1 tiles and KS is the largest divisor of the
// superstep count with KS * (base + 1) streaming waves at most (chunk-major order: up to 12 tiles
// per CU at K <= 6144); taller matrices run many blocks of 8 / KS tiles x KS <= 4 (Q8) or 2 (Q4) slices (tile-major
// order).
__host__ __device__ inline void pack_split(PackGeom* g) {
    int KS = 1;
    const int max_items = kPackWaves - pack_stage_waves(g->K);
    // (chunk-major offsets are 32-bit: matrices up to 2 GiB)
    if (max_items >= 1 && g->tiles <= max_items * kPackCUs && g->q_bytes < ((size_t)1 << 31)) {
        const int blocks = g->tiles < kPackCUs ? g->tiles : kPackCUs;
        const int tw = g->tiles / blocks + (g->tiles % blocks ? 1 : 0);
        for (int d = 1; d <= g->nss && d * tw <= max_items; ++d)
            if (g->nss % d == 0) KS = d;
        g->il = 1;
    } else {
        // slices per tile: 4 for Q8, 2 for Q4, whose dequantisation costs twice the vector work
        // per byte (248320 x 4096 heads: Q8 170 us at 4 slices, 182 at 2; Q4 125 us at 4, 110 at 2)
        const int ks_max = g->quant == 1 ? 2 : 4;
        while (KS < ks_max && g->nss % (2 * KS) == 0) KS *= 2;
        g->il = 0;
    }
    g->KS = KS;
    g->nss_w = g->nss / KS;
    g->CPS = g->U == 4 ? 2 : 1;
    g->CL = g->NI / g->CPS;
    g->CS = g->U / g->CPS;
    g->nch = g->nss_w * g->CPS;
    g->items = g->tiles * KS;
}

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
    pack_split(g);
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

// chunk index of (item, chunk) in memory order
__host__ __device__ inline size_t pack_chunk(const PackGeom& g, int item, int q) {
    return g.il ? (size_t)q * g.items + item : (size_t)item * g.nch + q;
}

// offset of the 16-byte piece (T, S, v, lane) in the packed quants
__host__ __device__ inline size_t pack_piece(const PackGeom& g, int T, int S, int v, int lane) {
    const int item = T * g.KS + S / g.nss_w, q = (S % g.nss_w) * g.CPS + v / g.CL;
    return (pack_chunk(g, item, q) * g.CL + v % g.CL) * 1024 + (size_t)lane * 16;
}

// offset of scale u (0..U-1) of (T, S, lane) in the packed scales
__host__ __device__ inline size_t pack_scale(const PackGeom& g, int T, int S, int lane, int u) {
    const int item = T * g.KS + S / g.nss_w, q = (S % g.nss_w) * g.CPS + u / g.CS;
    return (pack_chunk(g, item, q) * 64 + lane) * g.CS + u % g.CS;
}

// Reference layout -> tile order on the device (q, s: reference quants and scales).
int launch_pack_matrix(const PackGeom& g, const void* q, const float* s, void* qp, float* sp, hipStream_t st);

}  // namespace snl
