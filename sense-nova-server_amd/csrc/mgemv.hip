// Matrix-core skinny block-quantised GEMV for decode (M = 1..4 token rows), gfx950.
//
// y[m, n] = sum_b s[n, b] * sum_{i<32} q[n, 32b + i] * x[m, 32b + i]
//
// Weights are the reference's Q8_0 / Q4_0 blocks (src/weights.rs:48-55, src/engine.rs:84-108;
// Q4_0 nibble i of little-endian word w = element 8w + i) with f32 scales, held in the tile
// order of packing.h, so that every wave load is one contiguous KiB.
//
// The dot products run on v_mfma_f32_16x16x32_f16, which takes the place of the per-element
// convert-and-FMA of a vector-ALU GEMV (that costs ~3.5 VALU lane-ops per weight byte at M=2,
// close to the whole VALU budget at full HBM rate).  Both operands are exact:
//   * quants become f16 exactly: Q8 bytes, stored in offset binary (q + 128), are paired with 0x64
//     by v_perm (the f16 1024 + byte) and one packed f16 subtract of 1152 leaves q; Q4 nibbles are
//     only masked, and read as f16 subnormals n * 2^-24 (low nibble of a byte) or 16n * 2^-24 (high
//     nibble, whose token values are staged divided by 16); the offset 8 comes back per block as
//     -8 * (the block's sum of staged token values), formed by the staging, after the MFMAs;
//   * each token row x (f32) is split into two f16 parts, hi = f16(x) and lo = f16(x - hi), whose
//     sum carries 22 significant bits; a power of two per token and superstep scales the part's
//     largest |x| into [2^13, 2^14), so hi cannot overflow and small rows keep their bits.
// The accumulation is f32 throughout.
//
// MFMA orientation.  A (16 x 32) holds x, B (32 x 16) holds 16 weight rows.  The 4 lane groups of
// B (k-groups) each cover one 16-element half-block, so each lane has one quant block per load.
// A row i = 4*slot + combo (combo = token-in-pair x {hi, lo}) is non-zero only in the k-group of
// its slot.  The 16x16 result then leaves lane (row j, group g) with the block dot products of
// weight row j for the block of group g, one register per combo, and that lane scales them by
// its own block scale s[j, block] and accumulates.  One MFMA group handles one pair of tokens;
// M = 3, 4 runs a second A against the same converted B.
//
// Work split.  A tile is 16 weight rows (SwiGLU: 8 gate rows and the matching 8 up rows).  A
// superstep is 128*U elements of a row (U = 4 when K % 512 == 0, else 1), 8 KiB of a Q8 tile;
// K is cut into KS equal slices of supersteps.  Chunk-major matrices (packing.h) run one block per
// CU (at most 256 blocks, one resident per CU): block b owns the consecutive tiles
// [b*base + min(b, extra), +base + (b < extra)) (chunk-major shapes use extra = 0: base tiles per
// block, the last block the rest), its streaming wave w the item (tile w / KS, slice w % KS), so
// every active wave streams the same bytes, and pack_stage_waves(K) more waves stage the token
// rows.  Taller matrices (the vocabulary head) run many short blocks of 4 slices x 2 tiles
// (Q4: 2 x 4) whose waves do both.  The split depends on the matrix shape and quant type alone,
// never on M.  Weights stream through a three-chunk register ring (half supersteps; four chunks
// in blocks of at most 12 waves).  Slices are added in
// slice order through LDS, so a token's result does not depend on M, on its index or on timing
// (greedy output is then byte-identical with and without speculative drafting).
//
// Branch input (layers.wgsl:46-73 and :94-126): the plain x rows, RMSNorm(x0)*(1+w), or, inside
// the mHC range, RMSNorm(pre0*x0 + pre1*x1)*(1+w) with pre from this site's router sums, whose
// block partials the producing GEMV left; the 1/rms factor is applied to the dot products.
//
// Epilogues: plain store; residual add into stream 0 (merge mode 0, layers.wgsl:142-145); mHC
// merge (modes 1/2, layers.wgsl:150-161); SwiGLU (layers.wgsl:164-175).
#include "common.h"
#include "kernels.h"
#include "packing.h"

#pragma clang fp contract(off)

// two f32 through the raw buffer load intrinsic (clang's __builtin_amdgcn_raw_buffer_load_b64
// lowers to a single dword load here)
typedef float snl_f32x2_t __attribute__((ext_vector_type(2)));
__device__ snl_f32x2_t snl_raw_buffer_load_f32x2(__amdgpu_buffer_rsrc_t rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.ptr.buffer.load.v2f32");

namespace snl {

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMaxWaves = 16;
constexpr int kRing4Waves = 12;           // largest block of the four-chunk ring
constexpr int kCUs = 256;                 // MI355X compute units
constexpr int kLdsLimit = 150 * 1024;     // dynamic LDS per block
constexpr int kZeroBytes = 64;            // zero A fragment read by the lanes outside their slot

template <int EPI>
__device__ __forceinline__ int tile_row(const GemvArgs& a, int T, int j) {
    if constexpr (EPI == GEMV_SWIGLU) {
        const int c = T * 8 + (j & 7);
        if (c >= a.inter) return -1;
        return j < 8 ? c : a.inter + c;
    } else {
        const int r = T * 16 + j;
        return r < a.N ? r : -1;
    }
}

__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));


// Raw buffer descriptor over [base, base + bytes): a load at or past `bytes` returns zeros and
// touches no memory, so a wave can issue its weight ring unconditionally past the end of its
// slice.  Word 3 is the gfx9 raw (untyped) dword format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Block barrier that orders LDS only: this wave's LDS operations complete before the barrier and
// vector memory loads stay in flight across it.  (A full __syncthreads also orders global memory,
// so the compiler keeps every global access on its side of it.)
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// 16 bytes per lane from global memory straight into LDS (lane i at dst + 16 i), by DMA: no
// register receives the data.  Issued as inline assembly, so the compiler's wait insertion does
// not see it; the reader waits on the vector memory count itself.
__device__ __forceinline__ void copy16_to_lds(const char* base, unsigned voff, unsigned dst) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(dst), "v"(voff), "s"(base)
                 : "memory", "m0");
}

// Makes a loaded value opaque to the compiler at this point (no instruction is emitted), so that
// its first use, and the wait for the load, cannot be hoisted above: the staging waves issue every
// load of the prologue first and consume them only after the block barrier that orders the weight
// stream behind them.  (Without it the compiler waited for the first loads before issuing the rest.)
__device__ __forceinline__ void opaque(float& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void opaque(f32x4_t& v) { asm volatile("" : "+v"(v)); }

// 8 weights of one 16-byte load as exact f16: MFMA i (0..NM-1) of the load.
// Q8 order: elements 8i..8i+7.  Q4 order (word i): elements 8i + {0, 4, 1, 5, 2, 6, 3, 7}.
// Q8: the packed bytes are offset binary (q + 128, packing.h); v_perm pairs each with 0x64, the f16
// 1024 + byte, and one packed subtract of 1152 leaves q.  Q4: nibble pairs (i, i + 4) are masked
// in place (element i in the low half of a 16-bit lane, i + 4 in the high half), n from the low
// nibble of a byte and 16n from the high one, and taken as they are, f16 subnormals n * 2^-24 and
// 16n * 2^-24 (exact): 5 vector instructions per 8 weights.  The offset of 8 and the 2^24 are
// applied per block after the MFMAs (Q4 block correction, stage and compute).
template <int QT>
__device__ __forceinline__ half8_t dequant8(const uint4& w, int i) {
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    if constexpr (QT == 0) {
        const half2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
        const uint32_t u0 = wd[2 * i], u1 = wd[2 * i + 1];
        const half2_t p0 = as_h2(__builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u)) - bias;
        const half2_t p1 = as_h2(__builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u)) - bias;
        const half2_t p2 = as_h2(__builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u)) - bias;
        const half2_t p3 = as_h2(__builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u)) - bias;
        return half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
    } else {
        // the nibbles as they lie, read as f16 subnormals: n * 2^-24 for the low nibble of a byte, 16n *
        // 2^-24 for the high one (whose token values are staged divided by 16); the MFMA's sum of n * x
        // then becomes the block dot with 2^24 and the block's -8 * sum(x) (compute, below)
        const uint32_t v = wd[i], v8 = v >> 8;
        const half2_t p0 = as_h2(v & 0x000F000Fu), p1 = as_h2(v & 0x00F000F0u);
        const half2_t p2 = as_h2(v8 & 0x000F000Fu), p3 = as_h2(v8 & 0x00F000F0u);
        return half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
    }
}

// position of element e (0..31) of a block inside its staged A fragment
template <int QT>
__device__ __forceinline__ int a_pos(int e) {
    if constexpr (QT == 0) return e;
    else return (e & ~7) + 2 * (e & 3) + ((e >> 2) & 1);
}

// QT: 0 Q8_0, 1 Q4_0.  P: token pairs (M <= 2P).  U: quant blocks per lane group per superstep.
// UPT: 8-element units of each token row per staging thread.  IL: 1 chunk-major, 0 tile-major.
//
// Wave roles.  Chunk-major launches (one block per CU) run two kinds of waves: waves [0, sw0)
// stream the weights (one (tile, slice) item each) and waves [sw0, nwv) stage the token rows.
// The streaming waves issue their whole three-chunk ring at once and wait at the one block
// barrier; a wave stalled at issue behind its own weights is then not holding up the prologue,
// and the HBM stream starts with the kernel.  Tile-major launches (sw0 = 0) have every wave do
// both, the first chunk before the staging and the others after it.
//
// The staging needs no block barrier of its own.  Each staged superstep of a token (512 or 128
// elements) is one wave's lanes, which find its largest |value| by themselves and scale it by a
// power of two into [2^13, 2^14) before the f16 hi + lo split; the main loop multiplies each
// chunk's block scales by the superstep's inverse power of two (exact).  The RMSNorm factor
// 1/rms of the branch input is applied to the dot products in the epilogue, from the staging
// waves' sums of squares; the mHC pre-mix coefficients come from the router sums, which every
// staging wave adds up itself from the producer's partials.
//
// IL 2 is chunk-major with a four-chunk ring, for blocks of at most 12 waves (a wave may then hold
// 170 registers): the deeper ring keeps the memory pipe fed while the staging of a normed or mHC
// branch input is still running.
template <int QT, int P, int EPI, int PRO, int U, int UPT, int IL>
__global__ __launch_bounds__(IL == 2 ? kRing4Waves * 64 : kMaxWaves * 64) void mgemv_kernel(
    GemvArgs a, int M, int KS, int base, int extra, int nss_w, int tiles, int sw0) {
    constexpr int il = IL ? 1 : 0;
    constexpr int RING = IL == 2 ? 4 : 3;
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ float red_s[kMaxWaves * 16 * 2 * P];  // [wave][row j][token]
    __shared__ float ssq_s[kMaxWaves][2 * P];        // staging waves' sums of squares, per token
    __shared__ float cf_s[2 * P][8];                 // mHC token coefficients (MHC epilogue)
    __shared__ float raw_s[2 * P][9];                // last block: this site's router sums (NORM_MHC)
    __shared__ float pr_s[kMaxWaves * 16 / 32][2 * P][9];  // next-site router sums per 32-row group
    __shared__ float rt_s[9 * 2 * P * 16];                 // one tile: [sum][token][row] of them
    constexpr int NI = QT == 0 ? 2 * U : U;   // 16-byte loads per lane per superstep
    constexpr int NM = QT == 0 ? 2 : 4;       // MFMAs per load
    constexpr int SSU = 16 * U;               // 8-element units per superstep
    const int K = a.K, nb = K >> 5, K4 = K >> 2, nss = K / (128 * U);
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nthr = blockDim.x, nwv = nthr >> 6;
    const int bi = blockIdx.x;
    const int tile0 = bi * base + (bi < extra ? bi : extra);                 // first tile of the block
    const int cnt = min(base + (bi < extra ? 1 : 0), tiles - tile0);        // its tiles
    const int tw = wave / KS, ks = wave - tw * KS;
    const bool active = tw < cnt;  // staging waves (tw >= base + 1) and spare ones stream nothing
    const bool stager = wave >= sw0;
    const int Tl = tile0 + (active ? tw : 0);
    const int j = lane & 15, g = lane >> 4;
    const int tw_max = base + (extra ? 1 : 0);
    // LDS: token fragments [P][nb][256 B], a zero fragment, the next site's router rows (rpart),
    // then the superstep multipliers [P][nss][2]
    const int zero_off = P * nb * 256;
    const int rrow_off = zero_off + kZeroBytes;
    float* const mult_s = reinterpret_cast<float*>(lds + rrow_off + (a.rpart ? tw_max * 16 * M * 64 : 0));
    // Weights stream through a ring of three chunks of CL loads (half a superstep when U == 4)
    // with the CS = U*CL/NI scales of their quant blocks.  Chunk q of this wave's item
    // i = T*KS + ks is at chunk index q*items + i (chunk-major, il) or i*nch + q (tile-major) of
    // the packed matrix (packing.h): in both, a base for the item plus q times a stride.
    // Every issue is unconditional: the descriptor ends at the item's last chunk, so a chunk past
    // it reads zero without a memory access, and the loads keep one fixed order in which each
    // wait names exactly the chunk it needs.
    constexpr int CL = U == 4 ? NI / 2 : NI;  // loads per chunk
    constexpr int CPS = NI / CL;              // chunks per superstep
    constexpr int CS = U / CPS;               // scales per chunk
    uint4 w0[CL], w1[CL], w2[CL], w3[CL];
    float s0[CS], s1[CS], s2[CS], s3[CS];
    const int nch = nss_w * CPS;
    const size_t item = (size_t)Tl * KS + ks;
    const size_t items = (size_t)tiles * KS;
    const size_t cbase = il ? item : item * nch;         // chunk index of chunk 0
    const unsigned cstride = il ? (unsigned)items : 1u;  // chunk indices between chunks q and q + 1
    const __amdgpu_buffer_rsrc_t wr =
        make_rsrc(static_cast<const uint8_t*>(a.wq) + cbase * CL * 1024,
                  active ? ((unsigned)(nch - 1) * cstride + 1u) * CL * 1024 : 0u);
    const __amdgpu_buffer_rsrc_t sr =
        make_rsrc(a.ws + cbase * 64 * CS, active ? ((unsigned)(nch - 1) * cstride + 1u) * 64 * CS * 4 : 0u);
    const int wv = lane * 16, sv = lane * CS * 4;
    // The scales first, then the quants; the scheduling barrier keeps chunks in issue order.  The
    // whole offset goes in the per-lane operand: the range check covers that operand and the
    // instruction offset.  Both carry the non-temporal hint (cache-policy argument 2): a decode
    // pass reads every weight once, and at normal priority that stream would evict the token
    // rows, recurrent state and key/value cache that the following kernels read again.
    auto issue = [&](uint4 (&w)[CL], float (&sc)[CS], int q) {
        const int so = sv + q * (int)cstride * 64 * CS * 4;
        if constexpr (CS == 2) {
            const snl_f32x2_t t = snl_raw_buffer_load_f32x2(sr, so, 0, 2);
            sc[0] = t.x, sc[1] = t.y;
        } else {
            sc[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sr, so, 0, 2));
        }
        const int wo = wv + q * (int)cstride * CL * 1024;
#pragma unroll
        for (int v = 0; v < CL; ++v)
            w[v] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, wo + v * 1024, 0, 2));
        __builtin_amdgcn_sched_barrier(0);
    };
    // ---- prologue, part 1: every load of the token rows comes before the first weight load ----
    // Vector loads complete in issue order, so a row load issued after the weights would wait for
    // them.  Staging thread ts owns the 8-element units ts + u*nst (u < UPT) of every token row.
    const int ts = tid - sw0 * 64, nst = nthr - sw0 * 64;
    const int row0 = a.row_base ? *a.row_base : 0;
    const int K8 = K >> 3;
    // Every staging load is a range-checked buffer load without a branch: a token past M, a unit
    // past the row or a GNORM head past the buffer reads zero.  (A branch would join the loaded
    // value with a constant, and that join waits for the load.)
    const unsigned row_bytes = (unsigned)(PRO == GEMV_NORM_MHC ? 2 * K : K) * 4;
    __amdgpu_buffer_rsrc_t xr[2 * P];
#pragma unroll
    for (int m = 0; m < 2 * P; ++m)
        xr[m] = make_rsrc(a.x + (size_t)(row0 + (m < M ? m : 0)) * a.x_stride, m < M ? row_bytes : 0u);
    auto ld4 = [](__amdgpu_buffer_rsrc_t r, int off) {
        return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
    };
    // mHC: the staging waves add this site's router sums 0, 1 and 8 of each token
    // (layers.wgsl:94-102) from the producer's block partials, laid out [m][o][block]: lane l takes
    // blocks l, l + 64, ... in order.  The first 256 partials of each sum go to the wave's own LDS
    // slots by DMA (global_load_lds: no registers, so nothing is consumed before the barrier);
    // more producer blocks than 256 are added later from global memory.  The last block also needs
    // the site's other sums (o = 2..7) for the token coefficients: the 6M of them are spread over
    // its staging waves, kXtra each.
    constexpr int kRinO[3] = {0, 1, 8};
    constexpr int kXtra = 3;                         // 6M <= 12 sums over >= 4 staging waves
    constexpr int kRinSlots = 2 * P * 3 + kXtra;     // 1 KiB LDS slots per staging wave
    const unsigned rin_off = ((unsigned)(reinterpret_cast<unsigned char*>(mult_s) - lds) + (unsigned)P * nss * 8 + 15u) & ~15u;
    const unsigned rin_w = rin_off + (unsigned)(wave - sw0) * kRinSlots * 1024;  // this wave's slots
    // Q4: the block corrections [P][nb][4 combos], -8 * (sum of the block's staged values, high-nibble
    // ones times 16), after the router partial slots
    float* const corr_s = reinterpret_cast<float*>(
        lds + rin_off + (PRO == GEMV_NORM_MHC ? (unsigned)(nwv - sw0) * kRinSlots * 1024 : 0u));
    f32x4_t sb[2] = {f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}};  // the 8 router biases
    // NORM_MHC: xb is stream 1 of the row.  GNORM: gp holds the head's column-group partial sums
    // of squares.
    f32x4_t xa[2 * P][UPT][2], xb[2 * P][UPT][2], nw[UPT][2], gp[2 * P][UPT];
    auto stage_loads = [&]() {
    if constexpr (PRO == GEMV_NORM_MHC) {
        {
            const unsigned lds_base = (unsigned)(uintptr_t)(__attribute__((address_space(3))) void*)lds;
            // the 256-partial window may run past a shorter producer into other sums (masked when
            // added) but stays inside the partials buffer (kPartBlocks rows per sum)
#pragma unroll
            for (int m = 0; m < 2 * P; ++m)
#pragma unroll
                for (int c = 0; c < 3; ++c)
                    if (m < M)
                        copy16_to_lds(reinterpret_cast<const char*>(a.rin + (size_t)(9 * m + kRinO[c]) * a.rin_n),
                                      (unsigned)lane * 16u, lds_base + rin_w + (unsigned)(m * 3 + c) * 1024u);
            if (blockIdx.x == gridDim.x - 1)
#pragma unroll
                for (int x = 0; x < kXtra; ++x) {
                    const int k = (wave - sw0) + (nwv - sw0) * x;  // sum index m*6 + (o - 2)
                    if (k < 6 * M)
                        copy16_to_lds(reinterpret_cast<const char*>(a.rin + (size_t)(9 * (k / 6) + 2 + k % 6) * a.rin_n),
                                      (unsigned)lane * 16u, lds_base + rin_w + (unsigned)(2 * P * 3 + x) * 1024u);
                }
            const __amdgpu_buffer_rsrc_t br = make_rsrc(a.site_w + (size_t)16 * K, 32u);
            sb[0] = ld4(br, 0);
            sb[1] = ld4(br, 16);
        }
    }
    {
        const __amdgpu_buffer_rsrc_t nr = make_rsrc(a.norm_w, (PRO == GEMV_NORM || PRO == GEMV_NORM_MHC) ? (unsigned)K * 4 : 0u);
        // GNORM: the head partials [M][K/128][4]
        const __amdgpu_buffer_rsrc_t gr = make_rsrc(a.rin, PRO == GEMV_GNORM ? (unsigned)(M * (K / 128) * 16) : 0u);
#pragma unroll
        for (int u = 0; u < UPT; ++u) {
            const int k8 = ts + u * nst;
            const int ko = k8 < K8 ? k8 * 32 : row_bytes;  // byte offset of the unit (past the row: zero)
            if constexpr (PRO == GEMV_NORM || PRO == GEMV_NORM_MHC) {
                nw[u][0] = ld4(nr, ko);
                nw[u][1] = ld4(nr, ko + 16);
            }
#pragma unroll
            for (int m = 0; m < 2 * P; ++m) {
                xa[m][u][0] = ld4(xr[m], ko);
                xa[m][u][1] = ld4(xr[m], ko + 16);
                if constexpr (PRO == GEMV_NORM_MHC) {
                    xb[m][u][0] = ld4(xr[m], K * 4 + ko);
                    xb[m][u][1] = ld4(xr[m], K * 4 + ko + 16);
                } else if constexpr (PRO == GEMV_GNORM) {
                    gp[m][u] = ld4(gr, m < M && k8 < K8 ? (m * (K / 128) + k8 / 16) * 16 : (int)(M * (K / 128) * 16));
                }
            }
        }
    }
    };

    // Thread tid owns output tid of the block (cnt*16*M outputs, all in streaming waves); the
    // residual it will update is read now, also ahead of the weights.
    const int e_m = tid % M, e_r = tid / M;
    const int e_T = tile0 + (e_r >> 4), e_j = e_r & 15;
    const int e_row = tid < cnt * 16 * M && !(EPI == GEMV_SWIGLU && e_j >= 8) ? tile_row<EPI>(a, e_T, e_j) : -1;
    float e_y0 = 0.0f, e_y1 = 0.0f;
    float cfv = 0.0f;  // the site's token coefficients (MHC epilogue), left by its NORM_MHC launch
    float nr0[8], nr1[8];  // router rows of the next mHC site at this output's row
#pragma unroll
    for (int o = 0; o < 8; ++o) nr0[o] = nr1[o] = 0.0f;
    auto epilogue_loads = [&]() {
    if constexpr (EPI == GEMV_ADD || EPI == GEMV_MHC) {
        if (e_row >= 0) {
            const float* yr = a.y + (size_t)e_m * a.y_stride;
            e_y0 = yr[e_row];
            if constexpr (EPI == GEMV_MHC) e_y1 = yr[a.h + e_row];
        }
    }
    if constexpr (EPI == GEMV_MHC) {
        if (tid < 8 * M) cfv = a.coef[tid];
    }
    if constexpr (EPI == GEMV_ADD || EPI == GEMV_MHC) {
        if (a.rpart && e_row >= 0)
#pragma unroll
            for (int o = 0; o < 8; ++o) {
                nr0[o] = a.next_w[(size_t)o * 2 * a.h + e_row];
                nr1[o] = a.next_w[(size_t)o * 2 * a.h + a.h + e_row];
            }
    }
    };

    // ---- prologue, part 2: the staging, wave by wave ----
    float ssq[2 * P];  // this thread's sum of squares of the branch input, per token
#pragma unroll
    for (int m = 0; m < 2 * P; ++m) ssq[m] = 0.0f;
    // sum n of this wave's partial slot: lane l adds blocks l, l + 64, ... in order
    auto rin_sum = [&](int slot, int n) {
        const float* pl = reinterpret_cast<const float*>(lds + rin_w + slot * 1024);
        float t = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int b = lane + 64 * r;
            t = t + (b < a.rin_n ? pl[b] : 0.0f);
        }
        for (int b = lane + 256; b < a.rin_n; b += 64) t = t + a.rin[(size_t)n * a.rin_n + b];
        return t;
    };
    auto stage = [&]() {
        if (stager) {
            if constexpr (PRO == GEMV_NORM_MHC) __builtin_amdgcn_s_waitcnt(0);  // the DMA slots have landed
#pragma unroll
            for (int u = 0; u < UPT; ++u) {
                if constexpr (PRO == GEMV_NORM || PRO == GEMV_NORM_MHC) opaque(nw[u][0]), opaque(nw[u][1]);
#pragma unroll
                for (int m = 0; m < 2 * P; ++m) {
                    opaque(xa[m][u][0]);
                    opaque(xa[m][u][1]);
                    if constexpr (PRO == GEMV_NORM_MHC) opaque(xb[m][u][0]), opaque(xb[m][u][1]);
                    if constexpr (PRO == GEMV_GNORM) opaque(gp[m][u]);
                }
            }
            if constexpr (PRO == GEMV_NORM_MHC) opaque(sb[0]), opaque(sb[1]);
            const float sw0f = sb[0].x, sw1f = sb[0].y;
            float pre0[2 * P], pre1[2 * P];
#pragma unroll
            for (int m = 0; m < 2 * P; ++m) pre0[m] = 1.0f, pre1[m] = 0.0f;
            if constexpr (PRO == GEMV_NORM_MHC) {
                float rs[2 * P * 3];
#pragma unroll
                for (int m = 0; m < 2 * P; ++m)
#pragma unroll
                    for (int c = 0; c < 3; ++c) rs[m * 3 + c] = m < M ? rin_sum(m * 3 + c, 9 * m + kRinO[c]) : 0.0f;
                wave_sum_n(rs);
#pragma unroll
                for (int m = 0; m < 2 * P; ++m) {
                    if (m >= M) continue;
                    const float rr = 1.0f / sqrtf(rs[m * 3 + 2] / (float)(2 * K) + 1e-6f);
                    pre0[m] = 1.0f / (1.0f + __expf(-(rs[m * 3 + 0] * rr + sw0f)));
                    pre1[m] = 1.0f / (1.0f + __expf(-(rs[m * 3 + 1] * rr + sw1f)));
                }
                if (blockIdx.x == gridDim.x - 1) {
                    // the further sums, added in the same order, and all nine to LDS for the
                    // coefficients after the prologue barrier
                    float xs[kXtra];
#pragma unroll
                    for (int x = 0; x < kXtra; ++x) {
                        const int k = (wave - sw0) + (nwv - sw0) * x;
                        xs[x] = k < 6 * M ? rin_sum(2 * P * 3 + x, 9 * (k / 6) + 2 + k % 6) : 0.0f;
                    }
                    wave_sum_n(xs);
                    if (lane == 0) {
#pragma unroll
                        for (int x = 0; x < kXtra; ++x) {
                            const int k = (wave - sw0) + (nwv - sw0) * x;
                            if (k < 6 * M) raw_s[k / 6][2 + k % 6] = xs[x];
                        }
                        if (wave == sw0)
#pragma unroll
                            for (int m = 0; m < 2 * P; ++m)
                                if (m < M) raw_s[m][0] = rs[m * 3], raw_s[m][1] = rs[m * 3 + 1], raw_s[m][8] = rs[m * 3 + 2];
                    }
                }
            }
            // the branch input of each unit (layers.wgsl:57-73: pre-mix, then the (1 + w) weight; the
            // 1/rms factor waits for the epilogue), its sum of squares, and its largest |value|
            float umax[2 * P][UPT];
#pragma unroll
            for (int u = 0; u < UPT; ++u) {
                const bool on = ts + u * nst < K8;
#pragma unroll
                for (int m = 0; m < 2 * P; ++m) {
                    umax[m][u] = 0.0f;
                    if (!on || m >= M) continue;
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        f32x4_t t = xa[m][u][hh];
                        if constexpr (PRO == GEMV_GNORM) {  // the head factor of linear.wgsl:131-133
                            const f32x4_t pp = gp[m][u];
                            const float var_o = (((pp.x + pp.y) + pp.z) + pp.w) / 128.0f;
                            const float rr = 1.0f / sqrtf(var_o + a.eps);
                            t.x = t.x * rr;
                            t.y = t.y * rr;
                            t.z = t.z * rr;
                            t.w = t.w * rr;
                        }
                        if constexpr (PRO == GEMV_NORM_MHC) {
                            const f32x4_t v1 = xb[m][u][hh];
                            t.x = pre0[m] * t.x + pre1[m] * v1.x;
                            t.y = pre0[m] * t.y + pre1[m] * v1.y;
                            t.z = pre0[m] * t.z + pre1[m] * v1.z;
                            t.w = pre0[m] * t.w + pre1[m] * v1.w;
                        }
                        if constexpr (PRO == GEMV_NORM || PRO == GEMV_NORM_MHC) {
                            ssq[m] = fmaf(t.x, t.x, ssq[m]);
                            ssq[m] = fmaf(t.y, t.y, ssq[m]);
                            ssq[m] = fmaf(t.z, t.z, ssq[m]);
                            ssq[m] = fmaf(t.w, t.w, ssq[m]);
                            const f32x4_t w = nw[u][hh];
                            t.x = t.x * (1.0f + w.x);
                            t.y = t.y * (1.0f + w.y);
                            t.z = t.z * (1.0f + w.z);
                            t.w = t.w * (1.0f + w.w);
                        }
                        xa[m][u][hh] = t;
                        umax[m][u] = fmaxf(umax[m][u], fmaxf(fmaxf(fabsf(t.x), fabsf(t.y)), fmaxf(fabsf(t.z), fabsf(t.w))));
                    }
                }
            }
            // superstep maxima: the SSU units of a superstep are SSU consecutive lanes of this wave
#pragma unroll
            for (int u = 0; u < UPT; ++u)
#pragma unroll
                for (int m = 0; m < 2 * P; ++m) {
                    float v = umax[m][u];
                    v = xor_max<1>(v);
                    v = xor_max<2>(v);
                    v = xor_max<4>(v);
                    v = xor_max<8>(v);
                    if constexpr (SSU == 64) {
                        v = xor_max<16>(v);
                        v = xor_max<32>(v);
                    }
                    umax[m][u] = v;
                }
            // power-of-two scale per (token, superstep): the largest |value| lands in [2^13, 2^14), so
            // the f16 high part cannot overflow and keeps 11 bits, the low part 11 more
#pragma unroll
            for (int u = 0; u < UPT; ++u) {
                const int k8 = ts + u * nst;
                if (k8 >= K8) continue;
                const int S = k8 / SSU;
#pragma unroll
                for (int m = 0; m < 2 * P; ++m) {
                    const float mx = umax[m][u];
                    int e = mx > 0.0f ? ilogbf(mx) - 13 : 0;
                    e = e < -120 ? -120 : (e > 120 ? 120 : e);
                    const float f = ldexpf(1.0f, -e);
                    if (k8 % SSU == 0) mult_s[((m >> 1) * nss + S) * 2 + (m & 1)] = ldexpf(1.0f, e);
                    // unit k8 of token m -> 8 hi then 8 lo f16 in fragment order inside region (pair, block, token)
                    const float v[8] = {xa[m][u][0].x, xa[m][u][0].y, xa[m][u][0].z, xa[m][u][0].w,
                                        xa[m][u][1].x, xa[m][u][1].y, xa[m][u][1].z, xa[m][u][1].w};
                    half8_t hi, lo;
                    float shi = 0.0f, slo = 0.0f;  // Q4: the unit's staged values, high-nibble ones times 16
#pragma unroll
                    for (int e8 = 0; e8 < 8; ++e8) {
                        // Q4: an odd element (the high nibble of its byte) meets 16n, so it is staged / 16
                        const float y = QT == 1 && (e8 & 1) ? v[e8] * f * 0.0625f : v[e8] * f;
                        const _Float16 hv = (_Float16)y;
                        const _Float16 lv = (_Float16)(y - (float)hv);
                        const int pidx = a_pos<QT>(e8);
                        hi[pidx] = hv;
                        lo[pidx] = lv;
                        if constexpr (QT == 1) {
                            const float w = (e8 & 1) ? 16.0f : 1.0f;
                            shi = shi + (float)hv * w;
                            slo = slo + (float)lv * w;
                        }
                    }
                    unsigned char* bp =
                        lds + ((size_t)(m >> 1) * nb + (k8 >> 2)) * 256 + (m & 1) * 128 + (k8 & 3) * 16;
                    *reinterpret_cast<half8_t*>(bp) = hi;
                    *reinterpret_cast<half8_t*>(bp + 64) = lo;
                    if constexpr (QT == 1) {
                        // the block's four units are four neighbouring lanes (all staged or none)
                        shi = xor_sum<2>(xor_sum<1>(shi));
                        slo = xor_sum<2>(xor_sum<1>(slo));
                        if ((k8 & 3) == 0) {
                            const float c = -8.0f;  // (exact: the sums are exact in f32)
                            *reinterpret_cast<float2*>(corr_s + (((m >> 1) * nb + (k8 >> 2)) * 4 + (m & 1) * 2)) =
                                make_float2(shi * c, slo * c);
                        }
                    }
                }
            }
            if constexpr (PRO == GEMV_NORM || PRO == GEMV_NORM_MHC) {
                wave_sum_n(ssq);
                if (lane == 0)
#pragma unroll
                    for (int m = 0; m < 2 * P; ++m) ssq_s[wave][m] = ssq[m];
            }
        }
    };
    // small LDS items: the zero fragment, the next site's router rows, the token coefficients
    auto side_lds = [&]() {
        if (tid < kZeroBytes / 16)
            reinterpret_cast<float4*>(lds + zero_off)[tid] = make_float4(0, 0, 0, 0);
        // the next site's router rows wait in LDS until the epilogue, instead of holding 16 registers
        // through the main loop
        if constexpr (EPI == GEMV_ADD || EPI == GEMV_MHC) {
            if (a.rpart && e_row >= 0) {
                float4* st = reinterpret_cast<float4*>(lds + rrow_off) + tid * 4;
                st[0] = make_float4(nr0[0], nr0[1], nr0[2], nr0[3]);
                st[1] = make_float4(nr0[4], nr0[5], nr0[6], nr0[7]);
                st[2] = make_float4(nr1[0], nr1[1], nr1[2], nr1[3]);
                st[3] = make_float4(nr1[4], nr1[5], nr1[6], nr1[7]);
            }
        }
        if constexpr (EPI == GEMV_MHC) {
            if (tid < 8 * M) cf_s[tid >> 3][tid & 7] = cfv;
        }
    };
    auto sinkhorn = [&]() {
        if constexpr (PRO == GEMV_NORM_MHC) {
            // The last block's last wave (a staging wave, idle during the main loop) stores the
            // site's nine router sums of each token, which its staging waves left in LDS, and turns
            // them into the token coefficients (2x2 Sinkhorn) for the MHC epilogue of the same site,
            // a later launch.  It touches no global memory before its stores: a load here would
            // queue behind the block's weight stream.
            if (blockIdx.x == gridDim.x - 1 && wave == nwv - 1) {
                if (lane < M) {
                    float raw[9], bias8[8], cf[8];
#pragma unroll
                    for (int o = 0; o < 9; ++o) raw[o] = raw_s[lane][o];
#pragma unroll
                    for (int o = 0; o < 9; ++o) a.raw[lane * 9 + o] = raw[o];
#pragma unroll
                    for (int o = 0; o < 4; ++o) bias8[o] = sb[0][o], bias8[4 + o] = sb[1][o];
                    mhc_coefficients_b(raw, bias8, 2 * K, a.iterations, cf);
#pragma unroll
                    for (int o = 0; o < 8; ++o) a.coef[lane * 8 + o] = cf[o];
                }
            }
        }

    };

    // NORM prologue with norm_out: block 0's staging threads store the normed rows themselves (the
    // final norm of a decode pass, layers.wgsl:46-73), from their staged values and the sums of
    // squares of every staging wave, added in wave order
    auto store_norm_rows = [&]() {
        if constexpr (PRO == GEMV_NORM) {
            if (a.norm_out && blockIdx.x == 0 && stager) {
#pragma unroll
                for (int m = 0; m < 2 * P; ++m) {
                    if (m >= M) continue;
                    float ss = 0.0f;
                    for (int w = sw0; w < nwv; ++w) ss = ss + ssq_s[w][m];
                    const float of = 1.0f / sqrtf(ss / (float)K + a.eps);
#pragma unroll
                    for (int u = 0; u < UPT; ++u) {
                        const int k8 = ts + u * nst;
                        if (k8 >= K8) continue;
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh) {
                            const f32x4_t t = xa[m][u][hh];
                            const float4 o = make_float4(t.x * of, t.y * of, t.z * of, t.w * of);
                            reinterpret_cast<float4*>(a.norm_out + (size_t)m * K + k8 * 8)[hh] = o;
                            if (a.norm_last && m == M - 1) reinterpret_cast<float4*>(a.norm_last + k8 * 8)[hh] = o;
                        }
                    }
                }
            }
        }
    };

    // ---- main loop ----
    f32x4_t acc[P];
#pragma unroll
    for (int p = 0; p < P; ++p) acc[p] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    auto main_loop = [&]() {
        // lane (j, g) feeds A row j = 4*slot + combo; it carries data only when slot == g
        const int slot = j >> 2, combo = j & 3;
        const bool a_on = slot == g;

        auto compute = [&](const uint4 (&w)[CL], const float (&sc)[CS], int q) {
            const int S = ks * nss_w + q / CPS;  // superstep within the row
            float2 mm[P];                        // its power-of-two multipliers, token 0 and 1 of each pair
#pragma unroll
            for (int p = 0; p < P; ++p) mm[p] = *reinterpret_cast<const float2*>(mult_s + (p * nss + S) * 2);
            // the chunk's A fragments first: all LDS reads in flight together instead of one
            // read-wait-MFMA round trip per fragment (one token pair: two would not fit the
            // registers, and they read each fragment next to its MFMA)
            constexpr bool kAhead = P == 1;
            half8_t av[CL][NM][P];
            auto read_a = [&](int i0) {
                const int v = (q % CPS) * CL + i0;                              // load within the superstep
                const int blk = S * 4 * U + U * g + (QT == 0 ? (v >> 1) : v);  // quant block of this load
                const int eoff = QT == 0 ? (v & 1) * 16 : 0;                  // first element in the block
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const int abase = a_on ? ((p * nb + blk) * 4 + combo) * 64 + eoff * 2 : zero_off;
#pragma unroll
                    for (int i = 0; i < NM; ++i)
                        av[i0][i][p] = *reinterpret_cast<const half8_t*>(lds + abase + (a_on ? 16 * i : 0));
                }
            };
            if constexpr (kAhead) {
#pragma unroll
                for (int i0 = 0; i0 < CL; ++i0) read_a(i0);
                // keep the reads ahead, and each load's dequantisation next to its own MFMAs (so
                // the converted weights of only one load are live while the fragments are in flight)
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int i0 = 0; i0 < CL; ++i0) {
                if constexpr (!kAhead) read_a(i0);
                f32x4_t d[P];
#pragma unroll
                for (int p = 0; p < P; ++p) d[p] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int i = 0; i < NM; ++i) {
                    const half8_t b = dequant8<QT>(w[i0], i);
#pragma unroll
                    for (int p = 0; p < P; ++p) d[p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i0][i][p], b, d[p], 0, 0, 0);
                }
                const float scale = sc[QT == 0 ? (i0 >> 1) : i0];
                if constexpr (QT == 1) {
                    // the block dot from the MFMAs' sum of n * x (times 2^-24): times 2^24, minus 8 * sum(x)
                    const int blk = S * 4 * U + U * g + (q % CPS) * CL + i0;
#pragma unroll
                    for (int p = 0; p < P; ++p) {
                        const float4 cr = *reinterpret_cast<const float4*>(corr_s + (p * nb + blk) * 4);
                        d[p][0] = fmaf(d[p][0], 0x1p24f, cr.x);
                        d[p][1] = fmaf(d[p][1], 0x1p24f, cr.y);
                        d[p][2] = fmaf(d[p][2], 0x1p24f, cr.z);
                        d[p][3] = fmaf(d[p][3], 0x1p24f, cr.w);
                    }
                }
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    // combos 0, 1: token 0 hi, lo; combos 2, 3: token 1
                    const float sm0 = scale * mm[p].x, sm1 = scale * mm[p].y;
                    acc[p][0] = fmaf(sm0, d[p][0], acc[p][0]);
                    acc[p][1] = fmaf(sm0, d[p][1], acc[p][1]);
                    acc[p][2] = fmaf(sm1, d[p][2], acc[p][2]);
                    acc[p][3] = fmaf(sm1, d[p][3], acc[p][3]);
                }
                if constexpr (kAhead) __builtin_amdgcn_sched_barrier(0);
            }
        };

        // Steady state: compute a chunk, issue the one RING ahead.  The last 2 RING - 1 chunks or fewer
        // run as a straight-line tail that issues nothing past the slice.
        const int nrun = active ? nch : 0;
        int q = 0;
        if constexpr (RING == 4) {
            for (; q + 7 < nrun; q += 4) {
                compute(w0, s0, q);
                issue(w0, s0, q + 4);
                compute(w1, s1, q + 1);
                issue(w1, s1, q + 5);
                compute(w2, s2, q + 2);
                issue(w2, s2, q + 6);
                compute(w3, s3, q + 3);
                issue(w3, s3, q + 7);
            }
            const int rem = nrun - q;  // 0 (idle wave) .. 7
            if (rem >= 1) compute(w0, s0, q);
            if (rem >= 5) issue(w0, s0, q + 4);
            if (rem >= 2) compute(w1, s1, q + 1);
            if (rem >= 6) issue(w1, s1, q + 5);
            if (rem >= 3) compute(w2, s2, q + 2);
            if (rem >= 7) issue(w2, s2, q + 6);
            if (rem >= 4) compute(w3, s3, q + 3);
            if (rem >= 5) compute(w0, s0, q + 4);
            if (rem >= 6) compute(w1, s1, q + 5);
            if (rem >= 7) compute(w2, s2, q + 6);
            return;
        }
        for (; q + 5 < nrun; q += 3) {
            compute(w0, s0, q);
            issue(w0, s0, q + 3);
            compute(w1, s1, q + 1);
            issue(w1, s1, q + 4);
            compute(w2, s2, q + 2);
            issue(w2, s2, q + 5);
        }
        const int rem = nrun - q;  // 0 (idle wave) .. 5
        if (rem >= 1) compute(w0, s0, q);
        if (rem >= 4) issue(w0, s0, q + 3);
        if (rem >= 2) compute(w1, s1, q + 1);
        if (rem >= 5) issue(w1, s1, q + 4);
        if (rem >= 3) compute(w2, s2, q + 2);
        if (rem >= 4) compute(w0, s0, q + 3);
        if (rem >= 5) compute(w1, s1, q + 4);

    };

    // Every wave of the block has issued its row loads before any wave issues weights, so the rows
    // are not queued behind the block's weight stream (issued after it they arrived ~6 us later).
    // The staging waves reach this barrier without waiting for any load.  The two roles run in
    // separate branches from their first load on, each with its own copy of the barrier: a staging
    // wave holds no weight ring and a streaming wave no token rows, and the compiler's wait
    // tracking sees no join where a streaming wave might still owe a staging load.  (With the
    // staging loads in a branch that joined the streaming path before the barrier, every streaming
    // wave waited for its epilogue loads before issuing its second chunk.)
    if constexpr (IL >= 1) {
        if (stager) {
            stage_loads();
            __builtin_amdgcn_s_barrier();
            stage();
            side_lds();
            lds_barrier();
            sinkhorn();
            store_norm_rows();
        } else {
            epilogue_loads();
            __builtin_amdgcn_s_barrier();
            // streaming-only waves send the whole ring at once
            issue(w0, s0, 0);
            issue(w1, s1, 1);
            issue(w2, s2, 2);
            if constexpr (RING == 4) issue(w3, s3, 3);
            side_lds();
            lds_barrier();
            main_loop();
        }
    } else {
        // Tile-major launches (the vocabulary head: many short blocks, several resident per CU):
        // the odd waves send their second chunk before the staging too (168 -> 163 us per
        // 248320 x 4096 Q8_0 head), the others after it.
        stage_loads();
        epilogue_loads();
        __builtin_amdgcn_s_barrier();
        issue(w0, s0, 0);
        const bool early = (wave & 1) != 0;
        if (early) issue(w1, s1, 1);
        stage();
        side_lds();
        if (!early) issue(w1, s1, 1);
        issue(w2, s2, 2);
        lds_barrier();
        sinkhorn();
        store_norm_rows();
        main_loop();
    }

    // ---- reduction: hi + lo, then the 4 lane groups, then the K slices in order ----
#pragma unroll
    for (int p = 0; p < P; ++p) {
        float t0 = acc[p][0] + acc[p][1], t1 = acc[p][2] + acc[p][3];
        t0 = xor_sum<16>(t0);
        t1 = xor_sum<16>(t1);
        t0 = xor_sum<32>(t0);
        t1 = xor_sum<32>(t1);
        if (g == 0) {
            red_s[(wave * 16 + j) * 2 * P + 2 * p] = t0;
            red_s[(wave * 16 + j) * 2 * P + 2 * p + 1] = t1;
        }
    }
    __syncthreads();
    float x0n = 0.0f, x1n = 0.0f;  // the new residual of this output's row (ADD / MHC)
    if (e_row >= 0) {
        const int t2 = e_r >> 4;
        float v = 0.0f;
        for (int k = 0; k < KS; ++k) v = v + red_s[((t2 * KS + k) * 16 + e_j) * 2 * P + e_m];
        // the RMSNorm factor of the branch input, from the staging waves' sums in wave order
        float of = 1.0f;
        if constexpr (PRO == GEMV_NORM || PRO == GEMV_NORM_MHC) {
            float ss = 0.0f;
            for (int w = sw0; w < nwv; ++w) ss = ss + ssq_s[w][e_m];
            of = 1.0f / sqrtf(ss / (float)K + a.eps);
        }
        v = v * of;
        float* y = a.y + (size_t)e_m * a.y_stride;
        if constexpr (EPI == GEMV_SWIGLU) {
            float u = 0.0f;
            for (int k = 0; k < KS; ++k) u = u + red_s[((t2 * KS + k) * 16 + e_j + 8) * 2 * P + e_m];
            u = u * of;
            y[e_T * 8 + e_j] = v / (1.0f + expf(-v)) * u;
        } else if constexpr (EPI == GEMV_STORE) {
            y[a.n_off + e_row] = v;
        } else if constexpr (EPI == GEMV_ADD) {  // merge mode 0, layers.wgsl:142-145
            x0n = e_y0 + v;
            x1n = x0n;
            y[e_row] = x0n;
            if (a.expand) y[a.h + e_row] = x0n;  // mode 3 of the next visit, layers.wgsl:146-149
        } else {  // GEMV_MHC, modes 1 and 2, layers.wgsl:150-161
            const float* cf = cf_s[e_m];
            const float n0 = (cf[4] * e_y0 + cf[5] * e_y1) + cf[2] * v;
            const float n1 = (cf[6] * e_y0 + cf[7] * e_y1) + cf[3] * v;
            x0n = a.merge_mode == 2 ? 0.5f * (n0 + n1) : n0;
            x1n = a.merge_mode == 2 ? e_y1 : n1;  // mode 2 leaves stream 1 as it was
            if (a.expand) x1n = x0n;
            y[e_row] = x0n;
            if (a.merge_mode != 2 || a.expand) y[a.h + e_row] = x1n;
        }
    }
    if constexpr (EPI == GEMV_ADD || EPI == GEMV_MHC) {
        if (a.rpart) {
            // partial router sums of the next site over this block's rows, in an order that is the
            // same for every M (one tile: the rows in order; more: 32-row butterflies, then the
            // groups in order)
            float c[9];
            if (e_row >= 0) {
                const float4* st = reinterpret_cast<const float4*>(lds + rrow_off) + tid * 4;
                const float4 q0 = st[0], q1 = st[1], q2 = st[2], q3 = st[3];
                const float r0[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
                const float r1[8] = {q2.x, q2.y, q2.z, q2.w, q3.x, q3.y, q3.z, q3.w};
#pragma unroll
                for (int o = 0; o < 8; ++o) c[o] = r0[o] * x0n + r1[o] * x1n;
            } else {
#pragma unroll
                for (int o = 0; o < 8; ++o) c[o] = 0.0f;
            }
            c[8] = x0n * x0n + x1n * x1n;
            const int groups = (cnt * 16 + 31) / 32;
            if (groups == 1) {
                // one tile: every output sits in wave 0 (lane r*M + m: row r, token m).  The rows'
                // values go through LDS and lane o*M + m adds sum o of token m over the 16 rows in
                // row order (16 pipelined reads instead of 9 butterflies of 5 dependent swaps)
                if (tid < 64) {
                    if (tid < 16 * M)
#pragma unroll
                        for (int o = 0; o < 9; ++o) rt_s[(o * 2 * P + e_m) * 16 + e_r] = c[o];
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
                    if (tid < 9 * M) {
                        const int m = tid % M, o = tid / M;
                        const float* rv = rt_s + (o * 2 * P + m) * 16;
                        float t = rv[0];
#pragma unroll
                        for (int r = 1; r < 16; ++r) t = t + rv[r];
                        a.rpart[(size_t)(m * 9 + o) * gridDim.x + blockIdx.x] = t;
                    }
                }
            } else {
                // butterflies over the 32 rows of a token (lanes M apart), through DPP and permlane
                // swaps, then the 32-row groups in order
                if (M == 2) {
#pragma unroll
                    for (int o = 0; o < 9; ++o) c[o] = xor_sum<32>(xor_sum<16>(xor_sum<8>(xor_sum<4>(xor_sum<2>(c[o])))));
                } else {
#pragma unroll
                    for (int o = 0; o < 9; ++o) c[o] = xor_sum<16>(xor_sum<8>(xor_sum<4>(xor_sum<2>(xor_sum<1>(c[o])))));
                }
                if (((tid / M) & 31) == 0 && tid < cnt * 16 * M)
#pragma unroll
                    for (int o = 0; o < 9; ++o) pr_s[(tid / M) >> 5][tid % M][o] = c[o];
                __syncthreads();
                if (tid < 9 * M) {
                    const int m = tid / 9, o = tid - 9 * (tid / 9);
                    float t = 0.0f;
                    for (int gi = 0; gi < groups; ++gi) t = t + pr_s[gi][m][o];
                    a.rpart[(size_t)(m * 9 + o) * gridDim.x + blockIdx.x] = t;
                }
            }
        }
    }
}

using KernelFn = void (*)(GemvArgs, int, int, int, int, int, int, int);

template <int QT, int U, int UPT>
KernelFn pick_fn(int P, int epi, int pro, int il) {
#define SNL_G(E, PR)                                                                   \
    if (epi == E && pro == PR)                                                         \
        return il == 2 ? &mgemv_kernel<QT, 1, E, PR, U, UPT, 2> : &mgemv_kernel<QT, 1, E, PR, U, UPT, 1>;
    if (il == 0) {
        // tile-major (the vocabulary head, the draft's with its final norm): the plain store
        if constexpr (UPT <= 2) {
            if (P == 1 && epi == GEMV_STORE && pro == GEMV_PLAIN) return &mgemv_kernel<QT, 1, GEMV_STORE, GEMV_PLAIN, U, UPT, 0>;
            if (P == 1 && epi == GEMV_STORE && pro == GEMV_NORM) return &mgemv_kernel<QT, 1, GEMV_STORE, GEMV_NORM, U, UPT, 0>;
        }
        if constexpr (UPT == 1)
            if (P == 2 && epi == GEMV_STORE && pro == GEMV_PLAIN) return &mgemv_kernel<QT, 2, GEMV_STORE, GEMV_PLAIN, U, 1, 0>;
        return nullptr;
    }
    if (P == 1) {
        SNL_G(GEMV_STORE, GEMV_PLAIN)
        SNL_G(GEMV_ADD, GEMV_PLAIN)
        SNL_G(GEMV_MHC, GEMV_PLAIN)
        // a normed branch input, the mHC pre-mix of two residual streams of the hidden size and the
        // gated head norm of the DeltaNet output: at most 2 units per staging thread
        if constexpr (UPT <= 2) {
            SNL_G(GEMV_STORE, GEMV_NORM)
            SNL_G(GEMV_ADD, GEMV_NORM)
            SNL_G(GEMV_SWIGLU, GEMV_PLAIN)
            SNL_G(GEMV_SWIGLU, GEMV_NORM)
            SNL_G(GEMV_STORE, GEMV_NORM_MHC)
            SNL_G(GEMV_SWIGLU, GEMV_NORM_MHC)
            SNL_G(GEMV_ADD, GEMV_GNORM)
            SNL_G(GEMV_MHC, GEMV_GNORM)
            SNL_G(GEMV_STORE, GEMV_GNORM)
        }
    }
#undef SNL_G
    // two token pairs: the plain product with at most 2 units per staging thread (kernel-level
    // calls with M = 3, 4)
    if constexpr (UPT <= 2)
        if (P == 2 && epi == GEMV_STORE && pro == GEMV_PLAIN && il == 1)
            return &mgemv_kernel<QT, 2, GEMV_STORE, GEMV_PLAIN, U, UPT, 1>;
    return nullptr;
}

template <int UPT>
KernelFn pick_upt(int quant, int U, int P, int epi, int pro, int il) {
    if (quant == 0) return U == 4 ? pick_fn<0, 4, UPT>(P, epi, pro, il) : pick_fn<0, 1, UPT>(P, epi, pro, il);
    return U == 4 ? pick_fn<1, 4, UPT>(P, epi, pro, il) : pick_fn<1, 1, UPT>(P, epi, pro, il);
}

// UPT: 1 to 3 units per staging thread
KernelFn pick(int quant, int U, int UPT, int P, int epi, int pro, int il) {
    if (UPT == 1) return pick_upt<1>(quant, U, P, epi, pro, il);
    if (UPT == 2) return pick_upt<2>(quant, U, P, epi, pro, il);
    if (UPT == 3) return pick_upt<3>(quant, U, P, epi, pro, il);
    return nullptr;
}

// Reference layout -> packed order: thread i takes the 16-byte piece (T, S, v, lane) i in tile-major
// enumeration and writes it where packing.h places it.
__global__ __launch_bounds__(256) void pack_q_kernel(PackGeom g, const uint8_t* q, uint8_t* qp) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= g.q_bytes / 16) return;
    const int lane = (int)(i & 63);
    size_t r = i >> 6;
    const int v = (int)(r % g.NI);
    r /= g.NI;
    const int S = (int)(r % g.nss), T = (int)(r / g.nss);
    const int row = pack_row(g, T, lane & 15);
    uint4 val = make_uint4(0u, 0u, 0u, 0u);
    if (row >= 0) val = *reinterpret_cast<const uint4*>(q + (size_t)row * g.row_bytes + pack_row_offset(g, S, v, lane >> 4));
    if (g.quant == 0) {  // Q8 in offset binary
        val.x ^= 0x80808080u;
        val.y ^= 0x80808080u;
        val.z ^= 0x80808080u;
        val.w ^= 0x80808080u;
    }
    *reinterpret_cast<uint4*>(qp + pack_piece(g, T, S, v, lane)) = val;
}

__global__ __launch_bounds__(256) void pack_s_kernel(PackGeom g, const float* s, float* sp) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;  // (T, S, lane)
    if (i >= g.s_floats / g.U) return;
    const int lane = (int)(i & 63);
    const size_t r = i >> 6;
    const int S = (int)(r % g.nss), T = (int)(r / g.nss);
    const int row = pack_row(g, T, lane & 15);
    for (int u = 0; u < g.U; ++u)
        sp[pack_scale(g, T, S, lane, u)] =
            row >= 0 ? s[(size_t)row * (g.K / 32) + 4 * g.U * S + g.U * (lane >> 4) + u] : 0.0f;
}

}  // namespace

int launch_pack_matrix(const PackGeom& g, const void* q, const float* s, void* qp, float* sp, hipStream_t st) {
    const size_t nq = g.q_bytes / 16, ns = g.s_floats / g.U;
    hipLaunchKernelGGL(pack_q_kernel, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, st, g,
                       static_cast<const uint8_t*>(q), static_cast<uint8_t*>(qp));
    hipLaunchKernelGGL(pack_s_kernel, dim3((unsigned)((ns + 255) / 256)), dim3(256), 0, st, g, s, sp);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int mgemv_init() {
    for (int q = 0; q < 2; ++q)
        for (int U = 1; U <= 4; U += 3)
            for (int upt = 1; upt <= 3; ++upt)
                for (int P = 1; P <= 2; ++P)
                    for (int e = 0; e < 4; ++e)
                        for (int p = 0; p < 4; ++p)
                            for (int il = 0; il < 3; ++il) {
                                KernelFn f = pick(q, U, upt, P, e, p, il);
                                if (f && hipFuncSetAttribute(reinterpret_cast<const void*>(f),
                                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                                             kLdsLimit) != hipSuccess)
                                    return -2;
                            }
    return 0;
}

namespace {

// Launch shape, from the matrix shape only (the K split is the packing's, packing.h).
struct Shape {
    int KS, base, extra, blocks, waves, nss_w, upt;
    int sw0;           // streaming-only waves (chunk-major); 0: every wave stages and streams
    size_t lds_floor;  // dynamic LDS requested at least (keeps one block per CU)
};

// Chunk-major matrices: at most one block per CU, the same number of tiles in every block but the
// last, one streaming wave per (tile, slice) item and pack_stage_waves(K) staging waves; such a
// block asks for more than half a CU's LDS, so no CU holds two.
// Tile-major (the vocabulary head): short blocks of 2 tiles x KS slices, several per CU
// (measured: 248320 x 4096 Q8_0, 215 us with 1 slice x 8 tiles, 180 us at 4 x 2), at least 8
// waves, every wave staging.  A staging thread takes at most 3 units of 8 elements of a row.
bool mgemv_shape(const PackGeom& g, Shape* sh) {
    int TW;
    const int K8 = g.K / 8;
    if (g.il) {
        // TW tiles per block, the last block the rest: when the tiles do not divide over the CUs,
        // fewer blocks of equal work finish sooner than base / base + 1 (in_proj, 772 tiles: 193
        // blocks of 4, 12.8 instead of 13.2 us; qkv, 640 tiles: 214 of 3)
        const int b0 = g.tiles < kCUs ? g.tiles : kCUs;
        TW = (g.tiles + b0 - 1) / b0;
        sh->blocks = (g.tiles + TW - 1) / TW;
        sh->base = TW;
        sh->extra = 0;
        sh->lds_floor = 84 * 1024;
        sh->sw0 = g.KS * TW;
        sh->waves = sh->sw0 + pack_stage_waves(g.K);
    } else {
        TW = 8 / g.KS;
        sh->base = TW;
        sh->extra = 0;
        sh->blocks = (g.tiles + TW - 1) / TW;
        sh->lds_floor = 0;
        sh->sw0 = 0;
        int waves = g.KS * TW;
        if (waves < 8) waves = 8;
        while (waves < kMaxWaves && waves * 64 < K8) ++waves;  // one unit per thread where that fits
        sh->waves = waves;
    }
    if (sh->waves > kMaxWaves) return false;
    const int nst = (sh->waves - sh->sw0) * 64;
    const int upt = (K8 + nst - 1) / nst;
    if (upt > 3) return false;
    sh->KS = g.KS;
    sh->nss_w = g.nss_w;
    sh->upt = upt;
    return true;
}

// dynamic LDS: token fragments, the zero fragment, the next site's router rows, the multipliers,
// and (NORM_MHC) the staging waves' router partial slots, 9 KiB each
size_t lds_bytes(int M, int K, int U, size_t rrow_bytes, int rin_waves = 0, int quant = 0) {
    const int P = M <= 2 ? 1 : 2;
    const size_t b = (size_t)P * (K / 32) * 256 + kZeroBytes + rrow_bytes + (size_t)P * (K / (128 * U)) * 8;
    const size_t r = rin_waves ? ((b + 15) & ~(size_t)15) + (size_t)rin_waves * 9 * 1024 : b;
    // Q4: the block corrections, 16 bytes per (token pair, block)
    return quant == 1 ? ((r + 15) & ~(size_t)15) + (size_t)P * (K / 32) * 16 : r;
}
}  // namespace

int mgemv_blocks(int quant, int N, int K, int inter) {
    PackGeom g;
    Shape sh;
    if (!pack_geom(quant, N, K, inter, &g) || !mgemv_shape(g, &sh)) return 0;
    return sh.blocks;
}

bool mgemv_fits(int M, int K) {
    PackGeom g;
    Shape sh;
    if (!pack_geom(0, 16, K, 0, &g) || !mgemv_shape(g, &sh)) return false;
    return (M <= 2 || sh.upt <= 2) && lds_bytes(M, K, g.U, 0, 0, 1) <= (size_t)kLdsLimit;
}

// 0: launched; 1: this call is not served (M too large for LDS at this K); < 0 error.
// The weights are in tile order (packing.h) for (N, K, inter when SwiGLU).
int launch_mgemv(const GemvArgs& a, int quant, int M, hipStream_t s) {
    PackGeom g;
    if (!pack_geom(quant, a.N, a.K, a.epi == GEMV_SWIGLU ? a.inter : 0, &g)) return -1;
    Shape sh;
    if (!mgemv_shape(g, &sh)) return 1;
    const int P = M <= 2 ? 1 : 2;
    const int tw_max = sh.base + (sh.extra ? 1 : 0);
    const size_t need = lds_bytes(M, a.K, g.U, a.rpart ? (size_t)tw_max * 16 * M * 64 : 0,
                                  a.pro == GEMV_NORM_MHC ? sh.waves - sh.sw0 : 0, quant);
    if (need > (size_t)kLdsLimit || (P == 2 && sh.upt > 2)) return 1;
    const size_t lds = need > sh.lds_floor ? need : sh.lds_floor;
    if ((reinterpret_cast<uintptr_t>(a.wq) & 15) || (reinterpret_cast<uintptr_t>(a.ws) & 15) ||
        (reinterpret_cast<uintptr_t>(a.x) & 15) || (a.x_stride & 3))
        return -1;
    if (a.pro == GEMV_NORM_MHC && (!a.site_w || !a.raw || !a.coef || !a.rin || a.rin_n < 1 || M > 2)) return -1;
    if (a.pro == GEMV_GNORM && (!a.rin || a.rin_n != kDeltaGroups || a.K % 128)) return -1;
    if (a.norm_out && (a.pro != GEMV_NORM || (reinterpret_cast<uintptr_t>(a.norm_out) & 15) ||
                       (reinterpret_cast<uintptr_t>(a.norm_last) & 15)))
        return -1;
    if (a.epi == GEMV_MHC && !a.coef) return -1;
    if (a.rpart && (!a.next_w || (a.epi != GEMV_ADD && a.epi != GEMV_MHC) || (M & (M - 1)))) return -1;
    if (a.epi == GEMV_ADD && a.rpart && !a.expand) return -1;  // an ADD producer starts the mHC range
    // a chunk-major block of at most 12 waves with more than three chunks per wave streams through
    // the four-chunk ring (same arithmetic, same order)
    KernelFn f = nullptr;
    if (g.il == 1 && sh.waves <= kRing4Waves && sh.nss_w * g.CPS > 3) f = pick(quant, g.U, sh.upt, P, a.epi, a.pro, 2);
    if (!f) f = pick(quant, g.U, sh.upt, P, a.epi, a.pro, g.il);
    if (!f) return 1;
    hipLaunchKernelGGL(f, dim3(sh.blocks), dim3(sh.waves * 64), lds, s, a, M, sh.KS, sh.base, sh.extra, sh.nss_w,
                       g.tiles, sh.sw0);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace snl
