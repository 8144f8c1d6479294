// Gated GQA decode attention with partial rotate-half RoPE over the f16 KV cache
// (src/shaders/attention.wgsl: prep :59-127, attend :129-246, combine :248-269).
//
// Keys are split into fixed 64-key parts at absolute positions: part p covers keys
// [64p, 64p+64).  A token with `total` keys uses parts 0..ceil(total/64)-1, so its
// partition depends only on its own position, never on how many tokens share the call
// (the reference sizes its split from the whole step, src/engine.rs:827).  One block per
// (kv head, part) serves all M tokens and all 4 query heads of the GQA group, so each K/V
// byte is read once per call.  Each part writes (acc[256], max, sum) per (token, head);
// `combine` merges the parts in ascending order and applies the sigmoid output gate.
#include <float.h>
#include <hip/hip_fp16.h>

#include "common.h"
#include "kernels.h"

#pragma clang fp contract(off)

namespace snl {

namespace {

constexpr int HD = 256, G = 4, kPart = 64;

__device__ __forceinline__ float h2f(uint32_t b) { return __half2float(__ushort_as_half((uint16_t)b)); }

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// Block barrier that orders LDS only (vector memory loads stay in flight across it).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Raw buffer descriptor over [base, base + bytes): a load past `bytes` reads zero and touches no
// memory.  Word 3 is the gfx9 raw (untyped) dword format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));

// attention.wgsl:59-127 once per KV head, for contexts past kSplitPrepCtx: block kv head, thread d
// holds dim d of the group's 4 query rows and of this call's new key and value rows, per token.
// RMSNorm (1 + w), then rotate-half RoPE on the first rot_dim dims: the rotated queries go to qbuf,
// the new keys and values to the f16 cache.  The same operations as the fused prep of
// attend_kernel, so either path gives the same bits.
constexpr int kSplitPrepCtx = 8192;

template <int M>
__global__ __launch_bounds__(256) void prep_kernel(AttnArgs a) {
    constexpr int NS = G * M + M;
    __shared__ float qs[G * M][HD], ks[M][HD];
    __shared__ float red[4][NS];
    const int kh = blockIdx.x, d = threadIdx.x, lane = d & 63, w = d >> 6;
    const StepDev* st = a.step;
    const int q_dim = a.n_heads * HD, kv_dim = a.n_kv * HD;
    float qv0[G][M], kr0[M], vr0[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float* row = a.proj + (size_t)m * a.proj_stride;
#pragma unroll
        for (int j = 0; j < G; ++j) qv0[j][m] = row[(kh * G + j) * 2 * HD + d];
        kr0[m] = row[2 * q_dim + kh * HD + d];
        vr0[m] = row[2 * q_dim + kv_dim + kh * HD + d];
    }
    const float nq = a.norms[d], nk = a.norms[HD + d];
    const int half = a.rot_dim / 2;
    float rcs[M], rsn[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float2 rt = *reinterpret_cast<const float2*>(st->rope[m][half > 0 ? d % half : 0]);
        rcs[m] = d < a.rot_dim ? rt.x : 1.0f;
        rsn[m] = d < a.rot_dim ? rt.y : 0.0f;
    }
    const int pos0 = st->pos0;
    float ss[NS];
#pragma unroll
    for (int m = 0; m < M; ++m) {
#pragma unroll
        for (int j = 0; j < G; ++j) ss[j * M + m] = qv0[j][m] * qv0[j][m];
        ss[G * M + m] = kr0[m] * kr0[m];
    }
    wave_sum_n(ss);
    if (lane == 0)
#pragma unroll
        for (int i = 0; i < NS; ++i) red[w][i] = ss[i];
    __syncthreads();
#pragma unroll
    for (int m = 0; m < M; ++m) {
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const int i = j * M + m;
            const float total = (((0.0f + red[0][i]) + red[1][i]) + red[2][i]) + red[3][i];
            qs[i][d] = (qv0[j][m] * (1.0f / sqrtf(total / (float)HD + a.eps))) * (1.0f + nq);
        }
        const int i = G * M + m;
        const float total = (((0.0f + red[0][i]) + red[1][i]) + red[2][i]) + red[3][i];
        ks[m][d] = (kr0[m] * (1.0f / sqrtf(total / (float)HD + a.eps))) * (1.0f + nk);
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float cs = rcs[m], sn = rsn[m];
        auto rot = [&](const float* v) {
            if (d >= a.rot_dim) return v[d];
            return d < half ? v[d] * cs - v[d + half] * sn : v[d] * cs + v[d - half] * sn;
        };
#pragma unroll
        for (int j = 0; j < G; ++j) a.qbuf[(size_t)m * q_dim + (kh * G + j) * HD + d] = rot(qs[j * M + m]);
        const size_t c = (size_t)(pos0 + m) * kv_dim + kh * HD + d;
        a.kcache[c] = __builtin_bit_cast(uint16_t, (_Float16)rot(ks[m]));
        a.vcache[c] = __builtin_bit_cast(uint16_t, (_Float16)vr0[m]);
    }
}

// Block (kv head, part of kPart keys) for all M tokens and the 4 query heads of the GQA group,
// 256 threads = 4 waves, on v_mfma_f32_16x16x32_f16.  The 16 MFMA columns hold the head-token
// combinations: token m's 4 heads take columns 4 * ((pos0 + m) & 1) + head, so a token sits in the
// same columns whether it is decoded alone or in a pair, and its arithmetic never depends on M
// (the other columns are zero).
//  scores:  S^T = K Q^T: wave w takes keys [16w, 16w+16) of the part as the A operand (16 keys x
//           32 dims, exact f16 straight from the cache; rows past the part's last key read zero
//           through the buffer range check); B = the queries as f16 hi + lo under a per-column
//           power of two, so a score keeps the query's f32 precision;
//  softmax: exact within the part per combination (32 threads each); keys a token may not see
//           get weight 0;
//  values:  O^T = V^T P^T: the part's values pass through LDS (64 keys x 256 dims, f16, rows past
//           the last key zero) and each lane gathers the 8 keys of its A fragment for one dim;
//           B = the probabilities as f16 hi + lo; wave w takes dims [64w, 64w+64).
//
// FUSED: the block also forms its queries and this call's new keys (norms, RoPE: prep above) and
// writes the new cache rows, which suits short contexts where the key parts are few.  Otherwise
// (contexts past kSplitPrepCtx, hundreds of parts) prep_kernel has done that once per KV head and
// the block reads the rotated queries from qbuf and every key from the cache; the results are
// bitwise the same.
template <int M, bool FUSED>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void attend_kernel(AttnArgs a) {
    constexpr int NC = G * M;
    static_assert(NC == 4 || NC == 8, "M = 1 or 2");
    constexpr int VROW = HD + 16;  // V tile row in halfs (544 bytes: a transposed read's 4 rows on distinct banks)
    constexpr int NS = G * M + M;  // sums of squares: the group's queries (head, token), the new keys
    __shared__ __align__(16) _Float16 vt[kPart * VROW];
    __shared__ __align__(16) float sc[16][kPart];  // by MFMA column
    __shared__ float smax[16], ssum[16];
    __shared__ float red[4][NS];
    __shared__ __align__(16) _Float16 knew[M][HD], vnew[M][HD];  // this part's new keys (normed, rotated) and values
    // before the value tile is written, its space holds the queries and new keys: normed, then rotated
    float* const qs = reinterpret_cast<float*>(vt);  // [G * M][HD]
    float* const qr = qs + G * M * HD;               // [G * M][HD]
    float* const ks = qr + G * M * HD;               // [M][HD]
    static_assert((2 * G * M + M) * HD * 4 <= kPart * VROW * 2, "prep staging fits the value tile");
    const int kh = blockIdx.x, p = blockIdx.y;
    const StepDev* st = a.step;
    const int q_dim = a.n_heads * HD, kv_dim = a.n_kv * HD;
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    // ---- loads that do not need the position go out first: the position is a scalar load that
    // depends on another (the step record's address), and nothing else waits behind it ----
    // attention.wgsl:59-127 for the group's 4 query heads and this call's new key / value rows:
    // thread d holds dim d of each row
    const int d = tid;
    float qv0[G][M], kr0[M], vr0[M];
    float nq = 0.0f, nk = 0.0f;
    const int half = a.rot_dim / 2;
    float2 rt[M];
    if constexpr (FUSED) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float* row = a.proj + (size_t)m * a.proj_stride;
#pragma unroll
            for (int j = 0; j < G; ++j) qv0[j][m] = row[(kh * G + j) * 2 * HD + d];
            kr0[m] = row[2 * q_dim + kh * HD + d];
            vr0[m] = row[2 * q_dim + kv_dim + kh * HD + d];
        }
        nq = a.norms[d], nk = a.norms[HD + d];
        // the rotary cos / sin of this dim's frequency for each token, formed on the host (every
        // dim reads an entry; the dims past rot_dim drop it below)
#pragma unroll
        for (int m = 0; m < M; ++m) rt[m] = *reinterpret_cast<const float2*>(st->rope[m][half > 0 ? d % half : 0]);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int pos0 = st->pos0;
    const int kstart = p * kPart;
    const int total_max = pos0 + M;  // keys of the last token
    if (kstart >= total_max) return;
    const int nkeys = min(kPart, total_max - kstart);
    const int n = lane & 15, g = lane >> 4;  // MFMA column (combination) and k-group of this lane
    int cm = -1;                             // the token of column n, if any
#pragma unroll
    for (int m = 0; m < M; ++m)
        if ((n >> 2) == ((pos0 + m) & 1)) cm = m;
    const int chh = n & 3;  // its head in the group
    bool mine[M];           // token m's own key and value fall in this part
#pragma unroll
    for (int m = 0; m < M; ++m) mine[m] = pos0 + m >= kstart && pos0 + m < kstart + kPart;

    // ---- then the part's values (for the LDS tile) and this wave's keys, straight from the cache
    // (FUSED: the rows of this call's positions patch them below) ----
    const unsigned row_bytes = (unsigned)kv_dim * 2;
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(a.kcache + (size_t)kstart * kv_dim, (unsigned)nkeys * row_bytes);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(a.vcache + (size_t)kstart * kv_dim, (unsigned)nkeys * row_bytes);
    // not FUSED: the group's rotated queries first (vector loads complete in issue order, so they
    // are not waited for behind the keys and values), thread d taking dim d of each row, once per
    // block; they reach the lanes' fragments through LDS
    float qd[G][M];
    if constexpr (!FUSED) {
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int j = 0; j < G; ++j) qd[j][m] = a.qbuf[(size_t)m * q_dim + (kh * G + j) * HD + d];
    }
    // FUSED: (vector loads complete in issue order, so the waits for this call's rows do not
    // include the cache loads; issued first, they held the row prep back ~1 us)
    u32x4_t vv[kPart / 8];
    u32x4_t kf[HD / 32];
    if constexpr (FUSED) {
#pragma unroll
        for (int i = 0; i < kPart / 8; ++i)  // thread: keys tid / 32 + 8i, 16-byte segment tid % 32
            vv[i] = __builtin_amdgcn_raw_buffer_load_b128(vr, ((tid >> 5) + 8 * i) * (int)row_bytes + kh * HD * 2 + (tid & 31) * 16, 0, 0);
#pragma unroll
        for (int s = 0; s < HD / 32; ++s)  // key 16w + n, dims 32s + 8g .. + 7
            kf[s] = __builtin_amdgcn_raw_buffer_load_b128(kr, (16 * w + n) * (int)row_bytes + (kh * HD + 32 * s + 8 * g) * 2, 0, 0);
    } else {
#pragma unroll
        for (int s = 0; s < HD / 32; ++s)
            kf[s] = __builtin_amdgcn_raw_buffer_load_b128(kr, (16 * w + n) * (int)row_bytes + (kh * HD + 32 * s + 8 * g) * 2, 0, 0);
#pragma unroll
        for (int i = 0; i < kPart / 8; ++i)
            vv[i] = __builtin_amdgcn_raw_buffer_load_b128(vr, ((tid >> 5) + 8 * i) * (int)row_bytes + kh * HD * 2 + (tid & 31) * 16, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    float qv[HD / 32][8];
    float amax = 0.0f;
    if constexpr (FUSED) {
        // this call's key / value rows where they fall in this part, zeros elsewhere
        float kv0[M], vv0[M], rcs[M], rsn[M];
#pragma unroll
        for (int m = 0; m < M; ++m) {
            kv0[m] = mine[m] ? kr0[m] : 0.0f;
            vv0[m] = mine[m] ? vr0[m] : 0.0f;
            rcs[m] = d < a.rot_dim ? rt[m].x : 1.0f;
            rsn[m] = d < a.rot_dim ? rt[m].y : 0.0f;
        }
        // RMSNorm (1 + w) over each row's 256 dims: wave sums, then the 4 waves in order
        float ss[NS];
#pragma unroll
        for (int m = 0; m < M; ++m) {
#pragma unroll
            for (int j = 0; j < G; ++j) ss[j * M + m] = qv0[j][m] * qv0[j][m];
            ss[G * M + m] = kv0[m] * kv0[m];
        }
        wave_sum_n(ss);
        if (lane == 0)
#pragma unroll
            for (int i = 0; i < NS; ++i) red[w][i] = ss[i];
        __syncthreads();
#pragma unroll
        for (int m = 0; m < M; ++m) {
#pragma unroll
            for (int j = 0; j < G; ++j) {
                const int i = j * M + m;
                const float total = (((0.0f + red[0][i]) + red[1][i]) + red[2][i]) + red[3][i];
                qs[i * HD + d] = (qv0[j][m] * (1.0f / sqrtf(total / (float)HD + a.eps))) * (1.0f + nq);
            }
            if (mine[m]) {
                const int i = G * M + m;
                const float total = (((0.0f + red[0][i]) + red[1][i]) + red[2][i]) + red[3][i];
                ks[m * HD + d] = (kv0[m] * (1.0f / sqrtf(total / (float)HD + a.eps))) * (1.0f + nk);
            }
        }
        __syncthreads();
        // rotate-half RoPE on the first rot_dim dims; the new keys and values go to the cache
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float cs = rcs[m], sn = rsn[m];
            auto rot = [&](const float* v) {
                if (d >= a.rot_dim) return v[d];
                return d < half ? v[d] * cs - v[d + half] * sn : v[d] * cs + v[d - half] * sn;
            };
#pragma unroll
            for (int j = 0; j < G; ++j) {
                const float q = rot(qs + (j * M + m) * HD);
                qr[(j * M + m) * HD + d] = q;
                if (p == 0) a.qbuf[(size_t)m * q_dim + (kh * G + j) * HD + d] = q;
            }
            if (mine[m]) {
                const _Float16 kq = (_Float16)rot(ks + m * HD), vq = (_Float16)vv0[m];
                knew[m][d] = kq;
                vnew[m][d] = vq;
                const size_t c = (size_t)(pos0 + m) * kv_dim + kh * HD + d;
                a.kcache[c] = __builtin_bit_cast(uint16_t, kq);
                a.vcache[c] = __builtin_bit_cast(uint16_t, vq);
            }
        }
        __syncthreads();
        // the query fragments: lane (column n, k-group g) takes dims 32s + 8g .. + 7 of its column
#pragma unroll
        for (int s = 0; s < HD / 32; ++s) {
            float4 u0 = make_float4(0.f, 0.f, 0.f, 0.f), u1 = u0;
            if (cm >= 0) {
                const float4* qp = reinterpret_cast<const float4*>(qr + (chh * M + cm) * HD + 32 * s + 8 * g);
                u0 = qp[0];
                u1 = qp[1];
            }
            qv[s][0] = u0.x, qv[s][1] = u0.y, qv[s][2] = u0.z, qv[s][3] = u0.w;
            qv[s][4] = u1.x, qv[s][5] = u1.y, qv[s][6] = u1.z, qv[s][7] = u1.w;
#pragma unroll
            for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(qv[s][e]));
        }
        // the key rows of this call's positions come from knew, not from the cache loads above
#pragma unroll
        for (int m = 0; m < M; ++m)
            if (mine[m] && kstart + 16 * w + n == pos0 + m)
#pragma unroll
                for (int s = 0; s < HD / 32; ++s) kf[s] = *reinterpret_cast<const u32x4_t*>(&knew[m][32 * s + 8 * g]);
    } else {
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int j = 0; j < G; ++j) qr[(j * M + m) * HD + d] = qd[j][m];
        lds_barrier();
#pragma unroll
        for (int s = 0; s < HD / 32; ++s) {
            float4 u0 = make_float4(0.f, 0.f, 0.f, 0.f), u1 = u0;
            if (cm >= 0) {
                const float4* qp = reinterpret_cast<const float4*>(qr + (chh * M + cm) * HD + 32 * s + 8 * g);
                u0 = qp[0];
                u1 = qp[1];
            }
            qv[s][0] = u0.x, qv[s][1] = u0.y, qv[s][2] = u0.z, qv[s][3] = u0.w;
            qv[s][4] = u1.x, qv[s][5] = u1.y, qv[s][6] = u1.z, qv[s][7] = u1.w;
#pragma unroll
            for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(qv[s][e]));
        }
    }
    amax = xor_max<32>(xor_max<16>(amax));  // the 4 lanes of column n
    const int ex = amax > 0.0f ? max(ilogbf(amax) - 14, -110) : 0;
    const float down = ldexpf(1.0f, -ex), up = ldexpf(1.0f, ex) * a.scale;
    half8_t qh[HD / 32], ql[HD / 32];
#pragma unroll
    for (int s = 0; s < HD / 32; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float v = qv[s][e] * down;
            const _Float16 hv = (_Float16)v;
            qh[s][e] = hv;
            ql[s][e] = (_Float16)(v - (float)hv);
        }
    __syncthreads();  // the staging above is read: the value tile may now take its space
#pragma unroll
    for (int i = 0; i < kPart / 8; ++i) {
        const int r = (tid >> 5) + 8 * i;
        u32x4_t val = vv[i];
        if constexpr (FUSED)
#pragma unroll
            for (int m = 0; m < M; ++m)
                if (mine[m] && kstart + r == pos0 + m) val = *reinterpret_cast<const u32x4_t*>(&vnew[m][(tid & 31) * 8]);
        *reinterpret_cast<u32x4_t*>(vt + r * VROW + (tid & 31) * 8) = val;
    }

    // ---- scores: lane (column n, k-group g) ends with keys 16w + 4g + r ----
    f32x4_t c = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < HD / 32; ++s) {
        const half8_t kfr = __builtin_bit_cast(half8_t, kf[s]);
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kfr, qh[s], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kfr, ql[s], c, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[n][16 * w + 4 * g + r] = c[r] * up;
    lds_barrier();

    // ---- exact softmax over the part, 32 threads per combination ----
    if (tid < 32 * NC) {
        const int cc = tid >> 5, l = tid & 31;
        const int m = cc / G, col = 4 * ((pos0 + m) & 1) + cc % G;
        const int vk = min(nkeys, pos0 + m + 1 - kstart);
        const float s0 = l < vk ? sc[col][l] : -FLT_MAX, s1 = l + 32 < vk ? sc[col][l + 32] : -FLT_MAX;
        float mx = fmaxf(s0, s1);
        mx = xor_max<1>(xor_max<2>(xor_max<4>(xor_max<8>(xor_max<16>(mx)))));  // inside each 32-lane half
        const float e0 = l < vk ? expf(s0 - mx) : 0.0f, e1 = l + 32 < vk ? expf(s1 - mx) : 0.0f;
        sc[col][l] = e0;
        sc[col][l + 32] = e1;
        float sum = e0 + e1;
        sum = xor_sum<1>(xor_sum<2>(xor_sum<4>(xor_sum<8>(xor_sum<16>(sum)))));
        if (l == 0) {
            smax[col] = vk > 0 ? mx : -1e30f;
            ssum[col] = sum;
        }
    }
    lds_barrier();

    // ---- values: lane (column n, k-group g) ends with dims 64w + 16dt + 4g + r ----
    f32x4_t o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < kPart / 32; ++ks) {
        half8_t ph, pl;
        const float4 pa = *reinterpret_cast<const float4*>(&sc[n][32 * ks + 8 * g]);
        const float4 pb = *reinterpret_cast<const float4*>(&sc[n][32 * ks + 8 * g + 4]);
        const float pv[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const _Float16 hv = (_Float16)pv[e];
            ph[e] = hv;
            pl[e] = (_Float16)(pv[e] - (float)hv);
        }
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            // transposed reads (ds_read_b64_tr_b16): in each 16-lane group, lane 4a + b receives
            // element b of the 8 bytes addressed by lanes a, a + 4, a + 8, a + 12; lane s
            // addresses key 32ks + 8g + s / 4 (then + 4), dims 64w + 16dt + 4 (s % 4), so lane n
            // receives dim 64w + 16dt + n of its 8 keys
            const _Float16* vp = vt + (32 * ks + 8 * g + (n >> 2)) * VROW + 64 * w + 16 * dt + 4 * (n & 3);
            const short4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t*)(vp));
            const short4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t*)(vp + 4 * VROW));
            const half8_t va = __builtin_bit_cast(half8_t, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, ph, o[dt], 0, 0, 0);
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl, o[dt], 0, 0, 0);
        }
    }
    if (cm >= 0) {
        const int parts_max = (a.ctx + kPart - 1) / kPart;
        float* out = a.partial + (((size_t)cm * a.n_heads + kh * G + chh) * parts_max + p) * (HD + 2);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r) out[64 * w + 16 * dt + 4 * g + r] = o[dt][r];
        if (w == 0 && g == 0) {
            out[HD] = smax[n];
            out[HD + 1] = ssum[n];
        }
    }
}

// attention.wgsl:248-269: merge the token's parts, then the sigmoid gate.  Block (head, token, 32
// dims) of 512 threads: every part's scale e^(max_p - max) goes to LDS once, then thread (d, q)
// adds the parts q, q+16, ... of dim d and the 16 groups are added in order.  Many short chains
// keep a long context's partials (512 parts at 32K keys) in flight at once.  Past 512 parts
// (32K keys) thread t also takes the parts t + 512, t + 1024, ... for the maximum and the weights;
// the order of every sum depends on the token's part count alone.
constexpr int kCombThreads = 512, kCombDims = 32, kCombGroups = kCombThreads / kCombDims;

__global__ __launch_bounds__(kCombThreads) void combine_kernel(AttnArgs a) {
    __shared__ float fs[kAttnMaxParts];
    __shared__ float red[kCombThreads / 64];
    __shared__ float accq[kCombGroups][kCombDims];
    const int h = blockIdx.x, m = blockIdx.y, tid = threadIdx.x;
    const int dl = tid & (kCombDims - 1), q = tid / kCombDims;
    const int d = blockIdx.z * kCombDims + dl;
    const int parts_max = (a.ctx + kPart - 1) / kPart;
    const float* base = a.partial + ((size_t)m * a.n_heads + h) * parts_max * (HD + 2);
    // Every load that does not need the key count goes out first, in one round trip: the part
    // maxima and weights and this thread's first partial value (all inside the parts_max rows of
    // the buffer; parts past the count are masked below) and the output gate.
    const float mp0 = tid < parts_max ? base[(size_t)tid * (HD + 2) + HD] : -1e30f;
    const float lp0 = tid < parts_max ? base[(size_t)tid * (HD + 2) + HD + 1] : 0.0f;
    const float pv0 = q < parts_max ? base[(size_t)q * (HD + 2) + d] : 0.0f;
    const float gate = q == 0 ? a.proj[(size_t)m * a.proj_stride + h * 2 * HD + HD + d] : 0.0f;
    const int total = a.step->pos0 + m + 1;
    const int np = (total + kPart - 1) / kPart;
    // global max of the part maxima
    float mx = tid < np ? mp0 : -1e30f;
    for (int p = tid + kCombThreads; p < np; p += kCombThreads) mx = fmaxf(mx, base[(size_t)p * (HD + 2) + HD]);
    mx = wave_max(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < kCombThreads / 64; ++w) mx = fmaxf(mx, red[w]);
    __syncthreads();
    float lsum = 0.0f;
    if (tid < np) {
        const float f = expf(mp0 - mx);
        fs[tid] = f;
        lsum = lp0 * f;
    }
    for (int p = tid + kCombThreads; p < np; p += kCombThreads) {
        const float f = expf(base[(size_t)p * (HD + 2) + HD] - mx);
        fs[p] = f;
        lsum = lsum + base[(size_t)p * (HD + 2) + HD + 1] * f;
    }
    const float l = block_sum<kCombThreads>(lsum, red);  // the sum of the parts' weights
    float acc = 0.0f;
    if (q < np) acc = acc + pv0 * fs[q];
#pragma unroll 8
    for (int p = q + kCombGroups; p < np; p += kCombGroups) acc = acc + base[(size_t)p * (HD + 2) + d] * fs[p];
    accq[q][dl] = acc;
    __syncthreads();
    if (q == 0) {
        float v = accq[0][dl];
#pragma unroll
        for (int g = 1; g < kCombGroups; ++g) v = v + accq[g][dl];
        a.out[(size_t)m * a.n_heads * HD + h * HD + d] = v / l / (1.0f + expf(-gate));
    }
}

}  // namespace

int launch_attention(const AttnArgs& a, int M, hipStream_t s) {
    if (M < 1 || M > 2 || a.n_heads != G * a.n_kv || a.rot_dim > HD || a.rot_dim % 2) return -1;
    if (a.ctx > kMaxCtx) return -1;
    const int parts_max = (a.ctx + kPart - 1) / kPart;
    dim3 grid(a.n_kv, parts_max);
    // the context the engine was sized for (not the position) picks the path, so a captured pass
    // keeps one launch sequence
    const bool split = a.ctx > kSplitPrepCtx;
    if (split) {
        if (M == 1) hipLaunchKernelGGL(prep_kernel<1>, dim3(a.n_kv), dim3(256), 0, s, a);
        else hipLaunchKernelGGL(prep_kernel<2>, dim3(a.n_kv), dim3(256), 0, s, a);
    }
    if (M == 1) {
        if (split) hipLaunchKernelGGL((attend_kernel<1, false>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((attend_kernel<1, true>), grid, dim3(256), 0, s, a);
    } else {
        if (split) hipLaunchKernelGGL((attend_kernel<2, false>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((attend_kernel<2, true>), grid, dim3(256), 0, s, a);
    }
    hipLaunchKernelGGL(combine_kernel, dim3(a.n_heads, M, HD / kCombDims), dim3(kCombThreads), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace snl
