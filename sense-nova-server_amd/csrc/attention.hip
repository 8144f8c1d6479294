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

// attention.wgsl:59-127: block (slot, token); slots [0, nh) queries, then keys, then values.
__global__ __launch_bounds__(256) void prep_kernel(AttnArgs a) {
    __shared__ float sh[HD];
    __shared__ float red[4];
    const int slot = blockIdx.x, m = blockIdx.y, d = threadIdx.x;
    const StepDev* st = a.step;
    const int pos = st->pos0 + m;
    const int q_dim = a.n_heads * HD, kv_dim = a.n_kv * HD;
    const float* row = a.proj + (size_t)m * a.proj_stride;
    if (slot >= a.n_heads + a.n_kv) {
        const int kh = slot - a.n_heads - a.n_kv;
        const float v = row[2 * q_dim + kv_dim + kh * HD + d];
        a.vcache[(size_t)pos * kv_dim + kh * HD + d] = __half_as_ushort(__float2half_rn(v));
        return;
    }
    const bool is_q = slot < a.n_heads;
    float v = is_q ? row[slot * 2 * HD + d] : row[2 * q_dim + (slot - a.n_heads) * HD + d];
    const float total = block_sum<256>(v * v, red);
    v = (v * (1.0f / sqrtf(total / (float)HD + a.eps))) * (1.0f + a.norms[(is_q ? 0 : HD) + d]);
    sh[d] = v;
    __syncthreads();
    const int half = a.rot_dim / 2;
    if (d < a.rot_dim) {
        const int fi = d % half;
        const float inv_freq = powf(a.rope_theta, -(float)(2 * fi) / (float)a.rot_dim);
        const uint32_t* rp = st->rpos[m];
        uint32_t rot_pos = rp[0];
        if (fi % 3 == 1 && (uint32_t)fi < (a.mrope >> 16)) rot_pos = rp[1];
        else if (fi % 3 == 2 && (uint32_t)fi < (a.mrope & 0xFFFFu)) rot_pos = rp[2];
        const float ang = (float)rot_pos * inv_freq;
        const float cs = cosf(ang), sn = sinf(ang);
        v = d < half ? sh[d] * cs - sh[d + half] * sn : sh[d] * cs + sh[d - half] * sn;
    }
    if (is_q) {
        a.qbuf[(size_t)m * q_dim + slot * HD + d] = v;
    } else {
        const int kh = slot - a.n_heads;
        a.kcache[(size_t)pos * kv_dim + kh * HD + d] = __half_as_ushort(__float2half_rn(v));
    }
}

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

// Block (kv head, part of kPart keys) for all M tokens and the 4 query heads of the GQA group
// (NC = 4M head-token combinations).  256 threads = 4 waves.
//  loads:   the queries, then every key of the part, then every value, all in flight at once;
//           rows past the part's last key read zero through the buffer range check;
//  scores:  wave w takes keys [16w, 16w+16) of the part, 4 at a time: 16-lane row r of the wave
//           holds key 4i+r, lane j of the row dims [16j, 16j+16); the 16 lanes of a row are reduced
//           by a transposed butterfly (every combination takes the same shuffle sequence);
//  softmax: exact within the part, 32 threads per combination; keys a token may not see get
//           weight 0;
//  values:  thread (dim pair, key half) accumulates its 32 keys (weight 0 adds nothing).
// Each combination's arithmetic only depends on its own token's keys, so a token's result does
// not depend on M or on its row index.
template <int M>
__global__ __launch_bounds__(256) void attend_kernel(AttnArgs a) {
    constexpr int NC = G * M;
    static_assert(NC == 4 || NC == 8, "M = 1 or 2");
    constexpr int KI = kPart / 16;  // keys per 16-lane row
    constexpr int KH = kPart / 2;   // keys per value thread
    __shared__ __align__(16) float sc[NC][kPart];
    __shared__ float smax[NC], ssum[NC];
    __shared__ float2 vred[NC][128];
    const int kh = blockIdx.x, p = blockIdx.y;
    const StepDev* st = a.step;
    const int pos0 = st->pos0;
    const int kstart = p * kPart;
    const int total_max = pos0 + M;  // keys of the last token
    if (kstart >= total_max) return;
    const int nkeys = min(kPart, total_max - kstart);
    const int q_dim = a.n_heads * HD, kv_dim = a.n_kv * HD;
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane >> 4, j = lane & 15;
    int valid[M];
#pragma unroll
    for (int m = 0; m < M; ++m) valid[m] = min(nkeys, pos0 + m + 1 - kstart);

    // ---- loads: queries, keys, values ----
    float q[NC][16];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const float4* qp = reinterpret_cast<const float4*>(a.qbuf + (size_t)(c / G) * q_dim + (kh * G + c % G) * HD + 16 * j);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float4 t = qp[v];
            q[c][4 * v] = t.x, q[c][4 * v + 1] = t.y, q[c][4 * v + 2] = t.z, q[c][4 * v + 3] = t.w;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // the part's rows of the cache (all kv heads), nkeys of them in range
    const unsigned row_bytes = (unsigned)kv_dim * 2;
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(a.kcache + (size_t)kstart * kv_dim, (unsigned)nkeys * row_bytes);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(a.vcache + (size_t)kstart * kv_dim, (unsigned)nkeys * row_bytes);
    u32x4_t kraw[KI][2];
#pragma unroll
    for (int i = 0; i < KI; ++i) {
        const int t = 16 * w + 4 * i + r;  // key of this 16-lane row
        const int off = t * (int)row_bytes + (kh * HD + 16 * j) * 2;
        kraw[i][0] = __builtin_amdgcn_raw_buffer_load_b128(kr, off, 0, 0);
        kraw[i][1] = __builtin_amdgcn_raw_buffer_load_b128(kr, off + 16, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int dp = tid & 127, kh2 = tid >> 7;
    uint32_t vw[KH];
#pragma unroll
    for (int i = 0; i < KH; ++i) {
        const int t = kh2 * KH + i;
        vw[i] = __builtin_amdgcn_raw_buffer_load_b32(vr, t * (int)row_bytes + (kh * HD + 2 * dp) * 2, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- scores ----
#pragma unroll
    for (int i = 0; i < KI; ++i) {
        const int t = 16 * w + 4 * i + r;
        float kf[16];
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            const u32x4_t raw = kraw[i][v];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                kf[8 * v + 2 * e] = h2f(raw[e] & 0xFFFF);
                kf[8 * v + 2 * e + 1] = h2f(raw[e] >> 16);
            }
        }
        float d[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            float s = q[c][0] * kf[0];
#pragma unroll
            for (int e = 1; e < 16; ++e) s = fmaf(q[c][e], kf[e], s);
            d[c] = s;
        }
        // transposed butterfly over the 16 lanes of the row
        int n = NC;
#pragma unroll
        for (int mask = 8; mask >= 16 / NC && n > 1; mask >>= 1) {
            const bool up = j & mask;
            const int hn = n / 2;
#pragma unroll
            for (int e = 0; e < NC / 2; ++e) {
                if (e < hn) {
                    const float send = up ? d[e] : d[hn + e], keep = up ? d[hn + e] : d[e];
                    d[e] = keep + lane_xor_n(send, mask);
                }
            }
            n = hn;
        }
        float tot = d[0];
#pragma unroll
        for (int mask = 8 / NC; mask > 0; mask >>= 1) tot = tot + lane_xor_n(tot, mask);
        // lane j of the row holds combination j / (16 / NC)
        if ((j & (16 / NC - 1)) == 0) sc[j / (16 / NC)][t] = tot * a.scale;
    }
    lds_barrier();

    // ---- exact softmax over the part, 32 threads per combination ----
    if (tid < 32 * NC) {
        const int c = tid >> 5, l = tid & 31;
        const int vk = valid[c / G];
        const float s0 = l < vk ? sc[c][l] : -FLT_MAX, s1 = l + 32 < vk ? sc[c][l + 32] : -FLT_MAX;
        float mx = fmaxf(s0, s1);
        mx = xor_max<1>(xor_max<2>(xor_max<4>(xor_max<8>(xor_max<16>(mx)))));  // inside each 32-lane half
        const float e0 = l < vk ? expf(s0 - mx) : 0.0f, e1 = l + 32 < vk ? expf(s1 - mx) : 0.0f;
        sc[c][l] = e0;
        sc[c][l + 32] = e1;
        float sum = e0 + e1;
        sum = xor_sum<1>(xor_sum<2>(xor_sum<4>(xor_sum<8>(xor_sum<16>(sum)))));
        if (l == 0) {
            smax[c] = vk > 0 ? mx : -1e30f;
            ssum[c] = sum;
        }
    }
    lds_barrier();

    // ---- values: thread (dim pair dp, key half kh2) ----
    float2 acc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = make_float2(0.0f, 0.0f);
#pragma unroll
    for (int i4 = 0; i4 < KH; i4 += 4) {
        float4 wt[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) wt[c] = *reinterpret_cast<const float4*>(&sc[c][kh2 * KH + i4]);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const float v0 = h2f(vw[i4 + ii] & 0xFFFF), v1 = h2f(vw[i4 + ii] >> 16);
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const float wv = ii == 0 ? wt[c].x : ii == 1 ? wt[c].y : ii == 2 ? wt[c].z : wt[c].w;
                acc[c].x = fmaf(wv, v0, acc[c].x);
                acc[c].y = fmaf(wv, v1, acc[c].y);
            }
        }
    }
    if (kh2 == 1)
#pragma unroll
        for (int c = 0; c < NC; ++c) vred[c][dp] = acc[c];
    __syncthreads();
    if (kh2 == 0) {
        const int parts_max = (a.ctx + kPart - 1) / kPart;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int m = c / G, hh = kh * G + c % G;
            float* o = a.partial + (((size_t)m * a.n_heads + hh) * parts_max + p) * (HD + 2);
            const float2 u = vred[c][dp];
            o[2 * dp] = acc[c].x + u.x;
            o[2 * dp + 1] = acc[c].y + u.y;
            if (dp == 0) {
                o[HD] = smax[c];
                o[HD + 1] = ssum[c];
            }
        }
    }
}

// attention.wgsl:248-269: merge the token's parts, then the sigmoid gate.  Block (head, token, 64
// dims) of 1024 threads: every part's scale e^(max_p - max) goes to LDS once, then thread (d, q)
// adds the parts q, q+16, ... of dim d and the 16 groups are added in order.  Many short chains
// keep a long context's partials (512 parts at 32K keys) in flight at once.
constexpr int kCombThreads = 1024, kCombDims = 64, kCombGroups = kCombThreads / kCombDims, kMaxParts = 1024;

__global__ __launch_bounds__(kCombThreads) void combine_kernel(AttnArgs a) {
    __shared__ float fs[kMaxParts];
    __shared__ float red[kCombThreads / 64];
    __shared__ float accq[kCombGroups][kCombDims];
    const int h = blockIdx.x, m = blockIdx.y, tid = threadIdx.x;
    const int dl = tid & (kCombDims - 1), q = tid / kCombDims;
    const int d = blockIdx.z * kCombDims + dl;
    const int total = a.step->pos0 + m + 1;
    const int np = (total + kPart - 1) / kPart;
    const int parts_max = (a.ctx + kPart - 1) / kPart;
    const float* base = a.partial + ((size_t)m * a.n_heads + h) * parts_max * (HD + 2);
    // global max of the part maxima (np <= kMaxParts = kCombThreads: one part per thread)
    const float mp = tid < np ? base[(size_t)tid * (HD + 2) + HD] : -1e30f;
    const float lp = tid < np ? base[(size_t)tid * (HD + 2) + HD + 1] : 0.0f;
    float mx = wave_max(mp);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < kCombThreads / 64; ++w) mx = fmaxf(mx, red[w]);
    __syncthreads();
    const float f = tid < np ? expf(mp - mx) : 0.0f;
    if (tid < np) fs[tid] = f;
    const float l = block_sum<kCombThreads>(lp * f, red);  // the sum of the parts' weights
    float acc = 0.0f;
#pragma unroll 8
    for (int p = q; p < np; p += kCombGroups) acc = acc + base[(size_t)p * (HD + 2) + d] * fs[p];
    accq[q][dl] = acc;
    __syncthreads();
    if (q == 0) {
        float v = accq[0][dl];
#pragma unroll
        for (int g = 1; g < kCombGroups; ++g) v = v + accq[g][dl];
        const float gate = a.proj[(size_t)m * a.proj_stride + h * 2 * HD + HD + d];
        a.out[(size_t)m * a.n_heads * HD + h * HD + d] = v / l / (1.0f + expf(-gate));
    }
}

}  // namespace

int launch_attention(const AttnArgs& a, int M, hipStream_t s) {
    if (M < 1 || M > 2 || a.n_heads != G * a.n_kv || a.rot_dim > HD || a.rot_dim % 2) return -1;
    if ((a.ctx + kPart - 1) / kPart > kMaxParts) return -1;
    hipLaunchKernelGGL(prep_kernel, dim3(a.n_heads + 2 * a.n_kv, M), dim3(256), 0, s, a);
    const int parts_max = (a.ctx + kPart - 1) / kPart;
    dim3 grid(a.n_kv, parts_max);
    switch (M) {
        case 1: hipLaunchKernelGGL(attend_kernel<1>, grid, dim3(256), 0, s, a); break;
        case 2: hipLaunchKernelGGL(attend_kernel<2>, grid, dim3(256), 0, s, a); break;
        default: return -1;
    }
    hipLaunchKernelGGL(combine_kernel, dim3(a.n_heads, M, HD / kCombDims), dim3(kCombThreads), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace snl
