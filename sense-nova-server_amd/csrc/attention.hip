// Gated GQA decode attention with partial rotate-half RoPE over the f16 KV cache
// (src/shaders/attention.wgsl: prep :59-127, attend :129-246, combine :248-269).
//
// Keys are split into fixed 128-key parts at absolute positions: part p covers keys
// [128p, 128p+128).  A token with `total` keys uses parts 0..ceil(total/128)-1, so its
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

constexpr int HD = 256, G = 4, kPart = 128;

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

__device__ __forceinline__ float h2f(uint16_t b) { return __half2float(__ushort_as_half(b)); }

// Transposed butterfly: v[NV] per lane -> lane L returns the 64-lane sum of value L >> (6 - log2 NV).
template <int NV>
__device__ __forceinline__ float tsum(float (&v)[NV], int lane) {
    int n = NV;
#pragma unroll
    for (int mask = 32; mask >= 64 / NV && n > 1; mask >>= 1) {
        const bool up = lane & mask;
        const int hn = n / 2;
#pragma unroll
        for (int i = 0; i < NV / 2; ++i) {
            if (i < hn) {
                const float send = up ? v[i] : v[hn + i], keep = up ? v[hn + i] : v[i];
                v[i] = keep + __shfl_xor(send, mask, 64);
            }
        }
        n = hn;
    }
    float r = v[0];
#pragma unroll
    for (int mask = 32 / NV; mask > 0; mask >>= 1) r = r + __shfl_xor(r, mask, 64);
    return r;
}

// Block (kv head, part): scores for all M tokens x 4 heads over the part's keys, exact softmax
// inside the part, then the value sum.  256 threads = 4 waves; wave w scores keys
// [32w, 32w+32) of the part; lane l holds dims [4l, 4l+4).
template <int M>
__global__ __launch_bounds__(256) void attend_kernel(AttnArgs a) {
    constexpr int NC = G * M;  // (head, token) combinations
    __shared__ float sc[NC][kPart];
    __shared__ float smax[NC], ssum[NC];
    const int kh = blockIdx.x, p = blockIdx.y;
    const StepDev* st = a.step;
    const int pos0 = st->pos0;
    const int kstart = p * kPart;
    const int total_max = pos0 + M;  // keys of the last token
    if (kstart >= total_max) return;
    const int nkeys = min(kPart, total_max - kstart);
    const int q_dim = a.n_heads * HD, kv_dim = a.n_kv * HD;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;

    float q[NC][4];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int g = c % G, m = c / G;
        const float4 t = *reinterpret_cast<const float4*>(a.qbuf + (size_t)m * q_dim + (kh * G + g) * HD + 4 * lane);
        q[c][0] = t.x, q[c][1] = t.y, q[c][2] = t.z, q[c][3] = t.w;
    }
    // 16 keys at a time; each (head, token) combination is reduced by its own 16-value
    // butterfly, so a score's summation order never depends on M.
    const uint16_t* kbase = a.kcache + (size_t)kh * HD + 4 * lane;
#pragma unroll 1
    for (int k0 = w * 32; k0 < w * 32 + 32; k0 += 16) {
        if (k0 >= nkeys) break;
        float v[NC][16];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            float kf[4] = {0.f, 0.f, 0.f, 0.f};
            if (k0 + t < nkeys) {
                const uint2 raw = *reinterpret_cast<const uint2*>(kbase + (size_t)(kstart + k0 + t) * kv_dim);
                kf[0] = h2f(raw.x & 0xFFFF), kf[1] = h2f(raw.x >> 16), kf[2] = h2f(raw.y & 0xFFFF),
                kf[3] = h2f(raw.y >> 16);
            }
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                float d = q[c][0] * kf[0];
                d = fmaf(q[c][1], kf[1], d);
                d = fmaf(q[c][2], kf[2], d);
                d = fmaf(q[c][3], kf[3], d);
                v[c][t] = d;
            }
        }
        const int t = lane >> 2;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const float r = tsum<16>(v[c], lane);  // lane L holds key L >> 2
            if ((lane & 3) == 0 && k0 + t < nkeys) sc[c][k0 + t] = r * a.scale;
        }
    }
    __syncthreads();
    // exact softmax over the part, per (head, token); token m sees keys < pos0 + m + 1
    if (w == 0) {
        for (int c = 0; c < NC; ++c) {
            const int m = c / G;
            const int valid = min(nkeys, pos0 + m + 1 - kstart);
            float mx = -FLT_MAX;
            for (int t = lane; t < valid; t += 64) mx = fmaxf(mx, sc[c][t]);
            mx = wave_max(mx);
            float sum = 0.0f;
            for (int t = lane; t < kPart; t += 64) {
                float e = 0.0f;
                if (t < valid) e = expf(sc[c][t] - mx);
                sc[c][t] = e;
                sum += e;
            }
            sum = wave_sum(sum);
            if (lane == 0) {
                smax[c] = valid > 0 ? mx : -1e30f;
                ssum[c] = sum;
            }
        }
    }
    __syncthreads();
    // value sum: thread d owns dim d
    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = 0.0f;
    int valid[M];
#pragma unroll
    for (int m = 0; m < M; ++m) valid[m] = min(nkeys, pos0 + m + 1 - kstart);
    const uint16_t* vb = a.vcache + (size_t)kh * HD + tid;
    for (int t = 0; t < nkeys; ++t) {
        const float vv = h2f(vb[(size_t)(kstart + t) * kv_dim]);
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if (t < valid[c / G]) acc[c] = fmaf(sc[c][t], vv, acc[c]);
    }
    const int parts_max = (a.ctx + kPart - 1) / kPart;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int g = c % G, m = c / G;
        const int hh = kh * G + g;
        float* o = a.partial + (((size_t)m * a.n_heads + hh) * parts_max + p) * (HD + 2);
        o[tid] = acc[c];
        if (tid == 0) {
            o[HD] = smax[c];
            o[HD + 1] = ssum[c];
        }
    }
}

// attention.wgsl:248-269: merge the token's parts in order, then the sigmoid gate.
__global__ __launch_bounds__(256) void combine_kernel(AttnArgs a) {
    const int h = blockIdx.x, m = blockIdx.y, d = threadIdx.x;
    const int total = a.step->pos0 + m + 1;
    const int np = (total + kPart - 1) / kPart;
    const int parts_max = (a.ctx + kPart - 1) / kPart;
    const float* base = a.partial + ((size_t)m * a.n_heads + h) * parts_max * (HD + 2);
    float mx = -1e30f;
    for (int p = 0; p < np; ++p) mx = fmaxf(mx, base[(size_t)p * (HD + 2) + HD]);
    float l = 0.0f, acc = 0.0f;
    for (int p = 0; p < np; ++p) {
        const float* o = base + (size_t)p * (HD + 2);
        const float f = expf(o[HD] - mx);
        l = l + o[HD + 1] * f;
        acc = acc + o[d] * f;
    }
    const float gate = a.proj[(size_t)m * a.proj_stride + h * 2 * HD + HD + d];
    a.out[(size_t)m * a.n_heads * HD + h * HD + d] = acc / l / (1.0f + expf(-gate));
}

}  // namespace

int launch_attention(const AttnArgs& a, int M, hipStream_t s) {
    if (M < 1 || M > SNL_MAX_M || M == 3 || a.n_heads != G * a.n_kv || a.rot_dim > HD || a.rot_dim % 2) return -1;
    hipLaunchKernelGGL(prep_kernel, dim3(a.n_heads + 2 * a.n_kv, M), dim3(256), 0, s, a);
    const int parts_max = (a.ctx + kPart - 1) / kPart;
    dim3 grid(a.n_kv, parts_max);
    switch (M) {
        case 1: hipLaunchKernelGGL(attend_kernel<1>, grid, dim3(256), 0, s, a); break;
        case 2: hipLaunchKernelGGL(attend_kernel<2>, grid, dim3(256), 0, s, a); break;
        case 4: hipLaunchKernelGGL(attend_kernel<4>, grid, dim3(256), 0, s, a); break;
        default: return -1;
    }
    hipLaunchKernelGGL(combine_kernel, dim3(a.n_heads, M), dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace snl
