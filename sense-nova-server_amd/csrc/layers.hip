// Norms, mHC routing, residual merges, SwiGLU, embedding gather and the greedy pick.
// Semantics follow src/shaders/layers.wgsl, src/engine.rs:777-790 and src/sampler.rs:169-177.
#include <float.h>

#include <mutex>

#include "../../include/snl.h"
#include "common.h"
#include "kernels.h"

#pragma clang fp contract(off)

namespace snl {

namespace {

__global__ __launch_bounds__(256) void embed_kernel(const StepDev* step, const int8_t* __restrict__ eq,
                                                     const float* __restrict__ es, int vocab, int h,
                                                     float* __restrict__ x, int M, const float* carry_src,
                                                     float* carry_dst, const Pick* draft, int one_stream) {
    const int m = blockIdx.x;
    if (m == M) {  // the carried row (launched only with carry_src)
        for (int i = threadIdx.x; i * 4 < h; i += 256)
            reinterpret_cast<float4*>(carry_dst)[i] = reinterpret_cast<const float4*>(carry_src)[i];
        return;
    }
    // a verify pass launched right behind the MTP draft takes the draft's token from its pick
    uint32_t tok = draft && ((step->draft_rows >> m) & 1u) ? draft->token : step->tokens[m];
    if (tok >= (uint32_t)vocab) tok = 0;  // the host rejects out-of-range ids before launching
    const int8_t* q = eq + (size_t)tok * h;
    const float* s = es + (size_t)tok * (h / 32);
    float* xr = x + (size_t)m * (one_stream ? 1 : 2) * h;
    // piece p: 16 consecutive quants (half of quant block p / 2), one 16-byte load and its scale,
    // both issued before any store
    for (int p = threadIdx.x; p * 16 < h; p += 256) {
        const uint4 w = *reinterpret_cast<const uint4*>(q + 16 * p);
        const float sc = s[p >> 1];
        const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
        float4* o = reinterpret_cast<float4*>(xr + 16 * p);
        float4* z = reinterpret_cast<float4*>(xr + h + 16 * p);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t v = wd[k];
            o[k] = make_float4((float)(int8_t)(v & 0xffu) * sc, (float)(int8_t)((v >> 8) & 0xffu) * sc,
                               (float)(int8_t)((v >> 16) & 0xffu) * sc, (float)(int8_t)(v >> 24) * sc);
            if (!one_stream) z[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
}

// layers.wgsl:46-73 branch_norm; one block per output row.
__global__ __launch_bounds__(256) void branch_norm_kernel(NormArgs a) {
    __shared__ float red[8];
    const int r = blockIdx.x;
    const int row = a.first + r + (a.row_base ? *a.row_base : 0);
    const float4* x0 = reinterpret_cast<const float4*>(a.x + (size_t)row * a.x_stride);
    float pre0 = 1.0f, pre1 = 0.0f;
    if (a.mode == 1) {
        pre0 = a.coef[(a.first + r) * 8];
        pre1 = a.coef[(a.first + r) * 8 + 1];
    }
    constexpr int kMaxPer = 8;  // h <= 8192: 2048 float4 over 256 threads
    const int h4 = a.h >> 2;
    float4 v[kMaxPer];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxPer; ++j) {
        const int i = threadIdx.x + 256 * j;
        float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < h4) {
            t = x0[i];
            if (a.mode == 1) {
                const float4 u = x0[h4 + i];
                t.x = pre0 * t.x + pre1 * u.x;
                t.y = pre0 * t.y + pre1 * u.y;
                t.z = pre0 * t.z + pre1 * u.z;
                t.w = pre0 * t.w + pre1 * u.w;
            }
        }
        v[j] = t;
        ss = fmaf(t.x, t.x, ss);
        ss = fmaf(t.y, t.y, ss);
        ss = fmaf(t.z, t.z, ss);
        ss = fmaf(t.w, t.w, ss);
    }
    const float total = block_sum<256>(ss, red);
    const float rinv = 1.0f / sqrtf(total / (float)a.h + a.eps);
    float4* ob = reinterpret_cast<float4*>(a.out + (size_t)r * a.out_stride);
    const float4* w4 = reinterpret_cast<const float4*>(a.w);
#pragma unroll
    for (int j = 0; j < kMaxPer; ++j) {
        const int i = threadIdx.x + 256 * j;
        if (i < h4) {
            const float4 w = w4[i];
            float4 o;
            o.x = (v[j].x * rinv) * (a.one + w.x);
            o.y = (v[j].y * rinv) * (a.one + w.y);
            o.z = (v[j].z * rinv) * (a.one + w.z);
            o.w = (v[j].w * rinv) * (a.one + w.w);
            ob[i] = o;
            if (a.last_copy && r == a.count - 1) reinterpret_cast<float4*>(a.last_copy)[i] = o;
        }
    }
}

// mHC router sums of one token per block (layers.wgsl:75-92): the 8 router-row dots with the
// 2-stream row [x0, x1] and its sum of squares, written as the token's single partial.  All loads
// of a batch are issued before their first use.
constexpr int kMhcThreads = 1024;

__global__ __launch_bounds__(kMhcThreads) void mhc_kernel(const float* x, const float* w, float* part, int h) {
    __shared__ float red[kMhcThreads / 64][9];
    const int m = blockIdx.x, tid = threadIdx.x, d = 2 * h, d4 = d / 4;
    const float4* xr = reinterpret_cast<const float4*>(x + (size_t)m * d);
    const float4* wr = reinterpret_cast<const float4*>(w);
    float acc[9];
#pragma unroll
    for (int o = 0; o < 9; ++o) acc[o] = 0.0f;
    for (int i0 = tid; i0 < d4; i0 += 2 * kMhcThreads) {
        const int i1 = i0 + kMhcThreads;
        const bool ok1 = i1 < d4;
        const float4 v0 = xr[i0], v1 = xr[ok1 ? i1 : i0];
        float4 u0[8], u1[8];
#pragma unroll
        for (int o = 0; o < 8; ++o) {
            u0[o] = wr[(size_t)o * d4 + i0];
            u1[o] = wr[(size_t)o * d4 + (ok1 ? i1 : i0)];
        }
#pragma unroll
        for (int o = 0; o < 8; ++o) {
            acc[o] = fmaf(u0[o].x, v0.x, acc[o]);
            acc[o] = fmaf(u0[o].y, v0.y, acc[o]);
            acc[o] = fmaf(u0[o].z, v0.z, acc[o]);
            acc[o] = fmaf(u0[o].w, v0.w, acc[o]);
        }
        acc[8] = fmaf(v0.x, v0.x, acc[8]);
        acc[8] = fmaf(v0.y, v0.y, acc[8]);
        acc[8] = fmaf(v0.z, v0.z, acc[8]);
        acc[8] = fmaf(v0.w, v0.w, acc[8]);
        if (ok1) {
#pragma unroll
            for (int o = 0; o < 8; ++o) {
                acc[o] = fmaf(u1[o].x, v1.x, acc[o]);
                acc[o] = fmaf(u1[o].y, v1.y, acc[o]);
                acc[o] = fmaf(u1[o].z, v1.z, acc[o]);
                acc[o] = fmaf(u1[o].w, v1.w, acc[o]);
            }
            acc[8] = fmaf(v1.x, v1.x, acc[8]);
            acc[8] = fmaf(v1.y, v1.y, acc[8]);
            acc[8] = fmaf(v1.z, v1.z, acc[8]);
            acc[8] = fmaf(v1.w, v1.w, acc[8]);
        }
    }
    wave_sum_n(acc);
    if ((tid & 63) == 0)
#pragma unroll
        for (int o = 0; o < 9; ++o) red[tid >> 6][o] = acc[o];
    __syncthreads();
    if (tid < 9) {
        float t = 0.0f;
        for (int wv = 0; wv < kMhcThreads / 64; ++wv) t = t + red[wv][tid];
        part[m * 9 + tid] = t;
    }
}

__global__ __launch_bounds__(256) void expand_kernel(float* x, int h, int M) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= M * h) return;
    const int m = idx / h, i = idx % h;
    x[(size_t)m * 2 * h + h + i] = x[(size_t)m * 2 * h + i];
}

// layers.wgsl:128-162 merge, modes 0..2
__global__ __launch_bounds__(256) void merge_kernel(float* x, const float* coef, const float* br, int h, int M,
                                                     int mode) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= M * h) return;
    const int m = idx / h, i = idx % h;
    float* x0 = x + (size_t)m * 2 * h + i;
    float* x1 = x0 + h;
    const float b = br[idx];
    if (mode == 0) {
        *x0 = *x0 + b;
        return;
    }
    const float* c = coef + m * 8;
    const float a0 = *x0, a1 = *x1;
    const float n0 = (c[4] * a0 + c[5] * a1) + c[2] * b;
    const float n1 = (c[6] * a0 + c[7] * a1) + c[3] * b;
    if (mode == 2) {
        *x0 = 0.5f * (n0 + n1);
    } else {
        *x0 = n0;
        *x1 = n1;
    }
}

__global__ __launch_bounds__(256) void swiglu_kernel(const float* proj, float* act, int inter, int M) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= M * inter) return;
    const int m = idx / inter, i = idx % inter;
    const float g = proj[(size_t)m * 2 * inter + i], u = proj[(size_t)m * 2 * inter + inter + i];
    act[idx] = g / (1.0f + expf(-g)) * u;
}

// ---- greedy pick: (max, first index of max, second largest) ----
struct Top2 {
    float v1;
    uint32_t i1;
    float v2;
};

__device__ __forceinline__ Top2 top2_merge(Top2 a, Top2 b) {
    Top2 r;
    const bool take_b = b.v1 > a.v1 || (b.v1 == a.v1 && b.i1 < a.i1);
    r.v1 = take_b ? b.v1 : a.v1;
    r.i1 = take_b ? b.i1 : a.i1;
    r.v2 = fmaxf(fminf(a.v1, b.v1), fmaxf(a.v2, b.v2));
    return r;
}

template <int O>
__device__ __forceinline__ Top2 top2_xor(Top2 t) {
    const Top2 u = {__uint_as_float(lane_xor_bits<O>(__float_as_uint(t.v1))), lane_xor_bits<O>(t.i1),
                    __uint_as_float(lane_xor_bits<O>(__float_as_uint(t.v2)))};
    return top2_merge(t, u);
}

__device__ __forceinline__ Top2 top2_wave(Top2 t) {
    t = top2_xor<32>(t);
    t = top2_xor<16>(t);
    t = top2_xor<8>(t);
    t = top2_xor<4>(t);
    t = top2_xor<2>(t);
    return top2_xor<1>(t);
}

__device__ __forceinline__ Top2 top2_block(Top2 t) {
    __shared__ float s1[4], s2[4];
    __shared__ uint32_t si[4];
    t = top2_wave(t);
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    __syncthreads();
    if (lane == 0) {
        s1[w] = t.v1;
        si[w] = t.i1;
        s2[w] = t.v2;
    }
    __syncthreads();
    Top2 r = {s1[0], si[0], s2[0]};
    for (int i = 1; i < 4; ++i) r = top2_merge(r, Top2{s1[i], si[i], s2[i]});
    return r;
}

// 2048 logits per block, 8 per thread, all loaded before the first comparison: the row is read in
// one round trip by ~120 blocks per row instead of a chain of dependent loads
constexpr int kPickPer = 8;
constexpr int kPickChunk = 256 * kPickPer;

__global__ __launch_bounds__(256) void pick_partial_kernel(const float* logits, int V, float* scratch, int nblk) {
    const int row = blockIdx.y, b = blockIdx.x;
    const float* lg = logits + (size_t)row * V;
    Top2 t = {-FLT_MAX, 0xFFFFFFFFu, -FLT_MAX};
    float vals[kPickPer];
    const int i0 = b * kPickChunk + threadIdx.x;
#pragma unroll
    for (int u = 0; u < kPickPer; ++u) vals[u] = i0 + 256 * u < V ? lg[i0 + 256 * u] : -FLT_MAX;
#pragma unroll
    for (int u = 0; u < kPickPer; ++u) {
        const int i = i0 + 256 * u;
        const float v = vals[u];
        if (i >= V) break;
        // strict > keeps the first index; elements arrive in ascending order per thread
        if (v > t.v1) {
            t.v2 = t.v1;
            t.v1 = v;
            t.i1 = (uint32_t)i;
        } else if (v > t.v2) {
            t.v2 = v;
        }
    }
    t = top2_block(t);
    if (threadIdx.x == 0) {
        float* o = scratch + ((size_t)row * nblk + b) * 3;
        o[0] = t.v1;
        o[1] = __uint_as_float(t.i1);
        o[2] = t.v2;
    }
}

__global__ __launch_bounds__(256) void pick_final_kernel(const float* scratch, int nblk, Pick* out, Pick* host_out) {
    const int row = blockIdx.x;
    Top2 t = {-FLT_MAX, 0xFFFFFFFFu, -FLT_MAX};
    for (int b = threadIdx.x; b < nblk; b += 256) {
        const float* o = scratch + ((size_t)row * nblk + b) * 3;
        t = top2_merge(t, Top2{o[0], __float_as_uint(o[1]), o[2]});
    }
    t = top2_block(t);
    if (threadIdx.x == 0) {
        const Pick r = {t.i1 == 0xFFFFFFFFu ? 0u : t.i1, t.v1, t.v2, 0u};
        out[row] = r;
        if (host_out) {  // pinned host memory: the host reads it after the stream synchronises
            host_out[row] = r;
            __threadfence_system();
        }
    }
}

// One block of 256 threads.  Every thread reads what it needs of the two records before the
// barrier; the records are rewritten after it.
__global__ __launch_bounds__(256) void spec_next_kernel(SpecArgs a) {
    const int tid = threadIdx.x;
    const Pick p0 = a.picks[0], p1 = a.picks[1];
    const uint32_t d = a.draft->token;
    const StepDev& v = *a.vstep;
    const int32_t pos0 = v.pos0, s_ck = v.s_ck, s_out = v.s_out;
    const uint32_t rope = v.rpos[0][0], tok0 = v.tokens[0], seq = v.seq;
    (void)tok0;
    __syncthreads();
    const bool acc = p0.token == d;
    const int adv = acc ? 2 : 1;
    const uint32_t nrope = rope + (uint32_t)adv;
    // a position past the table (it holds ctx + 4 rows, and decode positions stay below the
    // context) reads the last row and is reported through the outcome's flags
    auto tab = [&](uint32_t p, int f) {
        const uint32_t r = p < (uint32_t)a.rope_rows ? p : (uint32_t)a.rope_rows - 1;
        return *reinterpret_cast<const float2*>(a.rope_tab + ((size_t)r * SNL_ROPE_MAX + f) * 2);
    };
    const bool rope_out = nrope + 1u >= (uint32_t)a.rope_rows;
    // rotary cos / sin: threads 0-127 the verify's two rows, 128-255 the draft's two rows
    {
        const int row = (tid >> 6) & 1, f = tid & 63;
        if (tid < 128) {
            const float2 t = tab(nrope + (uint32_t)row, f);
            a.vstep->rope[row][f][0] = t.x;
            a.vstep->rope[row][f][1] = t.y;
        } else {
            const float2 t = tab(rope + (uint32_t)row, f);
            a.mstep->rope[row][f][0] = t.x;
            a.mstep->rope[row][f][1] = t.y;
        }
    }
    if (tid == 0) {
        StepDev& nv = *a.vstep;
        nv.pos0 = pos0 + adv;
        nv.m = 2;
        nv.ckpt = 1;
        nv.s_in = acc ? s_out : s_ck;
        nv.s_ck = (nv.s_in + 1) % 3;
        nv.s_out = (nv.s_in + 2) % 3;
        nv.r0 = 0;
        nv.x_off = 0;
        nv.draft_rows = 2u;
        nv.seq = seq + 1;
        nv.tokens[0] = acc ? p1.token : p0.token;
        nv.tokens[1] = 0u;
        for (int i = 0; i < 2; ++i)
            for (int k = 0; k < 4; ++k) nv.rpos[i][k] = k < 3 ? nrope + (uint32_t)i : 0u;
        // the next draft: after an accept the pairs (d, p1) at the verify's positions, after a
        // reject (p0) and a padding row (the same token at the next position), from hidden row 1
        StepDev& nm = *a.mstep;
        nm.pos0 = pos0;
        nm.m = 2;
        nm.ckpt = 0;
        nm.s_in = nm.s_ck = nm.s_out = 0;
        nm.r0 = 1;
        nm.x_off = acc ? 1 : 0;
        nm.draft_rows = 0u;
        nm.seq = 0u;
        nm.tokens[0] = acc ? d : p0.token;
        nm.tokens[1] = acc ? p1.token : p0.token;
        for (int i = 0; i < 2; ++i)
            for (int k = 0; k < 4; ++k) nm.rpos[i][k] = k < 3 ? rope + (uint32_t)i : 0u;
        SpecOut o;
        o.seq = seq;
        o.draft = d;
        o.accepted = acc ? 1u : 0u;
        o.flags = rope_out ? kSpecRopeRange : 0u;
        o.picks[0] = p0;
        o.picks[1] = p1;
        a.ring[seq % (uint32_t)a.ring_n] = o;
    }
    // the rollback's carried row
    if (!acc)
        for (int i = tid; i < a.h; i += 256) a.hlast[i] = a.hid1[i];
    if (tid == 0) __threadfence_system();
}

__global__ __launch_bounds__(256) void copy_kernel(float* dst, const float* src, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

inline int last_error() { return hipGetLastError() == hipSuccess ? 0 : -2; }

}  // namespace

int launch_embed(const StepDev* step, const int8_t* eq, const float* es, int vocab, int h, float* x, int M,
                 hipStream_t s, const float* carry_src, float* carry_dst, const Pick* draft, bool one_stream) {
    if (M < 1 || M > SNL_MAX_M || h % 32 || (reinterpret_cast<uintptr_t>(eq) & 15) ||
        (reinterpret_cast<uintptr_t>(x) & 15) || (carry_src && !carry_dst) ||
        (reinterpret_cast<uintptr_t>(carry_src) & 15) || (reinterpret_cast<uintptr_t>(carry_dst) & 15))
        return -1;
    hipLaunchKernelGGL(embed_kernel, dim3(M + (carry_src ? 1 : 0)), dim3(256), 0, s, step, eq, es, vocab, h, x, M,
                       carry_src, carry_dst, draft, one_stream ? 1 : 0);
    return last_error();
}

int launch_branch_norm(const NormArgs& a, hipStream_t s) {
    if (a.count < 1 || a.h > 8192 || a.h < 4 || a.h % 4 || a.x_stride % 4 || a.out_stride % 4 ||
        (reinterpret_cast<uintptr_t>(a.last_copy) & 15))
        return -1;
    hipLaunchKernelGGL(branch_norm_kernel, dim3(a.count), dim3(256), 0, s, a);
    return last_error();
}

int launch_mhc(const float* x, const float* w, float* part, int h, int M, hipStream_t s) {
    if (M < 1 || M > SNL_PF_M || h % 2) return -1;
    hipLaunchKernelGGL(mhc_kernel, dim3(M), dim3(kMhcThreads), 0, s, x, w, part, h);
    return last_error();
}

int launch_expand(float* x, int h, int M, hipStream_t s) {
    hipLaunchKernelGGL(expand_kernel, dim3((M * h + 255) / 256), dim3(256), 0, s, x, h, M);
    return last_error();
}

int launch_merge(float* x, const float* coef, const float* br, int h, int M, int mode, hipStream_t s) {
    if (mode < 0 || mode > 2) return -1;
    hipLaunchKernelGGL(merge_kernel, dim3((M * h + 255) / 256), dim3(256), 0, s, x, coef, br, h, M, mode);
    return last_error();
}

int launch_swiglu(const float* proj, float* act, int inter, int M, hipStream_t s) {
    hipLaunchKernelGGL(swiglu_kernel, dim3((M * inter + 255) / 256), dim3(256), 0, s, proj, act, inter, M);
    return last_error();
}

size_t pick_scratch_floats(int V, int rows) { return (size_t)rows * ((V + kPickChunk - 1) / kPickChunk) * 3; }

int launch_spec_next(const SpecArgs& a, hipStream_t s) {
    if (!a.vstep || !a.mstep || !a.picks || !a.draft || !a.rope_tab || a.rope_rows < 1 || !a.hid1 || !a.hlast ||
        a.h < 1 || !a.ring || a.ring_n < 1)
        return -1;
    hipLaunchKernelGGL(spec_next_kernel, dim3(1), dim3(256), 0, s, a);
    return last_error();
}

int launch_pick(const float* logits, int V, int rows, float* scratch, Pick* out, hipStream_t s, Pick* host_out) {
    if (rows < 1 || V < 1) return -1;
    const int nblk = (V + kPickChunk - 1) / kPickChunk;
    hipLaunchKernelGGL(pick_partial_kernel, dim3(nblk, rows), dim3(256), 0, s, logits, V, scratch, nblk);
    hipLaunchKernelGGL(pick_final_kernel, dim3(rows), dim3(256), 0, s, scratch, nblk, out, host_out);
    return last_error();
}

int launch_copy(float* dst, const float* src, size_t n, hipStream_t s) {
    hipLaunchKernelGGL(copy_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, dst, src, n);
    return last_error();
}

}  // namespace snl

// ---- greedy pick without device allocation ----
//
// The block partials of launch_pick live in this file-scope array instead of a buffer the caller
// or the library allocates.  Each GPU holds its own copy until the process ends; host code reaches
// it only through the address hipGetSymbolAddress returns on that device (the array's name is a
// host-side stand-in, not a device address).  pick_partial_kernel writes every partial that
// pick_final_kernel reads, so nothing needs clearing between calls.
namespace snl {
namespace {
constexpr int kNoAllocPickBlocks = 4096;  // rows * ceil(V / 2048) at most: 48 KiB
static __device__ __align__(256) float scratch[kNoAllocPickBlocks * 3];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up once per device.
int scratch_address(float** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return SNL_EDEVICE;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return SNL_EDEVICE;
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return SNL_OK;
}
}  // namespace

}  // namespace snl

extern "C" int snl_pick_rows_noalloc(const float* logits, int V, int rows, snl_pick* picks_out, void* stream) {
    using namespace snl;
    if (!logits || !picks_out || V < 1 || rows < 1 || rows > 64) return SNL_EARG;
    if ((size_t)rows * ((V + kPickChunk - 1) / kPickChunk) > (size_t)kNoAllocPickBlocks) return SNL_EARG;
    float* sp = nullptr;
    if (const int rc = scratch_address(&sp)) return rc;
    return launch_pick(logits, V, rows, sp, reinterpret_cast<Pick*>(picks_out), (hipStream_t)stream) ? SNL_EDEVICE
                                                                                                       : SNL_OK;
}
