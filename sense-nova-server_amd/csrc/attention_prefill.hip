// Gated GQA attention over a prefill chunk (src/shaders/attention.wgsl: prep :59-127, attend
// :129-246, combine :248-269), on the matrix cores.
//
// prep: block (slot, token) as in the decode kernel: RMSNorm (1 + w) of each q / k head, partial
// rotate-half RoPE at the token's rotary position, q rows to qbuf (f32), k / v rows into the f16
// cache at the token's cache position.
//
// attend: block (kv head, 16 queries, key part), wave w = query head 4*kv + w of the GQA group;
// the block streams its part of the keys [0, last query's position] (4096 keys per part) in steps
// of 32 through LDS (K rows and V rows, each staged with 16-byte copies; the V^T fragments come
// back from the V rows through the transposing LDS read, two 8-byte reads per fragment),
// shared by the group's 4 heads.
//   scores  S^T = K Q^T on v_mfma_f32_16x16x32_f16: A = 16 keys x 32 dims of K (exact f16),
//           B = the query's dims split into f16 hi + lo under a per-query power of two, so the
//           f32 score carries the decode kernel's precision; lane (query j, group g) ends with
//           keys 4g..4g+3 of each 16-key half;
//   softmax online per query (running max, rescaled partial sums), keys past the query's own
//           position weigh 0;
//   values  O^T += V^T P^T: B = the lane's own 8 probabilities as f16 hi + lo (keys 4g..4g+3 and
//           16+4g..16+4g+3, the same order in the V^T fragment), A = 16 dims x those keys.
// With one part the output is divided by the softmax sum and multiplied by the sigmoid gate, as in
// combine; with several, each part leaves (unnormalised output, running max, sum) and
// pf_combine_kernel merges the parts in order.
#include <float.h>
#include <hip/hip_fp16.h>

#include "common.h"
#include "kernels.h"

#pragma clang fp contract(off)

namespace snl {

namespace {

constexpr int HD = 256, G = 4;
constexpr int QTILE = 16, KB = 32;
constexpr int KPART = 4096;  // keys per part when a long context splits the key range
constexpr int KROW = HD + 8;  // K tile row (halfs): 528 bytes keeps the 16 rows of a read on distinct banks
constexpr int VROW = HD + 16;  // V row (halfs): 544 bytes, so the 4 rows of a transposed read hit distinct banks

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void pf_prep_kernel(AttnArgs a, const PrefillDev* st) {
    __shared__ float sh[HD];
    __shared__ float red[4];
    const int slot = blockIdx.x, m = blockIdx.y, d = threadIdx.x;
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

__global__ __launch_bounds__(256) void pf_attend_kernel(AttnArgs a, const PrefillDev* st, int M, float* part,
                                                        int parts_max) {
    __shared__ __align__(16) _Float16 ks[KB * KROW];
    __shared__ __align__(16) _Float16 vs[KB * VROW];
    const int kh = blockIdx.x, q0 = blockIdx.y * QTILE;
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hh = kh * G + w;
    const int pos0 = st->pos0;
    const int qn = min(QTILE, M - q0);
    const int kend = pos0 + q0 + qn;  // keys of the block's last query
    const int p = blockIdx.z, nparts = (kend + KPART - 1) / KPART;
    if (p >= nparts) return;
    const int kfirst = p * KPART, kstop = min(kend, kfirst + KPART);
    const int q_dim = a.n_heads * HD, kv_dim = a.n_kv * HD;
    const int j = lane & 15, g = lane >> 4;
    const int mq = q0 + j;
    const bool qvalid = j < qn;
    const int qlim = pos0 + mq;  // the last key this lane's query sees

    // ---- the query as B fragments (dims 32s + 8g + i), hi + lo under a power of two ----
    float qv[8][8];
    float amax = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const float4* qp = reinterpret_cast<const float4*>(a.qbuf + (size_t)(qvalid ? mq : q0) * q_dim + hh * HD + 32 * s + 8 * g);
        const float4 u0 = qp[0], u1 = qp[1];
        qv[s][0] = u0.x, qv[s][1] = u0.y, qv[s][2] = u0.z, qv[s][3] = u0.w;
        qv[s][4] = u1.x, qv[s][5] = u1.y, qv[s][6] = u1.z, qv[s][7] = u1.w;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (!qvalid) qv[s][i] = 0.0f;
            amax = fmaxf(amax, fabsf(qv[s][i]));
        }
    }
    amax = xor_max<32>(xor_max<16>(amax));
    const int e = amax > 0.0f ? max(ilogbf(amax) - 14, -110) : 0;
    const float down = ldexpf(1.0f, -e), up = ldexpf(1.0f, e) * a.scale;
    half8_t qh[8], ql[8];
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float v = qv[s][i] * down;
            const _Float16 hv = (_Float16)v;
            qh[s][i] = hv;
            ql[s][i] = (_Float16)(v - (float)hv);
        }

    f32x4_t o[16];
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) o[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float mrun = -1e30f, lpart = 0.0f;
    const uint16_t* kc = a.kcache + kh * HD;
    const uint16_t* vc = a.vcache + kh * HD;

    for (int kb = kfirst; kb < kstop; kb += KB) {
        __syncthreads();  // the previous step's tiles are consumed
        {   // K rows: thread (key t >> 3, 32 dims)
            const int key = tid >> 3, seg = tid & 7;
            const int kk = kb + key;
            uint4 r[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) r[i] = make_uint4(0u, 0u, 0u, 0u);
            if (kk < kstop) {
                const uint4* src = reinterpret_cast<const uint4*>(kc + (size_t)kk * kv_dim + seg * 32);
#pragma unroll
                for (int i = 0; i < 4; ++i) r[i] = src[i];
            }
            uint4* dst = reinterpret_cast<uint4*>(ks + key * KROW + seg * 32);
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[i] = r[i];
        }
        {   // V rows, as the K rows: thread (key t >> 3, 32 dims)
            const int key = tid >> 3, seg = tid & 7;
            const int kk = kb + key;
            uint4 r[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) r[i] = make_uint4(0u, 0u, 0u, 0u);
            if (kk < kstop) {
                const uint4* src = reinterpret_cast<const uint4*>(vc + (size_t)kk * kv_dim + seg * 32);
#pragma unroll
                for (int i = 0; i < 4; ++i) r[i] = src[i];
            }
            uint4* dst = reinterpret_cast<uint4*>(vs + key * VROW + seg * 32);
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[i] = r[i];
        }
        __syncthreads();

        // ---- scores: two 16-key halves ----
        f32x4_t sc[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            f32x4_t c = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const half8_t kf = *reinterpret_cast<const half8_t*>(ks + (16 * kt + j) * KROW + 32 * s + 8 * g);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qh[s], c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, ql[s], c, 0, 0, 0);
            }
            sc[kt] = c;
        }
        // ---- online softmax for this lane's query ----
        float val[8];
        bool ok[8];
        float bmax = -1e30f;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int kk = kb + 16 * kt + 4 * g + r;
                const int i = 4 * kt + r;
                ok[i] = qvalid && kk <= qlim && kk < kstop;
                val[i] = sc[kt][r] * up;
                if (ok[i]) bmax = fmaxf(bmax, val[i]);
            }
        bmax = xor_max<32>(xor_max<16>(bmax));
        const float mnew = fmaxf(mrun, bmax);
        const float factor = expf(mrun - mnew);
        half8_t ph, pl;
        float psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float p = ok[i] ? expf(val[i] - mnew) : 0.0f;
            psum = psum + p;
            const _Float16 hv = (_Float16)p;
            ph[i] = hv;
            pl[i] = (_Float16)(p - (float)hv);
        }
        lpart = lpart * factor + psum;
        mrun = mnew;
        // ---- values ----
#pragma unroll
        for (int dt = 0; dt < 16; ++dt) {
            o[dt] = o[dt] * factor;
            // transposed reads (ds_read_b64_tr_b16): in each 16-lane group, lane 4a + b receives
            // element b of the 8 bytes addressed by lanes a, a + 4, a + 8, a + 12; lane s
            // addresses key 4g + s / 4 (then 16 + 4g + s / 4), dims 16 dt + 4 (s % 4), so lane j
            // receives dim 16 dt + j of keys 4g .. 4g + 3 (then 16 + 4g ..)
            const _Float16* pa = vs + (4 * g + (j >> 2)) * VROW + 16 * dt + 4 * (j & 3);
            const half4_t va = __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) short4_t*)(pa)));
            const half4_t vb = __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) short4_t*)(pa + 16 * VROW)));
            const half8_t vf = half8_t{va[0], va[1], va[2], va[3], vb[0], vb[1], vb[2], vb[3]};
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, ph, o[dt], 0, 0, 0);
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pl, o[dt], 0, 0, 0);
        }
    }
    // ---- normalise, gate, store: lane (query j) holds dims 16dt + 4g + r ----
    const float l = xor_sum<32>(xor_sum<16>(lpart));
    if (!qvalid) return;
    if (parts_max > 1) {  // this part's unnormalised output, running max and sum for the combine
        float* pp = part + (((size_t)mq * a.n_heads + hh) * parts_max + p) * (HD + 2);
#pragma unroll
        for (int dt = 0; dt < 16; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r) pp[16 * dt + 4 * g + r] = o[dt][r];
        if (g == 0) {
            pp[HD] = mrun;
            pp[HD + 1] = l;
        }
        return;
    }
    const float* grow = a.proj + (size_t)mq * a.proj_stride + hh * 2 * HD + HD;
    float* orow = a.out + (size_t)mq * q_dim + hh * HD;
#pragma unroll
    for (int dt = 0; dt < 16; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int d = 16 * dt + 4 * g + r;
            orow[d] = o[dt][r] / l / (1.0f + expf(-grow[d]));
        }
}

// Merge the key parts of one (query, head): block (head, query), thread = dim.  Parts are added
// in order with weights e^(m_p - max); then the division by the softmax sum and the sigmoid gate.
__global__ __launch_bounds__(HD) void pf_combine_kernel(AttnArgs a, const PrefillDev* st, int M, const float* part,
                                                        int parts_max) {
    const int hh = blockIdx.x, m = blockIdx.y, d = threadIdx.x;
    const int q0 = m / QTILE * QTILE, qn = min(QTILE, M - q0);
    const int nparts = (st->pos0 + q0 + qn + KPART - 1) / KPART;
    const float* pp = part + ((size_t)m * a.n_heads + hh) * parts_max * (HD + 2);
    float mx = -1e30f;
    for (int p = 0; p < nparts; ++p) mx = fmaxf(mx, pp[(size_t)p * (HD + 2) + HD]);
    float acc = 0.0f, l = 0.0f;
    for (int p = 0; p < nparts; ++p) {
        const float* q = pp + (size_t)p * (HD + 2);
        const float f = expf(q[HD] - mx);
        acc = acc + q[d] * f;
        l = l + q[HD + 1] * f;
    }
    const float gate = a.proj[(size_t)m * a.proj_stride + hh * 2 * HD + HD + d];
    a.out[(size_t)m * a.n_heads * HD + hh * HD + d] = acc / l / (1.0f + expf(-gate));
}

}  // namespace

int attention_prefill_parts(int ctx) { return (ctx + KPART - 1) / KPART; }

int launch_attention_prefill(const AttnArgs& a, const PrefillDev* pstep, int M, int keys, float* part, int parts_max,
                             hipStream_t s) {
    if (M < 1 || M > SNL_PF_M || a.n_heads != G * a.n_kv || a.rot_dim > HD || a.rot_dim % 2 || !pstep) return -1;
    const int parts = (keys + KPART - 1) / KPART;  // parts of the pass's longest key range
    if (parts > 1 && (!part || parts > parts_max)) return -1;
    hipLaunchKernelGGL(pf_prep_kernel, dim3(a.n_heads + 2 * a.n_kv, M), dim3(256), 0, s, a, pstep);
    hipLaunchKernelGGL(pf_attend_kernel, dim3(a.n_kv, (M + QTILE - 1) / QTILE, parts), dim3(256), 0, s, a, pstep, M,
                       part, parts > 1 ? parts_max : 1);
    if (parts > 1)
        hipLaunchKernelGGL(pf_combine_kernel, dim3(a.n_heads, M), dim3(HD), 0, s, a, pstep, M, part, parts_max);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace snl
