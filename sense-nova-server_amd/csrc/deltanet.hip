// Gated DeltaNet decode step: causal depthwise conv (k=4) + SiLU, then the recurrent
// gated delta rule with L2-normalised q/k and the gated RMS norm, for M = 1..4 tokens
// (src/shaders/linear.wgsl:38-140 conv + delta, fused into one launch).
//
// One block per value head h (k-head h / (n_v / n_k)), 512 threads: thread (j, g) owns
// column j of the head's [128 (i), 128 (j)] f32 state, rows i in [32g, 32g+32), kept in
// registers for all M tokens.  The conv of the head's 384 channels (q, k of its k-head,
// v of the head) runs first, token by token, into LDS.
//
// Recurrent state lives in three slots per visit.  A call reads slot s_in, writes the
// state after its last token to s_out and, when ckpt > 0, the state after token ckpt-1
// to s_ck; s_out and s_ck are never s_in, so no block overwrites what another block
// still reads (two v-heads share each k-head's conv channels).  A rejected draft
// becomes a change of the current slot on the host instead of a copy.
#include "common.h"
#include "kernels.h"

#pragma clang fp contract(off)

namespace snl {

namespace {

constexpr int DK = 128, DV = 128, kThreads = 512, kRowsPer = DK / (kThreads / DV);

template <int M>
__global__ __launch_bounds__(kThreads) void deltanet_kernel(DeltaArgs a) {
    __shared__ float cq[M][DK], ck[M][DK], cv[M][DV];  // conv outputs (SiLU applied)
    __shared__ float qs[DK], ks[DK];
    __shared__ float part[4][DV];
    __shared__ float red[16];

    const StepDev* st = a.step;
    const int s_in = st->s_in, s_out = st->s_out, s_ck = st->s_ck, ckpt = st->ckpt;
    const int h = blockIdx.x, tid = threadIdx.x;
    const int j = tid & (DV - 1), g = tid >> 7;
    const int group = a.n_v / a.n_k, kh = h / group;
    const int key_dim = a.n_k * DK, cd = a.conv_dim;

    // ---- causal conv (linear.wgsl:38-66) of this head's channels ----
    if (tid < 3 * DK) {
        const int which = tid >> 7, c0 = tid & 127;
        const int ch = which == 0 ? kh * DK + c0 : which == 1 ? key_dim + kh * DK + c0 : 2 * key_dim + h * DV + c0;
        const float* lw = a.lw + (size_t)ch * 4;
        const float w0 = lw[0], w1 = lw[1], w2 = lw[2], w3 = lw[3];
        const float* cs = a.conv_state + (size_t)s_in * a.conv_slot;
        float r0 = cs[ch], r1 = cs[cd + ch], r2 = cs[2 * cd + ch];
        // k-head channels are shared by `group` v-heads: the first one owns their state
        const bool owner = which == 2 || (h % group) == 0;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float cur = a.proj[(size_t)m * a.proj_stride + ch];
            const float o = ((w0 * r0 + w1 * r1) + w2 * r2) + w3 * cur;
            const float v = o / (1.0f + expf(-o));
            if (which == 0) cq[m][c0] = v;
            else if (which == 1) ck[m][c0] = v;
            else cv[m][c0] = v;
            r0 = r1;
            r1 = r2;
            r2 = cur;
            if (m + 1 == ckpt && owner) {
                float* cc = a.conv_state + (size_t)s_ck * a.conv_slot;
                cc[ch] = r0;
                cc[cd + ch] = r1;
                cc[2 * cd + ch] = r2;
            }
        }
        if (owner) {
            float* co = a.conv_state + (size_t)s_out * a.conv_slot;
            co[ch] = r0;
            co[cd + ch] = r1;
            co[2 * cd + ch] = r2;
        }
    }

    // ---- state columns into registers ----
    const size_t hoff = (size_t)h * DK * DV;
    const float* S0 = a.state + (size_t)s_in * a.state_slot + hoff;
    float s[kRowsPer];
#pragma unroll
    for (int r = 0; r < kRowsPer; ++r) s[r] = S0[(size_t)(g * kRowsPer + r) * DV + j];

    const float* lwp = a.lw + (size_t)cd * 4;
    const float a_log = lwp[h], dt_bias = lwp[a.n_v + h], norm_w = lwp[2 * a.n_v + j];
    const int z_off = cd, b_off = cd + a.n_v * DV, a_off = b_off + a.n_v;
    __syncthreads();

#pragma unroll
    for (int m = 0; m < M; ++m) {
        // L2 norms of q and k (linear.wgsl:104-110)
        float q2 = 0.0f, k2 = 0.0f;
        if (tid < DK) {
            q2 = cq[m][tid] * cq[m][tid];
            k2 = ck[m][tid] * ck[m][tid];
        }
        const float sq = block_sum<kThreads>(q2, red);
        const float sk = block_sum<kThreads>(k2, red + 8);
        if (tid < DK) {
            qs[tid] = (cq[m][tid] * (1.0f / sqrtf(sq + 1e-6f))) * (1.0f / sqrtf((float)DK));
            ks[tid] = ck[m][tid] * (1.0f / sqrtf(sk + 1e-6f));
        }
        const float* prow = a.proj + (size_t)m * a.proj_stride;
        const float beta = 1.0f / (1.0f + expf(-prow[b_off + h]));
        const float araw = prow[a_off + h] + dt_bias;
        const float sp = araw <= 20.0f ? logf(1.0f + expf(araw)) : araw;
        const float decay = expf(-expf(a_log) * sp);
        __syncthreads();

        // kv_mem_j = sum_i decay*S[i][j] * k_i
        float kv = 0.0f;
#pragma unroll
        for (int r = 0; r < kRowsPer; ++r) {
            s[r] = s[r] * decay;
            kv = fmaf(s[r], ks[g * kRowsPer + r], kv);
        }
        part[g][j] = kv;
        __syncthreads();
        const float kv_mem = ((part[0][j] + part[1][j]) + part[2][j]) + part[3][j];
        const float dlt = (cv[m][j] - kv_mem) * beta;
        float o = 0.0f;
#pragma unroll
        for (int r = 0; r < kRowsPer; ++r) {
            s[r] = fmaf(ks[g * kRowsPer + r], dlt, s[r]);
            o = fmaf(s[r], qs[g * kRowsPer + r], o);
        }
        __syncthreads();
        part[g][j] = o;
        __syncthreads();
        const float oj = ((part[0][j] + part[1][j]) + part[2][j]) + part[3][j];
        // gated RMS norm over the head's 128 outputs (linear.wgsl:131-133), plain w
        const float ss = block_sum<kThreads>(g == 0 ? oj * oj : 0.0f, red);
        if (g == 0) {
            const float z = prow[z_off + h * DV + j];
            const float var_o = ss / (float)DV;
            a.out[(size_t)m * a.n_v * DV + h * DV + j] =
                ((oj * (1.0f / sqrtf(var_o + a.eps))) * norm_w) * (z / (1.0f + expf(-z)));
        }
        if (m + 1 == ckpt) {
            float* SC = a.state + (size_t)s_ck * a.state_slot + hoff;
#pragma unroll
            for (int r = 0; r < kRowsPer; ++r) SC[(size_t)(g * kRowsPer + r) * DV + j] = s[r];
        }
        __syncthreads();
    }
    float* SO = a.state + (size_t)s_out * a.state_slot + hoff;
#pragma unroll
    for (int r = 0; r < kRowsPer; ++r) SO[(size_t)(g * kRowsPer + r) * DV + j] = s[r];
}

}  // namespace

int launch_deltanet(const DeltaArgs& a, int M, hipStream_t s) {
    if (a.n_k < 1 || a.n_v % a.n_k) return -1;
    switch (M) {
        case 1: hipLaunchKernelGGL(deltanet_kernel<1>, dim3(a.n_v), dim3(kThreads), 0, s, a); break;
        case 2: hipLaunchKernelGGL(deltanet_kernel<2>, dim3(a.n_v), dim3(kThreads), 0, s, a); break;
        case 3: hipLaunchKernelGGL(deltanet_kernel<3>, dim3(a.n_v), dim3(kThreads), 0, s, a); break;
        case 4: hipLaunchKernelGGL(deltanet_kernel<4>, dim3(a.n_v), dim3(kThreads), 0, s, a); break;
        default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace snl
