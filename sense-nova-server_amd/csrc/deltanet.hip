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
constexpr int kWaves = kThreads / 64;

// Critical path per token: two barriers (the column sums of S^T k and S^T q).  Everything that
// does not depend on the recurrence -- conv, q/k norms, beta and decay, the gate z -- is loaded
// and computed before the token loop, and the gated RMS norm of all tokens runs after it.
template <int M>
__global__ __launch_bounds__(kThreads) void deltanet_kernel(DeltaArgs a) {
    __shared__ float cq[M][DK], ck[M][DK], cv[M][DV];  // conv outputs (SiLU applied)
    __shared__ float kvp[2][4][DV], op[2][4][DV];       // column partials, double-buffered by token
    __shared__ float ob[M][DV];                          // head outputs before the gated norm
    __shared__ float red[kWaves][2 * M];

    const StepDev* st = a.step;
    const int s_in = st->s_in, s_out = st->s_out, s_ck = st->s_ck, ckpt = st->ckpt;
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = tid & (DV - 1), g = tid >> 7;
    const int group = a.n_v / a.n_k, kh = h / group;
    const int key_dim = a.n_k * DK, cd = a.conv_dim;
    const int z_off = cd, b_off = cd + a.n_v * DV, a_off = b_off + a.n_v;

    // ---- every load up front: conv inputs, recurrent state, gate, per-token scalars ----
    const int which = tid >> 7, c0 = tid & 127;  // conv lanes: tid < 384
    const int ch = which == 0 ? kh * DK + c0 : which == 1 ? key_dim + kh * DK + c0 : 2 * key_dim + h * DV + c0;
    float w4[4] = {0.0f, 0.0f, 0.0f, 0.0f}, r0 = 0.0f, r1 = 0.0f, r2 = 0.0f, cur[M];
    if (tid < 3 * DK) {
        const float4 w = *reinterpret_cast<const float4*>(a.lw + (size_t)ch * 4);
        w4[0] = w.x, w4[1] = w.y, w4[2] = w.z, w4[3] = w.w;
        const float* cs = a.conv_state + (size_t)s_in * a.conv_slot;
        r0 = cs[ch];
        r1 = cs[cd + ch];
        r2 = cs[2 * cd + ch];
#pragma unroll
        for (int m = 0; m < M; ++m) cur[m] = a.proj[(size_t)m * a.proj_stride + ch];
    }
    const size_t hoff = (size_t)h * DK * DV;
    const float* S0 = a.state + (size_t)s_in * a.state_slot + hoff;
    float s[kRowsPer];
#pragma unroll
    for (int r = 0; r < kRowsPer; ++r) s[r] = S0[(size_t)(g * kRowsPer + r) * DV + j];
    float z[M];
#pragma unroll
    for (int m = 0; m < M; ++m) z[m] = g == 0 ? a.proj[(size_t)m * a.proj_stride + z_off + h * DV + j] : 0.0f;
    const float* lwp = a.lw + (size_t)cd * 4;
    const float a_log = lwp[h], dt_bias = lwp[a.n_v + h], norm_w = lwp[2 * a.n_v + j];
    float beta[M], decay[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {  // linear.wgsl:113-117
        const float* prow = a.proj + (size_t)m * a.proj_stride;
        beta[m] = 1.0f / (1.0f + expf(-prow[b_off + h]));
        const float araw = prow[a_off + h] + dt_bias;
        const float sp = araw <= 20.0f ? logf(1.0f + expf(araw)) : araw;
        decay[m] = expf(-expf(a_log) * sp);
    }

    // ---- causal conv (linear.wgsl:38-66) of this head's channels, and the q/k sums of squares ----
    float sq[M];
#pragma unroll
    for (int m = 0; m < M; ++m) sq[m] = 0.0f;
    if (tid < 3 * DK) {
        // k-head channels are shared by `group` v-heads: the first one owns their state
        const bool owner = which == 2 || (h % group) == 0;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float o = ((w4[0] * r0 + w4[1] * r1) + w4[2] * r2) + w4[3] * cur[m];
            const float v = o / (1.0f + expf(-o));
            if (which == 0) cq[m][c0] = v;
            else if (which == 1) ck[m][c0] = v;
            else cv[m][c0] = v;
            if (which < 2) sq[m] = v * v;
            r0 = r1;
            r1 = r2;
            r2 = cur[m];
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
    // waves 0-1 hold the q channels, waves 2-3 the k channels (linear.wgsl:104-110)
    wave_sum_n(sq);
    if (lane == 0 && wave < 4)
#pragma unroll
        for (int m = 0; m < M; ++m) red[wave][m] = sq[m];
    __syncthreads();
    float qscale[M], kscale[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        qscale[m] = (1.0f / sqrtf((red[0][m] + red[1][m]) + 1e-6f)) * (1.0f / sqrtf((float)DK));
        kscale[m] = 1.0f / sqrtf((red[2][m] + red[3][m]) + 1e-6f);
    }

    // ---- the recurrence, token by token (linear.wgsl:118-136) ----
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const int b = m & 1;
        // kv_mem_j = sum_i decay*S[i][j] * k_i
        float kv = 0.0f;
#pragma unroll
        for (int r = 0; r < kRowsPer; ++r) {
            s[r] = s[r] * decay[m];
            kv = fmaf(s[r], ck[m][g * kRowsPer + r] * kscale[m], kv);
        }
        kvp[b][g][j] = kv;
        __syncthreads();
        const float kv_mem = ((kvp[b][0][j] + kvp[b][1][j]) + kvp[b][2][j]) + kvp[b][3][j];
        const float dlt = (cv[m][j] - kv_mem) * beta[m];
        float o = 0.0f;
#pragma unroll
        for (int r = 0; r < kRowsPer; ++r) {
            s[r] = fmaf(ck[m][g * kRowsPer + r] * kscale[m], dlt, s[r]);
            o = fmaf(s[r], cq[m][g * kRowsPer + r] * qscale[m], o);
        }
        op[b][g][j] = o;
        __syncthreads();
        if (g == 0) ob[m][j] = ((op[b][0][j] + op[b][1][j]) + op[b][2][j]) + op[b][3][j];
        if (m + 1 == ckpt) {
            float* SC = a.state + (size_t)s_ck * a.state_slot + hoff;
#pragma unroll
            for (int r = 0; r < kRowsPer; ++r) SC[(size_t)(g * kRowsPer + r) * DV + j] = s[r];
        }
    }
    float* SO = a.state + (size_t)s_out * a.state_slot + hoff;
#pragma unroll
    for (int r = 0; r < kRowsPer; ++r) SO[(size_t)(g * kRowsPer + r) * DV + j] = s[r];

    // ---- gated RMS norm over the head's 128 outputs (linear.wgsl:131-133), plain w ----
    float ss[M];
#pragma unroll
    for (int m = 0; m < M; ++m) ss[m] = g == 0 ? ob[m][j] * ob[m][j] : 0.0f;
    wave_sum_n(ss);
    if (lane == 0 && wave < 2)
#pragma unroll
        for (int m = 0; m < M; ++m) red[wave][M + m] = ss[m];
    __syncthreads();
    if (g == 0)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float var_o = (red[0][M + m] + red[1][M + m]) / (float)DV;
            const float oj = ob[m][j];
            a.out[(size_t)m * a.n_v * DV + h * DV + j] =
                ((oj * (1.0f / sqrtf(var_o + a.eps))) * norm_w) * (z[m] / (1.0f + expf(-z[m])));
        }
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
