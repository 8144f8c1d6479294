// Gated DeltaNet decode step: causal depthwise conv (k=4) + SiLU, then the recurrent gated delta
// rule with L2-normalised q/k, for M = 1..4 tokens (src/shaders/linear.wgsl:38-140 conv + delta,
// fused into one launch).  Of the gated RMS norm over each head's 128 outputs (linear.wgsl:131-133),
// out = ((o * rsqrt(mean(o^2) + eps)) * w) * silu(z), this kernel applies the per-column part: it
// writes (o * w) * silu(z) and, per (token, head, column group), the partial sum of o^2.  The
// consumer multiplies by the head's rsqrt factor (the out_proj GEMV prologue, or
// gated_norm_kernel for the kernel-level entry).
//
// The recurrence of state column j only reads column j (kv_mem_j = sum_i S[i][j] k_i, then
// S[:, j] += k (v_j - kv_mem_j) beta, o_j = sum_i S[i][j] q_i), so each value head's 128 columns
// split over kCG blocks of kCols columns: 4 * n_v blocks, each streaming a quarter of the head's
// state.  Thread (wave w, lane c + 4 rg) owns column 4w + c of the group, rows [8 rg, 8 rg + 8);
// the sums over rows are 16-lane butterflies, so the token loop has no block barrier.
//
// Recurrent state lives in three slots per visit.  A call reads slot s_in, writes the state
// after its last token to s_out and, when ckpt > 0, the state after token ckpt-1 to s_ck; s_out
// and s_ck are never s_in, so no block overwrites what another block still reads (the blocks of
// the v-heads that share a k-head all read its conv channels).  A rejected draft becomes a change
// of the current slot on the host instead of a copy.
#include "common.h"
#include "kernels.h"

#pragma clang fp contract(off)

namespace snl {

namespace {

constexpr int DK = 128, DV = 128;
constexpr int kCG = kDeltaGroups, kCols = DV / kCG;  // column groups per head, columns per group
constexpr int kThreads = 512, kWaves = kThreads / 64, kRows = 8;  // rows per thread

template <int M>
__global__ __launch_bounds__(kThreads) void deltanet_kernel(DeltaArgs a) {
    __shared__ float cq[M][DK], ck[M][DK], cv[M][kCols];  // conv outputs (SiLU applied)
    __shared__ float red[kWaves][M];                       // q / k sums of squares (waves 0-3)
    __shared__ float ored[kWaves][M];                      // sums of o^2 per wave

    const StepDev* st = a.step;
    const int h = blockIdx.x / kCG, cg = blockIdx.x - (blockIdx.x / kCG) * kCG;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 3, rg = lane >> 2;
    const int jl = 4 * wave + c, j = cg * kCols + jl;  // column in the group, in the head
    const int group = a.n_v / a.n_k, kh = h / group;
    const int key_dim = a.n_k * DK, cd = a.conv_dim;
    const int b_off = cd + a.n_v * DV, a_off = b_off + a.n_v;

    // ---- every load up front: first those that do not need the step record (the slots: a scalar
    // load that depends on another), the conv state of all three slots among them, then the state
    // slice ----
    // conv lanes: tid < 128 q channel, < 256 k channel, < 288 v channel of this column group
    const int which = tid < DK ? 0 : tid < 2 * DK ? 1 : tid < 2 * DK + kCols ? 2 : 3;
    const int ch = which == 0 ? kh * DK + tid
                 : which == 1 ? key_dim + kh * DK + (tid - DK)
                              : 2 * key_dim + h * DV + cg * kCols + (tid - 2 * DK);
    // (branch-free: the other lanes read zeros through the buffer range, so no wait is forced)
    const bool cl = which < 3;
    const __amdgpu_buffer_rsrc_t lr = buffer_range(a.lw, (unsigned)cd * 16u);
    const __amdgpu_buffer_rsrc_t pr = buffer_range(a.proj, (unsigned)(M * a.proj_stride) * 4u);
    float w4[4], cur[M];
    {
        const float4 w = load_f32x4_or0(lr, (unsigned)ch * 16u, cl);
        w4[0] = w.x, w4[1] = w.y, w4[2] = w.z, w4[3] = w.w;
#pragma unroll
        for (int m = 0; m < M; ++m) cur[m] = load_f32_or0(pr, (unsigned)(m * a.proj_stride + ch) * 4u, cl);
    }
    const float* lwp = a.lw + (size_t)cd * 4;
    const float a_log = lwp[h], dt_bias = lwp[a.n_v + h], norm_w = lwp[2 * a.n_v + j];
    float zr[M];  // the output gate of column j
#pragma unroll
    for (int m = 0; m < M; ++m) zr[m] = load_f32_or0(pr, (unsigned)(m * a.proj_stride + cd + h * DV + j) * 4u, rg == 0);
    float rs[3][3];  // conv state row i of slot k
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const __amdgpu_buffer_rsrc_t sr = buffer_range(a.conv_state + (size_t)k * a.conv_slot, (unsigned)cd * 12u);
#pragma unroll
        for (int i = 0; i < 3; ++i) rs[k][i] = load_f32_or0(sr, (unsigned)(i * cd + ch) * 4u, cl);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int s_in = st->s_in, s_out = st->s_out, s_ck = st->s_ck, ckpt = st->ckpt;
    // the state slice last: vector loads return in issue order, so the conv waits only for its
    // own inputs and runs while the state is in flight
    __builtin_amdgcn_sched_barrier(0);
    const size_t hoff = (size_t)h * DK * DV;
    const float* S0 = a.state + (size_t)s_in * a.state_slot + hoff;
    float s[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) s[r] = S0[(size_t)(kRows * rg + r) * DV + j];
    __builtin_amdgcn_sched_barrier(0);
    float r0 = s_in == 0 ? rs[0][0] : s_in == 1 ? rs[1][0] : rs[2][0];
    float r1 = s_in == 0 ? rs[0][1] : s_in == 1 ? rs[1][1] : rs[2][1];
    float r2 = s_in == 0 ? rs[0][2] : s_in == 1 ? rs[1][2] : rs[2][2];
    float gz[M];  // silu of the output gate
#pragma unroll
    for (int m = 0; m < M; ++m) gz[m] = zr[m] / (1.0f + expf(-zr[m]));
    float beta[M], decay[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {  // linear.wgsl:113-117
        const float* prow = a.proj + (size_t)m * a.proj_stride;
        beta[m] = 1.0f / (1.0f + expf(-prow[b_off + h]));
        const float araw = prow[a_off + h] + dt_bias;
        const float sp = araw <= 20.0f ? logf(1.0f + expf(araw)) : araw;
        decay[m] = expf(-expf(a_log) * sp);
    }

    // ---- causal conv (linear.wgsl:38-66) and the q / k sums of squares ----
    float sq[M];
#pragma unroll
    for (int m = 0; m < M; ++m) sq[m] = 0.0f;
    if (which < 3) {
        // the k-head's q/k conv state is owned by the first column group of its first v-head
        const bool owner = which == 2 || ((h % group) == 0 && cg == 0);
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float o = ((w4[0] * r0 + w4[1] * r1) + w4[2] * r2) + w4[3] * cur[m];
            const float v = o / (1.0f + expf(-o));
            if (which == 0) cq[m][tid] = v;
            else if (which == 1) ck[m][tid - DK] = v;
            else cv[m][tid - 2 * DK] = v;
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
    float osq[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        // kv_mem_j = sum_i decay*S[i][j] * k_i
        float kv = 0.0f;
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            s[r] = s[r] * decay[m];
            kv = fmaf(s[r], ck[m][kRows * rg + r] * kscale[m], kv);
        }
        kv = xor_sum<32>(xor_sum<16>(xor_sum<8>(xor_sum<4>(kv))));
        const float dlt = (cv[m][jl] - kv) * beta[m];
        float o = 0.0f;
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            s[r] = fmaf(ck[m][kRows * rg + r] * kscale[m], dlt, s[r]);
            o = fmaf(s[r], cq[m][kRows * rg + r] * qscale[m], o);
        }
        o = xor_sum<32>(xor_sum<16>(xor_sum<8>(xor_sum<4>(o))));
        if (rg == 0) a.out[(size_t)m * a.n_v * DV + h * DV + j] = (o * norm_w) * gz[m];
        // this wave's 4 columns: o^2 added over lanes 0-3
        float q2 = o * o;
        q2 = xor_sum<1>(q2);
        q2 = xor_sum<2>(q2);
        osq[m] = q2;
        if (m + 1 == ckpt) {
            float* SC = a.state + (size_t)s_ck * a.state_slot + hoff;
#pragma unroll
            for (int r = 0; r < kRows; ++r) SC[(size_t)(kRows * rg + r) * DV + j] = s[r];
        }
    }
    float* SO = a.state + (size_t)s_out * a.state_slot + hoff;
#pragma unroll
    for (int r = 0; r < kRows; ++r) SO[(size_t)(kRows * rg + r) * DV + j] = s[r];

    // partial sums of o^2 of this column group, waves in order
    if (lane == 0)
#pragma unroll
        for (int m = 0; m < M; ++m) ored[wave][m] = osq[m];
    __syncthreads();
    if (tid < M) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) t = t + ored[w][tid];
        a.ssq[((size_t)tid * a.n_v + h) * kCG + cg] = t;
    }
}

// The head factor of the gated RMS norm (linear.wgsl:131-133) in place, for the kernel-level
// entry: block (head, token), thread j: out *= rsqrt(mean(o^2) + eps), the mean from the
// column-group partials added in order.
__global__ __launch_bounds__(DV) void gated_norm_kernel(DeltaArgs a) {
    const int h = blockIdx.x, m = blockIdx.y, j = threadIdx.x;
    const float* ps = a.ssq + ((size_t)m * a.n_v + h) * kCG;
    const float var_o = (((ps[0] + ps[1]) + ps[2]) + ps[3]) / (float)DV;
    float* o = a.out + (size_t)m * a.n_v * DV + h * DV + j;
    *o = *o * (1.0f / sqrtf(var_o + a.eps));
}

}  // namespace

int launch_deltanet(const DeltaArgs& a, int M, hipStream_t s) {
    if (a.n_k < 1 || a.n_v % a.n_k || !a.ssq) return -1;
    const dim3 grid(a.n_v * kCG);
    switch (M) {
        case 1: hipLaunchKernelGGL(deltanet_kernel<1>, grid, dim3(kThreads), 0, s, a); break;
        case 2: hipLaunchKernelGGL(deltanet_kernel<2>, grid, dim3(kThreads), 0, s, a); break;
        case 3: hipLaunchKernelGGL(deltanet_kernel<3>, grid, dim3(kThreads), 0, s, a); break;
        case 4: hipLaunchKernelGGL(deltanet_kernel<4>, grid, dim3(kThreads), 0, s, a); break;
        default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_deltanet_norm(const DeltaArgs& a, int M, hipStream_t s) {
    if (M < 1 || M > 4 || !a.ssq) return -1;
    hipLaunchKernelGGL(gated_norm_kernel, dim3(a.n_v, M), dim3(DV), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace snl
