// Per-token kernels of the chunked prefill pass (up to 512 token rows per launch): the embedding
// gather, the mHC token coefficients, and the Gated DeltaNet over a chunk.
//
// DeltaNet (src/shaders/linear.wgsl:38-140).  The causal conv, SiLU, q/k L2 normalisation and the
// per-token gates do not depend on the recurrent state, so they run for every token of the chunk
// at once (dn_conv_kernel, one block per (token, head)); the conv state then takes the chunk's
// last three inputs (dn_conv_state_kernel).  The recurrence itself runs token by token in
// dn_recur_kernel with the decode kernel's per-thread layout (8 rows of one state column): 8
// blocks of 4 waves per value head, each owning 16 state columns in registers.  The tokens go
// through the state 4 at a time in the blocked form of the delta rule (dn_pairs_kernel forms the
// block's k.k and k.q scalars); the sums over a column's 128 rows run as DPP rotations inside
// 16-lane rows plus two cross-row exchanges.  The
// tokens' inputs stream through LDS in slices of 16.  The state is updated in place in the
// current slot (a prefill pass has no checkpoint).
#include "common.h"
#include "kernels.h"

#pragma clang fp contract(off)

namespace snl {

namespace {

constexpr int DK = 128, DV = 128;
// the recurrence: 8 blocks of 16 state columns per value head, 4 waves each (one wave per SIMD
// on every CU for the 32 value heads of the 9B shape)
constexpr int kCG = kDeltaPrefillGroups, kCols = DV / kCG;
constexpr int kThreads = 256, kWaves = kThreads / 64, kRows = 8;

// x[m, 0:h] = dequant(embed[tokens[m]]), x[m, h:2h] = 0 (src/engine.rs:777-790)
__global__ __launch_bounds__(256) void pf_embed_kernel(const uint32_t* tokens, const int8_t* eq, const float* es,
                                                        int vocab, int h, float* x) {
    const int m = blockIdx.x;
    uint32_t tok = tokens[m];
    if (tok >= (uint32_t)vocab) tok = 0;  // the host rejects out-of-range ids before launching
    const int8_t* q = eq + (size_t)tok * h;
    const float* s = es + (size_t)tok * (h / 32);
    float* xr = x + (size_t)m * 2 * h;
    for (int i = threadIdx.x; i < h; i += 256) {
        xr[i] = (float)q[i] * s[i >> 5];
        xr[h + i] = 0.0f;
    }
}

// coef[m] = mhc_coefficients of the token's router sums part[m][0..8] (layers.wgsl:94-126)
__global__ __launch_bounds__(64) void mhc_coef_kernel(const float* part, const float* w, int d, int iterations,
                                                       float* coef, int M) {
    const int m = blockIdx.x * 64 + threadIdx.x;
    if (m >= M) return;
    mhc_coefficients(part + (size_t)m * 9, w, d, iterations, coef + (size_t)m * 8);
}

// Block (token m, slot): slots [0, n_k) the q heads, [n_k, 2n_k) the k heads, then the v heads.
// 128 threads, one channel each (linear.wgsl:38-66, :104-117).
__global__ __launch_bounds__(128) void dn_conv_kernel(DnPrefillArgs a) {
    __shared__ float red[2];
    const int m = blockIdx.x, slot = blockIdx.y, tid = threadIdx.x;
    const int n_k = a.n_k, n_v = a.n_v, cd = a.conv_dim, key_dim = n_k * DK;
    const int kind = slot < n_k ? 0 : slot < 2 * n_k ? 1 : 2;
    const int head = kind == 0 ? slot : kind == 1 ? slot - n_k : slot - 2 * n_k;
    const int ch = kind == 0 ? head * DK + tid : kind == 1 ? key_dim + head * DK + tid : 2 * key_dim + head * DV + tid;
    const float4 w = *reinterpret_cast<const float4*>(a.lw + (size_t)ch * 4);
    // input t of the chunk: proj row t, or conv state row 3 + t for t < 0 (oldest first)
    float in[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = m - 3 + i;
        in[i] = t >= 0 ? a.proj[(size_t)t * a.proj_stride + ch] : a.conv_state[(size_t)(3 + t) * cd + ch];
    }
    const float o = ((w.x * in[0] + w.y * in[1]) + w.z * in[2]) + w.w * in[3];
    const float v = o / (1.0f + expf(-o));
    if (kind == 2) {
        a.v[((size_t)m * n_v + head) * DV + tid] = v;
        const float z = a.proj[(size_t)m * a.proj_stride + cd + head * DV + tid];
        a.gz[((size_t)m * n_v + head) * DV + tid] = z / (1.0f + expf(-z));
        if (tid == 0) {  // linear.wgsl:113-117
            const float* lwp = a.lw + (size_t)cd * 4;
            const float* prow = a.proj + (size_t)m * a.proj_stride;
            const int b_off = cd + n_v * DV, a_off = b_off + n_v;
            a.beta[(size_t)m * n_v + head] = 1.0f / (1.0f + expf(-prow[b_off + head]));
            const float araw = prow[a_off + head] + lwp[n_v + head];
            const float sp = araw <= 20.0f ? logf(1.0f + expf(araw)) : araw;
            a.decay[(size_t)m * n_v + head] = expf(-expf(lwp[head]) * sp);
        }
        return;
    }
    // L2 normalisation over the head's 128 channels (two wave sums, added in wave order)
    const float s = wave_sum(v * v);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    if (kind == 0) {
        const float qs = (1.0f / sqrtf((red[0] + red[1]) + 1e-6f)) * (1.0f / sqrtf((float)DK));
        a.q[((size_t)m * n_k + head) * DK + tid] = v * qs;
    } else {
        const float ks = 1.0f / sqrtf((red[0] + red[1]) + 1e-6f);
        a.k[((size_t)m * n_k + head) * DK + tid] = v * ks;
    }
}

// Blocked recurrence: the chunk's tokens go through the state kBlk at a time.  Inside a block
// the scalars k_b.k_c (c < b) and k_c.q_b (c <= b) do not depend on the state; they are the same
// for every state column, so one block per (kBlk tokens, key head) forms them here (128 threads, one
// channel each; wave sums, the two waves added in order).
// 4 tokens per block measured best (190 us per 512-row visit token by token; 166 / 159 / 187 us
// for blocks of 2 / 4 / 8: the triangular scalar work grows as the square of the block)
constexpr int kBlk = 4, kKK = kBlk * (kBlk - 1) / 2, kPairs = kBlk * kBlk;
__device__ __forceinline__ int kk_idx(int b, int c) { return b * (b - 1) / 2 + c; }       // c < b
__device__ __forceinline__ int kq_idx(int c, int b) { return kKK + b * (b + 1) / 2 + c; } // c <= b

__global__ __launch_bounds__(128) void dn_pairs_kernel(DnPrefillArgs a, int M) {
    __shared__ float red[2][kPairs];
    const int blk = blockIdx.x, kh = blockIdx.y, tid = threadIdx.x, n_k = a.n_k;
    float kd[kBlk], qd[kBlk];
#pragma unroll
    for (int b = 0; b < kBlk; ++b) {
        const int t = blk * kBlk + b;
        kd[b] = t < M ? a.k[((size_t)t * n_k + kh) * DK + tid] : 0.0f;
        qd[b] = t < M ? a.q[((size_t)t * n_k + kh) * DK + tid] : 0.0f;
    }
    float v[kPairs];
#pragma unroll
    for (int b = 1; b < kBlk; ++b)
#pragma unroll
        for (int c = 0; c < b; ++c) v[kk_idx(b, c)] = kd[b] * kd[c];
#pragma unroll
    for (int b = 0; b < kBlk; ++b)
#pragma unroll
        for (int c = 0; c <= b; ++c) v[kq_idx(c, b)] = kd[c] * qd[b];
    wave_sum_n(v);
    if ((tid & 63) == 0)
#pragma unroll
        for (int i = 0; i < kPairs; ++i) red[tid >> 6][i] = v[i];
    __syncthreads();
    if (tid < kPairs) a.pairs[((size_t)blk * n_k + kh) * kPairs + tid] = red[0][tid] + red[1][tid];
}

// conv state := the chunk's last three inputs (from the old state when the chunk is shorter)
__global__ __launch_bounds__(256) void dn_conv_state_kernel(DnPrefillArgs a, int M) {
    const int ch = blockIdx.x * 256 + threadIdx.x;
    const int cd = a.conv_dim;
    if (ch >= cd) return;
    float r[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int t = M - 3 + i;
        r[i] = t >= 0 ? a.proj[(size_t)t * a.proj_stride + ch] : a.conv_state[(size_t)(3 + t) * cd + ch];
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) a.conv_state[(size_t)i * cd + ch] = r[i];
}

// Sum over the 16 row groups (lane >> 2) of the lanes that share lane & 3: rotations by 4 and 8
// inside each 16-lane row (DPP), then the two rows of each half and the two halves (permlane
// swaps).
__device__ __forceinline__ float rowgroup_sum(float v) {
    v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));
    v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
    v = xor_sum<16>(v);
    return xor_sum<32>(v);
}

// The recurrence over the chunk (linear.wgsl:118-136), kCG blocks per value head.  The tokens'
// inputs pass through LDS in slices of kTok tokens, the next slice loaded while this one runs.
constexpr int kTok = 16;
struct RecurSlice {
    float q[kTok][DK], k[kTok][DK];
    float v[kTok][kCols], gz[kTok][kCols];
    float beta[kTok], decay[kTok];
    float pr[kTok / kBlk][kPairs];  // the blocks' k.k / k.q scalars
};

__global__ __launch_bounds__(kThreads) void dn_recur_kernel(DnPrefillArgs a, int M) {
    extern __shared__ float ored[];  // [kWaves][M]
    __shared__ RecurSlice sl[2];
    const int h = blockIdx.x / kCG, cg = blockIdx.x % kCG;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 3, rg = lane >> 2;
    const int jl = 4 * wave + c, j = cg * kCols + jl;
    const int n_k = a.n_k, n_v = a.n_v, group = n_v / n_k, kh = h / group;
    const size_t hoff = (size_t)h * DK * DV;
    float* S = a.state + hoff;
    float s[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) s[r] = S[(size_t)(kRows * rg + r) * DV + j];
    const float norm_w = a.lw[(size_t)a.conv_dim * 4 + 2 * n_v + j];

    // slice loader: thread t takes q/k float4s t, t + kThreads, ... (kTok * 2 * DK / 4 = 1024 of
    // them), then v/gz of the group's columns (one per thread) and the per-token scalars.  Tokens
    // past the chunk load as k = q = 0, decay 1, beta 0: they leave the state as it is.
    constexpr int kQK = kTok * 2 * DK / 4 / kThreads;
    static_assert(kTok * kCols == kThreads, "one v / gz value per thread");
    static_assert(kTok % kBlk == 0 && kTok / kBlk * kPairs <= kThreads, "a slice's pair scalars, one per thread");
    float4 rq[kQK];
    float rv = 0.0f, rb = 0.0f, rp = 0.0f;
    const int nblk = (M + kBlk - 1) / kBlk;
    auto load = [&](int m0) {
#pragma unroll
        for (int u = 0; u < kQK; ++u) {
            const int f = tid + kThreads * u;  // 0..1023
            const int which = f >> 9, rem = f & 511, tk = rem >> 5, d4 = rem & 31;
            const int m = min(m0 + tk, M - 1);
            const float* src = (which ? a.k : a.q) + ((size_t)m * n_k + kh) * DK;
            rq[u] = m0 + tk < M ? reinterpret_cast<const float4*>(src)[d4] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        {   // kTok * kCols values of v, one per thread
            const int tk = tid / kCols, col = tid % kCols;
            const int m = min(m0 + tk, M - 1);
            rv = a.v[((size_t)m * n_v + h) * DV + cg * kCols + col];
        }
        {
            const int tk = tid & (kTok - 1), m = min(m0 + tk, M - 1);
            const bool in = m0 + tk < M;
            rb = tid < kTok ? (in ? a.beta[(size_t)m * n_v + h] : 0.0f)
               : tid < 2 * kTok ? (in ? a.decay[(size_t)m * n_v + h] : 1.0f) : 0.0f;
        }
        {
            const int bi = m0 / kBlk + tid / kPairs;
            rp = tid < kTok / kBlk * kPairs && bi < nblk ? a.pairs[((size_t)bi * n_k + kh) * kPairs + tid % kPairs] : 0.0f;
        }
    };
    float rg2 = 0.0f;
    auto load_gz = [&](int m0) {
        const int tk = tid / kCols, col = tid % kCols;
        const int m = min(m0 + tk, M - 1);
        rg2 = a.gz[((size_t)m * n_v + h) * DV + cg * kCols + col];
    };
    auto store = [&](RecurSlice& d) {
#pragma unroll
        for (int u = 0; u < kQK; ++u) {
            const int f = tid + kThreads * u;
            const int which = f >> 9, rem = f & 511, tk = rem >> 5, d4 = rem & 31;
            reinterpret_cast<float4*>(which ? d.k[tk] : d.q[tk])[d4] = rq[u];
        }
        d.v[tid / kCols][tid % kCols] = rv;
        d.gz[tid / kCols][tid % kCols] = rg2;
        if (tid < kTok) d.beta[tid] = rb;
        else if (tid < 2 * kTok) d.decay[tid - kTok] = rb;
        if (tid < kTok / kBlk * kPairs) d.pr[tid / kPairs][tid % kPairs] = rp;
    };
    load(0);
    load_gz(0);
    store(sl[0]);
    __syncthreads();
    for (int m0 = 0; m0 < M; m0 += kTok) {
        const int cur = (m0 / kTok) & 1;
        const bool more = m0 + kTok < M;
        if (more) {
            load(m0 + kTok);
            load_gz(m0 + kTok);
        }
        const RecurSlice& d = sl[cur];
        const int n = min(kTok, M - m0);
        for (int t0 = 0; t0 < n; t0 += kBlk) {
            const int nb = min(kBlk, n - t0);
            // the block's inputs (tokens past the chunk read as k = q = 0, decay 1, beta 0)
            float kf[kBlk][kRows], qf[kBlk][kRows], g[kBlk], be[kBlk], vj[kBlk], gzj[kBlk];
#pragma unroll
            for (int b = 0; b < kBlk; ++b) {
                const int tk = t0 + b;
                const float4* qp = reinterpret_cast<const float4*>(d.q[tk] + kRows * rg);
                const float4* kp = reinterpret_cast<const float4*>(d.k[tk] + kRows * rg);
                const float4 q0 = qp[0], q1 = qp[1], k0 = kp[0], k1 = kp[1];
                qf[b][0] = q0.x, qf[b][1] = q0.y, qf[b][2] = q0.z, qf[b][3] = q0.w;
                qf[b][4] = q1.x, qf[b][5] = q1.y, qf[b][6] = q1.z, qf[b][7] = q1.w;
                kf[b][0] = k0.x, kf[b][1] = k0.y, kf[b][2] = k0.z, kf[b][3] = k0.w;
                kf[b][4] = k1.x, kf[b][5] = k1.y, kf[b][6] = k1.z, kf[b][7] = k1.w;
                g[b] = d.decay[tk];
                be[b] = d.beta[tk];
                vj[b] = d.v[tk][jl];
                gzj[b] = d.gz[tk][jl];
            }
            // the starting state against the block's keys and queries: column j's 128-row sums
            float ak[kBlk], aq[kBlk];
#pragma unroll
            for (int b = 0; b < kBlk; ++b) {
                ak[b] = 0.0f;
                aq[b] = 0.0f;
#pragma unroll
                for (int r = 0; r < kRows; ++r) {
                    ak[b] = fmaf(s[r], kf[b][r], ak[b]);
                    aq[b] = fmaf(s[r], qf[b][r], aq[b]);
                }
            }
#pragma unroll
            for (int b = 0; b < kBlk; ++b) {
                ak[b] = rowgroup_sum(ak[b]);
                aq[b] = rowgroup_sum(aq[b]);
            }
            // With G_b = g_0 ... g_b and P_bc = g_{c+1} ... g_b, token b sees the state
            // G_b S + sum_{c<b} P_bc k_c u_c^T, so its delta (linear.wgsl:118-136) is
            // u_b = (v_b - G_b S^T k_b - sum_{c<b} P_bc (k_c . k_b) u_c) beta_b, its output
            // o_b = G_b S^T q_b + sum_{c<=b} P_bc (k_c . q_b) u_c, and after the block the state
            // is G_3 S + sum_c P_3c k_c u_c^T.
            const float* pr = d.pr[t0 / kBlk];
            float G[kBlk], u[kBlk];
            G[0] = g[0];
#pragma unroll
            for (int b = 1; b < kBlk; ++b) G[b] = G[b - 1] * g[b];
#pragma unroll
            for (int b = 0; b < kBlk; ++b) {
                float kvm = G[b] * ak[b], pbc = 1.0f;
#pragma unroll
                for (int c = b - 1; c >= 0; --c) {
                    pbc = pbc * g[c + 1];
                    kvm = kvm + pbc * pr[kk_idx(b, c)] * u[c];
                }
                u[b] = (vj[b] - kvm) * be[b];
            }
#pragma unroll
            for (int b = 0; b < kBlk; ++b) {
                if (b >= nb) break;
                float o = G[b] * aq[b] + pr[kq_idx(b, b)] * u[b], pbc = 1.0f;
#pragma unroll
                for (int c = b - 1; c >= 0; --c) {
                    pbc = pbc * g[c + 1];
                    o = o + pbc * pr[kq_idx(c, b)] * u[c];
                }
                const int m = m0 + t0 + b;
                if (rg == 0) a.out[(size_t)m * n_v * DV + h * DV + j] = (o * norm_w) * gzj[b];
                float q2 = o * o;
                q2 = xor_sum<1>(q2);
                q2 = xor_sum<2>(q2);
                if (lane == 0) ored[wave * M + m] = q2;
            }
            float pu[kBlk];  // P_3c u_c
            float pc = 1.0f;
            pu[kBlk - 1] = u[kBlk - 1];
#pragma unroll
            for (int c = kBlk - 2; c >= 0; --c) {
                pc = pc * g[c + 1];
                pu[c] = pc * u[c];
            }
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                float acc = G[kBlk - 1] * s[r];
#pragma unroll
                for (int c = 0; c < kBlk; ++c) acc = fmaf(kf[c][r], pu[c], acc);
                s[r] = acc;
            }
        }
        __syncthreads();  // every wave is done with sl[cur ^ 1]'s previous contents
        if (more) store(sl[cur ^ 1]);
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < kRows; ++r) S[(size_t)(kRows * rg + r) * DV + j] = s[r];
    for (int m = tid; m < M; m += kThreads) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) t = t + ored[w * M + m];
        a.ssq[((size_t)m * n_v + h) * kCG + cg] = t;
    }
}

}  // namespace

int launch_embed_tokens(const uint32_t* tokens, const int8_t* eq, const float* es, int vocab, int h, float* x, int M,
                        hipStream_t s) {
    if (M < 1) return -1;
    hipLaunchKernelGGL(pf_embed_kernel, dim3(M), dim3(256), 0, s, tokens, eq, es, vocab, h, x);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_mhc_coef(const float* part, const float* w, int h, int iterations, float* coef, int M, hipStream_t s) {
    if (M < 1) return -1;
    hipLaunchKernelGGL(mhc_coef_kernel, dim3((M + 63) / 64), dim3(64), 0, s, part, w, 2 * h, iterations, coef, M);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

size_t dn_pairs_floats(int M, int n_k) { return (size_t)((M + kBlk - 1) / kBlk) * n_k * kPairs; }

int launch_deltanet_prefill(const DnPrefillArgs& a, int M, hipStream_t s) {
    if (M < 1 || M > SNL_PF_M || a.n_k < 1 || a.n_v % a.n_k) return -1;
    hipLaunchKernelGGL(dn_conv_kernel, dim3(M, 2 * a.n_k + a.n_v), dim3(128), 0, s, a);
    hipLaunchKernelGGL(dn_conv_state_kernel, dim3((a.conv_dim + 255) / 256), dim3(256), 0, s, a, M);
    if (!a.pairs) return -1;
    hipLaunchKernelGGL(dn_pairs_kernel, dim3((M + kBlk - 1) / kBlk, a.n_k), dim3(128), 0, s, a, M);
    hipLaunchKernelGGL(dn_recur_kernel, dim3(a.n_v * kCG), dim3(kThreads), (size_t)kWaves * M * 4, s, a, M);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace snl
