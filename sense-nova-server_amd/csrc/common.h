// Shared device helpers and launch descriptors for the MTP decode-step kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define SNL_WAVE 64

// Largest token count one decode-kernel launch handles (rows of x / proj / logits).
#define SNL_MAX_M 4

#define SNL_HIP_CHECK(expr)                                      \
    do {                                                         \
        hipError_t _e = (expr);                                  \
        if (_e != hipSuccess) return snl::device_error(_e, #expr); \
    } while (0)

namespace snl {

int device_error(hipError_t e, const char* what);

// Per-call device-side step record.  The host writes it (one small copy) before
// replaying a captured pass, so a captured graph never bakes in a position.
struct StepDev {
    int32_t pos0;   // cache position of row 0
    int32_t m;      // rows in this call
    int32_t ckpt;   // > 0: also save the recurrent state after row ckpt-1
    int32_t s_in;   // recurrent-state slot read
    int32_t s_out;  // recurrent-state slot written after the last row
    int32_t s_ck;   // recurrent-state slot written after row ckpt-1
    int32_t r0;     // MTP: first row of `hid` paired with tokens[0]
    int32_t x_off;  // MTP draft head: the row whose logits give the draft
    uint32_t draft_rows;  // bit m set: row m's token is the MTP draft's pick on the device, not tokens[m]
    uint32_t seq;         // speculative step number (the outcome ring's index)
    uint32_t tokens[SNL_MAX_M];
    uint32_t rpos[SNL_MAX_M][4];  // rotary (t, h, w, 0) position of each row
    // cos and sin of each row's rotary angles (attention.wgsl:90-110), formed on the host with
    // the row's positions: rope[m][f] for frequency f < rot_dim / 2 (SNL_ROPE_MAX at most)
    float rope[SNL_MAX_M][64][2];
};
#define SNL_ROPE_MAX 64

// Token rows of one prefill pass (chunked prefill and the MTP head's catch-up over a prompt).
#define SNL_PF_M 512
struct PrefillDev {
    int32_t pos0;   // cache position of row 0
    int32_t m;      // rows
    int32_t _pad[2];
    uint32_t tokens[SNL_PF_M];
    uint32_t rpos[SNL_PF_M][4];  // rotary (t, h, w, 0) position of each row
};

// ---- butterfly exchanges in vector registers ----
// lane_xor<O>(v), O = 1, 2, 4, 8: the v of lane l ^ O, by DPP inside each 16-lane row (quad
// permutes for 1 and 2; row shifts by 4 under bank masks, banks 0 and 2 reading l + 4 and banks 1
// and 3 reading l - 4; a row rotation by 8).  xor_sum<O> / xor_max<O> add / take the max of v and
// lane l ^ O's v; for O = 16 and 32 the gfx950 permlane swaps bring the pair together, and both
// lanes combine (lower lane's value, upper lane's value), the same result as v + __shfl_xor(v, O)
// since the operation commutes.  None of them goes through the LDS as ds_bpermute does.
template <int O>
__device__ __forceinline__ float lane_xor(float v) {
    static_assert(O == 1 || O == 2 || O == 4 || O == 8, "DPP exchange inside a row");
    const int x = __float_as_int(v);
    if constexpr (O == 1) return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));
    else if constexpr (O == 2) return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));
    else if constexpr (O == 4) {
        const int t = __builtin_amdgcn_update_dpp(x, x, 0x104, 0xF, 0x5, false);  // row_shl:4, banks 0, 2
        return __int_as_float(__builtin_amdgcn_update_dpp(t, x, 0x114, 0xF, 0xA, false));  // row_shr:4, 1, 3
    } else {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false));  // row_ror:8
    }
}

// the 32-bit word of lane l ^ O, any O from 1 to 32 (permlane swaps for 16 and 32: of the swapped
// pair, a lane takes the half that came from its partner)
template <int O>
__device__ __forceinline__ uint32_t lane_xor_bits(uint32_t x) {
    if constexpr (O == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        return (threadIdx.x & 32) ? r[0] : r[1];
    } else if constexpr (O == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        return (threadIdx.x & 16) ? r[0] : r[1];
    } else {
        return __float_as_uint(lane_xor<O>(__uint_as_float(x)));
    }
}

// lane_xor for an exchange distance known once the caller's loop is unrolled (1, 2, 4, 8)
__device__ __forceinline__ float lane_xor_n(float v, int o) {
    switch (o) {
        case 1: return lane_xor<1>(v);
        case 2: return lane_xor<2>(v);
        case 4: return lane_xor<4>(v);
        case 8: return lane_xor<8>(v);
        default: return __shfl_xor(v, o, SNL_WAVE);
    }
}

template <int O>
__device__ __forceinline__ float xor_sum(float v) {
    if constexpr (O == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else if constexpr (O == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else {
        return v + lane_xor<O>(v);
    }
}

template <int O>
__device__ __forceinline__ float xor_max(float v) {
    if constexpr (O == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    } else if constexpr (O == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    } else {
        return fmaxf(v, lane_xor<O>(v));
    }
}

__device__ __forceinline__ float wave_sum(float v) {
    v = xor_sum<32>(v);
    v = xor_sum<16>(v);
    v = xor_sum<8>(v);
    v = xor_sum<4>(v);
    v = xor_sum<2>(v);
    return xor_sum<1>(v);
}

// N independent wave sums, level by level so the N exchanges of a level overlap; each value gets
// exactly the additions of wave_sum.
template <int N>
__device__ __forceinline__ void wave_sum_n(float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = xor_sum<32>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = xor_sum<16>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = xor_sum<8>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = xor_sum<4>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = xor_sum<2>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = xor_sum<1>(v[i]);
}

template <int N>
__device__ __forceinline__ void wave_max_n(float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = xor_max<32>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = xor_max<16>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = xor_max<8>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = xor_max<4>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = xor_max<2>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = xor_max<1>(v[i]);
}

__device__ __forceinline__ float wave_max(float v) {
    v = xor_max<32>(v);
    v = xor_max<16>(v);
    v = xor_max<8>(v);
    v = xor_max<4>(v);
    v = xor_max<2>(v);
    return xor_max<1>(v);
}

// Raw buffer descriptor over [base, base + bytes) (gfx9 raw dword format in word 3): a load at
// or past `bytes` returns 0 and touches no memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_range(const void* base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Loads that read 0 instead of memory when `ok` is false, without a branch: the offset moves past
// the descriptor's range.  (A load under a condition whose other side sets a constant makes the
// compiler wait for the load where the two sides join, i.e. right after issuing it, which
// serialises the memory round trips of the loads that follow.)
constexpr unsigned kPastRange = 0xFFFFFF00u;
__device__ __forceinline__ float load_f32_or0(__amdgpu_buffer_rsrc_t r, unsigned off, bool ok) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)(ok ? off : kPastRange), 0, 0));
}
__device__ __forceinline__ float4 load_f32x4_or0(__amdgpu_buffer_rsrc_t r, unsigned off, bool ok) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(ok ? off : kPastRange), 0, 0));
}

// Sum over a block of NT threads (NT a multiple of 64, at most 1024); every thread gets the total.
// The order is fixed by the thread layout, so the result does not depend on anything else.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
    constexpr int NW = NT / SNL_WAVE;
    v = wave_sum(v);
    const int lane = threadIdx.x & (SNL_WAVE - 1), w = threadIdx.x / SNL_WAVE;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < NW; ++i) t += red[i];
    return t;
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

// mHC router dots of one token -> [pre0, pre1, post0, post1, mix00, mix01, mix10, mix11]
// (layers.wgsl:94-126): raw = 8 router-row dots and the sum of squares of the 2-stream row of
// length d; bias = the router's 8 biases.  The 2x2 mix is `iterations` Sinkhorn steps (rows,
// then columns).  The reference runs them in log space, p -= log(exp(p) + exp(q)); here they run
// on the exponentiated matrix, a /= a + b, which is the same iteration in exact arithmetic at a
// reciprocal per row instead of an exp and a log, on one thread's critical path.  Exponents are
// taken relative to the largest logit and floored at -80, so no entry underflows.
__device__ inline void mhc_coefficients_b(const float* raw, const float (&bias)[8], int d, int iterations, float* cf) {
    const float rinv = 1.0f / sqrtf(raw[8] / (float)d + 1e-6f);
    float lg[8];
#pragma unroll
    for (int o = 0; o < 8; ++o) lg[o] = raw[o] * rinv + bias[o];
    const float mx = fmaxf(fmaxf(lg[4], lg[5]), fmaxf(lg[6], lg[7]));
    float a = __expf(fmaxf(lg[4] - mx, -80.0f)), b = __expf(fmaxf(lg[5] - mx, -80.0f));
    float c = __expf(fmaxf(lg[6] - mx, -80.0f)), e = __expf(fmaxf(lg[7] - mx, -80.0f));
    for (int it = 0; it < iterations; ++it) {
        const float r0 = __builtin_amdgcn_rcpf(a + b), r1 = __builtin_amdgcn_rcpf(c + e);
        a = a * r0;
        b = b * r0;
        c = c * r1;
        e = e * r1;
        const float c0 = __builtin_amdgcn_rcpf(a + c), c1 = __builtin_amdgcn_rcpf(b + e);
        a = a * c0;
        c = c * c0;
        b = b * c1;
        e = e * c1;
    }
    cf[0] = 1.0f / (1.0f + __expf(-lg[0]));
    cf[1] = 1.0f / (1.0f + __expf(-lg[1]));
    cf[2] = 2.0f / (1.0f + __expf(-lg[2]));
    cf[3] = 2.0f / (1.0f + __expf(-lg[3]));
    cf[4] = a;
    cf[5] = b;
    cf[6] = c;
    cf[7] = e;
}
// the same with the biases read from the router (mhc_w = router [8][d] then bias[8])
__device__ inline void mhc_coefficients(const float* raw, const float* mhc_w, int d, int iterations, float* cf) {
    float bias[8];
#pragma unroll
    for (int o = 0; o < 8; ++o) bias[o] = mhc_w[(size_t)8 * d + o];
    mhc_coefficients_b(raw, bias, d, iterations, cf);
}
__device__ __forceinline__ float sigmoidf_(float v) { return 1.0f / (1.0f + expf(-v)); }

}  // namespace snl
