/*
 * CPU oracle: a plain-C restatement of the reference's MTP speculative decode
 * step (dparnell/sense-nova-server, crate `sensenova-loop`).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this file: only tests/, __graft_entry__.smoke() and bench.py's CPU
 * baseline use it, and only as the reference results (or as the timed CPU baseline).
 *
 * Every kernel below follows one WGSL entry point of the reference, in the
 * same arithmetic order where the WGSL fixes it (explicit loops, tree
 * reductions over workgroup lanes, left-to-right vector dots).  Compile with
 * -ffp-contract=off so that a*b+c stays two roundings, as written.  What the
 * WGSL leaves to the driver (FMA contraction, the accuracy of exp/log/
 * inverseSqrt/pow/sin/cos, pack2x16float rounding) is not reproducible here;
 * this file uses IEEE libm and round-to-nearest-even f16 packing.
 *
 * Citations are path:line into the reference repository.
 *
 * How each part is pinned (the reference cannot run here: Rust + wgpu, no
 * toolchain or Vulkan; it ships no test vectors for this path):
 *   f16 packing          numpy float16 (round to nearest even)
 *   Q8_0/Q4_0 quantize   hand-derived known answers, half-away-from-zero ties,
 *                        Q4 sign convention and nibble layout
 *   gemv                 float64 dequant-matmul, one-hot columns, M=1 == rows of M=2
 *   branch_norm          float64, transformers Qwen3_5RMSNorm
 *   mhc_dots/mhc_finish  float64 router and Sinkhorn (doubly stochastic result)
 *   merge, swiglu        closed forms
 *   conv, delta          transformers causal_conv1d_update / recurrent gated delta
 *                        rule and RMSNormGated; decay/beta/normalisation invariants
 *   attn_prep, attend,   float64 RMSNorm + RoPE, transformers rotate-half, brute-force
 *   combine              softmax attention over the f16 cache, split-K invariance
 *   argmax               brute force, first index on ties
 *   engine (forward,     the op order (src/engine.rs:383-570) against an independent
 *   mtp, rollback,       composition of transformers' Qwen3.5 modules over the same
 *   snapshot, generate)  weights (stored logits, tests/golden/composition.npz): plain,
 *                        looped and mHC models, Q8_0 and Q4_0, prefill chunks, verify,
 *                        MTP catch-up and drafts; the mHC router by a zero-router closed
 *                        form; planted mistakes rejected.  Plus self-consistency:
 *                        stepwise == batched, rollback == never run, snapshot/restore,
 *                        MTP on == off.
 *   twin RNG, weights    the engine's own convention (no reference counterpart);
 *                        moments and determinism only.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <stdio.h>

#define ORC_API __attribute__((visibility("default")))

#ifdef _OPENMP
#include <omp.h>
#endif

/* Threads the OpenMP loops of this file use. */
ORC_API int orc_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* Seeded generator shared with the device-side initialiser.                 */
/* splitmix64 (Vigna) as a counter-based hash; normals from an Irwin-Hall    */
/* sum of four 16-bit uniforms, which is exact integer arithmetic plus one   */
/* rounding, so host and device produce identical bits.                      */
/* ------------------------------------------------------------------------ */
static inline uint64_t smix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}
ORC_API uint64_t orc_stream_key(uint64_t seed, uint64_t stream) {
    return smix(seed ^ smix(stream * 0xD1B54A32D192ED03ull));
}
#define ORC_INV_SD 0x1.bb67aep-16f /* 1/sqrt((65536^2-1)/3) */
#define ORC_LN16 0x1.62e43p+1f
ORC_API float orc_randn(uint64_t key, uint64_t i) {
    uint64_t r = smix(key + i);
    int32_t s = (int32_t)(r & 0xFFFF) + (int32_t)((r >> 16) & 0xFFFF) + (int32_t)((r >> 32) & 0xFFFF) +
                (int32_t)(r >> 48);
    return (float)(s - 131070) * ORC_INV_SD;
}
ORC_API float orc_randu(uint64_t key, uint64_t i) {
    uint64_t r = smix(key + i);
    return (float)(r >> 40) * 0x1p-24f;
}

/* ------------------------------------------------------------------------ */
/* f16 packing (attention.wgsl:75, :124 pack2x16float; RNE chosen here).     */
/* ------------------------------------------------------------------------ */
ORC_API uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to inf */
    if (ax < 0x38800000u) {                                     /* subnormal or zero in f16 */
        if (ax < 0x33000000u) return (uint16_t)sign;             /* < 2^-25: rounds to 0 */
        uint32_t e = ax >> 23;
        uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
        /* value = mant * 2^(e-150); in units of 2^-24 that is mant * 2^(e-126) */
        uint32_t shift = 126u - e;
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 112u; /* rebias 127 -> 15 */
    uint32_t mant = ax & 0x7FFFFFu;
    uint32_t h = (e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}
ORC_API float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {
            float v = (float)m * 0x1p-24f;
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7F800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ------------------------------------------------------------------------ */
/* Quantisation (src/weights.rs:123-162).                                     */
/* ------------------------------------------------------------------------ */
/* Rust f32::round: half away from zero, same as C roundf. */
ORC_API void orc_quantize_q8(const float* src, int64_t n, int8_t* q, float* scales) {
    /* weights.rs:123-133 */
    for (int64_t b = 0; b < n / 32; ++b) {
        const float* blk = src + b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(blk[i]));
        float d = amax / 127.0f;
        float id = d > 0.0f ? 1.0f / d : 0.0f;
        for (int i = 0; i < 32; ++i) {
            float r = roundf(blk[i] * id);
            if (r < -127.0f) r = -127.0f;
            if (r > 127.0f) r = 127.0f;
            q[b * 32 + i] = (int8_t)r;
        }
        scales[b] = d;
    }
}

ORC_API void orc_quantize_q4(const float* src, int64_t n, uint8_t* q, float* scales) {
    /* weights.rs:135-153: the largest-magnitude value maps to -8; nibble i of
     * 32-bit little-endian word w holds element w*8+i. */
    for (int64_t b = 0; b < n / 32; ++b) {
        const float* blk = src + b * 32;
        float mx = 0.0f;
        for (int i = 0; i < 32; ++i)
            if (fabsf(blk[i]) > fabsf(mx)) mx = blk[i];
        float d = mx / -8.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        for (int w = 0; w < 4; ++w) {
            uint32_t word = 0;
            for (int i = 0; i < 8; ++i) {
                float v = blk[w * 8 + i] * id + 8.5f;
                int32_t t = (int32_t)v; /* Rust `as i32`: truncation toward zero, saturating */
                if (v != v) t = 0;
                if (t < 0) t = 0;
                if (t > 15) t = 15;
                word |= (uint32_t)t << (4 * i);
            }
            q[b * 16 + w * 4 + 0] = (uint8_t)(word & 0xFF);
            q[b * 16 + w * 4 + 1] = (uint8_t)((word >> 8) & 0xFF);
            q[b * 16 + w * 4 + 2] = (uint8_t)((word >> 16) & 0xFF);
            q[b * 16 + w * 4 + 3] = (uint8_t)(word >> 24);
        }
        scales[b] = d;
    }
}

ORC_API void orc_dequant_q8_row(const int8_t* q, const float* scales, int64_t n, float* out) {
    /* weights.rs:155-162 */
    for (int64_t i = 0; i < n; ++i) out[i] = (float)q[i] * scales[i / 32];
}

ORC_API void orc_dequant_q4_row(const uint8_t* q, const float* scales, int64_t n, float* out) {
    /* matmul.wgsl:49-55 u4x4: nibble - 8, times the block scale */
    for (int64_t i = 0; i < n; ++i) {
        int64_t b = i / 32, e = i % 32, w = e / 8, nib = e % 8;
        uint32_t byte = q[b * 16 + w * 4 + nib / 2];
        uint32_t v = (nib & 1) ? (byte >> 4) : (byte & 15u);
        out[i] = ((float)v - 8.0f) * scales[b];
    }
}

/* Generate a [rows, cols] matrix of std*N(0,1) values from (key) and quantize it.
 * Element (r, c) uses counter r*cols + c. */
ORC_API void orc_gen_matrix(uint64_t key, int64_t rows, int64_t cols, float std, int quant, void* q, float* s) {
    int64_t nb = rows * cols / 32;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < nb; ++b) {
        float v[32];
        for (int i = 0; i < 32; ++i) v[i] = std * orc_randn(key, (uint64_t)(b * 32 + i));
        if (quant == 0)
            orc_quantize_q8(v, 32, (int8_t*)q + b * 32, s + b);
        else
            orc_quantize_q4(v, 32, (uint8_t*)q + b * 16, s + b);
    }
}

/* ------------------------------------------------------------------------ */
/* Quantised matrix-vector products (src/shaders/matmul.wgsl).               */
/* ------------------------------------------------------------------------ */
static inline float dot4(float a0, float a1, float a2, float a3, const float* x) {
    /* WGSL dot(a, b), evaluated left to right */
    return ((a0 * x[0] + a1 * x[1]) + a2 * x[2]) + a3 * x[3];
}

static inline float q8_block_dot(const int8_t* q, const float* x) {
    /* gpu.rs:247-252 block_dot_v for Q8: eight dot(i8x4(word), x4) added left to right */
    float r = dot4(q[0], q[1], q[2], q[3], x);
    for (int w = 1; w < 8; ++w) r = r + dot4(q[4 * w], q[4 * w + 1], q[4 * w + 2], q[4 * w + 3], x + 4 * w);
    return r;
}

static inline float q4_block_dot(const uint8_t* q, const float* x) {
    /* gpu.rs:285-291 block_dot_v for Q4: u4x4(word, 0) then u4x4(word, 16) per word */
    float r = 0.0f;
    for (int w = 0; w < 4; ++w) {
        uint32_t word = (uint32_t)q[4 * w] | ((uint32_t)q[4 * w + 1] << 8) | ((uint32_t)q[4 * w + 2] << 16) |
                        ((uint32_t)q[4 * w + 3] << 24);
        float lo = dot4((float)(word & 15u) - 8.0f, (float)((word >> 4) & 15u) - 8.0f,
                        (float)((word >> 8) & 15u) - 8.0f, (float)((word >> 12) & 15u) - 8.0f, x + 8 * w);
        float hi = dot4((float)((word >> 16) & 15u) - 8.0f, (float)((word >> 20) & 15u) - 8.0f,
                        (float)((word >> 24) & 15u) - 8.0f, (float)((word >> 28) & 15u) - 8.0f, x + 8 * w + 4);
        r = (w == 0) ? (lo + hi) : ((r + lo) + hi);
    }
    return r;
}

/* matvec / matvec1 / matvec2 (matmul.wgsl:59-198) for one output element:
 * lane L (of 32) accumulates acc += scale * block_dot over blocks L, L+32, ...;
 * then the lanes are tree-summed (s = 16, 8, 4, 2, 1). */
static float mv_row(int quant, const uint8_t* wq, const float* ws, int64_t row, int K, const float* x) {
    int nb = K / 32;
    float red[32];
    for (int lane = 0; lane < 32; ++lane) red[lane] = 0.0f;
    const float* srow = ws + row * (int64_t)nb;
    if (quant == 0) {
        const int8_t* qrow = (const int8_t*)wq + row * (int64_t)K;
        for (int b0 = 0; b0 < nb; b0 += 32)
            for (int lane = 0; lane < 32 && b0 + lane < nb; ++lane) {
                int b = b0 + lane;
                red[lane] = red[lane] + srow[b] * q8_block_dot(qrow + b * 32, x + b * 32);
            }
    } else {
        const uint8_t* qrow = wq + row * (int64_t)(K / 2);
        for (int b0 = 0; b0 < nb; b0 += 32)
            for (int lane = 0; lane < 32 && b0 + lane < nb; ++lane) {
                int b = b0 + lane;
                red[lane] = red[lane] + srow[b] * q4_block_dot(qrow + b * 16, x + b * 32);
            }
    }
    for (int s = 16; s > 0; s >>= 1)
        for (int lane = 0; lane < s; ++lane) red[lane] = red[lane] + red[lane + s];
    return red[0];
}

/* Tiled prefill matmul (matmul.wgsl:200-318): each output accumulates
 * (q * scale) * x over k in ascending order. */
static float mm_row(int quant, const uint8_t* wq, const float* ws, int64_t row, int K, const float* x) {
    float c = 0.0f;
    int nb = K / 32;
    for (int k = 0; k < K; ++k) {
        float q;
        if (quant == 0) {
            q = (float)((const int8_t*)wq)[row * (int64_t)K + k];
        } else {
            int e = k % 32, w = e / 8, nib = e % 8;
            uint32_t byte = wq[row * (int64_t)(K / 2) + (k / 32) * 16 + w * 4 + nib / 2];
            q = (float)((nib & 1) ? (byte >> 4) : (byte & 15u)) - 8.0f;
        }
        float w = q * ws[row * (int64_t)nb + k / 32];
        c = c + w * x[k];
    }
    return c;
}

/* y[m*y_stride + n] = sum_k x[m*x_stride + k] * W[n, k] for m < M, n < N.
 * M selects the reference kernel: 1..8 the lane-strided matvec kernels, more the tiled matmul
 * (gpu.rs:211-217 MatKind::for_rows). */
ORC_API void orc_gemv(int quant, const void* wq, const float* ws, const float* x, float* y, int M, int N, int K,
                      int x_stride, int y_stride) {
    const uint8_t* q = (const uint8_t*)wq;
    int tiled = M > 8;
#pragma omp parallel for schedule(static) if (N >= 256)
    for (int n = 0; n < N; ++n)
        for (int m = 0; m < M; ++m) {
            const float* xr = x + (int64_t)m * x_stride;
            y[(int64_t)m * y_stride + n] = tiled ? mm_row(quant, q, ws, n, K, xr) : mv_row(quant, q, ws, n, K, xr);
        }
}

/* ------------------------------------------------------------------------ */
/* Workgroup tree reductions, as the WGSL writes them.                        */
/* ------------------------------------------------------------------------ */
static float tree_sum(float* red, int n) {
    for (int s = n / 2; s > 0; s >>= 1)
        for (int i = 0; i < s; ++i) red[i] = red[i] + red[i + s];
    return red[0];
}

/* ------------------------------------------------------------------------ */
/* layers.wgsl                                                               */
/* ------------------------------------------------------------------------ */
/* branch_norm (layers.wgsl:46-73): out[w, :] = rmsnorm(branch input of row m) * (one + nw)
 * for w < count, m = w (+ step_m - 1 when last_row).  x_stride 0 means 2h. */
ORC_API void orc_branch_norm(const float* x, const float* coef, const float* nw, float* out, int h, int count,
                             int step_m, int mode, int last_row, float eps, float one, int x_stride) {
    float red[256];
    for (int w = 0; w < count; ++w) {
        int m = w + (last_row ? step_m - 1 : 0);
        const float* xb = x + (int64_t)m * (x_stride ? x_stride : 2 * h);
        float pre0 = 1.0f, pre1 = 0.0f;
        if (mode == 1) {
            pre0 = coef[m * 8];
            pre1 = coef[m * 8 + 1];
        }
        for (int lid = 0; lid < 256; ++lid) {
            float ss = 0.0f;
            for (int i = lid; i < h; i += 256) {
                float v = pre0 * xb[i];
                if (mode == 1) v = v + pre1 * xb[h + i];
                ss = ss + v * v;
            }
            red[lid] = ss;
        }
        float total = tree_sum(red, 256);
        float rinv = 1.0f / sqrtf(total / (float)h + eps);
        for (int i = 0; i < h; ++i) {
            float v = pre0 * xb[i];
            if (mode == 1) v = v + pre1 * xb[h + i];
            out[(int64_t)w * h + i] = (v * rinv) * (one + nw[i]);
        }
    }
}

/* mhc_dots (layers.wgsl:75-92): raw[m*9+o] = router row o . streams (o<8), sum of squares (o=8). */
ORC_API void orc_mhc_dots(const float* x, const float* w, float* raw, int h, int M) {
    int d = 2 * h;
    float red[256];
    for (int m = 0; m < M; ++m)
        for (int o = 0; o < 9; ++o) {
            for (int lid = 0; lid < 256; ++lid) {
                float acc = 0.0f;
                for (int i = lid; i < d; i += 256) {
                    float v = x[(int64_t)m * d + i];
                    acc = acc + (o < 8 ? w[(int64_t)o * d + i] * v : v * v);
                }
                red[lid] = acc;
            }
            raw[m * 9 + o] = tree_sum(red, 256);
        }
}

static inline float lse2(float a, float b) {
    float mx = fmaxf(a, b);
    return mx + logf(expf(a - mx) + expf(b - mx));
}

/* mhc_finish (layers.wgsl:94-126): coef = [pre0, pre1, post0, post1, mix00, mix01, mix10, mix11]. */
ORC_API void orc_mhc_finish(const float* raw, const float* w, float* coef, int h, int M, int iterations) {
    int d = 2 * h;
    for (int m = 0; m < M; ++m) {
        float rinv = 1.0f / sqrtf(raw[m * 9 + 8] / (float)d + 1e-6f);
        float lg[8];
        for (int o = 0; o < 8; ++o) lg[o] = raw[m * 9 + o] * rinv + w[(int64_t)8 * d + o];
        float a = lg[4], b = lg[5], c = lg[6], e = lg[7];
        for (int it = 0; it < iterations; ++it) {
            float r0 = lse2(a, b), r1 = lse2(c, e);
            a -= r0;
            b -= r0;
            c -= r1;
            e -= r1;
            float c0 = lse2(a, c), c1 = lse2(b, e);
            a -= c0;
            c -= c0;
            b -= c1;
            e -= c1;
        }
        float* cb = coef + m * 8;
        cb[0] = 1.0f / (1.0f + expf(-lg[0]));
        cb[1] = 1.0f / (1.0f + expf(-lg[1]));
        cb[2] = 2.0f / (1.0f + expf(-lg[2]));
        cb[3] = 2.0f / (1.0f + expf(-lg[3]));
        cb[4] = expf(a);
        cb[5] = expf(b);
        cb[6] = expf(c);
        cb[7] = expf(e);
    }
}

/* merge (layers.wgsl:128-162) */
ORC_API void orc_merge(float* x, const float* coef, const float* br, int h, int M, int mode) {
    for (int m = 0; m < M; ++m)
        for (int i = 0; i < h; ++i) {
            float* x0 = x + (int64_t)m * 2 * h + i;
            float* x1 = x0 + h;
            float b = br[(int64_t)m * h + i];
            if (mode == 0) {
                *x0 = *x0 + b;
                continue;
            }
            if (mode == 3) {
                *x1 = *x0;
                continue;
            }
            const float* c = coef + m * 8;
            float n0 = (c[4] * *x0 + c[5] * *x1) + c[2] * b;
            float n1 = (c[6] * *x0 + c[7] * *x1) + c[3] * b;
            if (mode == 2) {
                *x0 = 0.5f * (n0 + n1);
            } else {
                *x0 = n0;
                *x1 = n1;
            }
        }
}

/* swiglu (layers.wgsl:164-175) */
ORC_API void orc_swiglu(const float* proj, float* act, int inter, int M) {
    for (int m = 0; m < M; ++m)
        for (int i = 0; i < inter; ++i) {
            float g = proj[(int64_t)m * 2 * inter + i];
            float u = proj[(int64_t)m * 2 * inter + inter + i];
            act[(int64_t)m * inter + i] = g / (1.0f + expf(-g)) * u;
        }
}

/* ------------------------------------------------------------------------ */
/* linear.wgsl: Gated DeltaNet                                                */
/* ------------------------------------------------------------------------ */
/* conv (linear.wgsl:38-66): causal depthwise conv (k=4) + SiLU; conv_state is [3, conv_dim], oldest first. */
ORC_API void orc_conv(const float* proj, int proj_stride, float* conv_out, float* conv_state, const float* lw,
                      float* conv_ckpt, int conv_dim, int M, int ckpt) {
    for (int c = 0; c < conv_dim; ++c) {
        float w0 = lw[c * 4], w1 = lw[c * 4 + 1], w2 = lw[c * 4 + 2], w3 = lw[c * 4 + 3];
        float r0 = conv_state[c], r1 = conv_state[conv_dim + c], r2 = conv_state[2 * conv_dim + c];
        for (int m = 0; m < M; ++m) {
            float cur = proj[(int64_t)m * proj_stride + c];
            float o = ((w0 * r0 + w1 * r1) + w2 * r2) + w3 * cur;
            conv_out[(int64_t)m * conv_dim + c] = o / (1.0f + expf(-o));
            r0 = r1;
            r1 = r2;
            r2 = cur;
            if (m + 1 == ckpt) {
                conv_ckpt[c] = r0;
                conv_ckpt[conv_dim + c] = r1;
                conv_ckpt[2 * conv_dim + c] = r2;
            }
        }
        conv_state[c] = r0;
        conv_state[conv_dim + c] = r1;
        conv_state[2 * conv_dim + c] = r2;
    }
}

/* delta (linear.wgsl:84-140): recurrent gated delta rule + gated RMS norm.
 * state is [n_v][128 (i, key)][128 (j, value)]; lw = conv w | A_log[n_v] | dt_bias[n_v] | norm[128]. */
ORC_API void orc_delta(const float* proj, int proj_stride, const float* conv_out, float* state, const float* lw,
                       float* out, float* state_ckpt, int conv_dim, int n_k, int n_v, float eps, int M, int ckpt) {
    enum { DK = 128, DV = 128 };
    int key_dim = n_k * DK;
    int z_off = conv_dim, b_off = conv_dim + n_v * DV, a_off = b_off + n_v;
#pragma omp parallel for schedule(static) if (n_v >= 8)
    for (int h = 0; h < n_v; ++h) {
        float sl[DK * DV];
        float qs[DK], ks[DK], red[DK], red2[DK], o[DV];
        int kh = h / (n_v / n_k);
        float a_log = lw[conv_dim * 4 + h];
        float dt_bias = lw[conv_dim * 4 + n_v + h];
        const float* norm_w = lw + conv_dim * 4 + 2 * n_v;
        float* st = state + (int64_t)h * DK * DV;
        memcpy(sl, st, sizeof(sl));
        for (int m = 0; m < M; ++m) {
            const float* crow = conv_out + (int64_t)m * conv_dim;
            for (int j = 0; j < DK; ++j) {
                float qv = crow[kh * DK + j], kv = crow[key_dim + kh * DK + j];
                red[j] = qv * qv;
                red2[j] = kv * kv;
            }
            float sq = tree_sum(red, DK), sk = tree_sum(red2, DK);
            for (int j = 0; j < DK; ++j) {
                float qv = crow[kh * DK + j], kv = crow[key_dim + kh * DK + j];
                qs[j] = (qv * (1.0f / sqrtf(sq + 1e-6f))) * (1.0f / sqrtf((float)DK));
                ks[j] = kv * (1.0f / sqrtf(sk + 1e-6f));
            }
            const float* prow = proj + (int64_t)m * proj_stride;
            float beta = 1.0f / (1.0f + expf(-prow[b_off + h]));
            float araw = prow[a_off + h] + dt_bias;
            float sp = araw;
            if (araw <= 20.0f) sp = logf(1.0f + expf(araw));
            float decay = expf(-expf(a_log) * sp);
            for (int j = 0; j < DV; ++j) {
                float vv = crow[2 * key_dim + h * DV + j];
                float kv_mem = 0.0f;
                for (int i = 0; i < DK; ++i) {
                    sl[i * DV + j] = sl[i * DV + j] * decay;
                    kv_mem = kv_mem + sl[i * DV + j] * ks[i];
                }
                float dlt = (vv - kv_mem) * beta;
                float oj = 0.0f;
                for (int i = 0; i < DK; ++i) {
                    sl[i * DV + j] = sl[i * DV + j] + ks[i] * dlt;
                    oj = oj + sl[i * DV + j] * qs[i];
                }
                o[j] = oj;
                red[j] = oj * oj;
            }
            float var_o = tree_sum(red, DV) / (float)DV;
            for (int j = 0; j < DV; ++j) {
                float z = prow[z_off + h * DV + j];
                out[(int64_t)m * n_v * DV + h * DV + j] =
                    ((o[j] * (1.0f / sqrtf(var_o + eps))) * norm_w[j]) * (z / (1.0f + expf(-z)));
            }
            if (m + 1 == ckpt) memcpy(state_ckpt + (int64_t)h * DK * DV, sl, sizeof(sl));
        }
        memcpy(st, sl, sizeof(sl));
    }
}

/* ------------------------------------------------------------------------ */
/* attention.wgsl                                                             */
/* ------------------------------------------------------------------------ */
typedef struct orc_attn_p {
    int n_heads, n_kv, rot_dim, proj_stride;
    float rope_theta, eps, scale;
    uint32_t mrope;
} orc_attn_p;

/* prep (attention.wgsl:59-127): q/k RMSNorm(1+w) + rotate-half RoPE, K/V to the f16 cache at pos0+m.
 * rpos is [M][4] (t, h, w, 0). */
ORC_API void orc_attn_prep(const orc_attn_p* p, const float* proj, float* qbuf, uint16_t* kcache, uint16_t* vcache,
                           const float* norms, const uint32_t* rpos, int M, int pos0) {
    enum { HD = 256 };
    int q_dim = p->n_heads * HD, kv_dim = p->n_kv * HD;
    float red[HD], v[HD], sh[HD];
    for (int m = 0; m < M; ++m) {
        int pos = pos0 + m;
        const float* row = proj + (int64_t)m * p->proj_stride;
        for (int slot = 0; slot < p->n_heads + 2 * p->n_kv; ++slot) {
            if (slot >= p->n_heads + p->n_kv) {
                int kh = slot - p->n_heads - p->n_kv;
                for (int d = 0; d < HD; ++d)
                    vcache[(int64_t)pos * kv_dim + kh * HD + d] = orc_f32_to_f16(row[2 * q_dim + kv_dim + kh * HD + d]);
                continue;
            }
            int norm_off;
            for (int d = 0; d < HD; ++d) {
                if (slot < p->n_heads)
                    v[d] = row[slot * 2 * HD + d];
                else
                    v[d] = row[2 * q_dim + (slot - p->n_heads) * HD + d];
                red[d] = v[d] * v[d];
            }
            norm_off = slot < p->n_heads ? 0 : HD;
            float total = tree_sum(red, HD);
            float r = 1.0f / sqrtf(total / (float)HD + p->eps);
            for (int d = 0; d < HD; ++d) {
                v[d] = (v[d] * r) * (1.0f + norms[norm_off + d]);
                sh[d] = v[d];
            }
            int half_rot = p->rot_dim / 2;
            const uint32_t* rp = rpos + m * 4;
            for (int d = 0; d < p->rot_dim; ++d) {
                int fi = d % half_rot;
                float inv_freq = powf(p->rope_theta, -(float)(2 * fi) / (float)p->rot_dim);
                uint32_t rot_pos = rp[0];
                if (fi % 3 == 1 && (uint32_t)fi < (p->mrope >> 16))
                    rot_pos = rp[1];
                else if (fi % 3 == 2 && (uint32_t)fi < (p->mrope & 0xFFFFu))
                    rot_pos = rp[2];
                float ang = (float)rot_pos * inv_freq;
                float cs = cosf(ang), sn = sinf(ang);
                if (d < half_rot)
                    v[d] = sh[d] * cs - sh[d + half_rot] * sn;
                else
                    v[d] = sh[d] * cs + sh[d - half_rot] * sn;
            }
            if (slot < p->n_heads) {
                for (int d = 0; d < HD; ++d) qbuf[(int64_t)m * q_dim + slot * HD + d] = v[d];
            } else {
                int kh = slot - p->n_heads;
                for (int d = 0; d < HD; ++d) kcache[(int64_t)pos * kv_dim + kh * HD + d] = orc_f32_to_f16(v[d]);
            }
        }
    }
}

/* attend (attention.wgsl:129-246): GQA online softmax over 16-key tiles; part `part` of `parts`. */
ORC_API void orc_attend(const orc_attn_p* p, const float* proj, const float* qbuf, const uint16_t* kcache,
                        const uint16_t* vcache, float* out, float* partial, int M, int pos0, int parts) {
    enum { HD = 256, G = 4, KC = 16 };
    int q_dim = p->n_heads * HD, kv_dim = p->n_kv * HD;
    for (int kh = 0; kh < p->n_kv; ++kh)
        for (int m = 0; m < M; ++m)
            for (int part = 0; part < parts; ++part) {
                float qs[G][HD], acc[G][HD], m_sh[G], l_sh[G], corr[G], pr[G][KC];
                for (int g = 0; g < G; ++g) {
                    for (int d = 0; d < HD; ++d) {
                        qs[g][d] = qbuf[(int64_t)m * q_dim + (kh * G + g) * HD + d];
                        acc[g][d] = 0.0f;
                    }
                    m_sh[g] = -1e30f;
                    l_sh[g] = 0.0f;
                }
                int total = pos0 + m + 1;
                int chunk = (total + parts - 1) / parts;
                int start = part * chunk < total ? part * chunk : total;
                int end = start + chunk < total ? start + chunk : total;
                for (int t0 = start; t0 < end; t0 += KC) {
                    int n_keys = end - t0 < KC ? end - t0 : KC;
                    for (int g = 0; g < G; ++g)
                        for (int j = 0; j < KC; ++j) {
                            float partd[4];
                            for (int seg = 0; seg < 4; ++seg) {
                                float d = 0.0f;
                                if (j < n_keys)
                                    for (int w = 0; w < 32; ++w) {
                                        int word = w * 4 + seg;
                                        const uint16_t* kk = kcache + (int64_t)(t0 + j) * kv_dim + kh * HD + 2 * word;
                                        d = d + (qs[g][2 * word] * orc_f16_to_f32(kk[0]) +
                                                 qs[g][2 * word + 1] * orc_f16_to_f32(kk[1]));
                                    }
                                partd[seg] = d;
                            }
                            float sc = -1e30f;
                            if (j < n_keys) sc = (((partd[0] + partd[1]) + partd[2]) + partd[3]) * p->scale;
                            pr[g][j] = sc;
                        }
                    for (int g = 0; g < G; ++g) {
                        float mx = m_sh[g];
                        for (int j = 0; j < n_keys; ++j) mx = fmaxf(mx, pr[g][j]);
                        float c = expf(m_sh[g] - mx);
                        float sum = 0.0f;
                        for (int j = 0; j < KC; ++j) {
                            float pe = 0.0f;
                            if (j < n_keys) pe = expf(pr[g][j] - mx);
                            pr[g][j] = pe;
                            sum = sum + pe;
                        }
                        corr[g] = c;
                        m_sh[g] = mx;
                        l_sh[g] = l_sh[g] * c + sum;
                    }
                    for (int d = 0; d < HD; ++d) {
                        for (int g = 0; g < G; ++g) acc[g][d] = acc[g][d] * corr[g];
                        for (int j = 0; j < n_keys; ++j) {
                            float v = orc_f16_to_f32(vcache[(int64_t)(t0 + j) * kv_dim + kh * HD + d]);
                            for (int g = 0; g < G; ++g) acc[g][d] = acc[g][d] + v * pr[g][j];
                        }
                    }
                }
                for (int g = 0; g < G; ++g) {
                    int hh = kh * G + g;
                    if (parts == 1) {
                        for (int d = 0; d < HD; ++d) {
                            float gate = proj[(int64_t)m * p->proj_stride + hh * 2 * HD + HD + d];
                            out[(int64_t)m * q_dim + hh * HD + d] = acc[g][d] / l_sh[g] / (1.0f + expf(-gate));
                        }
                    } else {
                        int64_t pi = ((int64_t)m * p->n_heads + hh) * parts + part;
                        for (int d = 0; d < HD; ++d) partial[pi * (HD + 2) + d] = acc[g][d];
                        partial[pi * (HD + 2) + HD] = m_sh[g];
                        partial[pi * (HD + 2) + HD + 1] = l_sh[g];
                    }
                }
            }
}

/* combine (attention.wgsl:248-269) */
ORC_API void orc_combine(const orc_attn_p* p, const float* proj, const float* partial, float* out, int M, int parts) {
    enum { HD = 256 };
    int q_dim = p->n_heads * HD;
    for (int m = 0; m < M; ++m)
        for (int h = 0; h < p->n_heads; ++h) {
            int64_t base = ((int64_t)m * p->n_heads + h) * parts;
            float mx = -1e30f;
            for (int i = 0; i < parts; ++i) mx = fmaxf(mx, partial[(base + i) * (HD + 2) + HD]);
            for (int d = 0; d < HD; ++d) {
                float l = 0.0f, acc = 0.0f;
                for (int i = 0; i < parts; ++i) {
                    int64_t o = (base + i) * (HD + 2);
                    float f = expf(partial[o + HD] - mx);
                    l = l + partial[o + HD + 1] * f;
                    acc = acc + partial[o + d] * f;
                }
                float gate = proj[(int64_t)m * p->proj_stride + h * 2 * HD + HD + d];
                out[(int64_t)m * q_dim + h * HD + d] = acc / l / (1.0f + expf(-gate));
            }
        }
}

/* argmax (sampler.rs:169-177): first index of the maximum (strict >). */
ORC_API uint32_t orc_argmax(const float* v, int64_t n) {
    int64_t best = 0;
    for (int64_t i = 0; i < n; ++i)
        if (v[i] > v[best]) best = i;
    return (uint32_t)best;
}

#include "snl_oracle_engine.inc"
