// Launch descriptors and host-side launchers of the decode-step kernels.
// Every launcher returns 0 on success, < 0 on a bad argument or launch error.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace snl {

// ---------------------------------------------------------------- GEMV (gemv.hip)
enum GemvEpi { GEMV_STORE = 0, GEMV_ADD = 1, GEMV_MHC = 2, GEMV_SWIGLU = 3 };
// Prologue applied to the token rows before the product: none, RMSNorm (1 + w) of stream 0, the
// mHC pre-mix pre0*x0 + pre1*x1 of both streams (pre from the router sums) then RMSNorm, or the
// gated RMS norm of each 128-wide DeltaNet head (GNORM).
enum GemvPro { GEMV_PLAIN = 0, GEMV_NORM = 1, GEMV_NORM_MHC = 2, GEMV_GNORM = 3 };

struct GemvArgs {
    const void* wq;      // quants [N, K] (Q8) or [N, K/2] (Q4), or tile order when packed
    const float* ws;     // scales [N, K/32], or tile order when packed
    int packed;          // 1: wq/ws in the tile order of packing.h (matrix-core kernel)
    const float* x;      // token row m at x + (row0 + m) * x_stride, row0 = row_base ? *row_base : 0
    int x_stride;        //   (16-byte aligned, stride % 4 == 0; NORM_MHC: stream 1 at +K)
    const int32_t* row_base;
    float* y;            // STORE: y[m*y_stride + n_off + n]; ADD/MHC: residual rows (stream 0 at +0,
    int y_stride;        //   stream 1 at +h); SWIGLU: act[m*y_stride + i]
    int N, K;
    int n_off;
    int epi;
    int merge_mode;      // MHC: 1 mix, 2 mix then collapse to the mean
    int h;               // MHC: offset of stream 1
    int inter;           // SWIGLU: intermediate size (N == 2*inter; gate rows then up rows)
    int pro;             // GemvPro
    const float* norm_w; // NORM*: weights w of the (1 + w) RMSNorm [K]
    float eps;           // (GNORM: x is the gated DeltaNet output of 128-wide heads and rin the
                         //  partial sums of squares [M][K/128][4] of their raw values)
    // mHC router (layers.wgsl:75-126).  A site's router sums (the 8 router-row dots with the
    // 2-stream row and its sum of squares) arrive as per-block partials [M][9][blocks] from the
    // GEMV that produced the row.  The NORM_MHC launch of the site adds them in block order and
    // takes pre0/pre1; its block 0 stores the sums in raw and the token coefficients (post and
    // the Sinkhorn mix) in coef, which the MHC epilogue of the same site reads.
    const float* site_w; // NORM_MHC: router of this GEMV's site, [8][2h] then bias[8]
    float* raw;          // NORM_MHC: [M][9] site sums (block 0)
    float* coef;         // [M][8] token coefficients: written by NORM_MHC (block 0), read by MHC
    const float* rin;    // NORM_MHC: partials [M][9][rin_n]
    int rin_n;
    int iterations;      // NORM_MHC: Sinkhorn iterations
    const float* next_w; // ADD / MHC epilogue: router of the next site, whose partials this launch
    float* rpart;        //   writes to rpart[M][9][gridDim.x] (null: none)
    int expand;          //   and, at the start of the mHC range, stream 1 := stream 0 first
    // NORM prologue of a tile-major launch (the vocabulary head): block 0 also stores the normed
    // token rows, RMSNorm(x) * (1 + w), to norm_out [M][K] and the last of them to norm_last
    float* norm_out;
    float* norm_last;
};
// grid size of launch_gemv over tile-order weights (the partial count a producer leaves)
int mgemv_blocks(int quant, int N, int K, int inter);
// Kernel-level GEMV (snl_gemv): the matrix-core path for tile-order weights, else the vector-ALU
// fallback of gemv.hip / gemv_ksplit.hip for the reference's row-major layout at shapes the
// matrix-core kernel does not serve (K % 128 != 0; M = 3, 4 where two token pairs overflow LDS).
// The engine's passes never take the fallback.
int launch_gemv(const GemvArgs& a, int quant, int M, hipStream_t s);
// vector-ALU fallback, K split over blocks (kernel-level calls only)
int launch_gemv_ksplit(const GemvArgs& a, int quant, int M, hipStream_t s);
// Matrix-core path (mgemv.hip) over tile-order weights: 0 launched, 1 not served (M too large for
// LDS at this K), < 0 error.
int launch_mgemv(const GemvArgs& a, int quant, int M, hipStream_t s);
// whether launch_mgemv serves M token rows at this K (the staged rows fit in LDS)
bool mgemv_fits(int M, int K);
int mgemv_init();
// Set the LDS limit of every streaming-GEMV instantiation (call once, outside graph capture).
int gemv_init();

// ---------------------------------------------------------------- prefill GEMM (mgemm.hip)
// Token rows -> the GEMM's f16 hi/lo A fragments, with the branch input computed on the way:
// the rows as they are, RMSNorm(x0) * (1 + w), the mHC pre-mix then that norm (coef[m][0..1]),
// or the head factor of the DeltaNet gated norm (ssq partials [M][K/128][kDeltaPrefillGroups]).
enum RowsMode { ROWS_PLAIN = 0, ROWS_NORM = 1, ROWS_NORM_MHC = 2, ROWS_GNORM = 3 };
struct RowsArgs {
    const float* x;      // token row m at x + m * x_stride (NORM_MHC: stream 1 at +h)
    int x_stride;
    int M, K;
    int mode;
    const float* w;      // NORM*: (1 + w) weights [K]
    const float* coef;   // NORM_MHC: [M][8]
    int h;
    const float* ssq;    // GNORM
    float eps;
    int perm4;           // 1: element order of the Q4 nibble dequant
    void* frags;         // out: frags_bytes(M, K)
    float* xs;           // out: per-token scale [roundup(M, 16)]
};
struct GemmArgs {
    const void* wq;      // panel-order quants
    const float* ws;     // panel-order scales
    const void* frags;   // token fragments
    const float* xs;
    float* y;            // y[m * y_stride + n_off + n]
    int y_stride, n_off;
    int M, N, K;
};
size_t gemm_q_bytes(int quant, int N, int K);
size_t gemm_s_floats(int N, int K);
size_t frags_bytes(int M, int K);
// reference layout (q [N, K] Q8 / [N, K/2] Q4, s [N, K/32]) -> panel order
int launch_panel_pack(int quant, int N, int K, const void* q, const float* s, void* qp, float* sp, hipStream_t st);
int launch_rows_to_frags(const RowsArgs& a, hipStream_t s);
int launch_mgemm(const GemmArgs& a, int quant, hipStream_t s);

// ---------------------------------------------------------------- layers (layers.hip)
// x[m, 0:h] = dequant(embed[tokens[m]]), x[m, h:2h] = 0 (src/engine.rs:777-790); with carry_src, one
// more block copies h floats from carry_src to carry_dst in the same launch.  one_stream: rows of h
// floats (x[m*h ..]) and no second stream.
struct Pick;
// draft: the MTP draft's pick, the token of the rows step->draft_rows names
int launch_embed(const StepDev* step, const int8_t* eq, const float* es, int vocab, int h, float* x, int M,
                 hipStream_t s, const float* carry_src = nullptr, float* carry_dst = nullptr,
                 const Pick* draft = nullptr, bool one_stream = false);

// out[r] = rmsnorm(branch input of row first+r) * (one + w) for r < count (layers.wgsl:46-73).
// mode 1 mixes the two streams with coef[row][0..1].  Row `row` of x starts at
// x + (row + (row_base ? *row_base : 0)) * x_stride.
struct NormArgs {
    const float* x;
    int x_stride;
    const int32_t* row_base;
    const float* coef;
    const float* w;
    float* out;
    int out_stride;
    int h;
    int mode;
    int first;
    int count;
    float eps;
    float one;
    float* last_copy;  // nullable: the last row's output is also written here
};
int launch_branch_norm(const NormArgs& a, hipStream_t s);

// mHC router sums (layers.wgsl:75-92) for a site that no GEMV precedes, one block per token:
// part[m][0..7] = router rows . [x0, x1], part[m][8] = sum of squares (one partial per token).
int launch_mhc(const float* x, const float* w, float* part, int h, int M, hipStream_t s);

// x[m, h + i] = x[m, i] (merge mode 3, layers.wgsl:146-149)
int launch_expand(float* x, int h, int M, hipStream_t s);

// Plain merge (modes 0..2) and SwiGLU, for paths that do not fuse them into a GEMV.
int launch_merge(float* x, const float* coef, const float* br, int h, int M, int mode, hipStream_t s);
int launch_swiglu(const float* proj, float* act, int inter, int M, hipStream_t s);

// Greedy pick per logits row: first index of the maximum, the maximum and the second largest value.
struct Pick {
    uint32_t token;
    float top1;
    float top2;
    uint32_t _pad;
};
// One greedy speculative step's outcome, posted to pinned host memory by spec_next.
constexpr uint32_t kSpecRopeRange = 1u;
struct SpecOut {
    uint32_t seq, draft, accepted, flags;  // flags: kSpecRopeRange when a position ran past rope_tab
    Pick picks[2];
};
// After a speculative step's verify (src/worker.rs:236-255, greedy): accept when the verify's first
// pick equals the draft; on a reject, hlast <- hid row 1 (the rollback's carried row).  Rewrites the
// verify record vstep and the draft record mstep for the next step (positions advanced by 2 or 1,
// the state slots switched, rotary cos / sin from rope_tab) and posts the outcome to ring[seq % ring_n].
struct SpecArgs {
    StepDev* vstep;
    StepDev* mstep;
    const Pick* picks;     // the verify's 2 picks
    const Pick* draft;     // the draft's pick
    const float* rope_tab; // [rope_rows][SNL_ROPE_MAX][2]: cos / sin of text position p
    int rope_rows;
    const float* hid1;     // hid row 1
    float* hlast;
    int h;
    SpecOut* ring;         // pinned host memory (device address)
    int ring_n;
};
int launch_spec_next(const SpecArgs& a, hipStream_t s);
// host_out: pinned host memory (its device address) that also receives the picks
int launch_pick(const float* logits, int V, int rows, float* scratch, Pick* out, hipStream_t s,
                Pick* host_out = nullptr);
size_t pick_scratch_floats(int V, int rows);

int launch_copy(float* dst, const float* src, size_t n, hipStream_t s);

// ---------------------------------------------------------------- Gated DeltaNet (deltanet.hip)
struct DeltaArgs {
    const float* proj;   // [M, proj_stride]: qkv[conv_dim] | z[n_v*128] | b[n_v] | a[n_v]
    int proj_stride;
    const float* lw;     // conv w [conv_dim*4] | A_log[n_v] | dt_bias[n_v] | norm[128]
    float* conv_state;   // 3 slots of [3, conv_dim]
    float* state;        // 3 slots of [n_v, 128, 128]
    size_t conv_slot;    // floats per conv slot
    size_t state_slot;   // floats per state slot
    float* out;          // [M, n_v*128] (o * w) * silu(z), before the head factor of the norm
    float* ssq;          // [M, n_v, 4] partial sums of out^2 per column group of 32
    int conv_dim, n_k, n_v;
    float eps;
    const StepDev* step;  // s_in / s_out / s_ck / ckpt
};
constexpr int kDeltaGroups = 4;  // column groups per value head (partials per head in ssq)
// column groups per value head of the prefill recurrence (partials per head in its ssq)
constexpr int kDeltaPrefillGroups = 8;
int launch_deltanet(const DeltaArgs& a, int M, hipStream_t s);
// the gated RMS norm in place on out (kernel-level entry; the engine folds it into out_proj)
int launch_deltanet_norm(const DeltaArgs& a, int M, hipStream_t s);

// ---------------------------------------------------------------- chunked prefill (prefill.hip)
// x[m] = dequant(embed[tokens[m]]) (stream 0), stream 1 zero
int launch_embed_tokens(const uint32_t* tokens, const int8_t* eq, const float* es, int vocab, int h, float* x, int M,
                        hipStream_t s);
// coef[m][8] from the router sums part[m][9] of the 2-stream rows (h: stream width)
int launch_mhc_coef(const float* part, const float* w, int h, int iterations, float* coef, int M, hipStream_t s);

struct DnPrefillArgs {
    const float* proj;   // [M, proj_stride]: qkv[conv_dim] | z[n_v*128] | b[n_v] | a[n_v]
    int proj_stride;
    const float* lw;     // conv w [conv_dim*4] | A_log[n_v] | dt_bias[n_v] | norm[128]
    float* conv_state;   // this visit's [3, conv_dim], updated in place
    float* state;        // this visit's [n_v, 128, 128], updated in place
    float *q, *k;        // scratch [M][n_k][128]: normalised (q also times 1/sqrt(128))
    float *v, *gz;       // scratch [M][n_v][128]: conv output, silu(z)
    float *beta, *decay; // scratch [M][n_v]
    float* out;          // [M, n_v*128] (o * w) * silu(z), before the head factor of the norm
    float* ssq;          // [M, n_v, kDeltaPrefillGroups] partial sums of o^2 per column group
    float* pairs;        // scratch of dn_pairs_floats(M, n_k): k.k and k.q inside blocks of tokens
    int conv_dim, n_k, n_v;
};
int launch_deltanet_prefill(const DnPrefillArgs& a, int M, hipStream_t s);
size_t dn_pairs_floats(int M, int n_k);

// ---------------------------------------------------------------- sampler (sampler.hip)
// src/sampler.rs:99-106: repetition, presence and frequency penalties on logits[tok[i]] in place
int launch_penalties(float* logits, int V, const uint32_t* tok, const uint32_t* cnt, int n, float rep, float presence,
                     float frequency, hipStream_t s);
// the k (<= 2048) largest entries as keys (order bits of the value << 32 | ~index), descending;
// *result points into scratch (topk_scratch_keys(V, k) keys)
size_t topk_scratch_keys(int V, int k);
int launch_topk(const float* logits, int V, int k, unsigned long long* scratch, unsigned long long** result,
                hipStream_t s);

// ---------------------------------------------------------------- gated attention (attention.hip)
struct AttnArgs {
    const float* proj;   // [M, proj_stride] q+gate | k | v
    int proj_stride;
    float* qbuf;         // [M, n_heads*256]
    uint16_t* kcache;    // [ctx, kv_dim] f16
    uint16_t* vcache;
    const float* norms;  // q_norm[256] | k_norm[256]
    float* out;          // [M, n_heads*256]
    float* partial;      // [M, n_heads, ceil(ctx / 64), 258] split-K partials
    int n_heads, n_kv, rot_dim;
    float rope_theta, eps, scale;
    uint32_t mrope;
    int ctx;
    const StepDev* step;  // pos0, rpos
};
// prep + attend + combine for M = 1 or 2 tokens
int launch_attention(const AttnArgs& a, int M, hipStream_t s);
constexpr int kAttnPart = 64;  // keys per split-K part
// Largest context (KV positions per attention layer): the reference's default max_position
// (src/config.rs), 4096 decode parts of 64 keys.
constexpr int kMaxCtx = 262144;
constexpr int kAttnMaxParts = kMaxCtx / kAttnPart;

// Gated attention over a chunk (attention_prefill.hip): rows m < M at cache positions pos0 + m
// with rotary positions rpos[m]; q/k norm + RoPE, K/V into the f16 cache, then causal
// attention over every earlier key and the sigmoid gate.  Same AttnArgs, with `pstep` for the
// positions (step is unused).  keys = pos0 + M (host-side); past 4096 keys the key range splits
// into parts whose partials go to part [M][n_heads][parts_max][258].
int attention_prefill_parts(int ctx);
int launch_attention_prefill(const AttnArgs& a, const PrefillDev* pstep, int M, int keys, float* part, int parts_max,
                             hipStream_t s);

// ---------------------------------------------------------------- seeded initialiser (init.hip)
int launch_gen_matrix(uint64_t key, int64_t rows, int64_t cols, float stdv, int quant, void* q, float* sc,
                      hipStream_t s);
// kind: 0 = std*N, 1 = 1 + std*N, 2 = DeltaNet parameter vector (conv_dim given), 3 = mHC router (h given)
int launch_gen_vector(uint64_t key, int64_t n, int kind, float stdv, int aux0, int aux1, float* out, hipStream_t s);

}  // namespace snl
