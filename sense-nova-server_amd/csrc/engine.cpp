// The decode engine behind the C ABI: device-resident weights, KV caches and recurrent
// state, the per-visit op sequence of the reference's Engine, and one captured hipGraph
// per pass shape (forward M=1/M=2 with 0..2 logit rows and optional checkpoint, MTP head
// M=1/M=2 with or without a draft).  Mirrors src/engine.rs (op graph :383-493, MTP
// :495-580 and :713-774, forward_mm :801-936, rollback/snapshot/restore/reset :646-697).
// The worker's decode loop and prefix cache over these entry points are in worker.cpp.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/snl.h"
#include "kernels.h"
#include "packing.h"
#include "snl_file.h"

namespace snl {

// cos / sin of the rotary angles of the step's rows (the reference's prep, attention.wgsl:90-110):
// frequency f < rot_dim / 2 turns by pos * theta^(-2f / rot_dim), where pos is the row's t, h or w
// position by the M-RoPE interleave (f % 3 == 1 below 3 * section[1] takes h, f % 3 == 2 below
// 3 * section[2] takes w, the rest t).  The same float operations as a device-side prep.
void step_rope(StepDev& st, int rows, float theta, int rot_dim, const int32_t* section) {
    const int half = rot_dim / 2;
    for (int m = 0; m < rows; ++m)
        for (int f = 0; f < half && f < SNL_ROPE_MAX; ++f) {
            uint32_t rp = st.rpos[m][0];
            if (f % 3 == 1 && f < 3 * section[1]) rp = st.rpos[m][1];
            else if (f % 3 == 2 && f < 3 * section[2]) rp = st.rpos[m][2];
            const float inv_freq = powf(theta, -(float)(2 * f) / (float)rot_dim);
            const float ang = (float)rp * inv_freq;
            st.rope[m][f][0] = cosf(ang);
            st.rope[m][f][1] = sinf(ang);
        }
}

int device_error(hipError_t e, const char* what) {
    (void)e;
    (void)what;
    return SNL_EDEVICE;
}

namespace {

constexpr int kSnapshots = SNL_SNAPSHOTS;
constexpr int kLogitRows = 2;
constexpr int kDistMax = 1024;  // largest k the device top-k serves (SNL_DIST_MAX)
// Token rows per captured pass.  The kernels take up to SNL_MAX_M; passes use 1 or 2.
constexpr int kMaxM = 2;
// Hidden rows: row 0 carries the token before a pass, rows 1..M a pass's final-normed rows (up to
// SNL_PF_M), and one more row for the padding row a two-row draft over r0 = SNL_PF_M reads.
constexpr int kHidRows = SNL_PF_M + kMaxM;
constexpr int kSpecRing = 4;  // speculative step outcomes held in pinned memory

// Tensor kinds of the seeded initialiser: stream id = ((layer + 1) << 8) | kind for layer
// tensors (layer 0xFFF is the MTP head), kind alone for the globals.
enum Kind {
    K_EMBED = 1, K_LM_HEAD = 2, K_NORM = 3,
    K_IN_LN = 1, K_POST_LN = 2, K_QK_NORM = 3, K_LIN = 4, K_QKV = 5, K_O_PROJ = 6, K_IN_PROJ = 7,
    K_OUT_PROJ = 8, K_GATE_UP = 9, K_DOWN = 10, K_MHC_ATTN = 11, K_MHC_FFN = 12,
    K_FC_E = 20, K_FC_H = 21, K_NORM_E = 22, K_NORM_H = 23, K_MTP_NORM = 24
};
constexpr int kMtpLayer = 0xFFF;

// Name of tensor (layer, kind) in the reference's weight files (src/convert.rs:203-311): the
// main file holds the globals and l{i}.*, the MTP file mtp.*.
std::string tensor_name(int layer, int kind) {
    if (layer == -1) return kind == K_EMBED ? "embed" : kind == K_LM_HEAD ? "lm_head" : "norm";
    const std::string p = layer == kMtpLayer ? std::string("mtp.") : "l" + std::to_string(layer) + ".";
    switch (kind) {
        case K_IN_LN: return p + "in_ln";
        case K_POST_LN: return p + "post_ln";
        case K_QK_NORM: return p + "qk_norm";
        case K_LIN: return p + "lin";
        case K_QKV: return p + "qkv";
        case K_O_PROJ: return p + "o_proj";
        case K_IN_PROJ: return p + "in_proj";
        case K_OUT_PROJ: return p + "out_proj";
        case K_GATE_UP: return p + "gate_up";
        case K_DOWN: return p + "down";
        case K_MHC_ATTN: return p + "mhc_attn";
        case K_MHC_FFN: return p + "mhc_ffn";
        case K_FC_E: return p + "fc_e";
        case K_FC_H: return p + "fc_h";
        case K_NORM_E: return p + "norm_e";
        case K_NORM_H: return p + "norm_h";
        case K_MTP_NORM: return p + "norm";
    }
    return p + "?";
}

uint64_t host_smix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}
uint64_t stream_key(uint64_t seed, int layer, int kind) {
    uint64_t stream = layer < 0 ? (uint64_t)kind : (((uint64_t)(layer + 1) << 8) | (uint64_t)kind);
    return host_smix(seed ^ host_smix(stream * 0xD1B54A32D192ED03ull));
}

// mHC roles of a GEMV launch: `site` is the router of its own site (NORM_MHC prologue: sums from
// the partials in mhc_part, coefficients left in coef for the site's MHC epilogue), `next` the
// router of the next site whose partials its epilogue leaves in mhc_part (expand: stream 1 :=
// stream 0 first).
struct MhcRole {
    const float* site = nullptr;
    const float* next = nullptr;
    int expand = 0;
};

struct QW {
    void* q = nullptr;
    float* s = nullptr;
    int rows = 0, cols = 0, quant = 0;
    bool packed = false;  // tile order (packing.h); otherwise the reference's row-major layout
    int inter = 0;        // packed with SwiGLU pairing of gate/up rows when > 0
    void* pq = nullptr;   // panel order for the prefill GEMM (mgemm.hip), rows in reference order
    float* ps = nullptr;
};

struct Vec {
    float* p = nullptr;
    int n = 0;
};

struct Layer {
    bool full = false;
    Vec in_ln, post_ln, small, mhc_attn, mhc_ffn;
    QW mix_in, mix_out, gate_up, down;
};

std::string g_create_error;

}  // namespace
}  // namespace snl

using namespace snl;

struct snl_engine {
    snl_config cfg{};
    int ctx = 0, quant = 0;
    uint64_t seed = 0;
    int64_t max_position = 262144;  // ModelConfig::max_position, kept for snl_engine_save
    // weight files while snl_engine_load runs init (null: the seeded generator draws the weights)
    const SnlFile* src = nullptr;
    const SnlFile* msrc = nullptr;
    hipStream_t stream = nullptr;
    // Passes are captured on a stream of their own, idle whatever the engine's stream still runs
    // (graphs do not depend on the stream they were captured on).
    hipStream_t cap_stream = nullptr;
    std::vector<void*> allocs;
    // reference-layout staging of one matrix while the weights are drawn and packed (init only)
    uint8_t* gen_tmp_q = nullptr;
    float* gen_tmp_s = nullptr;
    size_t gen_tmp_n = 0;

    QW embed, lm_head;
    Vec final_norm;
    std::vector<Layer> layers;
    QW fc_e, fc_h, m_qkv, m_o, m_gate_up, m_down;
    Vec norm_e, norm_h, m_norm, m_in_ln, m_post_ln, m_qk_norm;

    std::vector<int> plan;
    int n_full = 0, n_lin = 0;
    int h = 0, q_dim = 0, kv_dim = 0, conv_dim = 0, lin_proj_rows = 0, attn_proj_rows = 0, lin_value_dim = 0;

    float *x = nullptr, *xn = nullptr, *proj = nullptr, *act = nullptr, *attn_out = nullptr, *qbuf = nullptr;
    float* dn_ssq = nullptr;  // DeltaNet partial sums of squares [M][n_v][kDeltaGroups]
    float *coef = nullptr, *mhc_raw = nullptr, *mhc_part = nullptr, *partial = nullptr, *logits = nullptr, *hid = nullptr,
          *hlast = nullptr;
    float *mx = nullptr, *hn = nullptr, *m_logits = nullptr;
    // chunked prefill: up to SNL_PF_M rows per pass, launched eagerly (prefill.hip, mgemm.hip,
    // attention_prefill.hip)
    float *pf_x = nullptr, *pf_proj = nullptr, *pf_act = nullptr, *pf_attn = nullptr, *pf_qbuf = nullptr,
          *pf_br = nullptr, *pf_xs = nullptr, *pf_part = nullptr, *pf_coef = nullptr, *pf_ssq = nullptr;
    float* pf_pairs = nullptr;  // prefill DeltaNet: k.k / k.q inside blocks of 4 tokens
    float *pf_dq = nullptr, *pf_dk = nullptr, *pf_dv = nullptr, *pf_gz = nullptr, *pf_beta = nullptr,
          *pf_decay = nullptr;
    void* pf_frags = nullptr;
    float* pf_apart = nullptr;  // attention key-part partials (contexts past one part)
    int pf_parts = 1;
    int pf_pos0 = 0;            // cache position of the current prefill pass's row 0
    PrefillDev *d_pstep = nullptr, *h_pstep = nullptr;  // h_pstep: pinned
    uint16_t *kcache = nullptr, *vcache = nullptr, *m_kc = nullptr, *m_vc = nullptr;
    float *lin_state = nullptr, *conv_state = nullptr;
    size_t state_floats = 0, conv_floats = 0;  // per visit
    float *snap_lin[kSnapshots] = {}, *snap_conv[kSnapshots] = {}, *snap_h[kSnapshots] = {};
    float* pick_scratch = nullptr;
    Pick *d_picks = nullptr, *d_mpick = nullptr;
    Pick* h_picks = nullptr;  // pinned, 3 entries: 2 forward rows + 1 draft, written by the pick kernels
    Pick* hd_picks = nullptr;  // the device's address of h_picks
    // speculative steps (run kind 2): two graph instances (parity), each with its events before
    // the draft, between the passes and after the verify; the outcome ring in pinned memory; the
    // rotary cos / sin of every text position
    hipEvent_t spec_ev[2][3] = {};
    SpecOut* h_ring = nullptr;   // pinned, kSpecRing entries
    SpecOut* hd_ring = nullptr;  // its device address
    uint32_t spec_seq = 0;       // number of the next speculative step
    float* rope_tab = nullptr;   // [rope_rows][SNL_ROPE_MAX][2]
    int rope_rows = 0;
    // h_step: pinned, 2 records (forward, MTP); d_step / d_mstep: their device copies, adjacent
    StepDev *d_step = nullptr, *d_mstep = nullptr, *h_step = nullptr;

    int cur = 0, ck_slot = -1;
    int pos = 0, hid_rows = 0;
    int logit_rows = 0;  // logits rows the last forward left in `logits`
    // sampler scratch: top-k keys, penalty lists, pinned readback
    unsigned long long* topk_keys = nullptr;
    uint32_t* pen_dev = nullptr;       // [2][vocab]: tokens, counts
    unsigned long long* topk_host = nullptr;  // pinned, kDistMax keys
    // Counts the calls that change the caches, the recurrent state or a snapshot slot, so that a
    // holder of cache bookkeeping (the worker) can tell whether someone else has moved the engine.
    uint64_t epoch = 0;
    std::map<std::tuple<int, int, int, int, int>, hipGraphExec_t> graphs;
    // Keys the decode attention launches of a captured pass cover (its grid, part count and
    // query-prep path): the context bucket of the positions the pass may reach, so the cost of a
    // decode pass follows the position, not the allocated context.  0 outside recording.
    int span = 0;
    std::string err;

    // Per-op timing of an eagerly launched pass (the reference's SENSENOVA_PROFILE mode,
    // src/engine.rs:859-886, with device timestamps instead of host wall clock).
    struct Mark {
        const char* name;
        double bytes;
        hipEvent_t ev;
    };
    std::vector<Mark>* marks = nullptr;
    void mark(const char* name, double bytes) {
        if (!marks) return;
        hipEvent_t ev = nullptr;
        hipEventCreate(&ev);
        hipEventRecord(ev, stream);
        marks->push_back({name, bytes, ev});
    }
    // Isolated-op timing: when `only` is set, a pass launches only the ops of that name.
    const char* only = nullptr;
    int only_launches = 0;
    double only_bytes = 0.0;
    // Marks the start of op `name` and says whether to launch it.
    bool op(const char* name, double bytes) {
        if (only) {
            if (strcmp(name, only) != 0) return false;
            ++only_launches;
            only_bytes += bytes;
            return true;
        }
        mark(name, bytes);
        return true;
    }
    // Algorithmic HBM bytes of one GEMV launch: quants + f32 scales + the M input rows +
    // the output (read and written back for the residual epilogues).
    static double gemv_bytes(const QW& w, int M, int epi, int inter) {
        const double n = w.rows, k = w.cols;
        double b = n * k * (w.quant == 0 ? 1.0 : 0.5) + n * (k / 32) * 4 + (double)M * k * 4;
        if (epi == GEMV_STORE) b += (double)M * n * 4;
        else if (epi == GEMV_ADD) b += 2.0 * M * n * 4;
        else if (epi == GEMV_MHC) b += 4.0 * M * n * 4;
        else b += (double)M * inter * 4;
        return b;
    }

    int fail(int code, const char* fmt, ...) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        err = buf;
        return code;
    }

    template <class T>
    int dalloc(T** p, size_t count) {
        void* v = nullptr;
        if (hipMalloc(&v, count * sizeof(T) > 0 ? count * sizeof(T) : 16) != hipSuccess) {
            *p = nullptr;
            return fail(SNL_ENOMEM, "hipMalloc of %zu bytes failed", count * sizeof(T));
        }
        allocs.push_back(v);
        *p = static_cast<T*>(v);
        return SNL_OK;
    }

    // Draw a rows x cols quantised matrix (reference layout, src/weights.rs:48-55).  GEMV matrices
    // (pack_inter >= 0) are then stored in tile order; pack_inter > 0 pairs gate and up rows; with
    // `panel` a second copy in the prefill GEMM's panel order is kept.
    // With a weight file the matrix is read from it instead (its own dtype; the shape must match).
    int gen_q(QW& w, int layer, int kind, int rows, int cols, int qt, int pack_inter = 0, bool panel = true) {
        const SnlFile* f = layer == kMtpLayer ? msrc : src;
        const FileTensor* ft = nullptr;
        if (f) {
            const std::string name = tensor_name(layer, kind);
            ft = f->find(name);
            if (!ft) return fail(SNL_EARG, "weight file is missing tensor `%s`", name.c_str());
            if (ft->dtype == FD_F32 || ft->shape.size() != 2 || ft->rows() != rows || ft->cols() != cols)
                return fail(SNL_EARG, "tensor `%s`: expected a quantised [%d, %d] matrix", name.c_str(), rows, cols);
            qt = ft->dtype == FD_Q8_0 ? 0 : 1;
        }
        w.rows = rows;
        w.cols = cols;
        w.quant = qt;
        const size_t n = (size_t)rows * cols;
        const size_t qn = qt == 0 ? n : n / 2;
        const uint64_t key = stream_key(seed, layer, kind);
        int rc;
        // fill reference-layout quants and scales, from the file or the generator
        auto fill = [&](void* q, float* sc) {
            if (ft)
                return hipMemcpyAsync(q, f->quants(*ft), qn, hipMemcpyHostToDevice, stream) != hipSuccess ||
                       hipMemcpyAsync(sc, f->scales(*ft), n / 32 * 4, hipMemcpyHostToDevice, stream) != hipSuccess;
            return launch_gen_matrix(key, rows, cols, 0.02f, qt, q, sc, stream) != 0;
        };
        if (pack_inter < 0) {
            uint8_t* q;
            if ((rc = dalloc(&q, qn))) return rc;
            w.q = q;
            if ((rc = dalloc(&w.s, n / 32))) return rc;
            if (fill(w.q, w.s)) return fail(SNL_EDEVICE, "weight init failed");
            return SNL_OK;
        }
        PackGeom g;
        if (!pack_geom(qt, rows, cols, pack_inter, &g))
            return fail(SNL_EARG, "a %d x %d GEMV matrix needs K %% 128 == 0", rows, cols);
        if (n > gen_tmp_n) {
            if (hipStreamSynchronize(stream) != hipSuccess) return fail(SNL_EDEVICE, "weight init failed");
            hipFree(gen_tmp_q);
            hipFree(gen_tmp_s);
            gen_tmp_q = nullptr;
            gen_tmp_s = nullptr;
            gen_tmp_n = 0;
            if (hipMalloc((void**)&gen_tmp_q, n) != hipSuccess || hipMalloc((void**)&gen_tmp_s, n / 32 * 4) != hipSuccess)
                return fail(SNL_ENOMEM, "hipMalloc of the %zu-byte weight staging buffer failed", n);
            gen_tmp_n = n;
        }
        uint8_t* q;
        if ((rc = dalloc(&q, g.q_bytes))) return rc;
        w.q = q;
        if ((rc = dalloc(&w.s, g.s_floats))) return rc;
        w.packed = true;
        w.inter = pack_inter;
        if (fill(gen_tmp_q, gen_tmp_s) || launch_pack_matrix(g, gen_tmp_q, gen_tmp_s, w.q, w.s, stream))
            return fail(SNL_EDEVICE, "weight init failed");
        if (panel) {
            uint8_t* pq;
            if ((rc = dalloc(&pq, gemm_q_bytes(qt, rows, cols))) || (rc = dalloc(&w.ps, gemm_s_floats(rows, cols))))
                return rc;
            w.pq = pq;
            if (launch_panel_pack(qt, rows, cols, gen_tmp_q, gen_tmp_s, w.pq, w.ps, stream))
                return fail(SNL_EDEVICE, "weight init failed");
        }
        return SNL_OK;
    }

    void free_gen_tmp() {
        if (gen_tmp_q || gen_tmp_s) hipStreamSynchronize(stream);
        hipFree(gen_tmp_q);
        hipFree(gen_tmp_s);
        gen_tmp_q = nullptr;
        gen_tmp_s = nullptr;
        gen_tmp_n = 0;
    }

    int gen_v(Vec& v, int layer, int kind, int n, int vkind, float stdv, int aux0 = 0, int aux1 = 0) {
        v.n = n;
        int rc = dalloc(&v.p, n);
        if (rc) return rc;
        if (const SnlFile* f = layer == kMtpLayer ? msrc : src) {
            const std::string name = tensor_name(layer, kind);
            const FileTensor* ft = f->find(name);
            if (!ft) return fail(SNL_EARG, "weight file is missing tensor `%s`", name.c_str());
            if (ft->dtype != FD_F32 || ft->rows() * ft->cols() != n)
                return fail(SNL_EARG, "tensor `%s`: expected %d f32 values", name.c_str(), n);
            if (hipMemcpyAsync(v.p, f->quants(*ft), (size_t)n * 4, hipMemcpyHostToDevice, stream) != hipSuccess)
                return fail(SNL_EDEVICE, "weight upload failed");
            return SNL_OK;
        }
        if (launch_gen_vector(stream_key(seed, layer, kind), n, vkind, stdv, aux0, aux1, v.p, stream))
            return fail(SNL_EDEVICE, "vector init launch failed");
        return SNL_OK;
    }

    bool is_mhc(int l) const { return cfg.mhc_streams > 0 && cfg.mhc_start <= l && l < cfg.mhc_end; }

    int init();
    int record_forward(int M, int rows, int ckpt);
    int record_mtp(int M, int draft);
    int record_prefill(int M, int rows);
    int record_mtp_prefill(int M, int r0);
    int prefill_chunk(const uint32_t* tokens, const uint32_t* pos3, int m, int cache_pos0, int rows, bool mtp, int r0);
    const uint32_t* pf_tokens() const {
        return reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(d_pstep) + offsetof(PrefillDev, tokens));
    }
    // token rows -> GEMM fragments (the branch input on the way) -> panel GEMM
    int pf_mat(const char* name, const QW& w, const float* xin, int x_stride, int M, int mode, const float* nw,
               float* y, int y_stride) {
        int rc = 0;
        if (op("rows", 0.0)) {
            RowsArgs r{};
            r.x = xin;
            r.x_stride = x_stride;
            r.M = M;
            r.K = w.cols;
            r.mode = mode;
            r.w = nw;
            r.coef = pf_coef;
            r.h = h;
            r.ssq = pf_ssq;
            r.eps = cfg.eps;
            r.perm4 = w.quant;
            r.frags = pf_frags;
            r.xs = pf_xs;
            rc |= launch_rows_to_frags(r, stream);
        }
        if (op(name, 0.0)) {
            GemmArgs g{};
            g.wq = w.pq;
            g.ws = w.ps;
            g.frags = pf_frags;
            g.xs = pf_xs;
            g.y = y;
            g.y_stride = y_stride;
            g.M = M;
            g.N = w.rows;
            g.K = w.cols;
            rc |= launch_mgemm(g, w.quant, stream);
        }
        return rc;
    }
    // an mHC site over prefill rows: router sums, then the token coefficients in pf_coef
    int pf_site(const float* w, int M) {
        if (!op("mhc", 0.0)) return 0;
        return launch_mhc(pf_x, w, pf_part, h, M, stream) |
               launch_mhc_coef(pf_part, w, h, cfg.mhc_iterations, pf_coef, M, stream);
    }
    int run(int kind, int M, int a, int b, int keys, bool upload = true);
    // The context bucket serving passes over up to `keys` cache positions: 2048 * 2^k, capped at
    // the allocated context.  Results do not depend on it (blocks past the live keys return, and
    // both query-prep paths give the same bits); only the launch shape does.
    int span_for(int keys) const {
        int b = 2048;
        while (b < keys && b < ctx) b *= 2;
        return std::min(b, ctx);
    }
    int ensure_rope_tab();
    int build_spec_pair(int keys);
    // Keys of the speculative steps that follow a prompt: the next prefill chunk builds their
    // graphs (and the rotary table) on the host while its passes run, instead of the first step.
    int spec_prebuild = 0;
    // the speculative step's graph (run kind 2): the MTP draft over M pairs, then the checkpointed
    // 2-row verify whose second token is the draft's pick, with event records around both passes
    int build_spec(int M, int parity, int sp, hipGraphExec_t* out);
    static constexpr int kPartBlocks = 4096;  // partial-sum slots of mhc_part per token
    int part_n = 0;                           // partials currently in mhc_part (0: none)
    // GEMV with an optional fused branch-input prologue (pro: GEMV_NORM with norm weights nw, or
    // GEMV_NORM_MHC) and the epilogue `epi`.
    int gemv(const char* name, const QW& w, const float* xin, int x_stride, float* y, int y_stride, int M, int epi,
             int merge_mode = 0, int pro = GEMV_PLAIN, const float* nw = nullptr, const int32_t* row_base = nullptr,
             MhcRole mr = {}) {
        if (mr.next) {  // this launch leaves the next site's partials, launched or not (isolated timing)
            const int n = mgemv_blocks(w.quant, w.rows, w.cols, epi == GEMV_SWIGLU ? cfg.intermediate : 0);
            if (n < 1 || n > kPartBlocks) return SNL_EDEVICE;
            part_n = n;
        }
        float *no = norm_out, *nl = norm_last;  // (cleared whether or not this call launches)
        norm_out = norm_last = nullptr;
        if (!op(name, gemv_bytes(w, M, epi, cfg.intermediate))) return 0;
        GemvArgs g{};
        g.packed = w.packed ? 1 : 0;
        g.wq = w.q;
        g.ws = w.s;
        g.x = xin;
        g.x_stride = x_stride;
        g.row_base = row_base;
        g.y = y;
        g.y_stride = y_stride;
        g.N = w.rows;
        g.K = w.cols;
        g.epi = epi;
        g.merge_mode = merge_mode;
        g.h = h;
        g.inter = cfg.intermediate;
        g.pro = pro;
        g.norm_w = nw;
        g.eps = cfg.eps;
        g.site_w = mr.site;
        g.raw = mhc_raw;
        g.coef = coef;
        g.rin = pro == GEMV_GNORM ? dn_ssq : mhc_part;
        g.rin_n = pro == GEMV_NORM_MHC ? consumed_n : pro == GEMV_GNORM ? kDeltaGroups : 0;
        g.iterations = cfg.mhc_iterations;
        g.next_w = mr.next;
        g.rpart = mr.next ? mhc_part : nullptr;
        g.expand = mr.expand;
        g.norm_out = no;
        g.norm_last = nl;
        return launch_gemv(g, w.quant, M, stream);
    }
    int consumed_n = 0;  // partial count a NORM_MHC launch adds up
    float *norm_out = nullptr, *norm_last = nullptr;  // the next gemv() call's normed-row outputs
    int norm(const float* xin, int x_stride, const int32_t* row_base, int mode, const float* w, float* out,
             int first, int count, float* last_copy = nullptr) {
        NormArgs a{};
        a.last_copy = last_copy;
        a.x = xin;
        a.x_stride = x_stride;
        a.row_base = row_base;
        a.coef = coef;
        a.w = w;
        a.out = out;
        a.out_stride = h;
        a.h = h;
        a.mode = mode;
        a.first = first;
        a.count = count;
        a.eps = cfg.eps;
        a.one = 1.0f;
        if (!op("norm", 0.0)) return 0;
        return launch_branch_norm(a, stream);
    }
    AttnArgs attn_args(const StepDev* st, uint16_t* kc, uint16_t* vc, const float* norms) const {
        AttnArgs a{};
        a.proj = proj;
        a.proj_stride = attn_proj_rows;
        a.qbuf = qbuf;
        a.kcache = kc;
        a.vcache = vc;
        a.norms = norms;
        a.out = attn_out;
        a.partial = partial;
        a.n_heads = cfg.n_heads;
        a.n_kv = cfg.n_kv_heads;
        a.rot_dim = cfg.rot_dim;
        a.rope_theta = cfg.rope_theta;
        a.eps = cfg.eps;
        a.scale = 1.0f / sqrtf((float)cfg.head_dim);
        a.mrope = ((uint32_t)(3 * cfg.mrope_section[1]) << 16) | (uint32_t)(3 * cfg.mrope_section[2]);
        a.ctx = span > 0 ? span : ctx;
        a.step = st;
        return a;
    }
};

// config.rs:195-240
static const char* validate(const snl_config* c) {
    if (c->head_dim != 256) return "head_dim must be 256";
    if (c->lin_k_dim != 128 || c->lin_v_dim != 128) return "linear head dims must be 128";
    if (c->conv_kernel != 4) return "linear conv kernel must be 4";
    if (c->hidden % 256 != 0 || c->hidden > 8192) return "hidden size must be a multiple of 256 (at most 8192)";
    if (c->n_layers < 1 || c->n_layers > 64) return "layer count must be 1..64";
    if (c->n_heads != 4 * c->n_kv_heads) return "attention must have 4 query heads per KV head";
    if (c->lin_k_heads < 1 || c->lin_v_heads % c->lin_k_heads != 0)
        return "linear value heads must be a multiple of key heads";
    if (c->rot_dim % 2 != 0 || c->rot_dim > c->head_dim || c->rot_dim < 2) return "invalid rotary dim";
    if (c->rot_dim > 2 * SNL_ROPE_MAX) return "rotary dim must be at most 128";
    if (c->mrope_section[0] + c->mrope_section[1] + c->mrope_section[2] != c->rot_dim / 2)
        return "M-RoPE sections must cover the rotary dims";
    if (!(c->loop_start < c->loop_end && c->loop_end <= c->n_layers && c->loop_count >= 1)) return "invalid loop range";
    if (c->intermediate % 32 != 0 || c->vocab < 2) return "invalid intermediate size or vocab";
    // the prefill GEMM takes rows of at most 16384 (the down projection's K)
    if (c->intermediate > 16384) return "intermediate size must be at most 16384";
    if (c->mhc_streams != 0) {
        if (c->mhc_streams != 2) return "only 2 mHC streams are supported";
        const int s = c->mhc_start, e = c->mhc_end;
        const bool ok = (0 <= s && e <= c->loop_start) || (c->loop_start <= s && e <= c->loop_end) ||
                        (c->loop_end <= s && e <= c->n_layers);
        if (!ok || s >= e) return "mHC range crosses a loop boundary";
    }
    if (c->n_eos < 0 || c->n_eos > 4) return "at most 4 EOS ids";
    return nullptr;
}

int snl_engine::init() {
    const snl_config& c = cfg;
    h = c.hidden;
    q_dim = c.n_heads * c.head_dim;
    kv_dim = c.n_kv_heads * c.head_dim;
    lin_value_dim = c.lin_v_heads * c.lin_v_dim;
    conv_dim = 2 * c.lin_k_heads * c.lin_k_dim + lin_value_dim;
    lin_proj_rows = conv_dim + lin_value_dim + 2 * c.lin_v_heads;
    attn_proj_rows = 2 * q_dim + 2 * kv_dim;
    for (int i = 0; i < c.loop_start; ++i) plan.push_back(i);
    for (int r = 0; r < c.loop_count; ++r)
        for (int i = c.loop_start; i < c.loop_end; ++i) plan.push_back(i);
    for (int i = c.loop_end; i < c.n_layers; ++i) plan.push_back(i);
    for (int l : plan) (c.full_attention[l] ? n_full : n_lin)++;

    if (hipStreamCreateWithFlags(&stream, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&cap_stream, hipStreamNonBlocking) != hipSuccess)
        return fail(SNL_EDEVICE, "hipStreamCreate failed");
    if (gemv_init()) return fail(SNL_EDEVICE, "GEMV LDS configuration failed");
    int rc;
    // ---- weights (convert.rs:228-311 layout; seeded values) ----
    if ((rc = gen_q(lm_head, -1, K_LM_HEAD, c.vocab, h, 0, 0, false))) return rc;
    if ((rc = gen_q(embed, -1, K_EMBED, c.vocab, h, 0, -1))) return rc;  // gathered by row
    if ((rc = gen_v(final_norm, -1, K_NORM, h, 0, 0.1f))) return rc;
    layers.resize(c.n_layers);
    for (int l = 0; l < c.n_layers; ++l) {
        Layer& L = layers[l];
        L.full = c.full_attention[l] != 0;
        if ((rc = gen_v(L.in_ln, l, K_IN_LN, h, 0, 0.1f))) return rc;
        if ((rc = gen_v(L.post_ln, l, K_POST_LN, h, 0, 0.1f))) return rc;
        if (L.full) {
            if ((rc = gen_v(L.small, l, K_QK_NORM, 2 * c.head_dim, 0, 0.1f))) return rc;
            if ((rc = gen_q(L.mix_in, l, K_QKV, attn_proj_rows, h, quant))) return rc;
            if ((rc = gen_q(L.mix_out, l, K_O_PROJ, h, q_dim, quant))) return rc;
        } else {
            const int n = conv_dim * 4 + 2 * c.lin_v_heads + c.lin_v_dim;
            if ((rc = gen_v(L.small, l, K_LIN, n, 2, 0.0f, conv_dim, c.lin_v_heads))) return rc;
            if ((rc = gen_q(L.mix_in, l, K_IN_PROJ, lin_proj_rows, h, 0))) return rc;
            if ((rc = gen_q(L.mix_out, l, K_OUT_PROJ, h, lin_value_dim, quant))) return rc;
        }
        if ((rc = gen_q(L.gate_up, l, K_GATE_UP, 2 * c.intermediate, h, quant, c.intermediate))) return rc;
        if ((rc = gen_q(L.down, l, K_DOWN, h, c.intermediate, quant))) return rc;
        if (is_mhc(l)) {
            if ((rc = gen_v(L.mhc_attn, l, K_MHC_ATTN, 16 * h + 8, 3, 0.0f, h))) return rc;
            if ((rc = gen_v(L.mhc_ffn, l, K_MHC_FFN, 16 * h + 8, 3, 0.0f, h))) return rc;
        }
    }
    if (c.has_mtp) {
        const int L = kMtpLayer;
        if ((rc = gen_q(fc_e, L, K_FC_E, h, h, 0))) return rc;
        if ((rc = gen_q(fc_h, L, K_FC_H, h, h, 0))) return rc;
        if ((rc = gen_q(m_qkv, L, K_QKV, attn_proj_rows, h, 0))) return rc;
        if ((rc = gen_q(m_o, L, K_O_PROJ, h, q_dim, 0))) return rc;
        if ((rc = gen_q(m_gate_up, L, K_GATE_UP, 2 * c.intermediate, h, 0, c.intermediate))) return rc;
        if ((rc = gen_q(m_down, L, K_DOWN, h, c.intermediate, 0))) return rc;
        if ((rc = gen_v(norm_e, L, K_NORM_E, h, 0, 0.1f))) return rc;
        if ((rc = gen_v(norm_h, L, K_NORM_H, h, 0, 0.1f))) return rc;
        if ((rc = gen_v(m_norm, L, K_MTP_NORM, h, 0, 0.1f))) return rc;
        if ((rc = gen_v(m_in_ln, L, K_IN_LN, h, 0, 0.1f))) return rc;
        if ((rc = gen_v(m_post_ln, L, K_POST_LN, h, 0, 0.1f))) return rc;
        if ((rc = gen_v(m_qk_norm, L, K_QK_NORM, 2 * c.head_dim, 0, 0.1f))) return rc;
    }
    free_gen_tmp();

    // ---- activations (src/engine.rs:244-256), sized for kMaxM rows ----
    const int proj_w = std::max(std::max(2 * c.intermediate, lin_proj_rows), attn_proj_rows);
    const int act_w = std::max(c.intermediate, conv_dim);
    const int attn_w = std::max(q_dim, lin_value_dim);
    const int M = SNL_MAX_M;
    const int parts_max = (ctx + kAttnPart - 1) / kAttnPart;
    if ((rc = dalloc(&x, (size_t)M * 2 * h)) || (rc = dalloc(&xn, (size_t)M * h)) ||
        (rc = dalloc(&proj, (size_t)M * proj_w)) || (rc = dalloc(&act, (size_t)M * act_w)) ||
        (rc = dalloc(&attn_out, (size_t)M * attn_w)) || (rc = dalloc(&qbuf, (size_t)M * q_dim)) ||
        (rc = dalloc(&coef, (size_t)M * 8)) || (rc = dalloc(&mhc_raw, (size_t)M * 9)) ||
        (rc = dalloc(&dn_ssq, (size_t)M * std::max(c.lin_v_heads, 1) * kDeltaGroups)) ||
        (rc = dalloc(&mhc_part, (size_t)kPartBlocks * M * 9)) ||
        (rc = dalloc(&partial, (size_t)M * c.n_heads * parts_max * (c.head_dim + 2))) ||
        (rc = dalloc(&logits, (size_t)kLogitRows * c.vocab)) || (rc = dalloc(&hid, (size_t)kHidRows * h)) ||
        (rc = dalloc(&hlast, (size_t)h)) || (rc = dalloc(&mx, (size_t)M * 2 * h)) ||
        (rc = dalloc(&hn, (size_t)M * h)) || (rc = dalloc(&m_logits, (size_t)c.vocab)) ||
        (rc = dalloc(&pick_scratch, pick_scratch_floats(c.vocab, kLogitRows))) || (rc = dalloc(&d_picks, 2)) ||
        (rc = dalloc(&d_mpick, 1)) || (rc = dalloc(&d_step, 2)))
        return rc;
    d_mstep = d_step + 1;
    // ---- sampler scratch ----
    if ((rc = dalloc(&topk_keys, topk_scratch_keys(c.vocab, kDistMax))) || (rc = dalloc(&pen_dev, (size_t)2 * c.vocab)))
        return rc;
    if (hipHostMalloc((void**)&topk_host, kDistMax * sizeof(unsigned long long), hipHostMallocDefault) != hipSuccess)
        return fail(SNL_ENOMEM, "pinned host allocation failed");
    // ---- chunked prefill rows ----
    {
        const size_t P = SNL_PF_M;
        const int kmax = std::max(std::max(h, c.intermediate), std::max(q_dim, lin_value_dim));
        const int nv = std::max(c.lin_v_heads, 1);
        const size_t key_dim = (size_t)c.lin_k_heads * c.lin_k_dim;
        if ((rc = dalloc(&pf_x, P * 2 * h)) || (rc = dalloc(&pf_proj, P * proj_w)) ||
            (rc = dalloc(&pf_act, P * c.intermediate)) || (rc = dalloc(&pf_attn, P * attn_w)) ||
            (rc = dalloc(&pf_qbuf, P * q_dim)) || (rc = dalloc(&pf_br, P * h)) || (rc = dalloc(&pf_xs, P)) ||
            (rc = dalloc(&pf_part, P * 9)) || (rc = dalloc(&pf_coef, P * 8)) ||
            (rc = dalloc(&pf_ssq, P * nv * kDeltaPrefillGroups)) ||
            (rc = dalloc(&pf_pairs, dn_pairs_floats((int)P, std::max(c.lin_k_heads, 1)))) || (rc = dalloc(&pf_dq, P * std::max<size_t>(key_dim, 1))) ||
            (rc = dalloc(&pf_dk, P * std::max<size_t>(key_dim, 1))) || (rc = dalloc(&pf_dv, P * lin_value_dim + 1)) ||
            (rc = dalloc(&pf_gz, P * lin_value_dim + 1)) || (rc = dalloc(&pf_beta, P * nv)) ||
            (rc = dalloc(&pf_decay, P * nv)) || (rc = dalloc((uint8_t**)&pf_frags, frags_bytes(SNL_PF_M, kmax))) ||
            (rc = dalloc(&d_pstep, 1)))
            return rc;
        pf_parts = attention_prefill_parts(ctx);
        if (pf_parts > 1 && (rc = dalloc(&pf_apart, P * c.n_heads * pf_parts * (c.head_dim + 2)))) return rc;
        if (hipHostMalloc((void**)&h_pstep, sizeof(PrefillDev), hipHostMallocDefault) != hipSuccess)
            return fail(SNL_ENOMEM, "pinned host allocation failed");
    }
    // ---- caches and recurrent state ----
    const size_t kvn = (size_t)ctx * kv_dim;
    if ((rc = dalloc(&kcache, kvn * std::max(n_full, 1))) || (rc = dalloc(&vcache, kvn * std::max(n_full, 1))) ||
        (rc = dalloc(&m_kc, c.has_mtp ? kvn : 1)) || (rc = dalloc(&m_vc, c.has_mtp ? kvn : 1)))
        return rc;
    state_floats = (size_t)c.lin_v_heads * c.lin_k_dim * c.lin_v_dim;
    conv_floats = (size_t)3 * conv_dim;
    const size_t nl = std::max(n_lin, 1);
    if ((rc = dalloc(&lin_state, 3 * nl * state_floats)) || (rc = dalloc(&conv_state, 3 * nl * conv_floats)))
        return rc;
    for (int i = 0; i < kSnapshots; ++i)
        if ((rc = dalloc(&snap_lin[i], nl * state_floats)) || (rc = dalloc(&snap_conv[i], nl * conv_floats)) ||
            (rc = dalloc(&snap_h[i], (size_t)h)))
            return rc;
    if (hipHostMalloc((void**)&h_picks, 3 * sizeof(Pick), hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc((void**)&h_step, 2 * sizeof(StepDev), hipHostMallocDefault) != hipSuccess)
        return fail(SNL_ENOMEM, "pinned host allocation failed");
    if (hipHostGetDevicePointer((void**)&hd_picks, h_picks, 0) != hipSuccess || !hd_picks)
        return fail(SNL_EDEVICE, "no device address for the pinned picks");
    memset(h_picks, 0, 3 * sizeof(Pick));
    if (hipHostMalloc((void**)&h_ring, kSpecRing * sizeof(SpecOut), hipHostMallocDefault) != hipSuccess)
        return fail(SNL_ENOMEM, "pinned host allocation failed");
    if (hipHostGetDevicePointer((void**)&hd_ring, h_ring, 0) != hipSuccess || !hd_ring)
        return fail(SNL_EDEVICE, "no device address for the pinned step ring");
    memset(h_ring, 0, kSpecRing * sizeof(SpecOut));
    // zero everything a pass may read before writing (the reference's buffers start zeroed)
    if (hipMemsetAsync(x, 0, sizeof(float) * M * 2 * h, stream) != hipSuccess ||
        hipMemsetAsync(mx, 0, sizeof(float) * M * 2 * h, stream) != hipSuccess ||
        hipMemsetAsync(hid, 0, sizeof(float) * kHidRows * h, stream) != hipSuccess ||
        hipMemsetAsync(hlast, 0, sizeof(float) * h, stream) != hipSuccess ||
        hipMemsetAsync(lin_state, 0, sizeof(float) * 3 * nl * state_floats, stream) != hipSuccess ||
        hipMemsetAsync(conv_state, 0, sizeof(float) * 3 * nl * conv_floats, stream) != hipSuccess ||
        hipMemsetAsync(kcache, 0, 2 * kvn * std::max(n_full, 1), stream) != hipSuccess ||
        hipMemsetAsync(vcache, 0, 2 * kvn * std::max(n_full, 1), stream) != hipSuccess ||
        hipMemsetAsync(m_kc, 0, 2 * (c.has_mtp ? kvn : 1), stream) != hipSuccess ||
        hipMemsetAsync(m_vc, 0, 2 * (c.has_mtp ? kvn : 1), stream) != hipSuccess)
        return fail(SNL_EDEVICE, "hipMemset failed");
    if (hipStreamSynchronize(stream) != hipSuccess) return fail(SNL_EDEVICE, "weight initialisation failed");
    return SNL_OK;
}

// One decoder pass over the execution plan (src/engine.rs:389-493), M token rows, then the
// final norm into hid rows 1..M and `rows` rows of LM head + greedy pick.
int snl_engine::record_forward(int M, int rows, int ckpt) {
    // the checkpoint request itself travels in the step record
    const snl_config& c = cfg;
    int rc = 0;
    // the same launch copies hlast into hid row 0 (the hidden of the token before this step)
    if (op("embed", 0.0))
        rc |= launch_embed(d_step, (const int8_t*)embed.q, embed.s, c.vocab, h, x, M, stream, hlast, hid, d_mpick);
    int fslot = 0, lslot = 0;
    const size_t kvn = (size_t)ctx * kv_dim;
    const size_t nl = std::max(n_lin, 1);
    part_n = 0;
    for (size_t vi = 0; vi < plan.size(); ++vi) {
        const int li = plan[vi];
        const Layer& L = layers[li];
        const bool mhc = is_mhc(li);
        const int ln = vi + 1 < plan.size() ? plan[vi + 1] : -1;  // layer of the next visit
        // An mHC site's router sums arrive as partials from the GEMV that produced the row (the
        // previous visit's down projection, or this visit's output projection); a site that no
        // GEMV precedes runs the stream copy (mode 3) and the router kernel instead.
        if (mhc && !part_n) {
            if (li == c.mhc_start && op("expand", 0.0)) rc |= launch_expand(x, h, M, stream);
            if (op("mhc", 0.0)) rc |= launch_mhc(x, L.mhc_attn.p, mhc_part, h, M, stream);
            part_n = 1;
        }
        // branch input: RMSNorm (1 + in_ln) of stream 0, or of the mHC pre-mix, fused into the GEMV
        const int pro = mhc ? GEMV_NORM_MHC : GEMV_NORM;
        consumed_n = mhc ? part_n : 0;
        const MhcRole site_attn{mhc ? L.mhc_attn.p : nullptr};
        // the output projection merges the attention site and leaves the FFN site's partials
        const MhcRole merge_attn{mhc ? L.mhc_attn.p : nullptr, mhc ? L.mhc_ffn.p : nullptr, 0};
        part_n = 0;
        if (L.full) {
            rc |= gemv("gemv_qkv", L.mix_in, x, 2 * h, proj, attn_proj_rows, M, GEMV_STORE, 0, pro, L.in_ln.p,
                       nullptr, site_attn);
            AttnArgs a = attn_args(d_step, kcache + kvn * fslot, vcache + kvn * fslot, L.small.p);
            if (op("attention", 0.0)) rc |= launch_attention(a, M, stream);
            rc |= gemv("gemv_o", L.mix_out, attn_out, q_dim, x, 2 * h, M, mhc ? GEMV_MHC : GEMV_ADD, 1, GEMV_PLAIN,
                       nullptr, nullptr, merge_attn);
            ++fslot;
        } else {
            rc |= gemv("gemv_in_proj", L.mix_in, x, 2 * h, proj, lin_proj_rows, M, GEMV_STORE, 0, pro, L.in_ln.p,
                       nullptr, site_attn);
            DeltaArgs d{};
            d.proj = proj;
            d.proj_stride = lin_proj_rows;
            d.lw = L.small.p;
            d.conv_state = conv_state + conv_floats * lslot;
            d.state = lin_state + state_floats * lslot;
            d.conv_slot = nl * conv_floats;
            d.state_slot = nl * state_floats;
            d.out = attn_out;
            d.ssq = dn_ssq;
            d.conv_dim = conv_dim;
            d.n_k = c.lin_k_heads;
            d.n_v = c.lin_v_heads;
            d.eps = c.eps;
            d.step = d_step;
            const double dn_bytes = 2.0 * 4.0 * (double)state_floats + (ckpt ? 4.0 * (double)state_floats : 0.0);
            if (op("deltanet", dn_bytes)) rc |= launch_deltanet(d, M, stream);
            // the gated head norm of the DeltaNet output is the prologue of the output projection
            rc |= gemv("gemv_out_proj", L.mix_out, attn_out, lin_value_dim, x, 2 * h, M, mhc ? GEMV_MHC : GEMV_ADD,
                       1, GEMV_GNORM, nullptr, nullptr, merge_attn);
            ++lslot;
        }
        consumed_n = mhc ? part_n : 0;
        rc |= gemv("gemv_gate_up", L.gate_up, x, 2 * h, act, c.intermediate, M, GEMV_SWIGLU, 0, pro, L.post_ln.p,
                   nullptr, MhcRole{mhc ? L.mhc_ffn.p : nullptr});
        // the down projection merges the FFN site and leaves the next visit's attention-site
        // partials: after a mode 1 merge into the mHC range, or with the stream copy (mode 3) when
        // the next visit starts the range
        const int mode = !mhc ? 0 : (li + 1 == c.mhc_end ? 2 : 1);
        const bool next_mhc = ln >= 0 && is_mhc(ln);
        const bool next_start = next_mhc && ln == c.mhc_start;
        const bool leave = next_start || (next_mhc && mhc && mode == 1);
        part_n = 0;
        rc |= gemv("gemv_down", L.down, act, c.intermediate, x, 2 * h, M, mhc ? GEMV_MHC : GEMV_ADD, mode,
                   GEMV_PLAIN, nullptr, nullptr,
                   MhcRole{mhc ? L.mhc_ffn.p : nullptr, leave ? layers[ln].mhc_attn.p : nullptr, next_start ? 1 : 0});
    }
    // the final norm into hid rows 1..M, the last row's output also into hlast (the hidden carried
    // to the next pass): with logits for every row, in the LM head's prologue (its block 0 stores
    // the normed rows), else on its own
    if (rows == M) {
        norm_out = hid + h;
        norm_last = hlast;
        rc |= gemv("gemv_lm_head", lm_head, x, 2 * h, logits, c.vocab, rows, GEMV_STORE, 0, GEMV_NORM, final_norm.p);
    } else {
        rc |= norm(x, 2 * h, nullptr, 0, final_norm.p, hid + h, 0, M, hlast);
        if (rows > 0)
            rc |= gemv("gemv_lm_head", lm_head, hid + (size_t)(M - rows + 1) * h, h, logits, c.vocab, rows, GEMV_STORE);
    }
    if (rows > 0 && op("pick", 0.0)) rc |= launch_pick(logits, c.vocab, rows, pick_scratch, d_picks, stream, hd_picks);
    mark("end", 0.0);
    return rc ? SNL_EDEVICE : SNL_OK;
}

// The MTP head (src/engine.rs:549-570, :736-761) over M pairs.
int snl_engine::record_mtp(int M, int draft) {
    const snl_config& c = cfg;
    int rc = 0;
    // x = fc_e(norm_e(emb)) + fc_h(norm_h(hid[r0..])): the embedding rows go to xn (fc_e writes mx),
    // and norm_e is fc_e's prologue
    if (op("embed", 0.0))
        rc |= launch_embed(d_mstep, (const int8_t*)embed.q, embed.s, c.vocab, h, xn, M, stream, nullptr, nullptr,
                           nullptr, true);
    rc |= gemv("gemv_fc_e", fc_e, xn, h, mx, 2 * h, M, GEMV_STORE, 0, GEMV_NORM, norm_e.p);
    rc |= gemv("gemv_fc_h", fc_h, hid, h, mx, 2 * h, M, GEMV_ADD, 0, GEMV_NORM, norm_h.p, &d_mstep->r0);
    rc |= gemv("gemv_mtp_qkv", m_qkv, mx, 2 * h, proj, attn_proj_rows, M, GEMV_STORE, 0, GEMV_NORM, m_in_ln.p);
    AttnArgs a = attn_args(d_mstep, m_kc, m_vc, m_qk_norm.p);
    if (op("attention", 0.0)) rc |= launch_attention(a, M, stream);
    rc |= gemv("gemv_mtp_o", m_o, attn_out, q_dim, mx, 2 * h, M, GEMV_ADD);
    rc |= gemv("gemv_mtp_gate_up", m_gate_up, mx, 2 * h, act, c.intermediate, M, GEMV_SWIGLU, 0, GEMV_NORM,
               m_post_ln.p);
    rc |= gemv("gemv_mtp_down", m_down, act, c.intermediate, mx, 2 * h, M, GEMV_ADD);
    if (draft) {
        // final norm of the draft's pair (the record's x_off: the last real one) fused into the LM head
        rc |= gemv("gemv_lm_head", lm_head, mx, 2 * h, m_logits, c.vocab, 1, GEMV_STORE, 0, GEMV_NORM, m_norm.p,
                   &d_mstep->x_off);
        if (op("pick", 0.0)) rc |= launch_pick(m_logits, c.vocab, 1, pick_scratch, d_mpick, stream, hd_picks + 2);
    }
    mark("end", 0.0);
    return rc ? SNL_EDEVICE : SNL_OK;
}

// One prefill pass of M token rows (up to SNL_PF_M) over the execution plan, the same op order as
// record_forward with the matrix products on the panel GEMM and the per-token work in prefill
// kernels: branch inputs become GEMM fragments (rows_to_frags), each mHC site computes its router
// sums and coefficients over all rows, and merges and SwiGLU run as their own launches.
int snl_engine::record_prefill(int M, int rows) {
    const snl_config& c = cfg;
    int rc = 0;
    const int X2 = 2 * h;
    if (op("embed", 0.0)) rc |= launch_embed_tokens(pf_tokens(), (const int8_t*)embed.q, embed.s, c.vocab, h, pf_x, M, stream);
    if (op("copy", 0.0)) rc |= launch_copy(hid, hlast, h, stream);  // row 0 = hidden of the token before
    int fslot = 0, lslot = 0;
    const size_t kvn = (size_t)ctx * kv_dim;
    const size_t nl = std::max(n_lin, 1);
    for (size_t vi = 0; vi < plan.size(); ++vi) {
        const int li = plan[vi];
        const Layer& L = layers[li];
        const bool mhc = is_mhc(li);
        if (mhc) {
            if (li == c.mhc_start && op("expand", 0.0)) rc |= launch_expand(pf_x, h, M, stream);
            rc |= pf_site(L.mhc_attn.p, M);
        }
        const int pro = mhc ? ROWS_NORM_MHC : ROWS_NORM;
        rc |= pf_mat(L.full ? "gemm_qkv" : "gemm_in_proj", L.mix_in, pf_x, X2, M, pro, L.in_ln.p, pf_proj,
                     L.mix_in.rows);
        if (L.full) {
            AttnArgs a = attn_args(nullptr, kcache + kvn * fslot, vcache + kvn * fslot, L.small.p);
            a.proj = pf_proj;
            a.qbuf = pf_qbuf;
            a.out = pf_attn;
            if (op("attention", 0.0)) rc |= launch_attention_prefill(a, d_pstep, M, pf_pos0 + M, pf_apart, pf_parts, stream);
            rc |= pf_mat("gemm_o", L.mix_out, pf_attn, q_dim, M, ROWS_PLAIN, nullptr, pf_br, h);
            ++fslot;
        } else {
            DnPrefillArgs d{};
            d.proj = pf_proj;
            d.proj_stride = lin_proj_rows;
            d.lw = L.small.p;
            d.conv_state = conv_state + ((size_t)cur * nl + lslot) * conv_floats;
            d.state = lin_state + ((size_t)cur * nl + lslot) * state_floats;
            d.q = pf_dq;
            d.k = pf_dk;
            d.v = pf_dv;
            d.gz = pf_gz;
            d.beta = pf_beta;
            d.decay = pf_decay;
            d.pairs = pf_pairs;
            d.out = pf_attn;
            d.ssq = pf_ssq;
            d.conv_dim = conv_dim;
            d.n_k = c.lin_k_heads;
            d.n_v = c.lin_v_heads;
            if (op("deltanet", 0.0)) rc |= launch_deltanet_prefill(d, M, stream);
            // the head factor of the gated norm is applied while the rows become fragments
            rc |= pf_mat("gemm_out_proj", L.mix_out, pf_attn, lin_value_dim, M, ROWS_GNORM, nullptr, pf_br, h);
            ++lslot;
        }
        if (op("merge", 0.0)) rc |= launch_merge(pf_x, pf_coef, pf_br, h, M, mhc ? 1 : 0, stream);
        if (mhc) rc |= pf_site(L.mhc_ffn.p, M);
        rc |= pf_mat("gemm_gate_up", L.gate_up, pf_x, X2, M, pro, L.post_ln.p, pf_proj, 2 * c.intermediate);
        if (op("swiglu", 0.0)) rc |= launch_swiglu(pf_proj, pf_act, c.intermediate, M, stream);
        rc |= pf_mat("gemm_down", L.down, pf_act, c.intermediate, M, ROWS_PLAIN, nullptr, pf_br, h);
        const int mode = !mhc ? 0 : (li + 1 == c.mhc_end ? 2 : 1);
        if (op("merge", 0.0)) rc |= launch_merge(pf_x, pf_coef, pf_br, h, M, mode, stream);
    }
    rc |= norm(pf_x, X2, nullptr, 0, final_norm.p, hid + h, 0, M);
    if (rows > 0) {
        rc |= gemv("gemv_lm_head", lm_head, hid + (size_t)(M - rows + 1) * h, h, logits, c.vocab, rows, GEMV_STORE);
        if (op("pick", 0.0)) rc |= launch_pick(logits, c.vocab, rows, pick_scratch, d_picks, stream, hd_picks);
    }
    if (op("copy", 0.0)) rc |= launch_copy(hlast, hid + (size_t)M * h, h, stream);
    mark("end", 0.0);
    return rc ? SNL_EDEVICE : SNL_OK;
}

// The MTP head over M pairs (hidden row r0 + i, token i) of a prompt chunk, as record_mtp without
// the draft (src/engine.rs:549-570, src/worker.rs:312-318).
int snl_engine::record_mtp_prefill(int M, int r0) {
    const snl_config& c = cfg;
    int rc = 0;
    const int X2 = 2 * h;
    if (op("embed", 0.0)) rc |= launch_embed_tokens(pf_tokens(), (const int8_t*)embed.q, embed.s, c.vocab, h, pf_x, M, stream);
    // x = fc_e(norm_e(emb)) + fc_h(norm_h(hid[r0..])): the fragments are taken before fc_e overwrites x
    rc |= pf_mat("gemm_fc_e", fc_e, pf_x, X2, M, ROWS_NORM, norm_e.p, pf_x, X2);
    rc |= pf_mat("gemm_fc_h", fc_h, hid + (size_t)r0 * h, h, M, ROWS_NORM, norm_h.p, pf_br, h);
    if (op("merge", 0.0)) rc |= launch_merge(pf_x, pf_coef, pf_br, h, M, 0, stream);
    rc |= pf_mat("gemm_mtp_qkv", m_qkv, pf_x, X2, M, ROWS_NORM, m_in_ln.p, pf_proj, attn_proj_rows);
    AttnArgs a = attn_args(nullptr, m_kc, m_vc, m_qk_norm.p);
    a.proj = pf_proj;
    a.qbuf = pf_qbuf;
    a.out = pf_attn;
    if (op("attention", 0.0)) rc |= launch_attention_prefill(a, d_pstep, M, pf_pos0 + M, pf_apart, pf_parts, stream);
    rc |= pf_mat("gemm_mtp_o", m_o, pf_attn, q_dim, M, ROWS_PLAIN, nullptr, pf_br, h);
    if (op("merge", 0.0)) rc |= launch_merge(pf_x, pf_coef, pf_br, h, M, 0, stream);
    rc |= pf_mat("gemm_mtp_gate_up", m_gate_up, pf_x, X2, M, ROWS_NORM, m_post_ln.p, pf_proj, 2 * c.intermediate);
    if (op("swiglu", 0.0)) rc |= launch_swiglu(pf_proj, pf_act, c.intermediate, M, stream);
    rc |= pf_mat("gemm_mtp_down", m_down, pf_act, c.intermediate, M, ROWS_PLAIN, nullptr, pf_br, h);
    if (op("merge", 0.0)) rc |= launch_merge(pf_x, pf_coef, pf_br, h, M, 0, stream);
    mark("end", 0.0);
    return rc ? SNL_EDEVICE : SNL_OK;
}

// Upload one prefill chunk's tokens and positions and run it (main model, or the MTP head over
// hidden rows r0..), waiting for it: the pinned record is reused by the next chunk.
int snl_engine::prefill_chunk(const uint32_t* tokens, const uint32_t* pos3, int m, int cache_pos0, int rows,
                              bool mtp, int r0) {
    PrefillDev& st = *h_pstep;
    st.pos0 = cache_pos0;
    pf_pos0 = cache_pos0;
    st.m = m;
    for (int i = 0; i < m; ++i) {
        st.tokens[i] = tokens[i];
        for (int k = 0; k < 3; ++k) st.rpos[i][k] = pos3 ? pos3[(size_t)i * 3 + k] : (uint32_t)(cache_pos0 + i);
        st.rpos[i][3] = 0;
    }
    if (hipMemcpyAsync(d_pstep, h_pstep, sizeof(PrefillDev), hipMemcpyHostToDevice, stream) != hipSuccess)
        return fail(SNL_EDEVICE, "prefill step upload failed");
    int rc = mtp ? record_mtp_prefill(m, r0) : record_prefill(m, rows);
    if (rc) return fail(SNL_EDEVICE, "prefill launch failed (M %d)", m);
    if (spec_prebuild > 0) {  // host work while the chunk runs
        const int keys = spec_prebuild;
        spec_prebuild = 0;
        // (on failure the first step builds them again and reports why)
        if (build_spec_pair(keys)) err.clear();
    }
    if (hipStreamSynchronize(stream) != hipSuccess) return fail(SNL_EDEVICE, "prefill failed on device");
    return SNL_OK;
}

// Replay (capturing on first use) the pass (kind, M, a, b): kind 0 forward (a = rows,
// b = ckpt), kind 1 MTP (a = draft).  The step record is copied first.
// Replays the captured pass of `kind` (0: forward of M rows, a logit rows, checkpoint b; 1: MTP
// head over M pairs, draft a; 2: a greedy speculative step, the MTP draft over M pairs then the
// checkpointed 2-row verify) after uploading its step records.
// Points the engine's launch stream at its capture stream for the life of a capture.
struct CaptureScope {
    hipStream_t& s;
    const hipStream_t keep;
    CaptureScope(hipStream_t& v, hipStream_t cap) : s(v), keep(v) { s = cap; }
    ~CaptureScope() { s = keep; }
};

int snl_engine::run(int kind, int M, int a, int b, int keys, bool upload) {
    const int first = kind == 1 ? 1 : 0, count = kind == 2 ? 2 : 1;
    if (upload &&
        hipMemcpyAsync(d_step + first, h_step + first, count * sizeof(StepDev), hipMemcpyHostToDevice, stream) !=
            hipSuccess)
        return fail(SNL_EDEVICE, "step upload failed");
    const int sp = span_for(keys);
    auto key = std::make_tuple(kind, M, a, b, sp);
    auto it = graphs.find(key);
    if (it == graphs.end() && kind == 2) {
        hipGraphExec_t ex = nullptr;
        if (int rc = build_spec(M, a, sp, &ex)) return rc;
        it = graphs.emplace(key, ex).first;
    }
    if (it == graphs.end()) {
        CaptureScope capture(stream, cap_stream);
        hipGraph_t g = nullptr;
        if (hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal) != hipSuccess)
            return fail(SNL_EDEVICE, "hipStreamBeginCapture failed");
        span = sp;
        int rc = kind == 0 ? record_forward(M, a, b) : record_mtp(M, a);
        span = 0;
        hipError_t ce = hipStreamEndCapture(stream, &g);
        if (rc || ce != hipSuccess) {
            if (g) hipGraphDestroy(g);
            return fail(SNL_EDEVICE, "pass capture failed (kind %d, M %d): %s", kind, M,
                        rc ? (err.empty() ? "a launch failed" : err.c_str()) : hipGetErrorString(ce));
        }
        hipGraphExec_t ex = nullptr;
        hipError_t ie = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
        hipGraphDestroy(g);
        if (ie != hipSuccess) return fail(SNL_EDEVICE, "hipGraphInstantiate failed");
        it = graphs.emplace(key, ex).first;
    }
    if (hipGraphLaunch(it->second, stream) != hipSuccess) return fail(SNL_EDEVICE, "hipGraphLaunch failed");
    return SNL_OK;
}

// The rotary cos / sin of every text position (the three rotary components equal, as decode
// positions are), bitwise as step_rope forms them, for the records the speculative step's control
// kernel writes.  Built with the first speculative step graph, so engines that never draft hold
// none.
int snl_engine::ensure_rope_tab() {
    if (rope_tab) return SNL_OK;
    const int rows = ctx + 4, half = cfg.rot_dim / 2;
    std::vector<float> tab((size_t)rows * SNL_ROPE_MAX * 2, 0.0f);
    float inv_freq[SNL_ROPE_MAX];
    for (int f = 0; f < half && f < SNL_ROPE_MAX; ++f)
        inv_freq[f] = powf(cfg.rope_theta, -(float)(2 * f) / (float)cfg.rot_dim);
    for (int p = 0; p < rows; ++p)
        for (int f = 0; f < half && f < SNL_ROPE_MAX; ++f) {
            const float ang = (float)p * inv_freq[f];
            tab[((size_t)p * SNL_ROPE_MAX + f) * 2] = cosf(ang);
            tab[((size_t)p * SNL_ROPE_MAX + f) * 2 + 1] = sinf(ang);
        }
    float* d = nullptr;
    if (int rc = dalloc(&d, tab.size())) return rc;
    if (hipMemcpy(d, tab.data(), tab.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
        return fail(SNL_EDEVICE, "rotary table upload failed");  // (d stays in allocs, freed with the engine)
    rope_tab = d;
    rope_rows = rows;
    return SNL_OK;
}

// Both instances of the speculative step graph (steps alternate between them).
int snl_engine::build_spec_pair(int keys) {
    const int sp = span_for(keys);
    for (int parity = 0; parity < 2; ++parity) {
        const auto key = std::make_tuple(2, kMaxM, parity, 0, sp);
        if (graphs.count(key)) continue;
        hipGraphExec_t ex = nullptr;
        if (int rc = build_spec(kMaxM, parity, sp, &ex)) return rc;
        graphs.emplace(key, ex);
    }
    return SNL_OK;
}

// The two passes are captured on their own, then joined in a parent graph between event record
// nodes (an event recorded inside a stream capture was refused here).
int snl_engine::build_spec(int M, int parity, int sp, hipGraphExec_t* out) {
    if (int rc = ensure_rope_tab()) return rc;
    for (auto& evs : spec_ev)  // (the graphs' event nodes record these)
        for (hipEvent_t& ev : evs)
            if (!ev && hipEventCreate(&ev) != hipSuccess) return fail(SNL_EDEVICE, "event creation failed");
    struct SpanScope {  // the span of this capture, cleared on every return
        int& s;
        SpanScope(int& v, int x) : s(v) { s = x; }
        ~SpanScope() { s = 0; }
    } scope(span, sp);
    CaptureScope on_cap(stream, cap_stream);
    hipGraph_t ga = nullptr, gb = nullptr, pg = nullptr;
    auto capture = [&](hipGraph_t* g, bool draft) -> int {
        if (const hipError_t be = hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal); be != hipSuccess) {
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            hipStreamIsCapturing(stream, &cs);
            return fail(SNL_EDEVICE, "hipStreamBeginCapture failed (%s pass): %s, capture status %d",
                        draft ? "draft" : "verify", hipGetErrorString(be), (int)cs);
        }
        int rc = draft ? record_mtp(M, 1) : record_forward(2, 2, 1);
        if (!rc && !draft) {
            SpecArgs sa{};
            sa.vstep = d_step;
            sa.mstep = d_mstep;
            sa.picks = d_picks;
            sa.draft = d_mpick;
            sa.rope_tab = rope_tab;
            sa.rope_rows = rope_rows;
            sa.hid1 = hid + h;
            sa.hlast = hlast;
            sa.h = h;
            sa.ring = hd_ring;
            sa.ring_n = kSpecRing;
            rc = launch_spec_next(sa, stream);
        }
        const hipError_t ce = hipStreamEndCapture(stream, g);
        if (rc || ce != hipSuccess)
            return fail(SNL_EDEVICE, "speculative step capture failed (%s pass): %s", draft ? "draft" : "verify",
                        rc ? "a launch failed" : hipGetErrorString(ce));
        return SNL_OK;
    };
    int rc = capture(&ga, true);
    if (!rc) rc = capture(&gb, false);
    hipGraphNode_t n0, na, n1, nb, n2;
    const char* what = nullptr;
    if (!rc) {
        if (hipGraphCreate(&pg, 0) != hipSuccess) what = "hipGraphCreate";
        else if (hipGraphAddEventRecordNode(&n0, pg, nullptr, 0, spec_ev[parity][0]) != hipSuccess) what = "event node";
        else if (hipGraphAddChildGraphNode(&na, pg, &n0, 1, ga) != hipSuccess) what = "draft node";
        else if (hipGraphAddEventRecordNode(&n1, pg, &na, 1, spec_ev[parity][1]) != hipSuccess) what = "event node";
        else if (hipGraphAddChildGraphNode(&nb, pg, &n1, 1, gb) != hipSuccess) what = "verify node";
        else if (hipGraphAddEventRecordNode(&n2, pg, &nb, 1, spec_ev[parity][2]) != hipSuccess) what = "event node";
        else if (hipGraphInstantiate(out, pg, nullptr, nullptr, 0) != hipSuccess) what = "hipGraphInstantiate";
        if (what) rc = fail(SNL_EDEVICE, "speculative step graph: %s failed", what);
    }
    if (pg) hipGraphDestroy(pg);
    if (gb) hipGraphDestroy(gb);
    if (ga) hipGraphDestroy(ga);
    return rc;
}

extern "C" {

const char* snl_create_error(void) { return g_create_error.c_str(); }

int snl_engine_create(const snl_config* cfg, uint64_t seed, int quant, int ctx, snl_engine** out) {
    if (!out) return SNL_EARG;
    *out = nullptr;
    if (!cfg) {
        g_create_error = "null config";
        return SNL_EARG;
    }
    if (const char* why = validate(cfg)) {
        g_create_error = std::string("unsupported model configuration: ") + why;
        return SNL_EARG;
    }
    if ((quant != 0 && quant != 1) || ctx < 2) {
        g_create_error = "bad quant or ctx";
        return SNL_EARG;
    }
    if (ctx > kMaxCtx) {
        g_create_error = "ctx " + std::to_string(ctx) + " exceeds the largest supported context (" +
                         std::to_string(kMaxCtx) + " positions)";
        return SNL_ECTX;
    }
    snl_engine* e = new snl_engine();
    e->cfg = *cfg;
    e->ctx = ctx;
    e->quant = quant;
    e->seed = seed;
    int rc = e->init();
    if (rc) {
        g_create_error = e->err;
        snl_engine_destroy(e);
        return rc;
    }
    *out = e;
    return SNL_OK;
}

// Engine::load (src/engine.rs:230-644) from the reference's weight files: `path` the text model,
// `mtp_path` (nullable) the MTP head.  ctx is clamped to the model's max_position as the
// reference does.
int snl_engine_load(const char* path, const char* mtp_path, int ctx, snl_engine** out) {
    if (!out) return SNL_EARG;
    *out = nullptr;
    if (!path) {
        g_create_error = "null path";
        return SNL_EARG;
    }
    SnlFile main_file, mtp_file;
    FileConfig fc;
    std::string err;
    if (!main_file.open(path, &err) || !main_file.config(&fc, &err) || (mtp_path && !mtp_file.open(mtp_path, &err))) {
        g_create_error = err;
        return SNL_EARG;
    }
    snl_config cfg = fc.cfg;
    cfg.has_mtp = mtp_path ? 1 : 0;
    if (const char* why = validate(&cfg)) {
        g_create_error = std::string("unsupported model configuration: ") + why;
        return SNL_EARG;
    }
    const std::string& q = main_file.quant();
    if (q != "q8_0" && q != "q4_0") {
        g_create_error = "unknown quantization `" + q + "`";
        return SNL_EARG;
    }
    if (fc.max_position < ctx) ctx = (int)fc.max_position;
    if (ctx < 2) {
        g_create_error = "bad ctx";
        return SNL_EARG;
    }
    if (ctx > kMaxCtx) {
        g_create_error = "ctx " + std::to_string(ctx) + " exceeds the largest supported context (" +
                         std::to_string(kMaxCtx) + " positions)";
        return SNL_ECTX;
    }
    snl_engine* e = new snl_engine();
    e->cfg = cfg;
    e->ctx = ctx;
    e->quant = q == "q4_0" ? 1 : 0;
    e->max_position = fc.max_position;
    e->src = &main_file;
    e->msrc = mtp_path ? &mtp_file : nullptr;
    int rc = e->init();
    // every upload from the mapped files has finished before they are unmapped
    if (e->stream && hipStreamSynchronize(e->stream) != hipSuccess && !rc) rc = e->fail(SNL_EDEVICE, "weight upload failed");
    e->src = e->msrc = nullptr;
    if (rc) {
        g_create_error = e->err;
        snl_engine_destroy(e);
        return rc;
    }
    *out = e;
    return SNL_OK;
}

namespace {

// The tensors of one file in the converter's order (src/convert.rs:203-311, plan_mtp and plan).
std::vector<std::pair<int, int>> file_tensors(const snl_config& c, bool mtp) {
    std::vector<std::pair<int, int>> t;
    if (mtp) {
        const int L = kMtpLayer;
        for (int k : {K_FC_E, K_FC_H, K_NORM_E, K_NORM_H, K_MTP_NORM, K_IN_LN, K_POST_LN, K_QK_NORM, K_QKV, K_O_PROJ,
                      K_GATE_UP, K_DOWN})
            t.emplace_back(L, k);
        return t;
    }
    t.emplace_back(-1, K_EMBED);
    t.emplace_back(-1, K_LM_HEAD);
    t.emplace_back(-1, K_NORM);
    for (int i = 0; i < c.n_layers; ++i) {
        t.emplace_back(i, K_IN_LN);
        t.emplace_back(i, K_POST_LN);
        t.emplace_back(i, c.full_attention[i] ? K_QK_NORM : K_LIN);
        if (c.mhc_streams > 0 && c.mhc_start <= i && i < c.mhc_end) {
            t.emplace_back(i, K_MHC_ATTN);
            t.emplace_back(i, K_MHC_FFN);
        }
    }
    for (int i = 0; i < c.n_layers; ++i) {
        if (c.full_attention[i]) {
            t.emplace_back(i, K_QKV);
            t.emplace_back(i, K_O_PROJ);
        } else {
            t.emplace_back(i, K_IN_PROJ);
            t.emplace_back(i, K_OUT_PROJ);
        }
        t.emplace_back(i, K_GATE_UP);
        t.emplace_back(i, K_DOWN);
    }
    return t;
}

int save_file(snl_engine* e, const char* path, bool mtp, const char* model_name) {
    const auto list = file_tensors(e->cfg, mtp);
    std::vector<WriteTensor> wt;
    for (const auto& lk : list) {
        int rows = 0, cols = 0;
        const int type = snl_tensor_info(e, lk.first, lk.second, &rows, &cols);
        if (type < 0) return e->fail(SNL_EDEVICE, "tensor `%s` is missing", tensor_name(lk.first, lk.second).c_str());
        WriteTensor w;
        w.name = tensor_name(lk.first, lk.second);
        w.dtype = type == 2 ? FD_F32 : type == 0 ? FD_Q8_0 : FD_Q4_0;
        if (type == 2) w.shape = {cols};
        else w.shape = {rows, cols};
        wt.push_back(w);
    }
    FileConfig fc;
    fc.cfg = e->cfg;
    fc.max_position = e->max_position;
    SnlWriter wr;
    std::vector<FileTensor> placed;
    std::string err;
    // the MTP file is always 8-bit (src/convert.rs:326)
    const std::string quant = mtp || e->quant == 0 ? "q8_0" : "q4_0";
    if (!wr.begin(path, model_name ? model_name : "", quant, fc, wt, &placed, &err)) return e->fail(SNL_EARG, "%s", err.c_str());
    std::vector<uint8_t> q;
    std::vector<float> sc;
    for (size_t i = 0; i < list.size(); ++i) {
        const FileTensor& ft = placed[i];
        q.resize(ft.quant_bytes());
        sc.resize(ft.scale_bytes() / 4);
        const int rc = snl_tensor_read(e, list[i].first, list[i].second, q.data(), sc.empty() ? nullptr : sc.data());
        if (rc) return rc;
        if (!wr.write_region(ft.offset, q.data(), q.size(), &err) ||
            (!sc.empty() && !wr.write_region(ft.scales_offset, sc.data(), sc.size() * 4, &err)))
            return e->fail(SNL_EARG, "%s", err.c_str());
    }
    if (!wr.finish(&err)) return e->fail(SNL_EARG, "%s", err.c_str());
    return SNL_OK;
}

}  // namespace

// The model configuration of an engine (a loaded engine's comes from its weight file).
int snl_engine_config(const snl_engine* e, snl_config* out) {
    if (!e || !out) return SNL_EARG;
    *out = e->cfg;
    return SNL_OK;
}

// The converter's output (src/convert.rs:316-427) for the engine's weights: the text model to
// `path` and, when mtp_path is given, the MTP head to mtp_path.
int snl_engine_save(snl_engine* e, const char* path, const char* mtp_path, const char* model_name) {
    if (!e || !path) return SNL_EARG;
    e->err.clear();
    if (mtp_path && !e->cfg.has_mtp) return e->fail(SNL_EARG, "the engine has no MTP head");
    int rc = save_file(e, path, false, model_name);
    if (!rc && mtp_path) rc = save_file(e, mtp_path, true, model_name);
    return rc;
}

void snl_engine_destroy(snl_engine* e) {
    if (!e) return;
    if (e->stream) hipStreamSynchronize(e->stream);
    for (auto& kv : e->graphs) hipGraphExecDestroy(kv.second);
    e->free_gen_tmp();
    for (void* p : e->allocs) hipFree(p);
    for (auto& evs : e->spec_ev)
        for (hipEvent_t ev : evs)
            if (ev) hipEventDestroy(ev);
    if (e->h_ring) hipHostFree(e->h_ring);
    if (e->h_picks) hipHostFree(e->h_picks);
    if (e->h_step) hipHostFree(e->h_step);
    if (e->h_pstep) hipHostFree(e->h_pstep);
    if (e->topk_host) hipHostFree(e->topk_host);
    if (e->stream) hipStreamDestroy(e->stream);
    if (e->cap_stream) hipStreamDestroy(e->cap_stream);
    delete e;
}

const char* snl_last_error(const snl_engine* e) { return e ? e->err.c_str() : ""; }

int snl_pos(const snl_engine* e) { return e->pos; }
int snl_ctx(const snl_engine* e) { return e->ctx; }
int snl_hid_rows(const snl_engine* e) { return e->hid_rows; }
int snl_has_mtp(const snl_engine* e) { return e->cfg.has_mtp != 0; }
int snl_prefill_chunk(const snl_engine* e) {
    (void)e;
    return SNL_PF_M;
}

int snl_forward(snl_engine* e, const uint32_t* tokens, int n, const uint32_t* pos3, int logit_rows, int ckpt,
                float* logits_out, snl_pick* picks_out) {
    if (!e) return SNL_EARG;
    ++e->epoch;
    e->err.clear();
    // src/engine.rs:810-821
    if (logit_rows < 0 || logit_rows > kLogitRows || (ckpt && n != 2))
        return e->fail(SNL_EARG, "forward: unsupported logits or checkpoint request");
    if (n <= 0 || !tokens) return e->fail(SNL_EARG, "forward called with no tokens");
    if (e->pos + n > e->ctx) return e->fail(SNL_ECTX, "context length exceeded (%d > %d)", e->pos + n, e->ctx);
    for (int i = 0; i < n; ++i)
        if (tokens[i] >= (uint32_t)e->cfg.vocab) return e->fail(SNL_ETOKEN, "token id %u out of range", tokens[i]);
    int rows = 0;
    if (n > kMaxM) {
        // chunked prefill: passes of up to SNL_PF_M rows (the reference's MAX_M, src/engine.rs:18);
        // the last holds the logit rows
        int last = n % SNL_PF_M ? n % SNL_PF_M : SNL_PF_M;
        if (last < logit_rows) last = logit_rows;
        for (int c0 = 0; c0 < n;) {
            const int rem = n - c0;
            const int m = rem == last ? last : std::min(SNL_PF_M, rem - last);
            rows = c0 + m == n ? std::min(logit_rows, m) : 0;
            int rc = e->prefill_chunk(tokens + c0, pos3 ? pos3 + (size_t)c0 * 3 : nullptr, m, e->pos, rows, false, 0);
            if (rc) return rc;
            e->ck_slot = -1;
            e->pos += m;
            e->hid_rows = m;
            c0 += m;
        }
    } else {
        // one captured decode pass of n <= kMaxM rows
        rows = std::min(logit_rows, n);
        StepDev& st = e->h_step[0];
        memset(&st, 0, sizeof st);
        st.pos0 = e->pos;
        st.m = n;
        st.ckpt = ckpt ? 1 : 0;
        st.s_in = e->cur;
        st.s_ck = (e->cur + 1) % 3;
        st.s_out = ckpt ? (e->cur + 2) % 3 : (e->cur + 1) % 3;
        for (int i = 0; i < n; ++i) {
            st.tokens[i] = tokens[i];
            for (int k = 0; k < 3; ++k) st.rpos[i][k] = pos3 ? pos3[i * 3 + k] : (uint32_t)(e->pos + i);
            st.rpos[i][3] = 0;
        }
        step_rope(st, n, e->cfg.rope_theta, e->cfg.rot_dim, e->cfg.mrope_section);
        int rc = e->run(0, n, rows, ckpt ? 1 : 0, e->pos + n);
        if (rc) return rc;
        // the step record is reused by the next call: wait for this one
        if (hipStreamSynchronize(e->stream) != hipSuccess) return e->fail(SNL_EDEVICE, "forward failed on device");
        e->ck_slot = ckpt ? st.s_ck : -1;
        e->cur = st.s_out;
        e->pos += n;
        e->hid_rows = n;
    }
    e->logit_rows = rows;
    if (rows > 0) {
        if (logits_out &&
            hipMemcpy(logits_out, e->logits, sizeof(float) * rows * e->cfg.vocab, hipMemcpyDeviceToHost) != hipSuccess)
            return e->fail(SNL_EDEVICE, "logits readback failed");
        // the pick kernel also wrote them to pinned host memory, complete once the stream synchronised
        if (picks_out) memcpy(picks_out, e->h_picks, sizeof(snl_pick) * rows);
    }
    return SNL_OK;
}

int snl_forward_profiled(snl_engine* e, const uint32_t* tokens, int n, const uint32_t* pos3, int logit_rows,
                         int ckpt, snl_op_time* recs, int max_recs, int* n_recs) {
    if (!e || !recs || !n_recs) return SNL_EARG;
    e->err.clear();
    ++e->epoch;
    *n_recs = 0;
    if (logit_rows < 0 || logit_rows > kLogitRows || (ckpt && n != 2) || n <= 0 || n > kMaxM || !tokens)
        return e->fail(SNL_EARG, "forward_profiled: one pass of 1..%d tokens", kMaxM);
    if (e->pos + n > e->ctx) return e->fail(SNL_ECTX, "context length exceeded (%d > %d)", e->pos + n, e->ctx);
    for (int i = 0; i < n; ++i)
        if (tokens[i] >= (uint32_t)e->cfg.vocab) return e->fail(SNL_ETOKEN, "token id %u out of range", tokens[i]);
    const int rows = std::min(logit_rows, n);
    StepDev& st = e->h_step[0];
    memset(&st, 0, sizeof st);
    st.pos0 = e->pos;
    st.m = n;
    st.ckpt = ckpt ? 1 : 0;
    st.s_in = e->cur;
    st.s_ck = (e->cur + 1) % 3;
    st.s_out = ckpt ? (e->cur + 2) % 3 : (e->cur + 1) % 3;
    for (int i = 0; i < n; ++i) {
        st.tokens[i] = tokens[i];
        for (int k = 0; k < 3; ++k) st.rpos[i][k] = pos3 ? pos3[i * 3 + k] : (uint32_t)(e->pos + i);
    }
    step_rope(st, n, e->cfg.rope_theta, e->cfg.rot_dim, e->cfg.mrope_section);
    if (hipMemcpyAsync(e->d_step, &st, sizeof(StepDev), hipMemcpyHostToDevice, e->stream) != hipSuccess)
        return e->fail(SNL_EDEVICE, "step upload failed");
    std::vector<snl_engine::Mark> marks;
    marks.reserve(2048);
    e->marks = &marks;
    e->span = e->span_for(e->pos + n);
    int rc = e->record_forward(n, rows, ckpt ? 1 : 0);
    e->span = 0;
    e->marks = nullptr;
    hipError_t se = hipStreamSynchronize(e->stream);
    int k = 0;
    for (size_t i = 0; i + 1 < marks.size(); ++i) {
        if (k < max_recs) {
            float ms = 0.0f;
            hipEventElapsedTime(&ms, marks[i].ev, marks[i + 1].ev);
            snprintf(recs[k].name, sizeof recs[k].name, "%s", marks[i].name);
            recs[k].bytes = marks[i].bytes;
            recs[k].ms = ms;
            ++k;
        }
    }
    for (auto& m : marks) hipEventDestroy(m.ev);
    *n_recs = k;
    if (rc || se != hipSuccess) return e->fail(SNL_EDEVICE, "profiled pass failed");
    e->ck_slot = ckpt ? st.s_ck : -1;
    e->cur = st.s_out;
    e->pos += n;
    e->hid_rows = n;
    return SNL_OK;
}

int snl_time_op(snl_engine* e, const char* name, int reps, double* ms_per_launch, double* bytes_per_launch,
                int* launches_per_pass) {
    if (!e || !name || reps < 1 || !ms_per_launch) return SNL_EARG;
    e->err.clear();
    ++e->epoch;
    if (!strcmp(name, "copy") || !strcmp(name, "norm"))
        return e->fail(SNL_EARG, "time_op: '%s' writes the carried hidden row", name);
    if (e->pos + 2 > e->ctx) return e->fail(SNL_ECTX, "context length exceeded (%d > %d)", e->pos + 2, e->ctx);
    // the timed passes write both state slots other than `cur`, one of which holds a pending
    // checkpoint after a checkpointed verify
    if (e->ck_slot >= 0)
        return e->fail(SNL_ESTATE, "time_op: a checkpoint is pending (roll back or run another pass first)");
    // a verify pass (2 rows, checkpoint) at the current position; nothing is committed
    StepDev& st = e->h_step[0];
    memset(&st, 0, sizeof st);
    st.pos0 = e->pos;
    st.m = 2;
    st.ckpt = 1;
    st.s_in = e->cur;
    st.s_ck = (e->cur + 1) % 3;
    st.s_out = (e->cur + 2) % 3;
    for (int i = 0; i < 2; ++i)
        for (int k = 0; k < 3; ++k) st.rpos[i][k] = (uint32_t)(e->pos + i);
    step_rope(st, 2, e->cfg.rope_theta, e->cfg.rot_dim, e->cfg.mrope_section);
    if (hipMemcpyAsync(e->d_step, &st, sizeof(StepDev), hipMemcpyHostToDevice, e->stream) != hipSuccess)
        return e->fail(SNL_EDEVICE, "step upload failed");
    hipEvent_t t0 = nullptr, t1 = nullptr;
    if (hipEventCreate(&t0) != hipSuccess || hipEventCreate(&t1) != hipSuccess)
        return e->fail(SNL_EDEVICE, "event creation failed");
    e->only = name;
    e->only_launches = 0;
    e->only_bytes = 0.0;
    e->span = e->span_for(e->pos + 2);
    int rc = e->record_forward(2, 2, 1);  // warm-up pass
    const int per_pass = e->only_launches;
    const double bytes = per_pass ? e->only_bytes / per_pass : 0.0;
    hipEventRecord(t0, e->stream);
    for (int r = 0; r < reps && !rc; ++r) rc |= e->record_forward(2, 2, 1);
    hipEventRecord(t1, e->stream);
    e->only = nullptr;
    e->span = 0;
    float ms = 0.0f;
    const hipError_t se = hipEventSynchronize(t1);
    hipEventElapsedTime(&ms, t0, t1);
    hipEventDestroy(t0);
    hipEventDestroy(t1);
    if (rc || se != hipSuccess) return e->fail(SNL_EDEVICE, "time_op pass failed");
    if (!per_pass) return e->fail(SNL_EARG, "time_op: no op named '%s' in a verify pass", name);
    *ms_per_launch = (double)ms / ((double)reps * per_pass);
    if (bytes_per_launch) *bytes_per_launch = bytes;
    if (launches_per_pass) *launches_per_pass = per_pass;
    return SNL_OK;
}

int snl_mtp(snl_engine* e, int r0, const uint32_t* tokens, int n, const uint32_t* pos3, int slot0, int draft,
            uint32_t* draft_out, snl_pick* pick_out, float* logits_out) {
    if (!e) return SNL_EARG;
    e->err.clear();
    ++e->epoch;
    if (!e->cfg.has_mtp) return e->fail(SNL_ESTATE, "this model has no MTP head");
    if (n <= 0 || !tokens || !pos3 || r0 < 0 || r0 + n > e->hid_rows + 1 || slot0 < 0 || slot0 + n > e->ctx)
        return e->fail(SNL_EARG, "mtp: rows out of range");
    for (int i = 0; i < n; ++i)
        if (tokens[i] >= (uint32_t)e->cfg.vocab) return e->fail(SNL_ETOKEN, "token id %u out of range", tokens[i]);
    int c0 = 0;
    if (n > kMaxM) {
        // a prompt's catch-up (src/worker.rs:312-318): prefill passes of up to SNL_PF_M pairs; a
        // drafting call leaves its last pair to the captured one-row pass below
        const int np = draft ? n - 1 : n;
        while (c0 < np) {
            const int m = std::min(SNL_PF_M, np - c0);
            int rc = e->prefill_chunk(tokens + c0, pos3 + (size_t)c0 * 3, m, slot0 + c0, 0, true, r0 + c0);
            if (rc) return rc;
            c0 += m;
        }
    }
    for (; c0 < n; c0 += kMaxM) {
        const int m = std::min(kMaxM, n - c0);
        const bool last = c0 + m == n;
        StepDev& st = e->h_step[1];
        memset(&st, 0, sizeof st);
        st.pos0 = slot0 + c0;
        st.m = m;
        st.r0 = r0 + c0;
        st.x_off = m - 1;
        for (int i = 0; i < m; ++i) {
            st.tokens[i] = tokens[c0 + i];
            for (int k = 0; k < 3; ++k) st.rpos[i][k] = pos3[(c0 + i) * 3 + k];
        }
        step_rope(st, m, e->cfg.rope_theta, e->cfg.rot_dim, e->cfg.mrope_section);
        int rc = e->run(1, m, last && draft ? 1 : 0, 0, slot0 + c0 + m);
        if (rc) return rc;
        if (hipStreamSynchronize(e->stream) != hipSuccess) return e->fail(SNL_EDEVICE, "mtp failed on device");
    }
    if (draft) {
        // written to pinned host memory by the pick kernel of the synchronised pass
        if (draft_out) *draft_out = e->h_picks[2].token;
        if (pick_out) memcpy(pick_out, e->h_picks + 2, sizeof(snl_pick));
        if (logits_out &&
            hipMemcpy(logits_out, e->m_logits, sizeof(float) * e->cfg.vocab, hipMemcpyDeviceToHost) != hipSuccess)
            return e->fail(SNL_EDEVICE, "logits readback failed");
    }
    return SNL_OK;
}

int snl_rollback(snl_engine* e) {
    if (!e) return SNL_EARG;
    if (e->ck_slot < 0) return e->fail(SNL_ESTATE, "rollback without a checkpointed 2-token step");
    ++e->epoch;
    e->cur = e->ck_slot;
    e->ck_slot = -1;
    if (launch_copy(e->hlast, e->hid + e->h, e->h, e->stream) || hipStreamSynchronize(e->stream) != hipSuccess)
        return e->fail(SNL_EDEVICE, "rollback failed");
    e->pos -= 1;
    e->hid_rows = 1;
    return SNL_OK;
}

int snl_snapshot(snl_engine* e, int slot) {
    if (!e || slot < 0 || slot >= kSnapshots) return SNL_EARG;
    ++e->epoch;
    const size_t nl = std::max(e->n_lin, 1);
    const size_t sb = nl * e->state_floats * 4, cb = nl * e->conv_floats * 4;
    if (hipMemcpyAsync(e->snap_lin[slot], e->lin_state + (size_t)e->cur * nl * e->state_floats, sb,
                       hipMemcpyDeviceToDevice, e->stream) != hipSuccess ||
        hipMemcpyAsync(e->snap_conv[slot], e->conv_state + (size_t)e->cur * nl * e->conv_floats, cb,
                       hipMemcpyDeviceToDevice, e->stream) != hipSuccess ||
        hipMemcpyAsync(e->snap_h[slot], e->hlast, (size_t)e->h * 4, hipMemcpyDeviceToDevice, e->stream) !=
            hipSuccess ||
        hipStreamSynchronize(e->stream) != hipSuccess)
        return e->fail(SNL_EDEVICE, "snapshot failed");
    return SNL_OK;
}

int snl_restore(snl_engine* e, int slot, int pos) {
    if (!e || slot < 0 || slot >= kSnapshots || pos < 0 || pos > e->ctx) return SNL_EARG;
    ++e->epoch;
    const size_t nl = std::max(e->n_lin, 1);
    const size_t sb = nl * e->state_floats * 4, cb = nl * e->conv_floats * 4;
    if (hipMemcpyAsync(e->lin_state + (size_t)e->cur * nl * e->state_floats, e->snap_lin[slot], sb,
                       hipMemcpyDeviceToDevice, e->stream) != hipSuccess ||
        hipMemcpyAsync(e->conv_state + (size_t)e->cur * nl * e->conv_floats, e->snap_conv[slot], cb,
                       hipMemcpyDeviceToDevice, e->stream) != hipSuccess ||
        hipMemcpyAsync(e->hlast, e->snap_h[slot], (size_t)e->h * 4, hipMemcpyDeviceToDevice, e->stream) !=
            hipSuccess ||
        hipStreamSynchronize(e->stream) != hipSuccess)
        return e->fail(SNL_EDEVICE, "restore failed");
    e->pos = pos;
    e->hid_rows = 0;
    e->ck_slot = -1;
    return SNL_OK;
}

int snl_reset(snl_engine* e) {
    if (!e) return SNL_EARG;
    ++e->epoch;
    const size_t nl = std::max(e->n_lin, 1);
    if (hipMemsetAsync(e->lin_state + (size_t)e->cur * nl * e->state_floats, 0, nl * e->state_floats * 4,
                       e->stream) != hipSuccess ||
        hipMemsetAsync(e->conv_state + (size_t)e->cur * nl * e->conv_floats, 0, nl * e->conv_floats * 4,
                       e->stream) != hipSuccess ||
        hipStreamSynchronize(e->stream) != hipSuccess)
        return e->fail(SNL_EDEVICE, "reset failed");
    e->pos = 0;
    e->hid_rows = 0;
    e->ck_slot = -1;
    e->err.clear();
    return SNL_OK;
}

}  // extern "C"

namespace snl {

uint64_t engine_epoch(const snl_engine* e) { return e->epoch; }

int engine_fail(snl_engine* e, int code, const char* msg) { return e->fail(code, "%s", msg); }

int engine_vocab(const snl_engine* e) { return e->cfg.vocab; }

// Greedy speculative steps (src/worker.rs:197-255).  A step is the MTP draft (Engine::mtp with a
// draft, src/engine.rs:736-774) over one or two pairs from hidden row r0 at cache slot slot0, then
// the checkpointed 2-token verify of [tok, draft] (src/engine.rs:801-936), whose second token the
// embedding reads from the draft's pick on the device, then spec_next_kernel, which takes the accept
// decision, copies the rollback's carried row on a reject, posts the outcome to the pinned ring and
// writes both records of the next step.  The three replay as one graph (two instances, so that one
// step can be queued while the previous one runs).  The draft pass always has two rows: with one
// pair the second is a padding row at the next position, whose cache entry the next draft
// overwrites before any pass reads it; the draft comes from the record's row x_off.

// The records of a step from the host's decode state (draft pairs mtok / mpos, verify token tok
// at rotary positions pos3).
int spec_prepare(snl_engine* e, int r0, const uint32_t* mtok, int mn, const uint32_t* mpos, int slot0, uint32_t tok,
                 const uint32_t* pos3) {
    e->err.clear();
    if (!e->cfg.has_mtp) return e->fail(SNL_ESTATE, "this model has no MTP head");
    if (mn < 1 || mn > kMaxM || !mtok || !mpos || !pos3 || r0 < 0 || r0 + mn > e->hid_rows + 1 || slot0 < 0 ||
        slot0 + kMaxM > e->ctx)
        return e->fail(SNL_EARG, "mtp: rows out of range");
    // the draft pass reads kMaxM hidden rows from r0, padding included
    if (r0 + kMaxM > kHidRows) return e->fail(SNL_EARG, "mtp: hidden rows %d..%d past the buffer", r0, r0 + kMaxM - 1);
    for (int i = 0; i < mn; ++i)
        if (mtok[i] >= (uint32_t)e->cfg.vocab) return e->fail(SNL_ETOKEN, "token id %u out of range", mtok[i]);
    if (tok >= (uint32_t)e->cfg.vocab) return e->fail(SNL_ETOKEN, "token id %u out of range", tok);
    if (e->pos + 2 > e->ctx) return e->fail(SNL_ECTX, "context length exceeded (%d > %d)", e->pos + 2, e->ctx);
    StepDev& ms = e->h_step[1];
    memset(&ms, 0, sizeof ms);
    ms.pos0 = slot0;
    ms.m = kMaxM;
    ms.r0 = r0;
    ms.x_off = mn - 1;
    for (int i = 0; i < kMaxM; ++i) {
        ms.tokens[i] = mtok[i < mn ? i : 0];
        for (int k = 0; k < 3; ++k) ms.rpos[i][k] = i < mn ? mpos[i * 3 + k] : mpos[k] + (uint32_t)i;
    }
    step_rope(ms, kMaxM, e->cfg.rope_theta, e->cfg.rot_dim, e->cfg.mrope_section);
    StepDev& vs = e->h_step[0];
    memset(&vs, 0, sizeof vs);
    vs.pos0 = e->pos;
    vs.m = 2;
    vs.ckpt = 1;
    vs.s_in = e->cur;
    vs.s_ck = (e->cur + 1) % 3;
    vs.s_out = (e->cur + 2) % 3;
    vs.draft_rows = 2u;
    vs.seq = e->spec_seq;
    vs.tokens[0] = tok;
    for (int i = 0; i < 2; ++i)
        for (int k = 0; k < 3; ++k) vs.rpos[i][k] = pos3[i * 3 + k];
    step_rope(vs, 2, e->cfg.rope_theta, e->cfg.rot_dim, e->cfg.mrope_section);
    return SNL_OK;
}

// Queues step `seq` (instance seq & 1): with upload, from the records spec_prepare wrote; without,
// from the records the previous step's control kernel left on the device.
int spec_launch(snl_engine* e, bool upload) {
    const int parity = (int)(e->spec_seq & 1u);
    // Keys: step seq's verify reaches pos + 2 (host position) and a step queued ahead of it pos + 4;
    // both instances of that context bucket are built before the first launch, so queueing a step
    // ahead never captures.
    const int keys = e->pos + 4;
    if (int rc = e->build_spec_pair(keys)) return rc;
    if (int rc = e->run(2, kMaxM, parity, 0, keys, upload)) return rc;
    ++e->spec_seq;
    return SNL_OK;
}

// Waits for step seq and applies it to the engine's host state: the verify's slots and position,
// then the rollback on a reject (whose carried row the control kernel copied).
int spec_finish(snl_engine* e, uint32_t seq, SpecOut* out, float* draft_ms, float* verify_ms) {
    hipEvent_t* ev = e->spec_ev[seq & 1u];
    if (hipEventSynchronize(ev[2]) != hipSuccess) return e->fail(SNL_EDEVICE, "speculative step failed on device");
    const SpecOut o = e->h_ring[seq % kSpecRing];
    if (o.seq != seq) return e->fail(SNL_EDEVICE, "speculative step %u: outcome of step %u in the ring", seq, o.seq);
    if (o.flags & kSpecRopeRange)
        return e->fail(SNL_ECTX, "speculative step %u: rotary position past the context's table", seq);
    ++e->epoch;
    e->ck_slot = (e->cur + 1) % 3;
    e->cur = (e->cur + 2) % 3;
    e->pos += 2;
    e->hid_rows = 2;
    e->logit_rows = 2;
    if (!o.accepted) {
        e->cur = e->ck_slot;
        e->ck_slot = -1;
        e->pos -= 1;
        e->hid_rows = 1;
    }
    if (out) *out = o;
    // (timing is informative only: a failed query reports zero and clears the error state)
    float t0 = 0.0f, t1 = 0.0f;
    if (hipEventElapsedTime(&t0, ev[0], ev[1]) != hipSuccess || hipEventElapsedTime(&t1, ev[1], ev[2]) != hipSuccess) {
        (void)hipGetLastError();
        t0 = t1 = 0.0f;
    }
    if (draft_ms) *draft_ms = t0;
    if (verify_ms) *verify_ms = t1;
    return SNL_OK;
}

// One step from the host's decode state, waited for.
int engine_spec_step(snl_engine* e, int r0, const uint32_t* mtok, int mn, const uint32_t* mpos, int slot0,
                     uint32_t tok, const uint32_t* pos3, SpecOut* out, float* draft_ms, float* verify_ms) {
    if (int rc = spec_prepare(e, r0, mtok, mn, mpos, slot0, tok, pos3)) return rc;
    const uint32_t seq = e->spec_seq;
    if (int rc = spec_launch(e, true)) return rc;
    return spec_finish(e, seq, out, draft_ms, verify_ms);
}

// Steps queued ahead of the host: step seq + 1 from the device's records while step seq runs.
// Queues it when its verify stays inside the context whatever step seq decides.
int engine_spec_ahead(snl_engine* e, bool* queued) {
    *queued = false;
    if (e->pos + 4 > e->ctx) return SNL_OK;
    if (int rc = spec_launch(e, false)) return rc;
    *queued = true;
    return SNL_OK;
}

uint32_t engine_spec_seq(const snl_engine* e) { return e->spec_seq; }

// Asks the next prefill chunk to build the speculative step graphs for `keys` cache positions
// while its passes run (0 withdraws the request).
void engine_prebuild_spec(snl_engine* e, int keys) { e->spec_prebuild = keys > 0 ? keys : 0; }

// Penalties on logits row `row` of the last forward (in place, as the reference mutates its logits),
// then its k largest entries (value descending, index ascending on ties): k <= kDistMax on the
// device; otherwise (k == 0: the whole vocabulary) the row is read back and sorted here.
int engine_top(snl_engine* e, int row, const uint32_t* pen_tok, const uint32_t* pen_cnt, int n_pen, float rep,
               float presence, float frequency, int k, std::vector<uint32_t>* tok, std::vector<float>* val) {
    const int V = e->cfg.vocab;
    if (row < 0 || row >= e->logit_rows) return e->fail(SNL_ESTATE, "no logits row %d from the last forward", row);
    if (n_pen < 0 || n_pen > V) return e->fail(SNL_EARG, "penalty list longer than the vocabulary");
    float* lr = e->logits + (size_t)row * V;
    if (n_pen > 0) {
        if (hipMemcpyAsync(e->pen_dev, pen_tok, (size_t)n_pen * 4, hipMemcpyHostToDevice, e->stream) != hipSuccess ||
            hipMemcpyAsync(e->pen_dev + V, pen_cnt, (size_t)n_pen * 4, hipMemcpyHostToDevice, e->stream) != hipSuccess ||
            launch_penalties(lr, V, e->pen_dev, e->pen_dev + V, n_pen, rep, presence, frequency, e->stream))
            return e->fail(SNL_EDEVICE, "penalty launch failed");
    }
    if (k <= 0 || k > V) k = V;
    tok->resize(k);
    val->resize(k);
    if (k <= kDistMax) {
        unsigned long long* res = nullptr;
        if (launch_topk(lr, V, k, e->topk_keys, &res, e->stream) ||
            hipMemcpyAsync(e->topk_host, res, (size_t)k * 8, hipMemcpyDeviceToHost, e->stream) != hipSuccess ||
            hipStreamSynchronize(e->stream) != hipSuccess)
            return e->fail(SNL_EDEVICE, "top-k failed");
        for (int i = 0; i < k; ++i) {
            const unsigned long long key = e->topk_host[i];
            const uint32_t ob = (uint32_t)(key >> 32);
            const uint32_t bits = (ob & 0x80000000u) ? (ob & 0x7FFFFFFFu) : ~ob;
            (*tok)[i] = 0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull);
            float v;
            memcpy(&v, &bits, 4);
            (*val)[i] = v;
        }
        return SNL_OK;
    }
    std::vector<float> host(V);
    if (hipMemcpyAsync(host.data(), lr, (size_t)V * 4, hipMemcpyDeviceToHost, e->stream) != hipSuccess ||
        hipStreamSynchronize(e->stream) != hipSuccess)
        return e->fail(SNL_EDEVICE, "logits readback failed");
    std::vector<uint32_t> idx(V);
    for (int i = 0; i < V; ++i) idx[i] = (uint32_t)i;
    std::sort(idx.begin(), idx.end(), [&](uint32_t a, uint32_t b) {
        return host[a] > host[b] || (host[a] == host[b] && a < b);
    });
    for (int i = 0; i < k; ++i) {
        (*tok)[i] = idx[i];
        (*val)[i] = host[idx[i]];
    }
    return SNL_OK;
}

}  // namespace snl

extern "C" {

// ---- inspection ----
static const void* find_tensor(const snl_engine* e, int layer, int kind, int* type, int* rows, int* cols,
                               const float** scales, const QW** qw = nullptr) {
    const QW* w = nullptr;
    const Vec* v = nullptr;
    if (layer == -1) {
        if (kind == K_EMBED) w = &e->embed;
        if (kind == K_LM_HEAD) w = &e->lm_head;
        if (kind == K_NORM) v = &e->final_norm;
    } else if (layer == kMtpLayer) {
        if (!e->cfg.has_mtp) return nullptr;
        switch (kind) {
            case K_FC_E: w = &e->fc_e; break;
            case K_FC_H: w = &e->fc_h; break;
            case K_QKV: w = &e->m_qkv; break;
            case K_O_PROJ: w = &e->m_o; break;
            case K_GATE_UP: w = &e->m_gate_up; break;
            case K_DOWN: w = &e->m_down; break;
            case K_NORM_E: v = &e->norm_e; break;
            case K_NORM_H: v = &e->norm_h; break;
            case K_MTP_NORM: v = &e->m_norm; break;
            case K_IN_LN: v = &e->m_in_ln; break;
            case K_POST_LN: v = &e->m_post_ln; break;
            case K_QK_NORM: v = &e->m_qk_norm; break;
        }
    } else if (layer >= 0 && layer < e->cfg.n_layers) {
        const Layer& L = e->layers[layer];
        switch (kind) {
            case K_IN_LN: v = &L.in_ln; break;
            case K_POST_LN: v = &L.post_ln; break;
            case K_QK_NORM: if (L.full) v = &L.small; break;
            case K_LIN: if (!L.full) v = &L.small; break;
            case K_QKV: if (L.full) w = &L.mix_in; break;
            case K_O_PROJ: if (L.full) w = &L.mix_out; break;
            case K_IN_PROJ: if (!L.full) w = &L.mix_in; break;
            case K_OUT_PROJ: if (!L.full) w = &L.mix_out; break;
            case K_GATE_UP: w = &L.gate_up; break;
            case K_DOWN: w = &L.down; break;
            case K_MHC_ATTN: if (L.mhc_attn.p) v = &L.mhc_attn; break;
            case K_MHC_FFN: if (L.mhc_ffn.p) v = &L.mhc_ffn; break;
        }
    }
    if (w) {
        *type = w->quant;
        *rows = w->rows;
        *cols = w->cols;
        *scales = w->s;
        if (qw) *qw = w;
        return w->q;
    }
    if (v) {
        *type = 2;
        *rows = 1;
        *cols = v->n;
        *scales = nullptr;
        return v->p;
    }
    return nullptr;
}

int snl_tensor_info(const snl_engine* e, int layer, int kind, int* rows, int* cols) {
    int type = -1;
    const float* s;
    if (!e || !find_tensor(e, layer, kind, &type, rows, cols, &s)) return -1;
    return type;
}

int snl_tensor_read(snl_engine* e, int layer, int kind, void* q, float* s) {
    int type, rows, cols;
    const float* sp;
    const QW* w = nullptr;
    const void* qp = find_tensor(e, layer, kind, &type, &rows, &cols, &sp, &w);
    if (!qp || !q) return SNL_EARG;
    if (hipStreamSynchronize(e->stream) != hipSuccess) return SNL_EDEVICE;
    const size_t n = (size_t)rows * cols;
    if (w && w->packed) {  // tile order -> the reference's row-major quants and scales
        PackGeom g;
        if (!pack_geom(w->quant, rows, cols, w->inter, &g)) return SNL_EDEVICE;
        std::vector<uint8_t> hq(g.q_bytes);
        std::vector<float> hs(g.s_floats);
        if (hipMemcpy(hq.data(), qp, g.q_bytes, hipMemcpyDeviceToHost) != hipSuccess ||
            hipMemcpy(hs.data(), sp, g.s_floats * 4, hipMemcpyDeviceToHost) != hipSuccess)
            return SNL_EDEVICE;
        uint8_t* qo = static_cast<uint8_t*>(q);
        if (w->quant == 0)  // packed Q8 bytes carry the offset-binary flip of packing.h
            for (uint8_t& b : hq) b ^= 0x80u;
        for (int T = 0; T < g.tiles; ++T)
            for (int S = 0; S < g.nss; ++S)
                for (int lane = 0; lane < 64; ++lane) {
                    const int row = pack_row(g, T, lane & 15);
                    if (row < 0) continue;
                    for (int v = 0; v < g.NI; ++v)
                        std::memcpy(qo + (size_t)row * g.row_bytes + pack_row_offset(g, S, v, lane >> 4),
                                    hq.data() + pack_piece(g, T, S, v, lane), 16);
                    if (s)
                        for (int u = 0; u < g.U; ++u)
                            s[(size_t)row * (cols / 32) + 4 * g.U * S + g.U * (lane >> 4) + u] =
                                hs[pack_scale(g, T, S, lane, u)];
                }
        return SNL_OK;
    }
    const size_t qb = type == 0 ? n : (type == 1 ? n / 2 : n * 4);
    if (hipMemcpy(q, qp, qb, hipMemcpyDeviceToHost) != hipSuccess) return SNL_EDEVICE;
    if (type != 2 && s && hipMemcpy(s, sp, n / 32 * 4, hipMemcpyDeviceToHost) != hipSuccess) return SNL_EDEVICE;
    return SNL_OK;
}

int snl_tensor_zero_rows(snl_engine* e, int layer, int kind, int first) {
    if (!e) return SNL_EARG;
    e->err.clear();
    int type, rows, cols;
    const float* sp;
    const QW* cw = nullptr;
    const void* qp = find_tensor(e, layer, kind, &type, &rows, &cols, &sp, &cw);
    if (!qp || !cw || type == 2 || first < 0 || first > rows) return e->fail(SNL_EARG, "zero_rows: bad tensor or row");
    QW& w = const_cast<QW&>(*cw);
    ++e->epoch;
    if (hipStreamSynchronize(e->stream) != hipSuccess) return e->fail(SNL_EDEVICE, "zero_rows: device error");
    const size_t nb = (size_t)cols / 32;
    if (!w.packed) {  // row-major scales
        if (first < rows && hipMemset(w.s + (size_t)first * nb, 0, (size_t)(rows - first) * nb * 4) != hipSuccess)
            return e->fail(SNL_EDEVICE, "zero_rows: memset failed");
        return SNL_OK;
    }
    PackGeom g;
    if (!pack_geom(w.quant, rows, cols, w.inter, &g)) return e->fail(SNL_EDEVICE, "zero_rows: no tile order");
    std::vector<float> hs(g.s_floats);
    if (hipMemcpy(hs.data(), w.s, g.s_floats * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return e->fail(SNL_EDEVICE, "zero_rows: scale readback failed");
    for (int T = 0; T < g.tiles; ++T)
        for (int S = 0; S < g.nss; ++S)
            for (int lane = 0; lane < 64; ++lane) {
                const int row = pack_row(g, T, lane & 15);
                if (row >= first)
                    for (int u = 0; u < g.U; ++u) hs[pack_scale(g, T, S, lane, u)] = 0.0f;
            }
    if (hipMemcpy(w.s, hs.data(), g.s_floats * 4, hipMemcpyHostToDevice) != hipSuccess)
        return e->fail(SNL_EDEVICE, "zero_rows: scale upload failed");
    if (w.pq) {  // the prefill GEMM's panel copy, packed again from the reference layout
        const size_t n = (size_t)rows * cols, qn = w.quant == 0 ? n : n / 2;
        std::vector<uint8_t> hq(qn);
        std::vector<float> rs(n / 32);
        if (int rc = snl_tensor_read(e, layer, kind, hq.data(), rs.data())) return e->fail(rc, "zero_rows: readback failed");
        void* tq = nullptr;
        float* ts = nullptr;
        int rc = SNL_OK;
        if (hipMalloc(&tq, qn) != hipSuccess || hipMalloc((void**)&ts, n / 32 * 4) != hipSuccess)
            rc = e->fail(SNL_ENOMEM, "zero_rows: staging allocation failed");
        else if (hipMemcpy(tq, hq.data(), qn, hipMemcpyHostToDevice) != hipSuccess ||
                 hipMemcpy(ts, rs.data(), n / 32 * 4, hipMemcpyHostToDevice) != hipSuccess ||
                 launch_panel_pack(w.quant, rows, cols, tq, ts, w.pq, w.ps, e->stream) ||
                 hipStreamSynchronize(e->stream) != hipSuccess)
            rc = e->fail(SNL_EDEVICE, "zero_rows: panel repack failed");
        hipFree(tq);
        hipFree(ts);
        return rc;
    }
    return SNL_OK;
}

size_t snl_buffer_size(const snl_engine* e, int id) {
    const size_t nl = std::max(e->n_lin, 1);
    switch (id) {
        case 0: return (size_t)kMaxM * 2 * e->h * 4;
        case 1: return (size_t)(kMaxM + 1) * e->h * 4;
        case 2: return (size_t)e->h * 4;
        case 3: return nl * e->state_floats * 4;
        case 4: return nl * e->conv_floats * 4;
        case 5: return (size_t)kMaxM * 2 * e->h * 4;
    }
    return 0;
}

int snl_buffer_read(snl_engine* e, int id, void* out, size_t bytes) {
    if (!e || !out || bytes > snl_buffer_size(e, id)) return SNL_EARG;
    const size_t nl = std::max(e->n_lin, 1);
    const void* src = nullptr;
    switch (id) {
        case 0: src = e->x; break;
        case 1: src = e->hid; break;
        case 2: src = e->hlast; break;
        case 3: src = e->lin_state + (size_t)e->cur * nl * e->state_floats; break;
        case 4: src = e->conv_state + (size_t)e->cur * nl * e->conv_floats; break;
        case 5: src = e->mx; break;
        default: return SNL_EARG;
    }
    if (hipStreamSynchronize(e->stream) != hipSuccess || hipMemcpy(out, src, bytes, hipMemcpyDeviceToHost) != hipSuccess)
        return SNL_EDEVICE;
    return SNL_OK;
}

// ---- kernel-level entry points ----
static std::mutex g_kstep_mu;
static StepDev* g_kstep = nullptr;

static StepDev* kernel_step(const StepDev& h, hipStream_t s) {
    if (!g_kstep && hipMalloc((void**)&g_kstep, sizeof(StepDev)) != hipSuccess) return nullptr;
    if (hipMemcpyAsync(g_kstep, &h, sizeof(StepDev), hipMemcpyHostToDevice, s) != hipSuccess) return nullptr;
    if (hipStreamSynchronize(s) != hipSuccess) return nullptr;
    return g_kstep;
}

int snl_gemv(int quant, const void* wq, const float* ws, const float* x, float* y, int M, int N, int K, int x_stride,
             int y_stride, void* stream) {
    if ((quant != 0 && quant != 1) || !wq || !ws || !x || !y || x_stride % 4 || x_stride < K || y_stride < N)
        return SNL_EARG;
    static const int init_rc = gemv_init();
    if (init_rc) return SNL_EDEVICE;
    hipStream_t st = (hipStream_t)stream;
    GemvArgs g{};
    g.wq = wq;
    g.ws = ws;
    g.x = x;
    g.x_stride = x_stride;
    g.y = y;
    g.y_stride = y_stride;
    g.N = N;
    g.K = K;
    g.epi = GEMV_STORE;
    // The engine's kernel reads tile order: pack the caller's reference-layout matrix into a
    // staging buffer first (held under the lock until the call has finished on the stream).
    static uint8_t* pq = nullptr;
    static float* ps = nullptr;
    static size_t cap_q = 0, cap_s = 0;
    std::lock_guard<std::mutex> lk(g_kstep_mu);
    PackGeom pg;
    if (pack_geom(quant, N, K, 0, &pg) && M >= 1 && M <= SNL_MAX_M && mgemv_fits(M, K)) {
        if (pg.q_bytes > cap_q || pg.s_floats > cap_s) {
            if (hipStreamSynchronize(st) != hipSuccess) return SNL_EDEVICE;
            hipFree(pq);
            hipFree(ps);
            pq = nullptr;
            ps = nullptr;
            cap_q = cap_s = 0;
            if (hipMalloc((void**)&pq, pg.q_bytes) != hipSuccess || hipMalloc((void**)&ps, pg.s_floats * 4) != hipSuccess)
                return SNL_ENOMEM;
            cap_q = pg.q_bytes;
            cap_s = pg.s_floats;
        }
        if (launch_pack_matrix(pg, wq, ws, pq, ps, st)) return SNL_EDEVICE;
        g.packed = 1;
        g.wq = pq;
        g.ws = ps;
    }
    int rc = launch_gemv(g, quant, M, st);
    if (rc == 0 && g.packed && hipStreamSynchronize(st) != hipSuccess) rc = -2;
    return rc == -1 ? SNL_EARG : (rc ? SNL_EDEVICE : SNL_OK);
}

int snl_gemm(int quant, const void* wq, const float* ws, const float* x, float* y, int M, int N, int K, int x_stride,
             int y_stride, void* stream) {
    if ((quant != 0 && quant != 1) || !wq || !ws || !x || !y || K % 128 || K > 16384 || M < 1 || M > SNL_PREFILL_M || N < 1 ||
        x_stride < K || y_stride < N)
        return SNL_EARG;
    hipStream_t st = (hipStream_t)stream;
    // panel-order weights and the token fragments in staging buffers held under the lock until the
    // call has finished on the stream
    static uint8_t* pq = nullptr;
    static float *ps = nullptr, *xs = nullptr;
    static void* fr = nullptr;
    static size_t cap_q = 0, cap_s = 0, cap_f = 0;
    std::lock_guard<std::mutex> lk(g_kstep_mu);
    const size_t qb = gemm_q_bytes(quant, N, K), sf = gemm_s_floats(N, K), fb = frags_bytes(SNL_PREFILL_M, K);
    if (qb > cap_q || sf > cap_s || fb > cap_f) {
        if (hipStreamSynchronize(st) != hipSuccess) return SNL_EDEVICE;
        hipFree(pq);
        hipFree(ps);
        hipFree(fr);
        hipFree(xs);
        pq = nullptr;
        ps = xs = nullptr;
        fr = nullptr;
        cap_q = cap_s = cap_f = 0;
        if (hipMalloc((void**)&pq, qb) != hipSuccess || hipMalloc((void**)&ps, sf * 4) != hipSuccess ||
            hipMalloc(&fr, fb) != hipSuccess || hipMalloc((void**)&xs, SNL_PREFILL_M * 4) != hipSuccess)
            return SNL_ENOMEM;
        cap_q = qb;
        cap_s = sf;
        cap_f = fb;
    }
    if (launch_panel_pack(quant, N, K, wq, ws, pq, ps, st)) return SNL_EDEVICE;
    RowsArgs r{};
    r.x = x;
    r.x_stride = x_stride;
    r.M = M;
    r.K = K;
    r.mode = ROWS_PLAIN;
    r.perm4 = quant;
    r.frags = fr;
    r.xs = xs;
    if (launch_rows_to_frags(r, st)) return SNL_EDEVICE;
    GemmArgs g{};
    g.wq = pq;
    g.ws = ps;
    g.frags = fr;
    g.xs = xs;
    g.y = y;
    g.y_stride = y_stride;
    g.M = M;
    g.N = N;
    g.K = K;
    if (launch_mgemm(g, quant, st) || hipStreamSynchronize(st) != hipSuccess) return SNL_EDEVICE;
    return SNL_OK;
}

// The decode GEMV alone (measurement): `copies` distinct N x K matrices in tile order, together at
// least 1 GB so that the 256 MB Infinity Cache cannot serve a repeat, launched in turn `reps`
// times between two HIP events on a stream of its own.
int snl_gemv_time(int quant, int N, int K, int M, int reps, double* ms_per_launch, double* bytes_per_launch,
                  int* copies_out) {
    if ((quant != 0 && quant != 1) || K % 128 || M < 1 || M > SNL_MAX_M || N < 16 || reps < 1 || !ms_per_launch)
        return SNL_EARG;
    static const int init_rc = gemv_init();
    if (init_rc) return SNL_EDEVICE;
    PackGeom pg;
    if (!pack_geom(quant, N, K, 0, &pg) || !mgemv_fits(M, K)) return SNL_EARG;
    const size_t mat = pg.q_bytes + pg.s_floats * 4;
    const int copies = (int)std::max<size_t>(2, ((size_t)1 << 30) / mat + 1);
    hipStream_t st = nullptr;
    if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) return SNL_EDEVICE;
    const size_t n = (size_t)N * K;
    uint8_t *q = nullptr, *pq = nullptr;
    float *s = nullptr, *ps = nullptr, *x = nullptr, *y = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = SNL_OK;
    if (hipMalloc((void**)&q, quant == 0 ? n : n / 2) != hipSuccess || hipMalloc((void**)&s, n / 32 * 4) != hipSuccess ||
        hipMalloc((void**)&pq, pg.q_bytes * copies) != hipSuccess ||
        hipMalloc((void**)&ps, pg.s_floats * 4 * copies) != hipSuccess ||
        hipMalloc((void**)&x, (size_t)M * K * 4) != hipSuccess || hipMalloc((void**)&y, (size_t)M * N * 4) != hipSuccess ||
        hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
        rc = SNL_ENOMEM;
    } else {
        if (launch_gen_matrix(0x5EEDull, N, K, 0.02f, quant, q, s, st) ||
            launch_gen_vector(0x5EEEull, (int64_t)M * K, 0, 1.0f, 0, 0, x, st))
            rc = SNL_EDEVICE;
        for (int c = 0; !rc && c < copies; ++c)
            if (launch_pack_matrix(pg, q, s, pq + pg.q_bytes * c, ps + pg.s_floats * c, st)) rc = SNL_EDEVICE;
        GemvArgs g{};
        g.packed = 1;
        g.x = x;
        g.x_stride = K;
        g.y = y;
        g.y_stride = N;
        g.N = N;
        g.K = K;
        g.epi = GEMV_STORE;
        auto launch = [&](int i) {
            const int c = i % copies;
            g.wq = pq + pg.q_bytes * c;
            g.ws = ps + pg.s_floats * c;
            return launch_gemv(g, quant, M, st);
        };
        for (int i = 0; !rc && i < copies; ++i)  // warm-up: every copy once
            if (launch(i)) rc = SNL_EDEVICE;
        float ms = 0.0f;
        if (!rc && hipEventRecord(e0, st) != hipSuccess) rc = SNL_EDEVICE;
        for (int i = 0; !rc && i < reps; ++i)
            if (launch(i)) rc = SNL_EDEVICE;
        if (!rc && (hipEventRecord(e1, st) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                    hipEventElapsedTime(&ms, e0, e1) != hipSuccess))
            rc = SNL_EDEVICE;
        if (!rc) {
            *ms_per_launch = (double)ms / reps;
            // algorithmic bytes: quants + f32 block scales + the M input rows + the M output rows
            if (bytes_per_launch)
                *bytes_per_launch = (double)n * (quant == 0 ? 1.0 : 0.5) + (double)(n / 32) * 4 + (double)M * K * 4 +
                                    (double)M * N * 4;
            if (copies_out) *copies_out = copies;
        }
    }
    (void)hipStreamSynchronize(st);
    for (void* p : {(void*)q, (void*)s, (void*)pq, (void*)ps, (void*)x, (void*)y}) (void)hipFree(p);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipStreamDestroy(st);
    return rc;
}

int snl_gemm_time(int quant, int N, int K, int M, int reps, double* ms_per_launch) {
    if ((quant != 0 && quant != 1) || K % 128 || K > 16384 || M < 1 || M > SNL_PREFILL_M || N < 1 || reps < 1 ||
        !ms_per_launch)
        return SNL_EARG;
    hipStream_t st = nullptr;
    if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) return SNL_EDEVICE;
    const size_t n = (size_t)N * K;
    uint8_t *q = nullptr, *pq = nullptr;
    float *s = nullptr, *ps = nullptr, *x = nullptr, *y = nullptr, *xs = nullptr;
    void* fr = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = SNL_OK;
    if (hipMalloc((void**)&q, quant == 0 ? n : n / 2) != hipSuccess || hipMalloc((void**)&s, n / 32 * 4) != hipSuccess ||
        hipMalloc((void**)&pq, gemm_q_bytes(quant, N, K)) != hipSuccess ||
        hipMalloc((void**)&ps, gemm_s_floats(N, K) * 4) != hipSuccess ||
        hipMalloc((void**)&x, (size_t)M * K * 4) != hipSuccess || hipMalloc((void**)&y, (size_t)M * N * 4) != hipSuccess ||
        hipMalloc(&fr, frags_bytes(M, K)) != hipSuccess || hipMalloc((void**)&xs, (size_t)(M + 15) / 16 * 64) != hipSuccess ||
        hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
        rc = SNL_ENOMEM;
    } else {
        RowsArgs r{};
        r.x = x;
        r.x_stride = K;
        r.M = M;
        r.K = K;
        r.mode = ROWS_PLAIN;
        r.perm4 = quant;
        r.frags = fr;
        r.xs = xs;
        GemmArgs g{};
        g.wq = pq;
        g.ws = ps;
        g.frags = fr;
        g.xs = xs;
        g.y = y;
        g.y_stride = N;
        g.M = M;
        g.N = N;
        g.K = K;
        float ms = 0.0f;
        if (launch_gen_matrix(0x5EEDull, N, K, 0.02f, quant, q, s, st) ||
            launch_gen_vector(0x5EEEull, (int64_t)M * K, 0, 1.0f, 0, 0, x, st) ||
            launch_panel_pack(quant, N, K, q, s, pq, ps, st) || launch_rows_to_frags(r, st) ||
            launch_mgemm(g, quant, st) || hipEventRecord(e0, st) != hipSuccess)
            rc = SNL_EDEVICE;
        for (int i = 0; !rc && i < reps; ++i)
            if (launch_mgemm(g, quant, st)) rc = SNL_EDEVICE;
        if (!rc && (hipEventRecord(e1, st) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                    hipEventElapsedTime(&ms, e0, e1) != hipSuccess))
            rc = SNL_EDEVICE;
        if (!rc) *ms_per_launch = (double)ms / reps;
    }
    (void)hipStreamSynchronize(st);
    for (void* p : {(void*)q, (void*)s, (void*)pq, (void*)ps, (void*)x, (void*)y, fr, (void*)xs}) (void)hipFree(p);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipStreamDestroy(st);
    return rc;
}

int snl_deltanet(const float* proj, int proj_stride, const float* lw, float* conv_state, float* state, float* out,
                 int conv_dim, int n_k, int n_v, float eps, int M, int ckpt, int s_in, int s_out, int s_ck,
                 void* stream) {
    if (!proj || !lw || !conv_state || !state || !out || M < 1 || M > SNL_MAX_M || ckpt < 0 || ckpt > M)
        return SNL_EARG;
    if (s_in < 0 || s_in > 2 || s_out < 0 || s_out > 2 || s_ck < 0 || s_ck > 2 || s_out == s_in ||
        (ckpt && (s_ck == s_in || s_ck == s_out)))
        return SNL_EARG;
    if (n_k < 1 || n_v % n_k || conv_dim != 2 * n_k * 128 + n_v * 128) return SNL_EARG;
    std::lock_guard<std::mutex> lk(g_kstep_mu);
    StepDev h{};
    h.m = M;
    h.ckpt = ckpt;
    h.s_in = s_in;
    h.s_out = s_out;
    h.s_ck = s_ck;
    hipStream_t s = (hipStream_t)stream;
    StepDev* d = kernel_step(h, s);
    if (!d) return SNL_EDEVICE;
    DeltaArgs a{};
    a.proj = proj;
    a.proj_stride = proj_stride;
    a.lw = lw;
    a.conv_state = conv_state;
    a.state = state;
    a.conv_slot = (size_t)3 * conv_dim;
    a.state_slot = (size_t)n_v * 128 * 128;
    a.out = out;
    a.conv_dim = conv_dim;
    a.n_k = n_k;
    a.n_v = n_v;
    a.eps = eps;
    a.step = d;
    // the partial sums of squares between the step and the gated norm: kernel-level scratch
    static float* g_ssq = nullptr;
    static size_t g_ssq_n = 0;
    const size_t nss = (size_t)M * n_v * kDeltaGroups;
    if (nss > g_ssq_n) {
        hipFree(g_ssq);
        g_ssq = nullptr;
        g_ssq_n = 0;
        if (hipMalloc((void**)&g_ssq, nss * sizeof(float)) != hipSuccess) return SNL_ENOMEM;
        g_ssq_n = nss;
    }
    a.ssq = g_ssq;
    if (launch_deltanet(a, M, s) || launch_deltanet_norm(a, M, s)) return SNL_EDEVICE;
    return hipStreamSynchronize(s) == hipSuccess ? SNL_OK : SNL_EDEVICE;
}

int snl_attention(const float* proj, int proj_stride, float* qbuf, uint16_t* kcache, uint16_t* vcache,
                  const float* norms, float* out, float* partial, int n_heads, int n_kv, int rot_dim, float rope_theta,
                  float eps, const int32_t* mrope_section, int ctx, int M, int pos0, const uint32_t* rpos,
                  void* stream) {
    if (!proj || !qbuf || !kcache || !vcache || !norms || !out || !partial || !mrope_section || !rpos) return SNL_EARG;
    if (M < 1 || M > 2 || pos0 < 0 || pos0 + M > ctx || n_heads != 4 * n_kv || rot_dim < 2 || rot_dim % 2 ||
        rot_dim > 2 * SNL_ROPE_MAX)
        return SNL_EARG;
    std::lock_guard<std::mutex> lk(g_kstep_mu);
    StepDev h{};
    h.pos0 = pos0;
    h.m = M;
    for (int i = 0; i < M; ++i)
        for (int k = 0; k < 3; ++k) h.rpos[i][k] = rpos[i * 3 + k];
    step_rope(h, M, rope_theta, rot_dim, mrope_section);
    hipStream_t s = (hipStream_t)stream;
    StepDev* d = kernel_step(h, s);
    if (!d) return SNL_EDEVICE;
    AttnArgs a{};
    a.proj = proj;
    a.proj_stride = proj_stride;
    a.qbuf = qbuf;
    a.kcache = kcache;
    a.vcache = vcache;
    a.norms = norms;
    a.out = out;
    a.partial = partial;
    a.n_heads = n_heads;
    a.n_kv = n_kv;
    a.rot_dim = rot_dim;
    a.rope_theta = rope_theta;
    a.eps = eps;
    a.scale = 1.0f / 16.0f;
    a.mrope = ((uint32_t)(3 * mrope_section[1]) << 16) | (uint32_t)(3 * mrope_section[2]);
    a.ctx = ctx;
    a.step = d;
    int rc = launch_attention(a, M, s);
    if (rc) return rc == -1 ? SNL_EARG : SNL_EDEVICE;
    return hipStreamSynchronize(s) == hipSuccess ? SNL_OK : SNL_EDEVICE;
}

int snl_pick_rows(const float* logits, int V, int rows, snl_pick* picks_out, void* stream) {
    if (!logits || !picks_out || V < 1 || rows < 1 || rows > 64) return SNL_EARG;
    float* scratch = nullptr;
    if (hipMalloc((void**)&scratch, pick_scratch_floats(V, rows) * 4) != hipSuccess) return SNL_ENOMEM;
    hipStream_t s = (hipStream_t)stream;
    int rc = launch_pick(logits, V, rows, scratch, reinterpret_cast<Pick*>(picks_out), s);
    hipError_t se = hipStreamSynchronize(s);
    hipFree(scratch);
    return rc || se != hipSuccess ? SNL_EDEVICE : SNL_OK;
}

}  // extern "C"
