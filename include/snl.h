/*
 * snl.h -- C ABI of the MI355X-native MTP speculative decode step.
 *
 * The reference (dparnell/sense-nova-server, crate `sensenova-loop`) has no FFI: its
 * worker calls the Rust `Engine` directly.  The engine entry points below replace those
 * methods one for one, with the reference's argument meaning and error classes; each
 * cites the method it replaces.  All pointers are plain host pointers unless a comment
 * says "device"; no call keeps a pointer after it returns.  One engine handle is used by
 * one thread at a time (the reference's Engine is owned by a single generation thread,
 * src/worker.rs:76-105).  Every engine call has finished on the device when it returns.
 */
#ifndef SNL_H
#define SNL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  After any error other than SNL_EARG the caller resets the engine, as the
 * reference worker does after a failed request (src/worker.rs:94-101). */
enum {
    SNL_OK = 0,
    SNL_EARG = 1,     /* bad argument (src/engine.rs:810-818, :716-718) */
    SNL_ECTX = 2,     /* context length exceeded (src/engine.rs:819-821) */
    SNL_ETOKEN = 3,   /* token id out of range (src/engine.rs:784-786) */
    SNL_EDEVICE = 4,  /* HIP runtime error */
    SNL_ENOMEM = 5,   /* device allocation failed */
    SNL_ESTATE = 6    /* call not valid in the engine's state (e.g. rollback without a checkpoint) */
};

/* Model hyper-parameters: ModelConfig (src/config.rs:6-37).  mhc_streams = 0 means no mHC. */
typedef struct snl_config {
    int32_t hidden, intermediate, vocab, n_layers;
    int32_t n_heads, n_kv_heads, head_dim, rot_dim;
    float rope_theta, eps;
    int32_t mrope_section[3];
    int32_t lin_k_heads, lin_v_heads, lin_k_dim, lin_v_dim, conv_kernel;
    int32_t loop_start, loop_end, loop_count;
    int32_t mhc_start, mhc_end, mhc_streams, mhc_iterations;
    int32_t has_mtp;
    int32_t n_eos;
    uint32_t eos[4];
    uint8_t full_attention[64];
} snl_config;

/* Greedy pick of one logits row: first index of the maximum (src/sampler.rs:169-177),
 * the maximum and the second largest value (top1 - top2 is the argmax tie margin). */
typedef struct snl_pick {
    uint32_t token;
    float top1;
    float top2;
    uint32_t _pad;
} snl_pick;

typedef struct snl_engine snl_engine;

/* ---- lifecycle ------------------------------------------------------------------------ */

/* Engine::load (src/engine.rs:230-644) with weights drawn on the device from `seed`
 * (quant 0 = Q8_0, 1 = Q4_0 for the matrices a Q4_0 file quantises; embedding, LM head,
 * DeltaNet in_proj and the MTP head stay Q8_0 as in src/convert.rs:228-311).
 * ctx = KV positions per attention layer, 2..262144 (the reference's default max_position;
 * larger values return SNL_ECTX).  Returns SNL_OK and *out, or an error. */
int snl_engine_create(const snl_config* cfg, uint64_t seed, int quant, int ctx, snl_engine** out);
/* Engine::load (src/engine.rs:230-644) from the reference's `.snl` weight files
 * (src/weights.rs:1-121): `path` the text model, `mtp_path` (nullable) the MTP head, as written
 * by the converter (src/convert.rs:316-427).  Matrices keep each tensor's dtype (q8_0 / q4_0);
 * ctx is clamped to the model's max_position, and above 262144 returns SNL_ECTX.  The vision
 * tower is not loaded.  Errors (missing or misshapen tensors, bad header) return SNL_EARG with
 * the message in snl_create_error(). */
int snl_engine_load(const char* path, const char* mtp_path, int ctx, snl_engine** out);
/* The converter's output (src/convert.rs:316-427) for the engine's current weights: the text model
 * to `path` and, when mtp_path is not NULL, the MTP head to mtp_path, so that snl_engine_load
 * (or the reference) reads them back unchanged.  model_name (nullable) goes in the header. */
int snl_engine_save(snl_engine* e, const char* path, const char* mtp_path, const char* model_name);
/* The engine's model configuration (for a loaded engine, the one its weight file holds). */
int snl_engine_config(const snl_engine* e, snl_config* out);
void snl_engine_destroy(snl_engine* e);
/* Message of the last failed call on this handle ("" if none). */
const char* snl_last_error(const snl_engine* e);
/* Message of the last snl_engine_create failure in this process. */
const char* snl_create_error(void);

/* ---- Engine API (src/engine.rs) --------------------------------------------------------- */

/* Engine::forward_mm (src/engine.rs:801-936) for text tokens: feed `tokens[n]` at the
 * current position.  pos3 gives each token's rotary (t, h, w) position ([n][3]) or NULL
 * for the cache position.  logit_rows (0..2) rows of logits are produced for the last
 * tokens; ckpt (requires n == 2) saves the recurrent state after the first token so that
 * snl_rollback can undo the second.  logits_out (nullable) receives rows x vocab floats,
 * picks_out (nullable) one snl_pick per row. */
int snl_forward(snl_engine* e, const uint32_t* tokens, int n, const uint32_t* pos3, int logit_rows, int ckpt,
                float* logits_out, snl_pick* picks_out);

/* One forward pass (n <= 2 tokens, same semantics as snl_forward) launched op by op with
 * a device timestamp between ops, as the reference's per-op profile mode
 * (SENSENOVA_PROFILE, src/engine.rs:859-886).  recs[max_recs] receives, per op, its name,
 * its algorithmic HBM bytes (GEMV: quants + scales + input rows + output; 0 where not
 * counted) and its duration in ms; *n_recs the number of records. */
typedef struct snl_op_time {
    char name[24];
    double bytes;
    double ms;
} snl_op_time;
int snl_forward_profiled(snl_engine* e, const uint32_t* tokens, int n, const uint32_t* pos3, int logit_rows,
                         int ckpt, snl_op_time* recs, int max_recs, int* n_recs);

/* Isolated-op timing (no reference counterpart; a measurement aid beside the profile mode
 * above): launches only the ops called `name` (an snl_op_time name, e.g. "gemv_gate_up") of a
 * 2-token verify pass at the current position, `reps` passes back to back between two device
 * events on the engine stream, and reports the mean time per launch, the algorithmic HBM bytes
 * per launch (0 where not counted) and the launches per pass.  Skipped ops leave the inputs as
 * they are; nothing is committed (position, state slot and carried hidden row are unchanged).
 * "copy" and "norm" (the final norm, which also writes the carried hidden row) are refused, and
 * so is any op while a checkpointed verify awaits its rollback (SNL_ESTATE). */
int snl_time_op(snl_engine* e, const char* name, int reps, double* ms_per_launch, double* bytes_per_launch,
                int* launches_per_pass);

/* Engine::mtp (src/engine.rs:713-774): run the MTP head on pairs (hidden row r0+i of the
 * last step, tokens[i]) into MTP cache slots slot0+i with rotary positions pos3[i].  With
 * draft != 0, *draft_out receives the draft token, pick_out (nullable) its pick and
 * logits_out (nullable) the vocab logits. */
int snl_mtp(snl_engine* e, int r0, const uint32_t* tokens, int n, const uint32_t* pos3, int slot0, int draft,
            uint32_t* draft_out, snl_pick* pick_out, float* logits_out);

/* Engine::rollback (src/engine.rs:688-697): undo the second token of the last 2-token
 * checkpointed forward. */
int snl_rollback(snl_engine* e);
/* Engine::snapshot / restore / reset (src/engine.rs:646-683). slot < SNL_SNAPSHOTS. */
int snl_snapshot(snl_engine* e, int slot);
int snl_restore(snl_engine* e, int slot, int pos);
int snl_reset(snl_engine* e);
/* Fields and getters the worker reads (src/engine.rs:700-706, src/worker.rs:124, :292). */
int snl_pos(const snl_engine* e);
int snl_ctx(const snl_engine* e);
int snl_hid_rows(const snl_engine* e);
int snl_has_mtp(const snl_engine* e);
int snl_prefill_chunk(const snl_engine* e);

/* ---- the greedy MTP decode loop (src/worker.rs:123-255) ---------------------------------- */

/* prefill_s, decode_s: host wall time of the prompt and of the decode steps.  draft_s, verify_s:
   the greedy decode's device time in the MTP draft passes and in the 2-token verify passes
   (stream events around each pass; the two passes of a step are launched together). */
typedef struct snl_gen_stats {
    int32_t generated, drafted, accepted, _pad;
    double prefill_s, decode_s, draft_s, verify_s;
} snl_gen_stats;

/* Worker::run for one text prompt with greedy sampling (temperature 0, no penalties) and no
 * prefix cache: prefill, then draft / verify / accept-or-rollback until max_tokens tokens
 * (or an EOS id).  spec = 0 decodes one token per forward.  The speculation self-pause of
 * src/worker.rs:222-234 is off.  out[max_tokens] receives the tokens; gaps (nullable) the
 * top-2 margin of the logits row each token was taken from. */
int snl_generate(snl_engine* e, const uint32_t* prompt, int n, int max_tokens, int spec, uint32_t* out,
                 float* gaps, snl_gen_stats* stats);

/* The same loop one step at a time: snl_decoder_create prefills the prompt (Worker::feed,
 * src/worker.rs:291-323) and holds the first sampled token; each snl_decoder_step emits the
 * pending token and runs one speculative step (draft, 2-token verify, accept or rollback),
 * emitting the draft too when it is accepted.  out[2] / gaps[2] (nullable) receive the
 * emitted tokens, *n_out their number (1 or 2). */
typedef struct snl_decoder snl_decoder;
int snl_decoder_create(snl_engine* e, const uint32_t* prompt, int n, int spec, snl_decoder** out);
int snl_decoder_step(snl_decoder* d, uint32_t* out, float* gaps, int* n_out);
/* `steps` calls of snl_decoder_step in one native loop (no counterpart in the reference, whose
 * loop stops at an EOS id): with speculation each step is queued on the device before the host
 * waits for the one before it, the step's records being written on the device from the previous
 * step's outcome.  Every queued step has completed when it returns.  out / gaps (nullable) hold
 * 2 * steps entries; *n_out receives the number of emitted tokens. */
int snl_decoder_steps(snl_decoder* d, int steps, uint32_t* out, float* gaps, int* n_out);
int snl_decoder_stats(const snl_decoder* d, snl_gen_stats* out);
void snl_decoder_destroy(snl_decoder* d);

/* ---- the generation worker with its prefix cache (src/worker.rs:57-272) ------------------- */

/* Snapshot slots of an engine (SNAPSHOTS, src/engine.rs:20). */
#define SNL_SNAPSHOTS 4

/* Finish (src/worker.rs:43-55) of one request: reason 0 = length, 1 = stop (EOS). */
typedef struct snl_finish {
    int32_t reason, prompt_tokens, completion_tokens, cached_tokens, drafted, accepted;
    double prefill_s, decode_s;
} snl_finish;

/* The Worker (src/worker.rs:57-73) over one engine.  It owns the engine's state between its
 * requests: the keys of the tokens the caches hold ("live") and what each snapshot slot holds,
 * with a last-used clock.  A call on the engine from elsewhere (snl_forward, snl_generate, ...)
 * makes the worker forget both at its next request.  self_pause = 1 keeps the reference's
 * speculation self-pause (src/worker.rs:222-234); 0 drafts in every request. */
typedef struct snl_worker snl_worker;
int snl_worker_create(snl_engine* e, int self_pause, snl_worker** out);
void snl_worker_destroy(snl_worker* w);

/* Worker::run (src/worker.rs:123-272) for one text prompt with greedy sampling: reuse the live
 * state or the snapshot whose keys are the longest strict prefix of the prompt (or reset),
 * feed the prompt, snapshot after its first snapshot_at tokens into the least recently used
 * slot when snapshot_at is past the reused part and short of n (< 0: none, as server.rs:262
 * sets it at the last <|im_start|>), then decode as snl_generate does, drafting when spec is
 * set, the model has an MTP head and no self-pause is running.  out receives
 * max(1, min(max_tokens, ctx - n)) tokens at most; gaps (nullable) the top-2 margins; fin
 * (nullable) the Finish record, whose cached_tokens counts the prompt tokens not fed again.
 * Unlike the reference, a snapshot is dropped once a request writes the attention caches
 * under its prefix with another sequence (a snapshot holds only the recurrent state).  On an
 * error the engine is reset and the cache emptied (src/worker.rs:94-101). */
int snl_worker_run(snl_worker* w, const uint32_t* prompt, int n, int snapshot_at, int max_tokens, int spec,
                   uint32_t* out, float* gaps, snl_finish* fin);

/* The cache bookkeeping: live length, and per slot the key count (-1 = empty) and last use. */
int snl_worker_cache(const snl_worker* w, int* live_len, int* snap_len, uint64_t* snap_used);

/* ---- sampling (src/sampler.rs) ------------------------------------------------------------ */

/* SamplingParams (src/sampler.rs:4-29).  temperature <= 1e-5 is greedy; top_k 0 = no top-k. */
typedef struct snl_sampling {
    float temperature, top_p, min_p, presence_penalty, frequency_penalty, repetition_penalty;
    int32_t top_k, _pad;
} snl_sampling;

/* The reference's StdRng (rand 0.10.3: ChaCha12 keyed by seed_from_u64) as used by Sampler:
 * snl_rng_f32 is random::<f32>().  snl_chacha_block is the block function (rounds 12 or 20). */
typedef struct snl_rng {
    uint32_t key[8];
    uint64_t counter;
    uint32_t buf[16];
    int32_t idx, _pad;
} snl_rng;
void snl_chacha_block(const uint32_t in[16], int rounds, uint32_t out[16]);
void snl_rng_seed(snl_rng* r, uint64_t seed);
uint32_t snl_rng_u32(snl_rng* r);
float snl_rng_f32(snl_rng* r);
/* Sampler::draw (src/sampler.rs:143-158) over a normalised list, excluding `exclude` (-1: none),
 * with the uniform u; and the tail of Sampler::distribution (:111-140) over candidate logits in
 * descending order (temperature softmax, min-p, top-p, renormalisation): probs[n] receives the
 * probabilities, the return value is how many are kept. */
uint32_t snl_draw(const uint32_t* tokens, const float* probs, int n, int64_t exclude, float u);
int snl_finish_distribution(const float* logits, int n, float temperature, float min_p, float top_p, float* probs);

/* Sampler (src/sampler.rs:32-96) over logits row `row` (0 or 1) of the engine's last forward: the
 * penalties and top-k run on the device (only k candidates are read back; top_k 0 or above 1024
 * reads the row back), the rest on the host.  accept() records a generated token for the
 * penalties; sample() and verify() are Sampler::sample / Sampler::verify (accept the draft with
 * probability p(draft), else draw from p without it); distribution() returns the kept list.
 * has_seed = 0 seeds from the OS, as StdRng::from_rng does. */
typedef struct snl_sampler snl_sampler;
int snl_sampler_create(snl_engine* e, const snl_sampling* p, uint64_t seed, int has_seed, snl_sampler** out);
void snl_sampler_destroy(snl_sampler* s);
void snl_sampler_accept(snl_sampler* s, uint32_t token);
int snl_sampler_sample(snl_sampler* s, int row, uint32_t* token);
int snl_sampler_verify(snl_sampler* s, int row, uint32_t draft, int* accepted, uint32_t* token);
int snl_sampler_distribution(snl_sampler* s, int row, uint32_t* tokens, float* probs, int cap, int* n_out);

/* Worker::run with the request's SamplingParams (src/worker.rs:193-252): as snl_worker_run, the
 * tokens drawn by a Sampler seeded with `seed` (has_seed = 0: from the OS).  Greedy parameters
 * without penalties take snl_worker_run's path. gaps are not reported. */
int snl_worker_run_sampled(snl_worker* w, const uint32_t* prompt, int n, int snapshot_at, int max_tokens, int spec,
                           const snl_sampling* params, uint64_t seed, int has_seed, uint32_t* out, snl_finish* fin);

/* ---- inspection (tests) ------------------------------------------------------------------- */

/* Shape of a generated tensor: layer -1 = embed(1)/lm_head(2)/norm(3); layer 0xFFF = MTP
 * head.  Returns the type (0 Q8_0, 1 Q4_0, 2 f32 vector) or -1. */
int snl_tensor_info(const snl_engine* e, int layer, int kind, int* rows, int* cols);
/* Copy a tensor to host memory: q (quants or f32 values) and s (scales; NULL for vectors). */
int snl_tensor_read(snl_engine* e, int layer, int kind, void* q, float* s);
/* Set the block scales of rows first.. of a quantised matrix to zero, so those rows dequantise to
 * exactly 0 (every copy the engine keeps of it).  No counterpart in the reference: on random
 * weights no draft is ever accepted, so tests and the bench confine the LM head's argmax to its
 * first rows this way to drive the accept branch of the decode loop.  Drops cached state. */
int snl_tensor_zero_rows(snl_engine* e, int layer, int kind, int first);
/* Copy an engine buffer to host: 0 x [2, 2H], 1 hid [3, H], 2 hlast [H], 3 DeltaNet state
 * (current slot, all visits), 4 conv state (current slot), 5 MTP residual [2, 2H]. */
int snl_buffer_read(snl_engine* e, int id, void* out, size_t bytes);
size_t snl_buffer_size(const snl_engine* e, int id);

/* ---- kernel-level entry points (device pointers; `stream` is a hipStream_t or NULL) ------ */

/* y[m*y_stride + n] = sum_k x[m*x_stride + k] * W[n, k], M in 1..4 (matmul.wgsl matvec1/2).
 * wq/ws: reference layout quants [N, K] (Q8) or [N, K/2] (Q4), f32 scales [N, K/32].  When
 * K % 128 == 0 the call packs W into the engine's tile order in a staging buffer the library
 * keeps, runs the matrix-core kernel and returns after it has finished on `stream`; other
 * shapes run the vector-ALU kernel on W as given. */
int snl_gemv(int quant, const void* wq, const float* ws, const float* x, float* y, int M, int N, int K,
             int x_stride, int y_stride, void* stream);

/* The prefill GEMM (src/shaders/matmul.wgsl:200-318, MatKind::Tiled): y[m*y_stride + n] =
 * sum_k x[m*x_stride + k] * W[n, k] for M in 1..SNL_PREFILL_M token rows, K % 128 == 0 and
 * K <= 16384, W in
 * the reference layout as for snl_gemv.  The call packs W into the GEMM's panel order and the
 * rows into f16 hi/lo fragments in staging buffers the library keeps, and returns after the
 * product has finished on `stream`. */
#define SNL_PREFILL_M 512
int snl_gemm(int quant, const void* wq, const float* ws, const float* x, float* y, int M, int N, int K,
             int x_stride, int y_stride, void* stream);
/* Times the decode GEMV alone (measurement; no reference counterpart, it serves the skinny GEMV
 * microbench over src/shaders/matmul.wgsl:102-198): enough distinct seeded N x K matrices in tile
 * order to span at least 1 GB (*copies_out, nullable), launched in turn `reps` times with M random
 * token rows between two HIP events on a stream of its own.  *ms_per_launch receives the mean and
 * *bytes_per_launch (nullable) the algorithmic bytes of one launch: quants, f32 block scales, the
 * M input rows and the M output rows. */
int snl_gemv_time(int quant, int N, int K, int M, int reps, double* ms_per_launch, double* bytes_per_launch,
                  int* copies_out);
/* Times the prefill GEMM alone (measurement): seeded N x K weights in panel order and M random
 * token rows, `reps` launches back to back between two HIP events on a stream of its own;
 * *ms_per_launch receives the mean. */
int snl_gemm_time(int quant, int N, int K, int M, int reps, double* ms_per_launch);

/* One Gated DeltaNet step over M = 1..4 tokens (linear.wgsl conv + delta).  conv_state and
 * state hold three slots each ([3][3, conv_dim] and [3][n_v, 128, 128]); the call reads
 * slot s_in, writes slot s_out and, if ckpt > 0, the state after token ckpt-1 to slot s_ck. */
int snl_deltanet(const float* proj, int proj_stride, const float* lw, float* conv_state, float* state, float* out,
                 int conv_dim, int n_k, int n_v, float eps, int M, int ckpt, int s_in, int s_out, int s_ck,
                 void* stream);

/* Gated attention for M = 1 or 2 tokens at cache positions pos0..pos0+M-1
 * (attention.wgsl prep + attend + combine).  rpos: host [M][3] rotary positions.
 * partial: device scratch of M * n_heads * ceil(ctx/64) * 258 floats. */
int snl_attention(const float* proj, int proj_stride, float* qbuf, uint16_t* kcache, uint16_t* vcache,
                  const float* norms, float* out, float* partial, int n_heads, int n_kv, int rot_dim,
                  float rope_theta, float eps, const int32_t* mrope_section, int ctx, int M, int pos0,
                  const uint32_t* rpos, void* stream);

/* Greedy pick of `rows` device logits rows of length V into device picks_out; 1 <= rows <= 64. */
int snl_pick_rows(const float* logits, int V, int rows, snl_pick* picks_out, void* stream);

/* snl_pick_rows without any device allocation.  No counterpart in the reference: it is for callers
 * that cannot allocate (code under HIP graph capture, serving loops or harnesses that forbid
 * hipMalloc).  The block partials live in a static 48 KiB device array, one per GPU, held until
 * the process ends, so rows * ceil(V / 2048) may be at most 4096 (e.g. 33 rows of a 248320-entry
 * vocabulary), and rows at most 64 as for snl_pick_rows; SNL_EARG beyond either limit.  The call only enqueues work on `stream`, a stream of the current
 * device, and returns; picks_out is ready when the stream reaches it.  Calls that overlap on one
 * GPU share the array and race. */
int snl_pick_rows_noalloc(const float* logits, int V, int rows, snl_pick* picks_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SNL_H */
