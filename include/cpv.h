/*
 * cpv.h — C ABI of the MI355X verify-step library (libcpv.so).
 *
 * Drop-in boundary for codpiece's speculative-decoding verify step.  Today the
 * reference reaches its arithmetic through codpiece-ggml-sys, raw bindgen
 * bindings over ggml (crates/codpiece-ggml-sys/wrapper.h:1-9,
 * crates/codpiece-ggml-sys/src/lib.rs:1-11), building a graph per shape in
 * crates/codpiece-model/src/qwen35.rs:2445-3198 and running it with
 * ggml_backend_graph_compute (qwen35.rs:3606-3620).  This header is what a
 * thin codpiece-hip-sys crate binds instead: plain C types, device pointers
 * owned by the caller, opaque handles owned by the library.
 *
 * Conventions
 *  - Every call returns a cpv_status; on failure cpv_last_error(ctx) holds a
 *    message.  Nothing aborts or throws across this boundary (the reference's
 *    rule: qwen35.rs:3616-3618, crates/codpiece-model/src/meta.rs:47-49).
 *  - A context is bound to one device and one HIP stream and is used from one
 *    thread at a time, like the engine thread that owns every ggml object
 *    (crates/codpiece-server/src/engine.rs:1-7).  Calls enqueue on the stream
 *    and return; cpv_sync waits.  Distinct contexts are independent.
 *  - Pointers named *_dev are device pointers the caller owns.
 *  - Type ids are GGUF's (crates/codpiece-gguf/src/lib.rs:173-185).
 */
#ifndef CPV_H
#define CPV_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int cpv_status;
enum {
    CPV_OK = 0,
    CPV_EINVAL = 1,        /* bad argument (shape, null, range) */
    CPV_ENOMEM = 2,        /* device allocation failed; the context stays usable */
    CPV_EDEVICE = 3,       /* HIP runtime error */
    CPV_EUNSUPPORTED = 4,  /* valid request this build does not implement */
};

enum { CPV_F32 = 0, CPV_F16 = 1, CPV_Q8_0 = 8, CPV_Q4_K = 12, CPV_Q6_K = 14 };

typedef struct cpv_ctx cpv_ctx;
typedef struct cpv_weight cpv_weight;

/* ---- context ------------------------------------------------------------ */
/* Replaces ggml_backend_cuda_init / the backend handle Weights::load creates
 * (crates/codpiece-model/src/lib.rs:128-311). */
cpv_status  cpv_init(int device, cpv_ctx** out);
void        cpv_free(cpv_ctx* ctx);
const char* cpv_last_error(const cpv_ctx* ctx);
/* Enqueue on the caller's hipStream_t from now on, verbatim: NULL is HIP's
 * default (null) stream.  A new context starts on a stream of its own. */
cpv_status  cpv_set_stream(cpv_ctx* ctx, void* hip_stream);
void*       cpv_get_stream(const cpv_ctx* ctx);
cpv_status  cpv_sync(cpv_ctx* ctx);

/* ---- weights ------------------------------------------------------------ */
/* Upload n_rows rows of k elements in ggml block layout (GGUF tensor bytes,
 * ne = [k, n_rows]) and repack them for the GEMM kernels.  Replaces
 * ggml_backend_tensor_set of a weight tensor after ggml_backend_alloc_ctx_tensors
 * (crates/codpiece-model/src/lib.rs:236-266).  Supported: Q8_0, Q4_K, Q6_K. */
cpv_status  cpv_weight_upload(cpv_ctx* ctx, int type, const void* host_bytes, int64_t n_rows,
                              int64_t k, cpv_weight** out);
/* The same from bytes already in device memory (not retained). */
cpv_status  cpv_weight_from_device(cpv_ctx* ctx, int type, const void* dev_bytes, int64_t n_rows,
                                   int64_t k, cpv_weight** out);
void        cpv_weight_free(cpv_weight* w);
/* shape / type / device bytes held; any out pointer may be NULL */
cpv_status  cpv_weight_info(const cpv_weight* w, int* type, int64_t* n_rows, int64_t* k,
                            int64_t* bytes);
/* Dequantize rows[i] of w into out_dev[i][k] (f32), as ggml_get_rows does for
 * the token embedding and out_ids (qwen35.rs:2545,2794).  rows_dev: int32. */
cpv_status  cpv_get_rows(cpv_ctx* ctx, const cpv_weight* w, const int32_t* rows_dev, int64_t n,
                         float* out_dev);

/* ---- kernels -------------------------------------------------------------- */
/* y[m][n] = x[m][:] . dequant(w[n][:]) — ggml_mul_mat(w, x) with ne
 * [k, n] x [k, m] -> [n, m] (crates/codpiece-ggml-sys/tests/smoke.rs:19),
 * quantizing x to ggml's CPU vec_dot_type (Q8_0 for Q8_0 weights, Q8_K for
 * K-quants).  Per block the integer dot is exact; each block's scaled term is
 * rounded to an integer grid 2^g (g from the largest weight-row and
 * activation-row scales) and the terms are summed exactly below 2^53, so the
 * result does not depend on how the K loop is split.
 * Replaces every ggml_mul_mat on the verify path (qwen35.rs:2779-2782,2797,
 * 3029,3047,3051,3197; mtp_graph.rs:184,209-212,230).  x_dev: f32 [m][k];
 * y_dev: f32 [m][n_rows]; 1 <= m <= 256 (Q4_K from 32 rows on: the wide
 * prefill kernel, the same sums). */
cpv_status  cpv_qgemm(cpv_ctx* ctx, const cpv_weight* w, const float* x_dev, int64_t m,
                      float* y_dev);

/* No counterpart in the reference: cpv_qgemm for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops and
 * harnesses that forbid hipMalloc).  The same kernels and the same results
 * as cpv_qgemm, with the quantized activations and the split-K accumulator in
 * a fixed per-device scratch array (10 MiB, held until the process ends)
 * instead of the context's workspace; the call allocates nothing.  Limits:
 * 1 <= m <= 16, the quantized activations within 2 MiB (k up to 65536 at
 * m = 16) and m * (n_rows rounded up to 64) <= 1048576 (else CPV_EINVAL).
 * Every call on one device shares that device's scratch: calls that overlap
 * on one device (two streams, two contexts) race. */
cpv_status  cpv_qgemm_noalloc(cpv_ctx* ctx, const cpv_weight* w, const float* x_dev, int64_t m,
                              float* y_dev);

/* Masked GQA attention over the f16 KV cache; replaces ggml_flash_attn_ext
 * with prec F32 and an f16 mask (qwen35.rs:3182-3187, mask fill :3551-3568).
 *   q_dev        f32 [t][h][d]
 *   k_cache_dev  f16 [n_ctx][h_kv * d], the FA cache layout (qwen35.rs:571-575)
 *   v_cache_t_dev f16 [h_kv * d][v_stride], the transposed V cache the
 *                reference keeps without FA (qwen35.rs:580-586)
 *   rows / columns [0, n_past) are context; n_past + i holds tree node i
 *   parent_dev   int32 [t]: parent of each node (-1 = child of the context,
 *                parents precede children), or NULL for a linear chain (the
 *                reference's causal mask).  Node i sees all context rows plus
 *                its ancestors and itself.
 *   out_dev      f32 [t][h * d]
 * Requires d in {64, 128}, t <= 64 for a tree (t <= 8192 for a chain),
 * v_stride >= n_past + t and a multiple of 8, 16-byte aligned caches. */
cpv_status  cpv_attn(cpv_ctx* ctx, const float* q_dev, const uint16_t* k_cache_dev,
                     const uint16_t* v_cache_t_dev, int64_t v_stride, int64_t n_past,
                     const int32_t* parent_dev, int t, int h, int h_kv, int d, float scale,
                     float* out_dev);

/* Row argmax, first maximum wins: ggml_argmax (qwen35.rs:2811-2818),
 * optionally of logits + noise (the gumbel branch).  x_dev [rows][n],
 * noise_dev [rows][n] or NULL, out_dev int32 [rows]. */
cpv_status  cpv_argmax_rows(cpv_ctx* ctx, const float* x_dev, const float* noise_dev, int64_t rows,
                            int64_t n, int32_t* out_dev);

/* ---- speculative acceptance ------------------------------------------------ */
/* SamplerParams (crates/codpiece-sample/src/lib.rs:29-47) minus the seed. */
typedef struct {
    float   temp;
    int32_t top_k;
    float   top_p;
    float   min_p;
    int32_t min_keep;
    float   penalty_repeat;
    float   penalty_freq;
    float   penalty_present;
    int32_t penalty_last_n;
} cpv_sampler_params;

enum { CPV_ACCEPT_GREEDY = 0, CPV_ACCEPT_REJECT = 1, CPV_ACCEPT_GUMBEL = 2 };

/* Sampler::distribution (crates/codpiece-sample/src/lib.rs:184-187, built by
 * Sampler::build :229-376) for `rows` independent logit rows: penalties over
 * the row's history window, then top-k / min-p / top-p narrowing, the
 * temperature and the softmax, with the CPU sampler's f32 results bit for
 * bit (its sums are sequential folds in candidate order).
 *   logits_dev  f32 [rows][v]
 *   hist_dev    int32 [rows][hist_len] history, oldest first, -1 = empty
 *               (NULL = none); the last penalty_last_n valid entries count
 *   ids_dev     int32 [rows][v]: candidate ids in candidate order (logit
 *               descending, id ascending after a narrowing filter, index
 *               order otherwise); the first n_dev[r] are the distribution
 *   probs_dev   f32 [rows][v]: their probabilities
 *   n_dev       int32 [rows]
 * 1 <= v <= 262144, hist_len <= 4096, min_p <= 1 (above 1 no candidate
 * survives and the reference panics). */
cpv_status  cpv_distribution(cpv_ctx* ctx, const float* logits_dev, int rows, int v,
                             const cpv_sampler_params* params, const int32_t* hist_dev, int hist_len,
                             int32_t* ids_dev, float* probs_dev, int32_t* n_dev);

/* Decide a speculative round for b sequences on the device: the acceptance
 * loop of crates/codpiece-server/src/engine.rs:2326-2461 with the target
 * distribution of Sampler::distribution (crates/codpiece-sample/src/lib.rs:
 * 184-187,229-376) and Dist::{prob_of, draw, draw_excluding} (:387-436).
 *   p_logits_dev  f32 [b][k+1][v]   target logits at the k+1 verified rows
 *   q_logits_dev  f32 [b][k][v] or NULL.  NULL = drafts are the draft head's
 *                 argmax (a point mass) and the reference rule applies:
 *                 accept with p(x), else draw from p without x.  Non-NULL =
 *                 drafts were sampled from q: accept iff u*q(x) < p(x), else
 *                 draw from max(0, p - q) renormalised.
 *   draft_dev     int32 [b][k]
 *   mode          CPV_ACCEPT_GREEDY (argmax match), _REJECT, _GUMBEL
 *   u_dev         f32 [b][k+1][2] uniforms by role (r0 = accept roll, or the
 *                 bonus draw at j = k; r1 = residual draw), or NULL to draw
 *                 them from Philox4x64-10 with key (philox_seed, 0) and
 *                 counter (b, j, r, philox_round), taking (x >> 40) / 2^24
 *                 (a request keeps its seed; each of its rounds takes its
 *                 own philox_round).
 *   noise_dev     f32 [b][k+1][v], T-scaled gumbel noise (GUMBEL mode only)
 *   hist_dev      int32 [b][hist_len] penalty window, oldest first, -1 empty
 *                 (only read when a penalty is active)
 *   out_tok_dev   int32 [b][k+1]: the accepted drafts then the next token
 *   out_n_dev     int32 [b]: number of accepted drafts (tokens = out_n + 1)
 * v <= 262144, k <= 15, hist_len <= 4096; params may be NULL in GREEDY mode.
 * Outputs equal the CPU loop's for the same uniforms, bit for bit. */
cpv_status  cpv_spec_accept(cpv_ctx* ctx, const float* p_logits_dev, const float* q_logits_dev,
                            const int32_t* draft_dev, int b, int k, int v,
                            const cpv_sampler_params* params, int mode, const float* u_dev,
                            uint64_t philox_seed, uint64_t philox_round, const float* noise_dev,
                            const int32_t* hist_dev, int hist_len, int32_t* out_tok_dev,
                            int32_t* out_n_dev);

/* ---- model and verify round ------------------------------------------------- */
typedef struct cpv_model cpv_model;
typedef struct cpv_session cpv_session;

/* Hparams of an all-attention qwen35 model (qwen35.rs:45-148 with
 * full_attention_interval = 1): n_layer trunk layers, plus the MTP layer
 * blk.{n_layer} when has_mtp. */
typedef struct {
    int32_t n_layer;
    int32_t n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab;
    int32_t n_rot;               /* rotary dims of head_dim */
    int32_t rope_sections[4];    /* IMROPE sections; text positions use streams (p, p, p, 0) */
    float   rms_eps, freq_base;
    int32_t has_mtp;
} cpv_hparams;

/* Weights::load (crates/codpiece-model/src/lib.rs:128-311): create a model,
 * hand it every tensor by its GGUF name (ggml ne order: ne0 = row length,
 * ne1 = rows; host or device bytes), then check it with cpv_model_ready.
 * Linear weights: Q8_0 / Q4_K / Q6_K; norms: F32. */
cpv_status  cpv_model_create(cpv_ctx* ctx, const cpv_hparams* hp, cpv_model** out);
cpv_status  cpv_model_set_tensor(cpv_model* m, const char* name, int type, const void* data, int on_device,
                                 int64_t ne0, int64_t ne1);
cpv_status  cpv_model_ready(cpv_model* m);
void        cpv_model_free(cpv_model* m);

/* ---- the model file (GGUF) -------------------------------------------------
 * cpv_gguf_scan: GgufFile::open and its validation
 * (crates/codpiece-gguf/src/lib.rs:345-458).  It reads the header, the
 * metadata and the tensor directory of a GGUF v1-v3 file.  Counts and lengths
 * are capped.  The alignment must be a power of two.  Tensor offsets must be
 * aligned, in file order without overlap, and inside the data section.
 * tensor_bytes is the sum of the sized tensors (tensor_bytes, :453-456).  No
 * GPU is used.  On failure errbuf (may be NULL) gets the reason.
 *
 * cpv_gguf_hparams: Hparams::from_gguf (crates/codpiece-model/src/qwen35.rs:
 * 75-130) for an all-attention qwen35 file.  n_layer = block_count -
 * nextn_predict_layers, n_vocab = the length of tokenizer.ggml.tokens, and
 * the same defaults for the optional keys.  full_attention_interval must be 1
 * and there is at most one nextn layer (else CPV_EUNSUPPORTED).  No GPU is
 * used.
 *
 * cpv_model_load_gguf: Weights::load (crates/codpiece-model/src/lib.rs:
 * 128-311) on one device.  It creates the model from the file's
 * hyper-parameters, hands every tensor to cpv_model_set_tensor by name (one
 * whole-tensor read and upload each), then calls cpv_model_ready. */
typedef struct {
    int32_t  version;
    int64_t  n_tensors, n_kv;
    uint64_t alignment, data_start, tensor_bytes;
} cpv_gguf_info;
cpv_status  cpv_gguf_scan(const char* path, cpv_gguf_info* info, char* errbuf, int errlen);
cpv_status  cpv_gguf_hparams(const char* path, cpv_hparams* hp, char* errbuf, int errlen);
cpv_status  cpv_model_load_gguf(cpv_ctx* ctx, const char* path, cpv_model** out);

/* Session::new_spec (qwen35.rs:528-649): a K and a V cache per layer, plus
 * the MTP cache (min(n_ctx, 16384) rows); max_batch bounds t of every call.
 * The caches hold each row's values rounded to f16 as the integer limbs the
 * attention's MFMAs take (written once per row; the same scores and outputs
 * as over f16 caches). */
cpv_status  cpv_session_create(cpv_model* m, int64_t n_ctx, int32_t max_batch, cpv_session** out);
void        cpv_session_free(cpv_session* s);
/* n_past / mtp_past, the round bookkeeping of engine.rs:2533-2540: a caller
 * rewinds a rejected tail with set_pos(n_past - over, mtp_past + n_keep + 1). */
cpv_status  cpv_session_set_pos(cpv_session* s, int64_t n_past, int64_t mtp_past);
cpv_status  cpv_session_get_pos(const cpv_session* s, int64_t* n_past, int64_t* mtp_past);
/* No counterpart in the reference: a debugging tap.  While set, every
 * attention call of cpv_prefill / cpv_verify_step also copies its output
 * ([t][n_head][head_dim] f32, before the output gate) to tap_dev, blocks
 * back to back in call order (trunk layers, then each MTP link), restarting
 * at offset 0 with each call; blocks past capacity_floats are dropped.
 * NULL clears it. */
cpv_status  cpv_session_set_attn_tap(cpv_session* s, float* tap_dev, int64_t capacity_floats);
/* Round replay, the counterpart of the reference's per-shape graph reuse
 * (qwen35.rs:1740-1748: one built graph kept per shape; the graph uid of
 * patches/ggml-codpiece.patch:1-15).  On (the default), a cpv_verify_step
 * round without noise, shortlist, tap or profiling replays a HIP graph of its
 * shape -- t, depth and the attention grids' 1024-row position ranges -- which
 * the session captures on the shape's second round; the round's positions and
 * tokens are set on the stream before the replay, and the results are the
 * eager round's bit for bit.  Off, every round launches its kernels. */
cpv_status  cpv_session_set_replay(cpv_session* s, int on);
/* No counterpart in the reference: rounds captured as graphs and rounds
 * replayed (a captured round counts in both) since the session was made. */
cpv_status  cpv_session_replay_stats(const cpv_session* s, int64_t* captured, int64_t* replayed);

/* Trunk only over t prompt tokens (step_greedy's bulk prefill, main.rs:776-781):
 * writes the KV cache and advances n_past by t. */
cpv_status  cpv_prefill(cpv_session* s, const int32_t* tokens_dev, int t);

/* FusedOut (qwen35.rs:817-828).  Device pointers owned by the session, valid
 * until its next call. */
typedef struct {
    int64_t  n_past;        /* after the round (advanced by t, as the reference) */
    int32_t* preds_dev;     /* [t] argmax of each verified row (of logits + noise) */
    int32_t* chain_dev;     /* [depth][t] draft ids, link-major */
    float*   conf_dev;      /* [depth][t] softmax peak of each link */
    float*   logits_dev;    /* [t][n_vocab] trunk logits */
    float*   hidden_dev;    /* [t][n_embd] normed trunk hidden */
} cpv_round_out;

/* Qwen35::step_fused_cached (qwen35.rs:1693-1948) for t tokens with a draft
 * chain of `depth` links (0 = verify only): trunk, LM head, argmax (of
 * logits + noise_dev when noise is given, the gumbel branch), MTP chain. */
cpv_status  cpv_verify_step(cpv_session* s, const int32_t* tokens_dev, int t, int depth,
                            const float* noise_dev, cpv_round_out* out);
/* The same with the draft head over a shortlist: step_fused_cached's `cands`
 * (MtpTail::n_cand, qwen35.rs:208-216, :1698-1707).  Each link projects onto
 * the head's rows cands_host[0..n_cand) (get_rows then mul_mat,
 * :2925-2931).  Its draft is cands[argmax] and its confidence the softmax
 * peak over those n_cand logits.  As in the reference graph, the next link
 * embeds the argmax itself (tok_src = ids, :2958); the reported chain holds
 * the mapped ids (:1904-1910).  Verification keeps the full vocabulary.
 * Candidates are host ids < n_vocab.  The gathered head is kept while the
 * shortlist stays the same.  n_cand = 0 is cpv_verify_step. */
cpv_status  cpv_verify_step_cands(cpv_session* s, const int32_t* tokens_dev, int t, int depth,
                                  const float* noise_dev, const int32_t* cands_host, int n_cand,
                                  cpv_round_out* out);

/* One standalone draft link: Qwen35::mtp_draft (qwen35.rs:2086-2192), whose
 * graph is build_mtp_impl (mtp_graph.rs:123-249).  From the trunk's normed
 * hidden row hidden_dev [n_embd] (a row of cpv_round_out.hidden_dev, or the
 * previous link's hidden_dev) and `token`, the token at the position after
 * that row: rms(embed(token)) * enorm ; rms(hidden) * hnorm, eh_proj, the MTP
 * layer at rope position `pos` with its K/V written at MTP row mtp_past and
 * rows 0..mtp_past attended, then rms with the head norm (the next link's
 * hidden) and the draft head.  mtp_past advances by 1, as in the reference
 * (:2189).  Also on the device: the draft, argmax of the logits with the first
 * maximum winning (the host argmax, qwen35.rs:3659-3669), and the confidence
 * gate of the engine's re-draft (crates/codpiece-server/src/engine.rs:
 * 2598-2606) and of the CLI spec path (crates/codpiece-cli/src/main.rs:
 * 1066-1069): keep = 0 when p_min > 0 and 1 / lse < p_min, lse the f32 sum in
 * index order of exp(l - max), decided exactly; else keep = 1.  Outputs are
 * session-owned device memory, valid until the session's next call.
 * 0 <= pos <= n_ctx + 1; a full MTP cache (mtp_past = min(n_ctx, 16384)) is
 * an error, where the reference would write past it. */
typedef struct {
    float*   logits_dev;    /* [n_vocab] the draft head's logits */
    float*   hidden_dev;    /* [n_embd] the link's hidden for the next link */
    int32_t* draft_dev;     /* [1] argmax of logits_dev */
    int32_t* keep_dev;      /* [1] the gate: 1 = keep the draft, 0 = stop */
} cpv_draft_out;
cpv_status  cpv_mtp_draft(cpv_session* s, const float* hidden_dev, int32_t token, int64_t pos, float p_min,
                          cpv_draft_out* out);

/* The argmax and the re-draft gate of cpv_mtp_draft for `rows` logit rows
 * [rows][v] (v <= 262144): argmax_dev [rows], keep_dev [rows] as above. */
cpv_status  cpv_redraft_gate(cpv_ctx* ctx, const float* logits_dev, int64_t rows, int64_t v, float p_min,
                             int32_t* argmax_dev, int32_t* keep_dev);

/* ---- draft trees ----------------------------------------------------------
 * No counterpart in the reference: its rounds verify a linear draft and rewind
 * the rejected tail (crates/codpiece-server/src/engine.rs:2533-2540,
 * Qwen35::step_verify qwen35.rs:1568-1674).  These extend that round to a
 * draft tree, with the same trunk, head and argmax.
 *
 * cpv_verify_tree: step_verify over t <= CPV_TREE_MAX nodes.  parent_host[i]
 * is node i's parent (-1: a child of the context), and parents precede their
 * children.  Node i is written at KV row n_past + i, placed at position
 * n_past + depth(i), and attends to the context plus its ancestors and itself
 * (the tree mask of cpv_attn).  preds_dev[i] is the argmax of node i's logits
 * (of logits + noise when noise_dev is given).  n_past advances by t, as
 * verify_step does.  No draft chain is produced.
 *
 * cpv_session_commit_branch: after a tree verify, keeps path_host[0..n), a
 * root-to-node path of that tree.  Its nodes become context rows
 * n_past0 .. n_past0 + n - 1 in every trunk layer's K and V caches, where
 * n_past0 is n_past before the verify, and n_past becomes n_past0 + n.  The
 * other nodes are dropped (n = 0 drops the tree).  Every later row is the same
 * as if the path had been verified as a chain.  Any other call that moves n_past
 * (prefill, verify_step, set_pos) ends the pending tree. */
#define CPV_TREE_MAX 64
cpv_status  cpv_verify_tree(cpv_session* s, const int32_t* tokens_dev, const int32_t* parent_host, int t,
                            const float* noise_dev, cpv_round_out* out);
cpv_status  cpv_session_commit_branch(cpv_session* s, const int32_t* path_host, int n);

/* ---- kernel timing -------------------------------------------------------
 * No counterpart in the reference (which times whole rounds with
 * Instant::now, crates/codpiece-server/src/engine.rs:2295,2324).  Between
 * start and stop, every GEMM and attention launch on the context is bracketed
 * by a pair of HIP events on its stream; stop waits for the stream and sums,
 * per kernel class, the launches, their event-timed milliseconds and their
 * algorithmic bytes (GEMM: the quantized weight + 4*m*k + 4*m*n; attention:
 * the K and V rows read once + q and the output in f32; sampler: the logit
 * rows read once).  The events add a little time between launches: time
 * throughput without them. */
enum { CPV_PROF_Q4_K = 0, CPV_PROF_Q6_K = 1, CPV_PROF_Q8_0 = 2, CPV_PROF_ATTN = 3, CPV_PROF_SAMPLE = 4,
       CPV_PROF_Q4_K_WIDE = 5, CPV_PROF_Q8_0_WIDE = 6, CPV_PROF_Q6_K_WIDE = 7, CPV_PROF_CLASSES = 8 };
typedef struct { int64_t launches; double ms; double bytes; } cpv_prof_stat;
cpv_status  cpv_profile_start(cpv_ctx* ctx);
cpv_status  cpv_profile_stop(cpv_ctx* ctx, cpv_prof_stat* out /* [CPV_PROF_CLASSES] */);
/* Launch again, back to back, every launch of class `cls` the last profile
 * recorded (same kernels, grids and arguments), `reps` times between one pair
 * of events: *ms_per_launch = elapsed / (reps * launches), free of the gaps
 * the per-launch events add; *bytes_per_launch (may be NULL) their mean
 * algorithmic bytes.  The buffers of the recorded calls (weights, sessions)
 * must still be allocated; their outputs are overwritten, and the GEMM
 * accumulator is left zero (as every GEMM expects it). */
cpv_status  cpv_profile_replay(cpv_ctx* ctx, int cls, int reps, double* ms_per_launch, double* bytes_per_launch);

#ifdef __cplusplus
}
#endif
#endif
