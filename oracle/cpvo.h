/*
 * cpvo — CPU oracle for the codpiece verify step.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: tests/, the smoke
 * entry point and bench.py's cpu_baseline leg may load it; the product path
 * (codpiece_amd/, libcpv.so) never links, loads or calls it.
 *
 * It restates, in plain C, the arithmetic the reference's verify step relies
 * on.  The reference runs that arithmetic in ggml b10423 (not vendored, so not
 * buildable here) driven from Rust (no Rust toolchain here), so every
 * function below cites the reference call site it follows and states the
 * exact float contract it implements.  The GPU kernels implement the same
 * contracts; parity tests compare the two bit for bit where the contract is
 * exact, and against a tolerance where it is not (attention).
 *
 * Contracts (one line each; details at each function):
 *  - fp16 <-> fp32: IEEE binary16, round-to-nearest-even.
 *  - weights: ggml block formats Q8_0 / Q4_K / Q6_K (GGUF type ids 8/12/14).
 *  - activations: quantized as ggml's CPU vec_dot_type does — Q8_0 for Q8_0
 *    weights, Q8_K for K-quants.
 *  - qgemm: per block integer dots (exact), per block f64 scale products,
 *    summed EXACTLY in an int64 fixed-point window, rounded once per output.
 *    The result is independent of any summation order.
 *  - rms_norm: exact fixed-point sum of f32 squares, then ggml's f32 tail.
 *  - rope: NEOX pairs with ggml's f32 theta recurrence; cos/sin from libm.
 *  - attention: Q rounded to f16 (ggml CPU FA), scores/softmax/output in f64.
 *  - sampler: bit-faithful restatement of crates/codpiece-sample/src/lib.rs.
 *  - exp: cpvo_expf, a restatement of libm's expf equal to it on every input.
 *  - Philox4x64-10 (Salmon et al., SC'11) for explicit uniforms.
 */
#ifndef CPVO_H
#define CPVO_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type ids (crates/codpiece-gguf/src/lib.rs:173-185). */
enum { CPVO_F32 = 0, CPVO_F16 = 1, CPVO_Q8_0 = 8, CPVO_Q4_K = 12, CPVO_Q6_K = 14, CPVO_Q8_K = 15 };

#pragma pack(push, 1)
typedef struct { uint16_t d; int8_t qs[32]; } cpvo_block_q8_0;                       /* 34 B  */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } cpvo_block_q4_K; /* 144 B */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } cpvo_block_q6_K; /* 210 B */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } cpvo_block_q8_K;      /* 292 B */
#pragma pack(pop)

/* ---- scalar helpers ---------------------------------------------------- */
uint16_t cpvo_fp32_to_fp16(float f);
float    cpvo_fp16_to_fp32(uint16_t h);
void     cpvo_fp32_to_fp16_n(const float* x, int64_t n, uint16_t* y);
void     cpvo_fp16_to_fp32_n(const uint16_t* x, int64_t n, float* y);
float    cpvo_expf(float x);
void     cpvo_expf_n(const float* x, int64_t n, float* y);
void     cpvo_exp_table(uint64_t out[32]);   /* the 2^(i/32) table cpvo_expf uses */
/* count x in [lo, hi] (as float bit patterns, stepping every `stride` values)
 * where cpvo_expf(x) != libm expf(x); returns the number of mismatches. */
int64_t  cpvo_expf_vs_libm(float lo, float hi, int64_t stride);

/* ---- RNGs --------------------------------------------------------------- */
void     cpvo_philox4x64(const uint64_t ctr[4], const uint64_t key[2], uint64_t out[4]);
float    cpvo_u01(uint64_t x);                       /* (x >> 40) / 2^24, as next_f32 */
/* u[b][j][r] = cpvo_u01(philox((b, j, r, round), (seed, 0))[0]) for j in [0,k], r in {0,1} */
void     cpvo_philox_uniforms(uint64_t seed, uint64_t round, int B, int k, float* u);
/* xoshiro256++ seeded by splitmix64 (crates/codpiece-sample/src/lib.rs:88-130) */
void     cpvo_rng_seed(uint64_t seed, uint64_t s[4]);
uint64_t cpvo_rng_next_u64(uint64_t s[4]);
float    cpvo_rng_next_f32(uint64_t s[4]);

/* ---- block formats ------------------------------------------------------ */
int64_t  cpvo_type_block(int type);                 /* elements per block */
int64_t  cpvo_type_size(int type);                  /* bytes per block   */
int64_t  cpvo_row_bytes(int type, int64_t k);       /* -1 if k not block-aligned */
int      cpvo_quantize(int type, const float* x, int64_t n, void* out);
int      cpvo_dequantize(int type, const void* q, int64_t n, float* y);
/* activation quantizers (ggml quantize_row_q8_0_ref / quantize_row_q8_K_ref) */
void     cpvo_quantize_q8_0(const float* x, int64_t n, cpvo_block_q8_0* y);
void     cpvo_quantize_q8_K(const float* x, int64_t n, cpvo_block_q8_K* y);

/* ---- GEMM --------------------------------------------------------------- */
/* Y[M][N] = X[M][K] . dequant(W[N][K])^T in ggml's mul_mat convention
 * (ne: [K,N] x [K,M] -> [N,M], crates/codpiece-ggml-sys/tests/smoke.rs:19).
 * W is N rows of ggml blocks.  Returns 0, or -1 for an unsupported type / K. */
int      cpvo_qgemm(int type, const void* w, int64_t N, int64_t K,
                    const float* x, int64_t M, float* y, int n_threads);
/* plain f32 mul_mat (smoke.rs known answer) */
void     cpvo_mul_mat_f32(const float* w, int64_t N, int64_t K, const float* x,
                          int64_t M, float* y);
/* f64 reference of the same product over dequantized operands (no rounding
 * beyond the quantizers) — used to bound the exact contract. */
int      cpvo_qgemm_f64(int type, const void* w, int64_t N, int64_t K,
                        const float* x, int64_t M, double* y, int n_threads);
/* window exponent helpers shared with the tests */
int      cpvo_qgemm_window(int type, int64_t K);

/* ---- glue ops ----------------------------------------------------------- */
void     cpvo_rms_norm(const float* x, int64_t n, float eps, const float* w, float* y);
/* cs[p][i][0..1] = (cos, sin) of pos p for pair i, ggml's theta recurrence */
void     cpvo_rope_table(int n_pos, int n_rot, float freq_base, float* cs);
/* the same with IMROPE's interleaved sections (positions (p, p, p, 0)) */
void     cpvo_rope_table_sections(int n_pos, int n_rot, float freq_base, const int32_t* sections,
                                  float* cs);
/* rotate one head vector of length hd in place (NEOX pairs over n_rot dims) */
void     cpvo_rope_neox(float* x, int n_rot, const float* cs_row);

/* masked GQA attention over an f16 cache.
 * q: [T][H][D] f32; kc, vc: [n_ctx][Hkv*D] f16; rows [0, n_past) are context,
 * rows n_past + t hold node t.  parent: [T] tree parents (-1 = root, i.e. a
 * child of the context), or NULL for a linear chain.  Node t sees all context
 * rows plus its ancestors and itself.  out: [T][H*D].
 * cpvo_attn is the exact-window contract (cpvo_glue.c), order-free;
 * cpvo_attn_f64 the same attention in binary64 (q rounded to f16), the
 * accuracy reference. */
#define CPVO_ATTN_CHUNK 128
#define CPVO_ATTN_PBITS 22   /* a row's weight e in (0, 1] as rint(e 2^22) */
#define CPVO_ATTN_VBITS 14   /* an f16 value v as rint(v 2^14): |vq| < 2^30 */
/* vq of an f16 cache value (f16_tab must be initialised: any cpvo_attn call does it) */
int64_t  cpvo_attn_vq(uint16_t h);
void     cpvo_attn(const float* q, const uint16_t* kc, const uint16_t* vc, int64_t n_past,
                   const int32_t* parent, int T, int H, int Hkv, int D, float scale,
                   float* out);
void     cpvo_attn_f64(const float* q, const uint16_t* kc, const uint16_t* vc, int64_t n_past,
                       const int32_t* parent, int T, int H, int Hkv, int D, float scale,
                       float* out);

/* ---- sampler (crates/codpiece-sample/src/lib.rs) ------------------------ */
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
} cpvo_sampler_params;

/* Sampler::distribution (lib.rs:184-187, build :229-376).  hist: the penalty
 * window, oldest first (already capped at penalty_last_n).  Writes the
 * candidate ids and probabilities in candidate order; tlogit (optional) gets
 * the tempered logits build() leaves behind.  Returns the candidate count. */
int      cpvo_distribution(const cpvo_sampler_params* p, const float* logits, int V,
                           const int32_t* hist, int n_hist,
                           int32_t* ids, float* probs, float* tlogit);
int32_t  cpvo_dist_draw(const int32_t* ids, const float* probs, int n, float r);
int32_t  cpvo_dist_draw_excluding(const int32_t* ids, const float* probs, int n,
                                  int32_t token, float r);
float    cpvo_dist_prob_of(const int32_t* ids, const float* probs, int n, int32_t token);
float    cpvo_dist_peak(const float* probs, int n);
int32_t  cpvo_sample_coupled(const cpvo_sampler_params* p, const float* logits, int V,
                             const int32_t* hist, int n_hist, const float* noise_t);
int32_t  cpvo_argmax(const float* x, int64_t n);
/* The draft gate of the engine's post-commit re-draft (crates/codpiece-server/
 * src/engine.rs:2598-2606) and of the CLI spec path (softmax_prob at the
 * argmax, crates/codpiece-cli/src/main.rs:946-954, 1066-1069): 1 / lse with
 * lse = sum over i, in index order, of exp(l_i - max) in f32 (max the f32::max
 * fold from -inf).  The caller compares it with p_min. */
float    cpvo_softmax_peak_seq(const float* l, int64_t n);

/* ---- acceptance (crates/codpiece-server/src/engine.rs:2326-2461) -------- */
enum { CPVO_ACCEPT_GREEDY = 0, CPVO_ACCEPT_REJECT = 1, CPVO_ACCEPT_GUMBEL = 2 };
/* p_logits [B][k+1][V]; q_logits [B][k][V] or NULL (point-mass drafts, the
 * reference rule); draft [B][k]; u [B][k+1][2] uniforms by role (r0 = accept
 * roll / bonus draw, r1 = residual draw); noise_t [B][k+1][V] (gumbel mode);
 * hist [B][hist_len] (oldest first, -1 = empty slot).  out_tok [B][k+1],
 * out_n [B] = number of accepted drafts; out_tok[b][0..out_n] are valid. */
int      cpvo_spec_accept(const float* p_logits, const float* q_logits, const int32_t* draft,
                          int B, int k, int V, const cpvo_sampler_params* p, int mode,
                          const float* u, const float* noise_t,
                          const int32_t* hist, int hist_len,
                          int32_t* out_tok, int32_t* out_n);
/* The engine loop verbatim for one sequence with the reference's sequential
 * RNG (point-mass drafts).  Records the uniform consumed for each role in
 * u_used [k+1][2] (NaN where none was drawn).  Returns n_accept. */
int      cpvo_spec_accept_rng(const float* p_logits, const int32_t* draft, int k, int V,
                              const cpvo_sampler_params* p, uint64_t rng[4],
                              const int32_t* hist, int n_hist,
                              int32_t* out_tok, float* u_used);

/* ---- model restatement (crates/codpiece-model/src/qwen35.rs) ------------ */
typedef struct {
    int32_t n_layer;
    int32_t n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab;
    int32_t n_rot;
    int32_t rope_sections[4];
    float   rms_eps, freq_base;
    int32_t has_mtp;
} cpvo_hparams;
typedef struct cpvo_model cpvo_model;
typedef struct cpvo_session cpvo_session;
cpvo_model*   cpvo_model_create(const cpvo_hparams* hp);
void          cpvo_model_free(cpvo_model* m);
/* tensors by GGUF name, ggml ne order (ne0 = row length, ne1 = rows) */
int           cpvo_model_set(cpvo_model* m, const char* name, int type, const void* data, int64_t ne0, int64_t ne1);
cpvo_session* cpvo_session_create(cpvo_model* m, int64_t n_ctx);
void          cpvo_session_free(cpvo_session* s);
void          cpvo_session_set_pos(cpvo_session* s, int64_t n_past, int64_t mtp_past);
/* Inject the attention outputs of another implementation (consecutive
 * [T][H][head_dim] f32 blocks, one per attention call, in call order): each
 * block() checks its own attention against the injected block and continues
 * with the injected values, so every op outside attention can be compared
 * exactly.  NULL turns it off.  inject_ratio = max |inj - ref| / (2e-5 +
 * 2e-4|ref|) seen since the last set (inf when the blocks ran out). */
void          cpvo_session_set_attn_inject(cpvo_session* s, const float* att, int64_t n_floats);
double        cpvo_session_inject_ratio(const cpvo_session* s);
void          cpvo_session_get_pos(const cpvo_session* s, int64_t* n_past, int64_t* mtp_past);
/* Planted mistakes, for tests that show the independent f64 forward catches a
 * wrong composition (0 = none, the faithful restatement):
 *   1 Q and the output gate swapped in their attn_q slots
 *   2 the sigmoid gate applied after wo instead of before it
 *   3 the MTP concat in the wrong order, [hnorm(h) ; enorm(e)]
 *   4 the MTP link hands on its hidden before shared_head_norm
 *   5 the post-attention norm dropped (the FFN reads the raw residual)
 *   6 enorm and hnorm weights swapped in the MTP concat */
void          cpvo_set_fault(int code);
/* The round's attention in binary64 (cpvo_attn_f64) instead of the chunked
 * contract, so that a composition check is not blurred by the contract's
 * f16 probabilities (0 = the contract, the default). */
void          cpvo_set_attn_f64(int on);
/* Every mul_mat of the round on the f32 activation rows as they are (no
 * activation quantization), summed in binary64: with cpvo_set_attn_f64 the
 * round becomes a smooth function of its inputs, for composition checks
 * against a float64 forward (0 = ggml's quantized activations, the default). */
void          cpvo_set_smooth(int on);
/* threads of the model round's GEMMs and attention (default 8) */
void          cpvo_set_threads(int n);
int           cpvo_prefill(cpvo_session* s, const int32_t* tok, int t);
/* step_fused_cached: preds [t], chain [depth][t], conf [depth][t] (nullable),
 * logits [t][V] and hidden [t][E] (nullable); noise [t][V] or NULL */
int           cpvo_verify_step(cpvo_session* s, const int32_t* tok, int t, int depth, const float* noise,
                               int32_t* preds, int32_t* chain, float* conf, float* logits, float* hidden);
int           cpvo_verify_step_cands(cpvo_session* s, const int32_t* tok, int t, int depth, const float* noise,
                                     const int32_t* cands, int n_cand, int32_t* preds, int32_t* chain, float* conf,
                                     float* logits_out, float* hidden_out);
/* Qwen35::mtp_draft (qwen35.rs:2086-2192), the graph of build_mtp_impl
 * (mtp_graph.rs:123-249): one draft link from the trunk's normed hidden row
 * `hidden` [E] and `token`, the token at the position after it, placed at rope
 * position `pos`: rms(embed(token)) * enorm ; rms(hidden) * hnorm, eh_proj,
 * the MTP layer's attention (its K/V written at MTP row mtp_past, attending
 * rows 0..mtp_past) and FFN, then rms with the head norm (hidden_out [E]) and
 * the draft head (logits_out [V]).  mtp_past advances by 1.  Returns -1 (and
 * does nothing) when the MTP cache is full or pos is past the rope table. */
int           cpvo_mtp_draft(cpvo_session* s, const float* hidden, int32_t token, int64_t pos, float* logits_out,
                             float* hidden_out);
/* cmd_fused: returns the number of committed tokens; stats = {accepted, proposed, rounds} */
int           cpvo_fused_generate(cpvo_session* s, const int32_t* prompt, int n_prompt, int n_gen, int depth,
                                  int tail, int bulk, int32_t* committed, int64_t* stats);

#ifdef __cplusplus
}
#endif
#endif
