/*
 * ne.h - C-ABI of the MI355X (gfx950) training_dynamic step: forward, backward, AdamW and
 * the KV-cached token loop, over device-resident weights.
 *
 * This library replaces the reference's ANE dispatch and staging layer and the CPU ops
 * between the ANE kernels.  Reference paths below are relative to the reference repo,
 * TD = ane-training/training/training_dynamic.  Conventions follow the reference's own
 * exported C-ABI precedent (ane-training/bridge/ane_bridge.h:15-94): an opaque handle,
 * NULL on create failure, int status (0 ok, negative error), caller-owned host buffers.
 *
 * Status codes: 0 success; -1 bad argument/shape; -2 bad state; -3 file I/O; -4 bad
 * checkpoint format; -5 out of memory; -1000-hipError_t for a HIP runtime error.
 * ne_last_error() gives a thread-local message for the last failure.  The library never
 * prints and never exits.
 *
 * Threading: one context per thread; each context owns one HIP stream.  Calls return after
 * their stream work completes, except ne_train_step (work may stay queued until the next
 * synchronising call: ne_sync, ne_get_tensor, ne_optimizer_step with gnorm_out, ...).
 */
#ifndef NE_H
#define NE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ne_ctx ne_ctx;

/* Model and step shape.  Replaces the compile-time model headers
 * TD/models/{stories110m,qwen3_06b,qwen3_06b_seq512}.h:6-19 (DIM, HIDDEN, HEADS, KV_HEADS,
 * HD, SEQ, NLAYERS, VOCAB) plus the values hardcoded in the reference: RoPE base 10000
 * (TD/cpu_ops.h:466), residual scale 1/sqrt(2*NLAYERS) (TD/train.m:181), eps 1e-5
 * (TD/cpu_ops.h:42).  qk_norm adds Qwen3's per-head RMSNorm on q and k (absent in the
 * reference). */
typedef struct ne_config {
  int32_t dim, hidden, n_heads, kv_heads, head_dim, n_layers, vocab;
  int32_t seq;          /* training sequence length S (multiple of 64) */
  int32_t batch;        /* training sequences per step B (T = B*S tokens) */
  int32_t qk_norm;      /* 0: reference (no QK-norm), 1: per-head QK-RMSNorm */
  float rope_theta;     /* reference: 10000 */
  float res_alpha;      /* residual branch scale; TD/train.m:181 uses 1/sqrt(2L), generate.py 1 */
  float norm_eps;       /* 1e-5 */
  int32_t decode_batch; /* max sequences of ne_decode (0: no decode buffers) */
  int32_t decode_ctx;   /* max prompt + generated tokens of ne_decode */
  int32_t dtype;        /* 16-bit format of activations and the weight shadow: NE_FP16 or NE_BF16 */
} ne_config;

/* 16-bit formats.  NE_FP16 (IEEE half: 10-bit mantissa, the reference's own ANE format) is
 * the training default; its backward runs at an internal power-of-two gradient scale with
 * overflow detection (see ne_optimizer_step).  NE_BF16 trades precision for range. */
enum { NE_BF16 = 0, NE_FP16 = 1 };

/* Counters of the v4 checkpoint header (TD/config.h:82-91 CkptHdr). */
typedef struct ne_train_state {
  int32_t step, total_steps;
  float lr, loss;
  double cum_compile, cum_train, cum_wall;
  int32_t cum_steps, cum_batches, adam_t;
} ne_train_state;

/* Tensor kinds for ne_set_tensor / ne_get_tensor. */
enum { NE_PARAM = 0, NE_GRAD = 1, NE_ADAM_M = 2, NE_ADAM_V = 3 };

/* ---------------------------------------------------------------- context ---- */

/* Allocate device-resident fp32 master weights, grads, Adam m/v, the 16-bit weight shadow and
 * all activation/workspace buffers.  Replaces ane_init (TD/config.h:99-107), the per-layer
 * host allocations (TD/config.h:110-176, TD/train.m:199-210), kernel compilation
 * (TD/train.m:25-94, TD/io.h:135-171) and IOSurface/request setup (TD/train.m:304-329).
 * Weights start at zero (gains at 1); load them with ne_set_tensor or ne_load_ckpt_v4. */
ne_ctx *ne_create(const ne_config *cfg);
/* Frees everything.  Replaces free_kern / free_per_layer (TD/io.h:172-181, 412-419). */
void ne_destroy(ne_ctx *ctx);
/* Thread-local message for the last failing call. */
const char *ne_last_error(void);
/* Wait for all queued work of the context. */
int ne_sync(ne_ctx *ctx);

/* Tensor ids follow the checkpoint order (TD/train.m:111-129): for layer l,
 * 9*l + {0:Wq[Q,D] 1:Wk[KV,D] 2:Wv[KV,D] 3:Wo[D,Q] 4:W1[H,D] 5:W2[D,H] 6:W3[H,D]
 * 7:rms_att[D] 8:rms_ffn[D]}; then 9L: rms_final[D]; 9L+1: embed[V,D]; with qk_norm,
 * 9L+2+2l: q_norm[HD] and 9L+3+2l: k_norm[HD]. */
int ne_num_tensors(const ne_ctx *ctx);
int64_t ne_tensor_numel(const ne_ctx *ctx, int tensor_id);
/* Copy fp32 host data in/out of one tensor (row-major, reference layout).  Setting a
 * parameter also refreshes its 16-bit shadow.  Replaces the per-layer stage_* / transpose
 * restaging of TD/io.h:263-409 and TD/train.m:261-274 (weights never leave the device
 * during training). */
int ne_set_tensor(ne_ctx *ctx, int kind, int tensor_id, const float *host, size_t n);
int ne_get_tensor(ne_ctx *ctx, int kind, int tensor_id, float *host, size_t n);

/* ------------------------------------------------------------ training step ---- */

/* One forward + backward over B sequences: tokens is [B, S+1] int32 (inputs [:, :S],
 * targets [:, 1:]).  Gradients (times loss_scale) ACCUMULATE into the context's grads.
 * loss_out (may be NULL; non-NULL synchronises) receives the mean token loss
 * -log(p_tgt + 1e-10).  Replaces the step body of TD/train.m:403-757: embed_lookup, the 28
 * sdpaFwd/ffnFused + 5 backward ANE evals per layer (TD/io.h:190-229), the CPU RMSNorm /
 * residual / RoPE / GQA ops, cross_entropy_loss (TD/cpu_ops.h:348-382), the dW sgemms and
 * embed_backward. */
int ne_train_step(ne_ctx *ctx, const int32_t *tokens, float loss_scale, float *loss_out);
/* Replay the step, and each position of ne_decode, from captured HIP graphs (default on;
 * the step's graph is used only while ne_overlap_weight_grads is off and per-kernel
 * profiling is disabled: the two-stream step runs faster from eager launches).  The step's graph is
 * captured on first use per (fresh accumulation, loss_scale, internal gradient scale), the
 * decode graphs per (batch size, greedy or sampling); they replace the reference's
 * per-kernel ANE dispatch (TD/io.h:190-229).  Off: every kernel is launched eagerly. */
int ne_use_graphs(ne_ctx *ctx, int on);
/* Run the step's weight-gradient GEMMs (and the embedding gradient of the classifier) on a
 * second HIP stream beside the chain of activation gradients, handed over once per layer
 * (default on; off: one stream, in order, replayed from a graph if ne_use_graphs is on).
 * Results are identical either way: every kernel writes its own outputs and the second
 * stream is joined before the gain-gradient sums and the embedding scatter.
 * Mirrors the reference's dW scheduling: its cblas weight-gradient sgemms are queued on a
 * concurrent dispatch queue beside the ANE backward evals (TD/train.m:377-378, 521, 554,
 * 588, 628) and awaited once before the update (TD/train.m:756).  The switch has no
 * counterpart there: it is for timing, and for checking that the two orders agree. */
int ne_overlap_weight_grads(ne_ctx *ctx, int on);

/* Which RMSNorm backward the step uses for the attention, FFN and final norms.  ref = 0
 * (default): the exact gradient of y = x*r*g, dx = r*g*dy - x*r^3*sum(dy*x*g)/D.  ref = 1:
 * the reference's formula, dx = (dy - x*r^2*sum(dy*x*g)/D)*r*g, as rmsnorm_bwd /
 * rmsnorm_bwd_add compute it (TD/cpu_ops.h:146-153, 188-189, 255-256; called from TD/train.m:527, 603, 751);
 * its projection term carries one more gain factor, so the two agree while the gains are
 * 1.0 and drift apart as they train.  For runs that must follow a reference run's trajectory.
 * The gain gradients are the same under both; the QK-norm backward (no counterpart in the
 * reference) stays exact. */
int ne_rmsnorm_bwd_formula(ne_ctx *ctx, int ref);

/* Scale grads by grad_scale, global L2 norm, clip to `clip` (if > 0), AdamW with
 * bias-corrected moments (t = ++adam_t), weight decay wd on matrices and the embedding
 * (0 on the RMSNorm / QK-norm gains), refresh the 16-bit shadow, zero the grads.  gnorm_out
 * (may be NULL) receives the pre-clip norm.  If any 16-bit value of the accumulated
 * micro-steps overflowed, the update is skipped (weights, moments and adam_t unchanged,
 * grads zeroed), the internal gradient scale is halved and 1 is returned; otherwise 0.
 * Synchronises.  Replaces TD/train.m:782-903 and adam_update (TD/cpu_ops.h:266-303). */
int ne_optimizer_step(ne_ctx *ctx, float lr, float b1, float b2, float eps, float wd,
                      float grad_scale, float clip, float *gnorm_out);
/* Zero all gradients.  Replaces layer_grads_zero (TD/config.h:164-170). */
int ne_zero_grads(ne_ctx *ctx);
/* Internal gradient scale of the 16-bit backward, the number of skipped (overflowed)
 * optimizer steps and, for the last skipped step, a bit mask of the conversion sites that
 * overflowed (bit i: 0 norm fwd, 1 qkv, 2 h1|h3, 3 swiglu gate, 4 dlogits, 5 norm bwd,
 * 6 dh1|dh3, 7 d(attn out), 8 dv, 9 dq|dk).  Any pointer may be NULL.  No reference
 * counterpart (the ANE path had a fixed loss scale 256, TD/train.m:180). */
int ne_grad_scale_info(const ne_ctx *ctx, float *scale, int32_t *skipped_steps,
                       int32_t *overflow_sites);
/* Norms of the gradient the last ne_optimizer_step used, before the clip and after its
 * grad_scale: out[0] the global norm, out[1] the attention matrices (Wq, Wk, Wv, Wo of every
 * layer), out[2] the FFN matrices (W1, W2, W3), out[3] the embedding; the gains count only
 * in out[0].  Valid until the next ne_train_step, ne_zero_grads or gradient write
 * (NE_ERR_STATE otherwise, and after a skipped step).  Replaces the attn_sq / ffn_sq /
 * embed_sq sums printed with the global norm (TD/train.m:786-830). */
int ne_grad_norm_parts(ne_ctx *ctx, float out[4]);
/* Range of the last ne_train_step's final hidden state x (the last layer's output, before the
 * final RMSNorm) and of the gradient dy of the loss times loss_scale with respect to the
 * first layer's input, in the reference's scale (d(mean loss * loss_scale)/dx):
 * out = {x_min, x_max, dy_min, dy_max}.  Synchronises.  Replaces the vDSP_minv / vDSP_maxv of
 * the step line (TD/train.m:770-777). */
int ne_step_stats(ne_ctx *ctx, float out[4]);
int ne_get_state(const ne_ctx *ctx, ne_train_state *st);
int ne_set_state(ne_ctx *ctx, const ne_train_state *st);

/* ------------------------------------------------------------- checkpoints ---- */

/* v4 checkpoint (TD/train.m:97-165, header TD/config.h:82-91): 96-byte header, per layer
 * Wq Wk Wv Wo W1 W2 W3 rms_att rms_ffn then their (m, v), rms_final+m+v, embed+m+v, all
 * fp32.  With qk_norm a trailer "QKN1" + per layer q_norm,m,v,k_norm,m,v follows (v4
 * readers stop before it).  Load checks magic, version, dims against the context and the
 * file size.  st may be NULL. */
int ne_load_ckpt_v4(ne_ctx *ctx, const char *path, ne_train_state *st);
int ne_save_ckpt_v4(ne_ctx *ctx, const char *path, const ne_train_state *st);

/* ------------------------------------------------------------- token loop ---- */

/* Vocabulary compaction (TD/cpu_ops.h:384-431; used at TD/train.m:286-292, 401, 497-523,
 * 802): the classifier and the softmax run over the embedding rows ids[0..cv) only (compact
 * id c stands for full id ids[c]); every target must be among them; the compact embedding
 * gradient is added back to its rows of the full one.  The reference builds ids from the
 * training data: the distinct ids in ascending order.  ids must be distinct and in
 * [0, vocab).  cv = 0 (ids NULL) restores the full vocabulary.  Call before a step that
 * starts an accumulation window (after ne_optimizer_step or ne_zero_grads); returns
 * NE_ERR_STATE otherwise. */
int ne_set_vocab_map(ne_ctx *ctx, const int32_t *ids, int cv);

/* KV-cached autoregressive generation (TD/tools/generate.py:113-228) for B sequences
 * sharing one prompt length P: prompt is [B, P] int32, out_tokens receives [B, n_new].
 * temperature < 1e-6 selects greedy argmax; otherwise softmax(logits/temperature), an
 * optional top-p mask (top_p < 1) and inverse-CDF sampling in vocabulary order with
 * uniforms[b*n_new + j] in [0,1) (the draw of numpy's RandomState.choice, generate.py:215).
 * Uses the 16-bit weight shadow with fp32 activations and an fp32 KV cache.  Requires
 * B <= decode_batch and P + n_new <= decode_ctx. */
int ne_decode(ne_ctx *ctx, const int32_t *prompt, int B, int P, int n_new, float temperature,
              float top_p, const double *uniforms, int32_t *out_tokens);
/* ne_decode with the sampling draws taken from a seed, as generate.py's --seed makes them
 * (np.random.seed(seed), then one np.random.choice per sampled token: generate.py:198-215,
 * 248-249): MT19937 seeded by the 32-bit integer seed (seed >= 2^32 is rejected, as numpy
 * rejects it), each draw the 53-bit double numpy's RandomState.random_sample returns.  With
 * B > 1 the draws go position by position, the sequences of a position in order.
 * temperature < 1e-6 is greedy and draws nothing. */
int ne_decode_seeded(ne_ctx *ctx, const int32_t *prompt, int B, int P, int n_new, float temperature,
                     float top_p, uint64_t seed, int32_t *out_tokens);
/* The first n draws of that generator: out[k] = RandomState(seed).random_sample() in order.
 * Host only (no device work). */
int ne_mt19937_uniforms(uint64_t seed, int64_t n, double *out);

/* ------------------------------------------------------------- profiling ---- */

/* Per-kernel-family HIP-event timing on the context's stream (off by default).
 * ne_prof_enable takes a bit mask of families (1 << NE_PROF_*; 0 disables); only the
 * selected families get an event pair around their launches. */
enum {
  NE_PROF_GEMM_FWD = 0, NE_PROF_GEMM_BWD, NE_PROF_ATTN_FWD, NE_PROF_ATTN_BWD, NE_PROF_NORM,
  NE_PROF_CE, NE_PROF_ADAM, NE_PROF_GNORM, NE_PROF_EMBED, NE_PROF_DECODE, NE_PROF_COUNT
};
int ne_prof_enable(ne_ctx *ctx, int mask);
int ne_prof_reset(ne_ctx *ctx);
/* Total milliseconds and launch count of one family since the last reset (synchronises). */
int ne_prof_get(ne_ctx *ctx, int family, double *ms, int64_t *count);

/* Phase timeline of the training step (off by default).  While on, ne_train_step and
 * ne_optimizer_step record HIP timing events at their phase boundaries without changing
 * the schedule (the two-stream step stays two-stream; the single-stream step launches
 * eagerly instead of from its graph).  ne_step_timeline (synchronises) returns the last
 * step's phases in milliseconds of GPU time on the step stream: out[NE_TL_WAIT] the wait for
 * the previous update before the embedding lookup, NE_TL_FWD the forward through the final
 * RMSNorm, NE_TL_CLS the classifier and cross-entropy forward and backward through the
 * final RMSNorm's backward, NE_TL_BWD the layers' backward chain, NE_TL_DWAIT the wait for
 * the weight-gradient stream, NE_TL_TAIL the gain sums and embedding scatter, NE_TL_STEP
 * first to last event; for the last optimizer call NE_TL_OPT the norm and clip on the step
 * stream and NE_TL_UPDATE the AdamW pass, first launch to last (NaN if none was recorded).
 * layer_fwd / layer_bwd (may be NULL) receive n_layers times each.  Replaces the per-phase
 * timers of the step line (TD/train.m:763-767). */
enum {
  NE_TL_WAIT = 0, NE_TL_FWD, NE_TL_CLS, NE_TL_BWD, NE_TL_DWAIT, NE_TL_TAIL, NE_TL_STEP, NE_TL_OPT,
  NE_TL_UPDATE, NE_TL_COUNT
};
int ne_timeline(ne_ctx *ctx, int on);
int ne_step_timeline(ne_ctx *ctx, float out[NE_TL_COUNT], float *layer_fwd, float *layer_bwd);
/* Launches of the AdamW pass that a training step runs beside its forward after an optimizer
 * step on two streams: the gains, one per layer, then the embedding's rows in the classifier's
 * vocabulary pieces (a measurement aid for the pass's per-launch roofline; the reference's
 * update, TD/train.m:861-897, is one CPU loop over the tensors).  Negative for a NULL ctx. */
int ne_update_launches(const ne_ctx *ctx);

/* ------------------------------------------------------ kernel-level entry points ---- */
/* Device-pointer entry points of the individual kernels, for testing and for callers
 * composing their own step.  16-bit buffers hold NE_FP16 or NE_BF16 bit patterns as
 * selected by dtype.  stream: a hipStream_t or NULL.  They launch asynchronously and return
 * the launch status. */

/* y[T,D] 16-bit = x*r*g, r[T] = (mean(x^2)+eps)^-1/2.  TD/cpu_ops.h:20-60 rmsnorm. */
int ne_k_rmsnorm_fwd(int dtype, const float *x, const float *g, void *y, float *r, int T, int D,
                     float eps, void *stream);
/* Exact RMSNorm backward + residual (may be NULL); dg += dg_scale * sum_t dy*x*r; dxb (may
 * be NULL) receives 16-bit(bscale*dx).  TD/cpu_ops.h:108-261 rmsnorm_bwd(_add). */
int ne_k_rmsnorm_bwd(int dtype, const float *dy, const float *x, const float *g, const float *r,
                     const float *resid, float *dx, void *dxb, float bscale, float *dg,
                     float dg_scale, int T, int D, void *stream);
/* C = epi(alpha * A.B) on 16-bit MFMA.  layout 0: A[M,K] B[N,K] (forward, weights [out,in]);
 * 2: A[M,K] B[K,N] (input gradient); 3: A[K,M] B[K,N] (weight gradient).  epi 0: C 16-bit,
 * 1: C fp32, 2: C fp32 +=, 3: C fp32 = R fp32 + result, 4: SwiGLU backward (result =
 * dgate, R = h13 16-bit [M,2N], C = dh13 16-bit [M,2N]), 7: SwiGLU forward (layout 0, B =
 * [W1;W3] [N,K]: C = h13 16-bit [M,N] and R, written here, = gate silu(h1)*h3 16-bit [M,N/2];
 * N a multiple of 128).  M, N, K multiples of 64.
 * Replaces the matmuls of TD/mil_dynamic.h:14-35, 57-234, 238-306, 320-576 and the
 * cblas_sgemm calls of TD/train.m:500-524, 554-738. */
int ne_k_gemm(int dtype, int layout, int epi, int M, int N, int K, const void *A, int64_t lda,
              const void *B, int64_t ldb, void *C, int64_t ldc, const void *R, int64_t ldr,
              float alpha, void *stream);
/* The weight-gradient GEMMs of one layer as one launch: C_p[M_p,N_p] fp32 (= or, with
 * accumulate, +=) alpha * A_p^T.B_p for p < n (n <= 4), A_p[K,M_p] (row pitch lda[p]) and
 * B_p[K,N_p] (ldb[p]) 16-bit, on 256x256 tiles each over the whole K range (no split-K).  Only
 * for shapes the step runs this way: every M_p and N_p a multiple of 256, K >= 8192 and a
 * multiple of 64, at least 192 tiles in all (else NE_ERR_ARG).  Replaces the per-layer
 * cblas_sgemm weight gradients of TD/train.m:554-738 that the reference runs on its
 * concurrent dispatch queue. */
int ne_k_gemm_wgrad_group(int dtype, int n, const int *M, const int *N, int K, const void *const *A,
                          const int64_t *lda, const void *const *B, const int64_t *ldb, float *const *C,
                          int accumulate, float alpha, void *stream);
/* Per-head QK-RMSNorm (gq/gk NULL: off) + interleaved RoPE of the q and k column blocks of
 * qkv [T, ld] at positions t % S with fp32 tables cos/sin [S, HD/2]; writes qr, kr and the
 * norm factors rq [T,NH], rk [T,NKV].  TD/mil_dynamic.h:133-169. */
int ne_k_qk_prep_fwd(int dtype, const void *qkv, int64_t ld, const float *cosb,
                     const float *sinb, const float *gq, const float *gk, void *qr, void *kr,
                     float *rq, float *rk, int T, int S, int NH, int NKV, int HD, float eps,
                     void *stream);
/* Backward of ne_k_qk_prep_fwd: dq [T,NH*HD], dk [T,NKV*HD] fp32 -> q/k column blocks of
 * dqkv; gain grads (times dg_scale) accumulate into dgq/dgk.  TD/cpu_ops.h:510-537. */
int ne_k_qk_prep_bwd(int dtype, const float *dq, const float *dk, const void *qkv, int64_t ld,
                     const float *cosb, const float *sinb, const float *gq, const float *gk,
                     const float *rq, const float *rk, void *dqkv, float *dgq, float *dgk,
                     float dg_scale, int T, int S, int NH, int NKV, int HD, void *stream);
/* Causal GQA flash attention forward: o [T,NH*HD] and lse [T,NH] fp32 (natural log of the
 * row sum of exp(scale*q.k)).  Rows are t = b*S + s.  TD/mil_dynamic.h:171-223. */
int ne_k_attn_fwd(int dtype, const void *q, int64_t ldq, const void *k, int64_t ldk,
                  const void *v, int64_t ldv, void *o, int64_t ldo, float *lse, int B, int S,
                  int NH, int NKV, int HD, float scale, void *stream);
/* Backward: dq [T,NH*HD] fp32, dk [T,NKV*HD] fp32, dv 16-bit (GQA-reduced); delta [T,NH] is
 * scratch.  TD/mil_dynamic.h:583-707, TD/cpu_ops.h:585-605. */
int ne_k_attn_bwd(int dtype, const void *q, int64_t ldq, const void *k, int64_t ldk,
                  const void *v, int64_t ldv, const void *o, int64_t ldo, const float *lse,
                  const void *dout, int64_t lddo, float *delta, float *dq, int64_t lddq,
                  float *dk, int64_t lddk, void *dv, int64_t lddv, int B, int S, int NH, int NKV,
                  int HD, float scale, void *stream);
/* ne_k_attn_bwd without the delta argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops): it allocates nothing on any call.  No
 * counterpart in the reference.  Its delta scratch [B*S, NH] lives in a fixed device array
 * of 2^20 floats (4 MiB per GPU, held until the process ends): B*S*NH above 2^20 is rejected
 * with NE_ERR_ARG.  Every call on a GPU shares that GPU's array, so calls that overlap on one
 * GPU (other streams, other threads) race; calls ordered on one stream do not. */
int ne_k_attn_bwd_noalloc(int dtype, const void *q, int64_t ldq, const void *k, int64_t ldk,
                          const void *v, int64_t ldv, const void *o, int64_t ldo, const float *lse,
                          const void *dout, int64_t lddo, float *dq, int64_t lddq, float *dk,
                          int64_t lddk, void *dv, int64_t lddv, int B, int S, int NH, int NKV,
                          int HD, float scale, void *stream);
/* Fused LM-head + softmax cross-entropy (TD/train.m:493-524, TD/cpu_ops.h:348-382):
 * logits = x[T,D] . E[V,D]^T are produced tile by tile and never stored.  Forward writes
 * lse[T] and loss[0] = mean(-log(p_tgt + 1e-10)); part is scratch [T, V/64*2] floats
 * and tgt_logit/loss_rows scratch [T]. */
int ne_k_ce_fwd(int dtype, const void *x, const void *E, const int32_t *targets, int T, int D,
                int V, float *part, float *tgt_logit, float *lse, float *loss_rows, float *loss,
                void *stream);
/* Backward: dlogits 16-bit [T,V] = (softmax - onehot) * scale, recomputing the logits. */
int ne_k_ce_bwd(int dtype, const void *x, const void *E, const int32_t *targets,
                const float *lse, int T, int D, int V, float scale, void *dlogits, void *stream);
/* Forward and backward in one call, as the reference's cross_entropy_loss computes the loss
 * and dlogits together (TD/cpu_ops.h:348-382): ne_k_ce_fwd's outputs, and dlogits as
 * ne_k_ce_bwd defines it, without a second logits GEMM: the GEMM's epilogue stores each
 * logit as the 16-bit exp(logit - the max of its column tile) into dlogits, which one
 * streaming pass turns into (softmax - onehot) * scale once the rows' log-sum-exp is known
 * (the target's probability from its fp32 logit).  dlogits: 16-byte aligned [T, V]. */
int ne_k_ce_fwd_grad(int dtype, const void *x, const void *E, const int32_t *targets, int T, int D,
                     int V, float *part, float *tgt_logit, float *lse, float *loss_rows,
                     float *loss, float scale, void *dlogits, void *stream);
/* In-place AdamW over n fp32 elements; elements [0, n_decay) get weight decay.  The grad is
 * multiplied by *gscale (device scalar).  pb (may be NULL) receives the 16-bit weights; the
 * grad is zeroed when zero_grad.  TD/cpu_ops.h:266-303. */
int ne_k_adam(int dtype, float *p, float *g, float *m, float *v, void *pb, int64_t n,
              int64_t n_decay, float lr, float b1, float b2, float eps, float wd, int t,
              const float *gscale, int zero_grad, void *stream);
/* Global grad norm and clip factor: gscale[0] = grad_scale * min(1, clip/norm),
 * gnorm[0] = grad_scale * ||g||.  partials: scratch of 1024 doubles.  TD/train.m:785-849. */
int ne_k_grad_norm(const float *g, int64_t n, float grad_scale, float clip, double *partials,
                   float *gscale, float *gnorm, void *stream);
/* x[T,D] fp32 = E[tok[t]] (TD/cpu_ops.h:433-439); gE[tok[t]] += scale*dx[t]
 * (TD/cpu_ops.h:441-447). */
int ne_k_embed_fwd(const float *E, const int32_t *tok, float *x, int T, int D, void *stream);
int ne_k_embed_bwd(float *gE, const int32_t *tok, const float *dx, float scale, int T, int D,
                   void *stream);
/* gate[T,H] = silu(h1)*h3 with h13 = [h1 | h3] rows [T,2H] (TD/mil_dynamic.h:276-281). */
int ne_k_swiglu_fwd(int dtype, const void *h13, void *gate, int T, int H, void *stream);
/* MFMA issue ceiling, a measurement kernel with no counterpart in the reference (its
 * roofline figures are quoted against it next to the datasheet peak): `blocks` work-groups
 * of 4 waves, each wave running 8 independent accumulator chains of `iters` MFMAs of the
 * 16-bit format with no memory traffic in the loop; shape 0 = 32x32x16, 1 = 16x16x32.
 * out: blocks*256 floats (written so the work is kept).  Flops per launch:
 * blocks * 4 * 8 * iters * (2*32*32*16 or 2*16*16*32). */
int ne_k_mfma_ceiling(int dtype, int shape, int blocks, int iters, float *out, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* NE_H */
