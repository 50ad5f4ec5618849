/*
 * train.c - the `train` command line of the training_dynamic step over the MI355X C-ABI
 * (include/ne.h).  Drop-in for the reference's TD/train.m main (TD = ane-training/training/
 * training_dynamic): the same build (`make train MODEL=<models/NAME.h>`), the same flags
 * (TD/train.m:184-195), the same hyperparameter defaults (TD/train.m:173-183), the same data
 * sampling (TD/train.m:389-398), loss scale, gradient accumulation, clip, warmup + cosine LR
 * and AdamW cadence (TD/train.m:782-903), the same checkpoint file and save rule
 * (TD/train.m:97-165, 907-915) and the same stdout lines that TR/dashboard.py parses.
 *
 * As in the reference, the classifier and the softmax cover only the token ids present in the
 * data file (vocabulary compaction, TD/cpu_ops.h:384-431, TD/train.m:286-292).
 *
 * Differences, all on purpose: weights, gradients and Adam state live on the GPU and never
 * cross to the host during training; the RMSNorm backward is the exact gradient
 * (--rmsnorm-bwd-ref selects the reference's formula, TD/cpu_ops.h:146-153, 188-189, 255-256,
 * for runs that must follow a reference run).
 * Extensions: --full-vocab runs the full-vocabulary softmax instead of the compaction,
 * --tokens32 reads int32 token ids (uint16 cannot hold Qwen3's vocabulary), --qk-norm and
 * --rope-theta select Qwen3's per-head QK-RMSNorm and RoPE base, --ckpt overrides the
 * checkpoint path, --bf16 selects bf16 instead of fp16 activations.
 */
#define _DEFAULT_SOURCE
#include <fcntl.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

#include "ne.h"

/* the model header comes after ne.h: its macros (DIM, HD, ...) would rename ne.h's
 * parameter names */
#ifndef MODEL_HEADER
#error "no model selected: build with make train MODEL=<name of a header in models/>"
#endif
#include MODEL_HEADER

#define Q_DIM (HEADS * HD)
#define KV_DIM (KV_HEADS * HD)

static double now_ms(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec * 1e3 + ts.tv_nsec * 1e-6;
}

static int fail(const char *what, int rc) {
  printf("ERROR: %s failed (%d): %s\n", what, rc, ne_last_error());
  return 1;
}

/* Uniform +-scale init of TD/train.m:236-251 from srand48(42), in the same draw order
 * (per layer Wq Wk Wv Wo W1 W2 W3, then the embedding), uploaded tensor by tensor.  Each
 * element is rounded once, as there: the float scale times the double draw is formed in
 * double, then stored as float (the scale products scale_qd*res_scale and scale_d*res_scale
 * are float products, evaluated first). */
static int init_scratch(ne_ctx *ctx) {
  const float scale_d = 1.0f / sqrtf(DIM), scale_qd = 1.0f / sqrtf(Q_DIM), scale_h = 1.0f / sqrtf(HIDDEN);
  const float res_scale = 1.0f / sqrtf(2.0f * NLAYERS);
  const size_t sz[7] = {(size_t)Q_DIM * DIM, (size_t)KV_DIM * DIM, (size_t)KV_DIM * DIM, (size_t)DIM * Q_DIM,
                        (size_t)HIDDEN * DIM, (size_t)DIM * HIDDEN, (size_t)HIDDEN * DIM};
  const float sc[7] = {scale_d, scale_d, scale_d, scale_qd * res_scale, scale_h, scale_d * res_scale, scale_h};
  float *buf = malloc((size_t)VOCAB * DIM * sizeof(float));
  if (!buf) return -5; /* out of memory */
  int rc = 0;
  srand48(42);
  for (int L = 0; L < NLAYERS && !rc; L++)
    for (int j = 0; j < 7 && !rc; j++) {
      for (size_t i = 0; i < sz[j]; i++) buf[i] = (float)(sc[j] * (2 * drand48() - 1));
      rc = ne_set_tensor(ctx, NE_PARAM, 9 * L + j, buf, sz[j]);
    }
  for (size_t i = 0; i < (size_t)VOCAB * DIM && !rc; i++) buf[i] = (float)(0.02f * (2 * drand48() - 1));
  if (!rc) rc = ne_set_tensor(ctx, NE_PARAM, 9 * NLAYERS + 1, buf, (size_t)VOCAB * DIM);
  free(buf);
  return rc; /* RMSNorm (and QK-norm) gains start at 1 in a new context */
}

int main(int argc, char *argv[]) {
  setbuf(stdout, NULL);
  int total_steps = 10000;
  float max_lr = 3e-4f;
  const float adam_b1 = 0.9f, adam_b2 = 0.95f, adam_eps = 1e-8f, wd = 0.1f;
  int start_step = 0;
  int accum_steps = 10;
  int warmup_steps = 100;
  float grad_clip = 1.0f;
  const float loss_scale = 256.0f;
  const float res_alpha = 1.0f / sqrtf(2.0f * NLAYERS);
  const float min_lr_frac = 0.1f;
  int do_resume = 0, from_scratch = 0, tokens32 = 0, qk_norm = QK_NORM, bf16 = 0, full_vocab = 0, norm_ref = 0;
  float rope_theta = ROPE_THETA;
  const char *data_path = DEFAULT_DATA_PATH;
  const char *ckpt_path = CKPT_PATH;
  for (int i = 1; i < argc; i++) {
    if (strcmp(argv[i], "--resume") == 0) do_resume = 1;
    else if (strcmp(argv[i], "--scratch") == 0) from_scratch = 1;
    else if (strcmp(argv[i], "--steps") == 0 && i + 1 < argc) total_steps = atoi(argv[++i]);
    else if (strcmp(argv[i], "--lr") == 0 && i + 1 < argc) max_lr = (float)atof(argv[++i]);
    else if (strcmp(argv[i], "--accum") == 0 && i + 1 < argc) accum_steps = atoi(argv[++i]);
    else if (strcmp(argv[i], "--warmup") == 0 && i + 1 < argc) warmup_steps = atoi(argv[++i]);
    else if (strcmp(argv[i], "--clip") == 0 && i + 1 < argc) grad_clip = (float)atof(argv[++i]);
    else if (strcmp(argv[i], "--data") == 0 && i + 1 < argc) data_path = argv[++i];
    else if (strcmp(argv[i], "--ckpt") == 0 && i + 1 < argc) ckpt_path = argv[++i];
    else if (strcmp(argv[i], "--rope-theta") == 0 && i + 1 < argc) rope_theta = (float)atof(argv[++i]);
    else if (strcmp(argv[i], "--qk-norm") == 0) qk_norm = 1;
    else if (strcmp(argv[i], "--tokens32") == 0) tokens32 = 1;
    else if (strcmp(argv[i], "--bf16") == 0) bf16 = 1;
    else if (strcmp(argv[i], "--full-vocab") == 0) full_vocab = 1;
    else if (strcmp(argv[i], "--rmsnorm-bwd-ref") == 0) norm_ref = 1;
  }
  if (accum_steps < 1) accum_steps = 1;
  float lr = max_lr;

  ne_config cfg;
  memset(&cfg, 0, sizeof cfg);
  cfg.dim = DIM; cfg.hidden = HIDDEN; cfg.n_heads = HEADS; cfg.kv_heads = KV_HEADS; cfg.head_dim = HD;
  cfg.n_layers = NLAYERS; cfg.vocab = VOCAB; cfg.seq = SEQ; cfg.batch = 1; cfg.qk_norm = qk_norm;
  cfg.rope_theta = rope_theta; cfg.res_alpha = res_alpha; cfg.norm_eps = 1e-5f;
  cfg.dtype = bf16 ? NE_BF16 : NE_FP16;
  const double t_create = now_ms();
  ne_ctx *ctx = ne_create(&cfg);
  if (!ctx) {
    printf("ERROR: ne_create: %s\n", ne_last_error());
    return 1;
  }
  if (norm_ref && ne_rmsnorm_bwd_formula(ctx, 1) != 0) {
    printf("ERROR: ne_rmsnorm_bwd_formula: %s\n", ne_last_error());
    ne_destroy(ctx);
    return 1;
  }
  const double create_ms = now_ms() - t_create;

  double cum_train = 0, cum_wall = 0;
  int cum_steps = 0;
  float resume_loss = 0;
  int resuming = 0;
  if (do_resume) {
    ne_train_state st;
    if (ne_load_ckpt_v4(ctx, ckpt_path, &st) == 0) {
      resuming = 1;
      start_step = st.step; total_steps = st.total_steps; lr = st.lr; resume_loss = st.loss;
      cum_train = st.cum_train; cum_wall = st.cum_wall; cum_steps = st.cum_steps;
      printf("[RESUMED step %d, loss=%.4f]\n", start_step, resume_loss);
    }
  }
  if (!resuming) {
    printf("=== ANE Dynamic Training: %s (%d layers, GQA %d/%d heads) ===\n", MODEL_NAME, NLAYERS, HEADS, KV_HEADS);
    printf("dim=%d q_dim=%d kv_dim=%d hd=%d hidden=%d seq=%d vocab=%d\n", DIM, Q_DIM, KV_DIM, HD, HIDDEN, SEQ, VOCAB);
    const double lw = (double)Q_DIM * DIM + 2.0 * KV_DIM * DIM + (double)DIM * Q_DIM + 3.0 * HIDDEN * DIM;
    const double xformer_m = NLAYERS * (lw + 2.0 * DIM) / 1e6, embed_m = (double)VOCAB * DIM / 1e6;
    printf("Params: %.1fM (transformer %.1fM + embed %.1fM)\n", xformer_m + embed_m, xformer_m, embed_m);
    printf("Kernels: HIP gfx950 (MFMA GEMM, flash attention, RMSNorm, fused CE, AdamW), device-resident weights\n");
    printf("Accum %d steps, LR=%g\n", accum_steps, max_lr);
    const double fwd_flops = 2.0 * NLAYERS * lw * SEQ;
    printf("FLOPs/step: fwd=%.1fM total=%.1fM\n", fwd_flops / 1e6, 3.0 * fwd_flops / 1e6);
    if (from_scratch) {
      printf("  Training from scratch (random init)\n");
      int rc = init_scratch(ctx);
      if (rc) {
        ne_destroy(ctx);
        return fail("init", rc);
      }
    } else {
      printf("  ERROR: no checkpoint to resume (%s). Use --scratch.\n", ckpt_path);
      ne_destroy(ctx);
      return 1;
    }
  }

  /* token data: uint16 ids (TD/train.m:281-283), or int32 ids with --tokens32 */
  int fd = open(data_path, O_RDONLY);
  if (fd < 0) {
    printf("Cannot open %s\n", data_path);
    ne_destroy(ctx);
    return 1;
  }
  struct stat sb;
  fstat(fd, &sb);
  const size_t data_len = (size_t)sb.st_size;
  void *data = mmap(NULL, data_len, PROT_READ, MAP_PRIVATE, fd, 0);
  if (data == MAP_FAILED) {
    printf("mmap failed\n");
    close(fd);
    ne_destroy(ctx);
    return 1;
  }
  const size_t n_tokens = data_len / (tokens32 ? 4 : 2);
  printf("Token data: %zu tokens (%.1f MB)\n", n_tokens, data_len / 1e6);
  if (n_tokens < (size_t)SEQ + 2) {
    printf("Token data too short for seq %d\n", SEQ);
    munmap(data, data_len);
    close(fd);
    ne_destroy(ctx);
    return 1;
  }
  if (full_vocab) {
    printf("Vocab: full %d-way softmax (no compaction)\n", VOCAB);
  } else {
    /* vocab_map_build (TD/cpu_ops.h:391-414): the distinct ids in ascending order */
    unsigned char *used = (unsigned char *)calloc(VOCAB, 1);
    int32_t *ids = (int32_t *)malloc(sizeof(int32_t) * VOCAB);
    int cv = 0, bad = 0;
    for (size_t i = 0; i < n_tokens; i++) {
      const int64_t t = tokens32 ? ((const int32_t *)data)[i] : ((const uint16_t *)data)[i];
      if (t < 0 || t >= VOCAB) bad = 1;
      else used[t] = 1;
    }
    for (int v = 0; v < VOCAB; v++)
      if (used[v]) ids[cv++] = v;
    const int vrc = bad ? -1 : ne_set_vocab_map(ctx, ids, cv);
    free(used);
    free(ids);
    if (bad || vrc) {
      if (bad) printf("Token data holds ids outside [0, %d)\n", VOCAB);
      else printf("ERROR: ne_set_vocab_map: %s\n", ne_last_error());
      munmap(data, data_len);
      close(fd);
      ne_destroy(ctx);
      return 1;
    }
    printf("Vocab compaction: %d \u2192 %d active tokens (%.1fx reduction)\n", VOCAB, cv, (float)VOCAB / cv);
  }
  /* TD/train.m:302 (read by TR/dashboard.py's RE_COMPILED): nothing is compiled at run time
   * here, the gfx950 code objects are prebuilt into the library; the time is context creation */
  printf("Compiled 0 kernels in %.0fms (gfx950 code prebuilt; context created)\n\n", create_ms);
  /* phase timing of the printed steps (HIP events; the schedule is unchanged) */
  int rc = 0;
  if ((rc = ne_timeline(ctx, 1))) {
    fail("ne_timeline", rc);
    munmap(data, data_len);
    close(fd);
    ne_destroy(ctx);
    return 1;
  }

  int32_t tok[SEQ + 1];
  float last_loss = 999.0f;
  float best_loss = resume_loss > 0 ? resume_loss : 999.0f;
  double total_train_ms = 0;
  int total_steps_done = 0;
  const double t_wall_start = now_ms();
  srand48(42 + start_step);

  for (int step = start_step; step < total_steps; step++) {
    const double t_step = now_ms();
    /* TD/train.m:392-398: a random window of SEQ+1 ids */
    const size_t max_pos = n_tokens - SEQ - 1;
    const size_t pos = (size_t)(drand48() * max_pos);
    for (int t = 0; t <= SEQ; t++)
      tok[t] = tokens32 ? ((const int32_t *)data)[pos + t] : (int32_t)((const uint16_t *)data)[pos + t];
    const int adam_now = (step + 1) % accum_steps == 0 || step == total_steps - 1;
    const int print_now = step % 10 == 0 || step == start_step;
    const int ckpt_now = adam_now && (step + 1) % 100 == 0;
    float loss = NAN;
    /* the loss is read back (a synchronising copy) only when a line or a checkpoint needs it */
    if ((rc = ne_train_step(ctx, tok, loss_scale, (print_now || ckpt_now) ? &loss : NULL))) {
      fail("ne_train_step", rc);
      break;
    }
    if (print_now || ckpt_now) last_loss = loss;
    if (!adam_now) ne_sync(ctx);
    double step_ms = now_ms() - t_step;
    /* TD/train.m:763-778: timing, then the step line with the range of the final hidden state
     * and of the input gradient, printed before the update (the time excludes it) */
    if (print_now) {
      float xs[4] = {0.f, 0.f, 0.f, 0.f};
      if ((rc = ne_step_stats(ctx, xs))) {
        fail("ne_step_stats", rc);
        break;
      }
      /* TD/train.m:764-767.  GPU time of the step's phases on its stream: ane_fwd the forward
       * chain, io_fwd the wait for the previous update's share that the forward reads first
       * (the device counterpart of restaging weights), ane_bwd the backward chain, cls the
       * classifier and cross-entropy, dwait the wait for the weight-gradient stream; RMSNorm,
       * residual, GQA and RoPE run inside those chains (fused kernels, no separate phase) and
       * nothing is copied for the weight gradients, so rms, io_bwd, rms_bwd, resid, gqa, rope
       * and dw read 0; gap is the rest of the step's wall time (gain sums, embedding scatter,
       * host). */
      float ph[NE_TL_COUNT];
      if ((rc = ne_step_timeline(ctx, ph, NULL, NULL))) {
        fail("ne_step_timeline", rc);
        break;
      }
      const double timed = ph[NE_TL_FWD] + ph[NE_TL_WAIT] + ph[NE_TL_BWD] + ph[NE_TL_CLS] + ph[NE_TL_DWAIT];
      printf("  timing: ane_fwd=%.1f io_fwd=%.1f rms=%.1f ane_bwd=%.1f io_bwd=%.1f rms_bwd=%.1f cls=%.1f dw=%.1f "
             "dwait=%.1f resid=%.1f gqa=%.1f rope=%.1f [gap=%.1f]\n",
             ph[NE_TL_FWD], ph[NE_TL_WAIT], 0.0, ph[NE_TL_BWD], 0.0, 0.0, ph[NE_TL_CLS], 0.0, ph[NE_TL_DWAIT], 0.0, 0.0,
             0.0, step_ms - timed);
      printf("step %-4d loss=%.4f  lr=%.2e  %.1fms/step  x[%.2f,%.2f] dy[%.3e,%.3e]\n", step, loss, lr, step_ms,
             xs[0], xs[1], xs[2], xs[3]);
    }

    if (adam_now) {
      const double t_adam = now_ms();
      const float gsc = 1.0f / (accum_steps * loss_scale);
      /* TD/train.m:851-858 */
      if (step < warmup_steps) {
        lr = max_lr * ((float)(step + 1)) / warmup_steps;
      } else {
        const float decay_ratio = (float)(step - warmup_steps) / (float)(total_steps - warmup_steps);
        const float min_lr = max_lr * min_lr_frac;
        lr = min_lr + 0.5f * (1.0f + cosf((float)M_PI * decay_ratio)) * (max_lr - min_lr);
      }
      float gnorm = 0.f;
      const int orc = ne_optimizer_step(ctx, lr, adam_b1, adam_b2, adam_eps, wd, gsc, grad_clip, &gnorm);
      if (orc < 0) {
        rc = orc;
        fail("ne_optimizer_step", rc);
        break;
      }
      if (orc == 1) {
        float gs = 0.f;
        ne_grad_scale_info(ctx, &gs, NULL, NULL);
        printf("  [adam] step %d skipped: 16-bit gradient overflow, internal scale now %g\n", step, gs);
      } else if ((step + 1) % 10 == 0) {
        float gp[4] = {gnorm, 0.f, 0.f, 0.f};
        if ((rc = ne_grad_norm_parts(ctx, gp))) {
          fail("ne_grad_norm_parts", rc);
          break;
        }
        printf("  grad_norm=%.4f  attn=%.4f ffn=%.4f embed=%.4f\n", gnorm, gp[1], gp[2], gp[3]);
      }
      const double adam_ms = now_ms() - t_adam;
      printf("  [adam] step %d: %.1fms (update+zero)\n", step, adam_ms);
      if (ckpt_now && last_loss < best_loss) {
        best_loss = last_loss;
        const double wall = now_ms() - t_wall_start;
        ne_train_state st;
        ne_get_state(ctx, &st);
        st.step = step + 1;
        st.total_steps = total_steps;
        st.lr = lr;
        st.loss = last_loss;
        st.cum_compile = 0;
        st.cum_train = total_train_ms + step_ms + cum_train;
        st.cum_wall = wall + cum_wall;
        st.cum_steps = total_steps_done + 1 + cum_steps;
        if ((rc = ne_save_ckpt_v4(ctx, ckpt_path, &st))) {
          fail("ne_save_ckpt_v4", rc);
          break;
        }
        printf("  [ckpt saved, best_loss=%.4f]\n", best_loss);
      }
    }
    total_train_ms += step_ms;
    total_steps_done++;
  }

  const double wall = now_ms() - t_wall_start;
  printf("\n=== Efficiency Report ===\n");
  printf("Total steps:  %d\n", total_steps_done);
  printf("Compile:      %.0fms (one-time, %.1f%%)\n", create_ms, 100 * create_ms / (wall + cum_wall + create_ms));
  printf("Train time:   %.0fms (%.1fms/step)\n", total_train_ms,
         total_steps_done ? total_train_ms / total_steps_done : 0.0);
  printf("Wall time:    %.1fs\n", (wall + cum_wall) / 1000);
  munmap(data, data_len);
  close(fd);
  ne_destroy(ctx);
  return rc ? 1 : 0;
}
