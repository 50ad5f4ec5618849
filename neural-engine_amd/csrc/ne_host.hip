// Context, device memory plan, the training-step orchestration, the optimizer step and
// v4 checkpoint I/O.  Host code only; every numeric operation runs in the kernels of
// k_*.hip on the context's single stream.
//
// Device memory (all resident, nothing round-trips through the host during a step):
//   flat fp32 buffers P (master weights), G (grads), M, V (Adam) and the 16-bit shadow Pb
//   of P, one element order for all five:
//     per layer: Wqkv [Q+2KV, D] (= Wq;Wk;Wv rows), Wo [D,Q], W13 [2H, D] (= W1;W3 rows),
//                W2 [D,H]
//     E [V, D]
//     gains: per layer rms_att [D], rms_ffn [D] (+ q_norm, k_norm [HD]); rms_final [D]
//   so AdamW is one pass over all parameters and weight decay applies to the prefix
//   before the gains.  Activations are token-major [T, features] (T = B*S).
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "ne_ctx.h"

int decode_run(ne_ctx *ctx, const int32_t *prompt, int B, int P, int n_new, float temp, float top_p,
               const double *uniforms, int32_t *out);
int decode_alloc(ne_ctx *ctx);
void decode_free(ne_ctx *ctx);

namespace {

constexpr int CKPT_MAGIC = 0x424C5A54;
constexpr int QKN_TAG = 0x314E4B51;

#pragma pack(push, 4)
struct CkptHdr {  // TD/config.h:82-91, 96 bytes with native alignment
  int32_t magic, version, step, total_steps;
  int32_t n_layers, vocab_size, dim, hidden_dim, n_heads, seq_len;
  float lr, loss;
  double cum_compile, cum_train, cum_wall;
  int32_t cum_steps, cum_batches, adam_t;
  int32_t kv_heads, head_dim, q_dim;
};
#pragma pack(pop)
static_assert(sizeof(CkptHdr) == 96, "v4 header is 96 bytes");

}  // namespace

namespace {

// Two-pass bump allocator: sizes are summed first, then carved out of one allocation.
struct Plan {
  size_t total = 0;
  std::vector<std::pair<void **, size_t>> items;
  template <typename T>
  void add(T **p, size_t n) {
    items.push_back({(void **)p, n * sizeof(T)});
    total += (n * sizeof(T) + 255) & ~(size_t)255;
  }
  void assign(char *base) {
    size_t off = 0;
    for (auto &it : items) {
      *it.first = base + off;
      off += (it.second + 255) & ~(size_t)255;
    }
  }
};

void prof_begin(ne_ctx *c, int fam, hipEvent_t *e0, hipStream_t s) {
  if (!c->prof.on || !(c->prof.mask & (1 << fam))) return;
  *e0 = c->prof.get();
  hipEventRecord(*e0, s);
}
void prof_end(ne_ctx *c, int fam, hipEvent_t e0, hipStream_t s) {
  if (!c->prof.on || !(c->prof.mask & (1 << fam))) return;
  hipEvent_t e1 = c->prof.get();
  hipEventRecord(e1, s);
  c->prof.pending.push_back({fam, e0, e1});
}

// Event pair around the work of one kernel family enqueued on s (default: the step stream).
struct ProfScope {
  ne_ctx *c;
  int fam;
  hipStream_t s;
  hipEvent_t e0 = nullptr;
  ProfScope(ne_ctx *c_, int f, hipStream_t s_ = nullptr) : c(c_), fam(f), s(s_ ? s_ : c_->st) {
    prof_begin(c, fam, &e0, s);
  }
  ~ProfScope() { prof_end(c, fam, e0, s); }
};

// Make st follow the last optimizer update (every entry point that reads or writes
// parameters, moments or gradients, other than the next training step): a deferred pass is
// run on st now, in one launch; one still running on st2 is waited for.
int adam_join(ne_ctx *c) {
  if (c->upd_deferred) {
    c->upd_deferred = false;
    AdamArgs a = c->upd;
    a.max_groups = 0;
    hipEvent_t e0 = nullptr;
    prof_begin(c, NE_PROF_ADAM, &e0, c->st);
    NE_CHECK(launch_adam(c->dt, a, c->st));
    prof_end(c, NE_PROF_ADAM, e0, c->st);
  }
  if (!c->adam_pending) return 0;
  NE_HIP(hipStreamWaitEvent(c->st, c->ev_adam.back(), 0));
  c->adam_pending = false;
  return 0;
}

// Timeline event e on stream s (default st), when the timeline is on.
int tl_mark(ne_ctx *c, hipEvent_t e, hipStream_t s = nullptr) {
  if (!c->tl.on) return 0;
  NE_HIP(hipEventRecord(e, s ? s : c->st));
  return 0;
}

int prof_collect(ne_ctx *c) {
  if (c->prof.pending.empty()) return 0;
  NE_CHECK(adam_join(c));
  NE_HIP(hipStreamSynchronize(c->st));
  for (auto &r : c->prof.pending) {
    float ms = 0.f;
    hipEventElapsedTime(&ms, r.a, r.b);
    c->prof.ms[r.fam] += ms;
    c->prof.cnt[r.fam] += 1;
    c->prof.pool.push_back(r.a);
    c->prof.pool.push_back(r.b);
  }
  c->prof.pending.clear();
  return 0;
}

int gemm(ne_ctx *c, int fam, int site, int layout, int epi, int M, int N, int K, const void *A, long lda,
         const void *B, long ldb, void *C, long ldc, const void *R = nullptr, long ldr = 0, float alpha = 1.f) {
  ProfScope ps(c, fam);
  GemmArgs g = {};
  g.M = M; g.N = N; g.K = K;
  g.A = A; g.lda = lda; g.B = B; g.ldb = ldb; g.C = C; g.ldc = ldc; g.R = R; g.ldr = ldr;
  g.alpha = alpha;
  g.ovf = site >= 0 ? c->ovf + site : nullptr;
  g.ws = c->ws;
  g.ws_elems = c->ws_elems;
  return gemm_launch(c->dt, layout, epi, g, c->st);
}

// Weight-gradient GEMM C[M,N] (fp32, = or +=) of the step's backward; on st2 when the step
// forks (see Fork), else in order on st.
// Its split-K partials (if any) go to ws2 either way, so they never meet the dX partials
// that a consumer has yet to read from ws.
// sq (nullable): the sum-of-squares slots of C (GemmArgs::sq).
int gemm_dw(ne_ctx *c, bool side, int fam, int epi, int M, int N, int K, const h16_t *dY, long ldy, const h16_t *X,
            long ldx, float *C, float u, double *sq) {
  ProfScope ps(c, fam);
  GemmArgs g = {};
  g.M = M; g.N = N; g.K = K;
  g.A = dY; g.lda = ldy; g.B = X; g.ldb = ldx; g.C = C; g.ldc = N;
  g.alpha = u;
  g.ws = c->ws2;
  g.ws_elems = c->ws_elems;
  g.sq = sq;
  return gemm_launch(c->dt, GEMM_TN, epi, g, side ? c->st2 : c->st);
}

// Weight-gradient GEMMs of the backward, queued and run in batches by flush().  With `on`,
// the batches go to st2: flush() makes st2 wait for everything enqueued on st so far (inside a
// stream capture, a graph edge) and enqueues the batch there; join() makes st wait for st2.
// Without, a batch runs in order on st where flush() is called (per-kernel-family event
// timing records on st).
// A GEMM job with sq writes the sum of squares of each tile of G it finishes into its nsq
// slots (the global gradient norm's partials); also queued: the sum of squares of a part of
// G into its slots (sumsq(): the compact embedding gradient after its scatter).
struct WgradQueue {
  struct Job {
    int fam, epi, M, N, K;
    const h16_t *dY; long ldy; const h16_t *X; long ldx; float *C; float u;
    double *sq; long nsq;              // GEMM: its tiles' sum-of-squares slots (nullable)
    long n; int nparts; double *part;  // M == 0: sum of squares of C[0, n) into part[0, nparts)
  };
  ne_ctx *c;
  bool on;
  std::vector<Job> jobs;
  int run(const Job &j, bool side) {
    if (j.M == 0) return launch_sumsq(j.C, j.n, j.part, j.nparts, side ? c->st2 : c->st);
    if (j.sq && gemm_sq_parts(j.epi, j.M, j.N, j.K, c->ws_elems) != j.nsq)
      return ne_fail(NE_ERR_STATE, "weight gradient %dx%d: %ld norm slots planned, the launch writes %ld", j.M, j.N,
                     j.nsq, gemm_sq_parts(j.epi, j.M, j.N, j.K, c->ws_elems));
    return gemm_dw(c, side, j.fam, j.epi, j.M, j.N, j.K, j.dY, j.ldy, j.X, j.ldx, j.C, j.u, j.sq);
  }
  int push(const Job &j) {
    jobs.push_back(j);
    return 0;
  }
  int add(int fam, int epi, int M, int N, int K, const h16_t *dY, long ldy, const h16_t *X, long ldx, float *C,
          float u, double *sq = nullptr, long nsq = 0) {
    return push({fam, epi, M, N, K, dY, ldy, X, ldx, C, u, sq, nsq, 0, 0, nullptr});
  }
  int sumsq(const float *g, long n, long slot, int nparts) {
    return push({0, 0, 0, 0, 0, nullptr, 0, nullptr, 0, (float *)g, 0.f, nullptr, 0, n, nparts, c->gn_part + slot});
  }
  // Consecutive GEMM jobs with one epilogue, K and scale that gemm_group_fits (a long step's
  // weight gradients of a layer) run as one launch without split-K, in both schedules, so the
  // two give the same sums.
  int run_batch(bool side) {
    for (size_t i = 0; i < jobs.size();) {
      size_t e = i;
      GemmArgs ga[GEMM_GROUP_MAX];
      while (e < jobs.size() && e - i < (size_t)GEMM_GROUP_MAX && jobs[e].M > 0 && jobs[e].epi == jobs[i].epi &&
             jobs[e].K == jobs[i].K && jobs[e].u == jobs[i].u) {
        const Job &j = jobs[e];
        GemmArgs &g = ga[e - i];
        g = GemmArgs();
        g.M = j.M; g.N = j.N; g.K = j.K;
        g.A = j.dY; g.lda = j.ldy; g.B = j.X; g.ldb = j.ldx; g.C = j.C; g.ldc = j.N;
        g.alpha = j.u;
        g.sq = j.sq;
        e++;
      }
      if (e - i >= 2 && gemm_group_fits(ga, (int)(e - i))) {
        for (size_t k = i; k < e; k++)
          if (jobs[k].sq && jobs[k].nsq != (long)(jobs[k].M / 256) * (jobs[k].N / 256))
            return ne_fail(NE_ERR_STATE, "grouped weight gradient %dx%d: %ld norm slots planned", jobs[k].M,
                           jobs[k].N, jobs[k].nsq);
        ProfScope ps(c, jobs[i].fam);
        NE_CHECK(gemm_group_launch(c->dt, jobs[i].epi, ga, (int)(e - i), side ? c->st2 : c->st));
        i = e;
      } else {
        NE_CHECK(run(jobs[i], side));
        i++;
      }
    }
    jobs.clear();
    return 0;
  }
  int flush() {
    if (jobs.empty()) return 0;
    if (!on) return run_batch(false);
    NE_HIP(hipEventRecord(c->ev_fork, c->st));
    NE_HIP(hipStreamWaitEvent(c->st2, c->ev_fork, 0));
    return run_batch(true);
  }
  int join() {
    NE_CHECK(flush());
    if (!on) return 0;
    NE_HIP(hipEventRecord(c->ev_join, c->st2));
    NE_HIP(hipStreamWaitEvent(c->st, c->ev_join, 0));
    return 0;
  }
};

// On short steps the W1|W3 GEMM writes the SwiGLU gate itself (one launch instead of the GEMM
// and a pass over h13) when it would run unsplit: the same tile, sums and 16-bit roundings as
// the two kernels, so the same h13 and gate bit for bit.  With split-K the SwiGLU kernel sums
// the partials as before; on long steps (more than 2048 tokens) the separate pass, which
// streams at full bandwidth, is cheaper than the gate work in the GEMM's epilogue, where the
// waves of one work-group per CU all reach it together (16,384 tokens: 113.3 vs 114.3 ms per
// Qwen3-0.6B step).
bool swiglu_in_gemm(const ne_ctx *c) {
  return c->T <= 2048 && (2 * c->H) % 128 == 0 && gemm_splits(EPI_H16, c->T, 2 * c->H, c->D, c->ws_elems) == 1;
}

int gemm_swiglu_fwd(ne_ctx *c, const h16_t *x2n, const h16_t *w13, h16_t *h13, h16_t *gate) {
  ProfScope ps(c, NE_PROF_GEMM_FWD);
  GemmArgs g = {};
  g.M = c->T; g.N = 2 * c->H; g.K = c->D;
  g.A = x2n; g.lda = c->D; g.B = w13; g.ldb = c->D;
  g.C = h13; g.ldc = 2 * c->H; g.C2 = gate; g.ldc2 = c->H;
  g.alpha = 1.f;
  g.ovf = c->ovf + OVF_H13;
  g.ovf2 = c->ovf + OVF_SWIGLU;
  return gemm_launch(c->dt, GEMM_NT, EPI_SWIGLU_FWD, g, c->st);
}

// GEMM whose split-K reduction, when it splits, is left to the kernel that consumes C:
// *sp then describes the partials in c->ws (C unwritten), else has n = 0 (C written).  C must
// be [M, N] row-major with ldc = N; R (EPI_RESID) is the residual added after the sum.
int gemm_split(ne_ctx *c, int fam, int layout, int epi, int M, int N, int K, const void *A, long lda,
               const void *B, long ldb, void *C, SplitIn *sp, const float *R = nullptr, float alpha = 1.f,
               int *ovf = nullptr) {
  ProfScope ps(c, fam);
  GemmArgs g = {};
  g.M = M; g.N = N; g.K = K;
  g.A = A; g.lda = lda; g.B = B; g.ldb = ldb; g.C = C; g.ldc = N; g.R = R; g.ldr = N;
  g.alpha = alpha;
  g.ovf = ovf;  // 16-bit C written here (no split); with a split the consumer raises it
  g.ws = c->ws;
  g.ws_elems = c->ws_elems;
  g.defer_reduce = 1;
  int split = 1;
  NE_CHECK(gemm_launch(c->dt, layout, epi, g, c->st, &split));
  *sp = SplitIn();
  if (split > 1) {
    sp->part = c->ws;
    sp->n = split;
    sp->slice = (long)M * N;
    sp->base = R;
    sp->alpha = alpha;
  }
  return 0;
}

// Gain-gradient partial slab of an RMSNorm site (0: final norm; 1 + 2l: layer l's FFN norm;
// 2 + 2l: its attention norm) and of layer l's QK-norm pair.
float *norm_part(ne_ctx *c, int site) { return c->gpart + (long)site * c->rms_slab; }
float *qk_part(ne_ctx *c, int l) { return c->gpart + (long)(2 * c->L + 1) * c->rms_slab + (long)l * c->qk_slab; }

// Sum-of-squares partials of G, reduced in slot order by the optimizer: per layer the slots
// of its Wqkv, Wo (the attention block, G from lo[l].wqkv), W13 and W2 (the FFN block, from
// lo[l].w13) weight gradients, one per tile of each GEMM, written by the GEMM as it stores
// the tile; the embedding gradient's GEMM (its tiles); the gains; then one slot per token row
// for the change the embedding scatter makes to the row it updates.
constexpr int GN_GAINS = 16;
enum { GN_WQKV = 0, GN_WO, GN_W13, GN_W2 };
long gn_layer(const ne_ctx *c, int l) { return (long)l * c->gn_lay; }
long gn_job(const ne_ctx *c, int l, int j) {
  long o = gn_layer(c, l);
  for (int i = 0; i < j; i++) o += c->gn_n[i];
  return o;
}
long gn_attn_n(const ne_ctx *c) { return c->gn_n[GN_WQKV] + c->gn_n[GN_WO]; }
long gn_embed(const ne_ctx *c) { return (long)c->L * c->gn_lay; }
long gn_gains(const ne_ctx *c) { return gn_embed(c) + c->gn_emb; }
long gn_rows(const ne_ctx *c) { return gn_gains(c) + GN_GAINS; }
long gn_slots(const ne_ctx *c) { return gn_rows(c) + c->T; }
long layer_params(const ne_ctx *c) { return (long)(c->QKV + c->Q + 3L * c->H) * c->D; }
long layer_attn_params(const ne_ctx *c) { return (long)(c->QKV + c->Q) * c->D; }

// The slot counts: a layer's four weight gradients are queued as one batch (W2, W13, Wo,
// Wqkv), which runs as one grouped launch of 256x256 tiles when gemm_group_fits, else as four
// GEMMs tiled by gemm_launch's plan; the embedding gradient's GEMM runs alone.
void plan_gn(ne_ctx *c) {
  const int T = c->T, D = c->D, H = c->H;
  const int M[4] = {c->QKV, D, 2 * H, D}, N[4] = {D, c->Q, D, H};  // GN_WQKV .. GN_W2
  GemmArgs ga[4] = {};
  for (int j = 0; j < 4; j++) {
    ga[j].M = M[j];
    ga[j].N = N[j];
    ga[j].K = T;
  }
  c->gn_grouped = gemm_group_fits(ga, 4);
  c->gn_lay = 0;
  for (int j = 0; j < 4; j++) {
    c->gn_n[j] = c->gn_grouped ? (long)(M[j] / 256) * (N[j] / 256) : gemm_sq_parts(EPI_F32, M[j], N[j], T, c->ws_elems);
    c->gn_lay += c->gn_n[j];
  }
  // On short steps the embedding gradient's GEMM (V x D, K = T: at 256 tokens 622 MB of fp32
  // written by a GEMM with little to compute) runs in row blocks, one beside each layer's
  // backward: in one launch it slowed the two layers of the chain beside it by ~150 us.
  // Block boundaries on the coarsest of 256, 128, 64 rows that divides the vocabulary.
  const int gran = c->V % 256 == 0 ? 256 : c->V % 128 == 0 ? 128 : 64;
  c->de_pieces = T <= 4096 ? std::min(c->L, c->V / gran) : 1;
  c->de_rows.resize(c->de_pieces + 1);
  c->gn_emb = 0;
  for (int p = 0; p <= c->de_pieces; p++) c->de_rows[p] = (int)((long)(c->V / gran) * p / c->de_pieces) * gran;
  for (int p = 0; p < c->de_pieces; p++)
    c->gn_emb += gemm_sq_parts(EPI_F32, c->de_rows[p + 1] - c->de_rows[p], D, T, c->ws_elems);
}

// Sum of squares of all of G into the step's slots (the per-row change slots of the
// embedding scatter read 0), on st: for an optimizer step that follows a direct gradient
// write or no micro-step at all.
int gn_sum_all(ne_ctx *c) {
  for (int l = 0; l < c->L; l++) {
    const LayerOff &o = c->lo[l];
    const long na = gn_attn_n(c), nf = c->gn_lay - na;
    NE_CHECK(launch_sumsq(c->G + o.wqkv, layer_attn_params(c), c->gn_part + gn_layer(c, l), (int)na, c->st));
    NE_CHECK(launch_sumsq(c->G + o.w13, layer_params(c) - layer_attn_params(c), c->gn_part + gn_layer(c, l) + na,
                          (int)nf, c->st));
  }
  NE_CHECK(launch_sumsq(c->G + c->off_E, (long)c->V * c->D, c->gn_part + gn_embed(c), (int)c->gn_emb, c->st));
  NE_CHECK(launch_sumsq(c->G + c->n_decay, c->n_params - c->n_decay, c->gn_part + gn_gains(c), GN_GAINS, c->st));
  return launch_fill_f32((float *)(c->gn_part + gn_rows(c)), 0.f, 2L * c->T, c->st);
}

int validate(const ne_config *c) {
  if (!c) return ne_fail(NE_ERR_ARG, "null config");
  if (c->dim <= 0 || c->hidden <= 0 || c->n_heads <= 0 || c->kv_heads <= 0 || c->head_dim <= 0 ||
      c->n_layers <= 0 || c->vocab <= 0 || c->seq <= 0 || c->batch <= 0)
    return ne_fail(NE_ERR_ARG, "config: all dims must be positive");
  if (c->n_heads % c->kv_heads) return ne_fail(NE_ERR_ARG, "config: n_heads %% kv_heads != 0");
  if (c->head_dim != 64 && c->head_dim != 128) return ne_fail(NE_ERR_ARG, "config: head_dim must be 64 or 128");
  if (c->seq % 64) return ne_fail(NE_ERR_ARG, "config: seq must be a multiple of 64");
  if (c->dim % 64 || c->hidden % 64 || c->vocab % 64)
    return ne_fail(NE_ERR_ARG, "config: dim, hidden and vocab must be multiples of 64");
  if (c->dim > 2048) return ne_fail(NE_ERR_ARG, "config: dim > 2048 unsupported");
  if (c->decode_batch < 0 || c->decode_ctx < 0) return ne_fail(NE_ERR_ARG, "config: negative decode sizes");
  if (c->dtype != NE_BF16 && c->dtype != NE_FP16) return ne_fail(NE_ERR_ARG, "config: dtype must be NE_BF16 or NE_FP16");
  return 0;
}

void layout_params(ne_ctx *c) {
  const long D = c->D, H = c->H, Q = c->Q, KV = c->KV, HD = c->HD;
  long off = 0;
  c->lo.resize(c->L);
  for (int l = 0; l < c->L; l++) {
    LayerOff &o = c->lo[l];
    o.wqkv = off; off += (Q + 2 * KV) * D;
    o.wo = off; off += D * Q;
    o.w13 = off; off += 2 * H * D;
    o.w2 = off; off += D * H;
  }
  c->off_E = off; off += (long)c->V * D;
  c->n_decay = off;
  for (int l = 0; l < c->L; l++) {
    LayerOff &o = c->lo[l];
    o.g_att = off; off += D;
    o.g_ffn = off; off += D;
    if (c->c.qk_norm) {
      o.gq = off; off += HD;
      o.gk = off; off += HD;
    } else {
      o.gq = o.gk = -1;
    }
  }
  c->off_gfinal = off; off += D;
  c->n_params = off;
  // tensor ids in checkpoint order
  c->t_off.clear();
  c->t_numel.clear();
  auto push = [&](long o, long n) { c->t_off.push_back(o); c->t_numel.push_back(n); };
  for (int l = 0; l < c->L; l++) {
    const LayerOff &o = c->lo[l];
    push(o.wqkv, Q * D);
    push(o.wqkv + Q * D, KV * D);
    push(o.wqkv + (Q + KV) * D, KV * D);
    push(o.wo, D * Q);
    push(o.w13, H * D);
    push(o.w2, D * H);
    push(o.w13 + H * D, H * D);
    push(o.g_att, D);
    push(o.g_ffn, D);
  }
  push(c->off_gfinal, D);
  push(c->off_E, (long)c->V * D);
  if (c->c.qk_norm)
    for (int l = 0; l < c->L; l++) {
      push(c->lo[l].gq, HD);
      push(c->lo[l].gk, HD);
    }
}

float *kind_base(ne_ctx *c, int kind) {
  switch (kind) {
    case NE_PARAM: return c->P;
    case NE_GRAD: return c->G;
    case NE_ADAM_M: return c->M;
    case NE_ADAM_V: return c->Vm;
  }
  return nullptr;
}

}  // namespace

// ------------------------------------------------------------------------ lifetime ----

// Vocabulary pieces of the classifier's logits GEMM at most (ce_cut): a 256-token Qwen3-0.6B
// step has four (256, 256, 256 and 419 work-groups of 256 x 128 tiles).
constexpr int CE_PIECES_MAX = 8;

extern "C" ne_ctx *ne_create(const ne_config *cfg) {
  if (validate(cfg)) return nullptr;
  ne_ctx *c = new ne_ctx();
  c->c = *cfg;
  c->D = cfg->dim; c->H = cfg->hidden; c->NH = cfg->n_heads; c->NKV = cfg->kv_heads; c->HD = cfg->head_dim;
  c->L = cfg->n_layers; c->V = cfg->vocab; c->S = cfg->seq; c->B = cfg->batch; c->T = c->B * c->S;
  c->Q = c->NH * c->HD; c->KV = c->NKV * c->HD; c->QKV = c->Q + 2 * c->KV;
  c->dt = cfg->dtype;
  layout_params(c);
  const size_t T = c->T, D = c->D, H = c->H, Q = c->Q, KV = c->KV, QKV = c->QKV, NH = c->NH, NKV = c->NKV;
  Plan pl;
  pl.add(&c->P, c->n_params);
  pl.add(&c->G, c->n_params);
  pl.add(&c->M, c->n_params);
  pl.add(&c->Vm, c->n_params);
  pl.add(&c->Pb, c->n_params);
  c->act.resize(c->L);
  for (int l = 0; l < c->L; l++) {
    LayerAct &a = c->act[l];
    pl.add(&a.x_in, T * D); pl.add(&a.r1, T); pl.add(&a.xn, T * D);
    pl.add(&a.qkv, T * QKV); pl.add(&a.qr, T * Q); pl.add(&a.kr, T * KV);
    pl.add(&a.rq, T * NH); pl.add(&a.rk, T * NKV);
    pl.add(&a.attn, T * Q); pl.add(&a.lse, T * NH);
    pl.add(&a.x2, T * D); pl.add(&a.r2, T); pl.add(&a.x2n, T * D);
    pl.add(&a.h13, T * 2 * H); pl.add(&a.gate, T * H);
  }
  pl.add(&c->xL, T * D); pl.add(&c->rf, T); pl.add(&c->xf, T * D);
  pl.add(&c->dx, T * D); pl.add(&c->dx2, T * D); pl.add(&c->dtmp, T * D);
  pl.add(&c->dq, T * Q); pl.add(&c->dk, T * KV); pl.add(&c->delta, T * NH);
  c->attn_split = attn_bwd_split_heads(c->B, c->S, c->NH, c->NKV);
  pl.add(&c->attn_part, c->attn_split ? 2 * T * Q : 1);
  const size_t L = c->L;
  pl.add(&c->dbf, 2 * L * T * D); pl.add(&c->dh13, L * T * 2 * H); pl.add(&c->dattn, T * Q);
  pl.add(&c->dqkv, L * T * QKV);
  pl.add(&c->dlogits, T * (size_t)c->V);
  pl.add(&c->ce_part, T * (size_t)(c->V / 64) * 2);
  pl.add(&c->ce_tgt, T); pl.add(&c->ce_lse, T); pl.add(&c->ce_rows, T); pl.add(&c->loss, 4);
  pl.add(&c->tok_in, 4 * T);  // inputs, targets, id chains: filled by one copy
  pl.add(&c->cosb, (size_t)c->S * c->HD / 2); pl.add(&c->sinb, (size_t)c->S * c->HD / 2);
  pl.add(&c->gscale, 4);
  pl.add(&c->stats_part, 4 * NE_STATS_BLOCKS); pl.add(&c->gnorm, 4); pl.add(&c->ovf, 32);
  // split-K partials: up to 32 splits of a [T, D] result (the LM-head dX of a short step)
  c->ws_elems = std::min<long>(32L << 20, std::max<long>(8L << 20, (long)T * D * 32));
  pl.add(&c->ws, (size_t)c->ws_elems);
  pl.add(&c->ws2, (size_t)c->ws_elems);
  plan_gn(c);
  pl.add(&c->gn_part, (size_t)gn_slots(c));
  c->ce_cut.assign(CE_PIECES_MAX + 1, 0);
  c->ce_cut.resize(gemm_ce_pieces(T, c->V, D, CE_PIECES_MAX, c->ce_cut.data()) + 1);
  // gain-gradient partials of every norm site (2L+1 RMSNorms, L QK-norm pairs), summed by one
  // ordered launch at the end of the backward
  c->rms_slab = rmsnorm_bwd_part_elems(c->T, c->D);
  c->qk_slab = c->c.qk_norm ? qk_prep_bwd_part_elems(c->T, c->NH, c->NKV, c->HD) : 0;
  pl.add(&c->gpart, (size_t)(2 * c->L + 1) * c->rms_slab + (size_t)c->L * c->qk_slab);
  c->cs_njobs = 2 * c->L + 1 + (c->c.qk_norm ? 2 * c->L : 0);
  pl.add(&c->cs_jobs, (size_t)c->cs_njobs);

  int rc = 0;
  if ((rc = ne_hip_status(hipStreamCreateWithFlags(&c->st, hipStreamNonBlocking), "stream"))) goto fail;
  if ((rc = ne_hip_status(hipStreamCreateWithFlags(&c->st2, hipStreamNonBlocking), "stream"))) goto fail;
  if ((rc = ne_hip_status(hipEventCreateWithFlags(&c->ev_fork, hipEventDisableTiming), "event"))) goto fail;
  if ((rc = ne_hip_status(hipEventCreateWithFlags(&c->ev_join, hipEventDisableTiming), "event"))) goto fail;
  c->ev_adam.assign(c->L + c->ce_cut.size(), nullptr);
  c->tl.fwd_l.assign(c->L, nullptr);  // the step names them whether or not the timeline is on
  c->tl.bwd_l.assign(c->L, nullptr);
  for (auto &e : c->ev_adam)
    if ((rc = ne_hip_status(hipEventCreateWithFlags(&e, hipEventDisableTiming), "event"))) goto fail;
  if ((rc = ne_hip_status(hipEventCreateWithFlags(&c->ev_lookup, hipEventDisableTiming), "event"))) goto fail;
  if ((rc = ne_hip_status(hipMalloc(&c->arena, pl.total), "hipMalloc(arena)"))) goto fail;
  pl.assign((char *)c->arena);
  c->tok_tgt = c->tok_in + T;
  c->tok_nxt = c->tok_in + 2 * T;
  c->tok_first = c->tok_in + 3 * T;
  c->tok_last.assign(c->V, -1);
  {
    std::vector<ColsumJob> jobs;
    const int rows = rmsnorm_bwd_part_rows(c->T);
    for (int site = 0; site < 2 * c->L + 1; site++) {
      float *out = site == 0 ? c->G + c->off_gfinal
                             : c->G + ((site & 1) ? c->lo[(site - 1) / 2].g_ffn : c->lo[(site - 2) / 2].g_att);
      jobs.push_back({norm_part(c, site), out, rows, c->D});
    }
    if (c->c.qk_norm) {
      int rq, rk;
      qk_prep_bwd_part_rows(c->T, c->NH, c->NKV, c->HD, &rq, &rk);
      for (int l = 0; l < c->L; l++) {
        jobs.push_back({qk_part(c, l), c->G + c->lo[l].gq, rq, c->HD});
        jobs.push_back({qk_part(c, l) + (long)rq * c->HD, c->G + c->lo[l].gk, rk, c->HD});
      }
    }
    if ((rc = ne_hip_status(hipMemcpy(c->cs_jobs, jobs.data(), jobs.size() * sizeof(ColsumJob),
                                      hipMemcpyHostToDevice), "colsum jobs")))
      goto fail;
  }
  if ((rc = ne_hip_status(hipHostMalloc((void **)&c->h_tok, 8 * T * sizeof(int32_t), 0), "hipHostMalloc"))) goto fail;
  if ((rc = ne_hip_status(hipEventCreateWithFlags(&c->tok_ev[0], hipEventDisableTiming), "event"))) goto fail;
  if ((rc = ne_hip_status(hipEventCreateWithFlags(&c->tok_ev[1], hipEventDisableTiming), "event"))) goto fail;
  if ((rc = ne_hip_status(hipHostMalloc((void **)&c->h_scalar, 4 * sizeof(float), 0), "hipHostMalloc"))) goto fail;
  if ((rc = ne_hip_status(hipHostMalloc((void **)&c->h_ovf, 32 * sizeof(int), 0), "hipHostMalloc"))) goto fail;
  // zero weights, gains 1; zero grads and moments
  if ((rc = ne_hip_status(hipMemsetAsync(c->P, 0, c->n_params * 4, c->st), "memset"))) goto fail;
  if ((rc = ne_hip_status(hipMemsetAsync(c->G, 0, c->n_params * 4, c->st), "memset"))) goto fail;
  if ((rc = ne_hip_status(hipMemsetAsync(c->M, 0, c->n_params * 4, c->st), "memset"))) goto fail;
  if ((rc = ne_hip_status(hipMemsetAsync(c->Vm, 0, c->n_params * 4, c->st), "memset"))) goto fail;
  if ((rc = launch_fill_f32(c->P + c->n_decay, 1.f, c->n_params - c->n_decay, c->st))) goto fail;
  if ((rc = ne_hip_status(hipMemsetAsync(c->ovf, 0, 32 * sizeof(int), c->st), "memset"))) goto fail;
  if ((rc = launch_f32_to_h16(c->dt, c->P, c->Pb, c->n_params, c->st))) goto fail;
  {
    // RoPE tables [S, HD/2]: angle = pos * theta^(-2i/HD), evaluated in double
    const int half = c->HD / 2;
    std::vector<float> cs((size_t)c->S * half), sn((size_t)c->S * half);
    for (int p = 0; p < c->S; p++)
      for (int i = 0; i < half; i++) {
        const double freq = 1.0 / pow((double)cfg->rope_theta, 2.0 * i / c->HD);
        const double ang = p * freq;
        cs[(size_t)p * half + i] = (float)cos(ang);
        sn[(size_t)p * half + i] = (float)sin(ang);
      }
    if ((rc = ne_hip_status(hipMemcpy(c->cosb, cs.data(), cs.size() * 4, hipMemcpyHostToDevice), "rope"))) goto fail;
    if ((rc = ne_hip_status(hipMemcpy(c->sinb, sn.data(), sn.size() * 4, hipMemcpyHostToDevice), "rope"))) goto fail;
  }
  if (cfg->decode_batch > 0 && cfg->decode_ctx > 0)
    if ((rc = decode_alloc(c))) goto fail;
  if ((rc = ne_hip_status(hipStreamSynchronize(c->st), "create sync"))) goto fail;
  return c;
fail:
  ne_destroy(c);
  return nullptr;
}

extern "C" void ne_destroy(ne_ctx *c) {
  if (!c) return;
  if (c->st) hipStreamSynchronize(c->st);
  if (c->st2) hipStreamSynchronize(c->st2);
  for (auto &e : c->graphs) hipGraphExecDestroy(e.exec);
  if (c->ev_fork) hipEventDestroy(c->ev_fork);
  if (c->ev_join) hipEventDestroy(c->ev_join);
  for (auto e : c->ev_adam)
    if (e) hipEventDestroy(e);
  if (c->ev_lookup) hipEventDestroy(c->ev_lookup);
  for (int i = 0; i < 2; i++)
    if (c->tok_ev[i]) hipEventDestroy(c->tok_ev[i]);
  decode_free(c);
  for (auto &r : c->prof.pending) {
    hipEventDestroy(r.a);
    hipEventDestroy(r.b);
  }
  for (auto e : c->prof.pool) hipEventDestroy(e);
  for (hipEvent_t e : {c->tl.start, c->tl.lookup, c->tl.fwd, c->tl.cls, c->tl.bwd, c->tl.join, c->tl.end, c->tl.opt0,
                       c->tl.opt1, c->tl.upd0, c->tl.upd1})
    if (e) hipEventDestroy(e);
  for (auto e : c->tl.fwd_l)
    if (e) hipEventDestroy(e);
  for (auto e : c->tl.bwd_l)
    if (e) hipEventDestroy(e);
  if (c->arena) hipFree(c->arena);
  if (c->cids) hipFree(c->cids);
  if (c->cE) hipFree(c->cE);
  if (c->gcE) hipFree(c->gcE);
  if (c->h_tok) hipHostFree(c->h_tok);
  if (c->h_scalar) hipHostFree(c->h_scalar);
  if (c->h_ovf) hipHostFree(c->h_ovf);
  if (c->st2) hipStreamDestroy(c->st2);
  if (c->st) hipStreamDestroy(c->st);
  delete c;
}

extern "C" int ne_sync(ne_ctx *c) {
  if (!c) return ne_fail(NE_ERR_ARG, "null context");
  NE_CHECK(adam_join(c));
  NE_HIP(hipStreamSynchronize(c->st));
  return 0;
}

// ------------------------------------------------------------------------ tensors ----

extern "C" int ne_num_tensors(const ne_ctx *c) { return c ? (int)c->t_off.size() : 0; }

extern "C" int64_t ne_tensor_numel(const ne_ctx *c, int id) {
  if (!c || id < 0 || id >= (int)c->t_off.size()) return ne_fail(NE_ERR_ARG, "bad tensor id %d", id);
  return c->t_numel[id];
}

extern "C" int ne_set_tensor(ne_ctx *c, int kind, int id, const float *host, size_t n) {
  if (!c || !host) return ne_fail(NE_ERR_ARG, "null argument");
  NE_CHECK(adam_join(c));
  if (id < 0 || id >= (int)c->t_off.size()) return ne_fail(NE_ERR_ARG, "bad tensor id %d", id);
  if ((long)n != c->t_numel[id]) return ne_fail(NE_ERR_ARG, "tensor %d has %ld elements, got %zu", id, c->t_numel[id], n);
  float *base = kind_base(c, kind);
  if (!base) return ne_fail(NE_ERR_ARG, "bad tensor kind %d", kind);
  if (kind == NE_GRAD && c->grads_fresh) {  // materialise the logical zeros before a partial write
    NE_CHECK(launch_fill_f32(c->G, 0.f, c->n_params, c->st));
    c->grads_fresh = false;
  }
  if (kind == NE_GRAD) c->gn_ready = c->gn_parts_ok = false;  // the sum-of-squares partials no longer hold
  NE_HIP(hipMemcpyAsync(base + c->t_off[id], host, n * 4, hipMemcpyHostToDevice, c->st));
  if (kind == NE_PARAM) NE_CHECK(launch_f32_to_h16(c->dt, c->P + c->t_off[id], c->Pb + c->t_off[id], n, c->st));
  NE_HIP(hipStreamSynchronize(c->st));
  return 0;
}

extern "C" int ne_get_tensor(ne_ctx *c, int kind, int id, float *host, size_t n) {
  if (!c || !host) return ne_fail(NE_ERR_ARG, "null argument");
  NE_CHECK(adam_join(c));
  if (id < 0 || id >= (int)c->t_off.size()) return ne_fail(NE_ERR_ARG, "bad tensor id %d", id);
  if ((long)n != c->t_numel[id]) return ne_fail(NE_ERR_ARG, "tensor %d has %ld elements, got %zu", id, c->t_numel[id], n);
  float *base = kind_base(c, kind);
  if (!base) return ne_fail(NE_ERR_ARG, "bad tensor kind %d", kind);
  if (kind == NE_GRAD && c->grads_fresh) {  // logically zero since the last update
    memset(host, 0, n * 4);
    return 0;
  }
  NE_HIP(hipMemcpyAsync(host, base + c->t_off[id], n * 4, hipMemcpyDeviceToHost, c->st));
  NE_HIP(hipStreamSynchronize(c->st));
  return 0;
}

extern "C" int ne_get_state(const ne_ctx *c, ne_train_state *st) {
  if (!c || !st) return ne_fail(NE_ERR_ARG, "null argument");
  *st = c->state;
  return 0;
}

extern "C" int ne_set_state(ne_ctx *c, const ne_train_state *st) {
  if (!c || !st) return ne_fail(NE_ERR_ARG, "null argument");
  c->state = *st;
  return 0;
}

// ------------------------------------------------------------------- training step ----

// The deferred AdamW pass of the last optimizer step, enqueued on st2 by the training step
// that follows it, forked from st at the step's start.  Chunks in order: the gains
// (ev_adam[0]), layer l's matrices (ev_adam[1 + l]), then the embedding (ev_adam[L + 1]) after
// ev_lookup (the step's lookup, which computes the updated rows itself, has read them).  The
// forward waits for each chunk just before it reads what the chunk writes, the classifier for
// the embedding's.  The step enqueues the chunks as its forward goes, UPD_AHEAD layers ahead
// of the layer it enqueues: all of them up front kept the GPU's forward waiting 0.2-0.3 ms for
// the host.  Qwen3-0.6B, 256 tokens, one box, ms per step: the embedding last 7.94, its rows
// in pieces after each of the last 14 layers 7.95, after every layer 8.06; the embedding
// first with the lookup waiting for it (the former order) 8.02-8.03.  The forward runs at the
// pace of the pass beside it (~140-150 us per layer against ~60 alone); over the forward the
// two move ~19.4 GB in ~4 ms, about 90% of what a plain device copy streams.
constexpr int UPD_AHEAD = 2;
// The chunks beside the forward run at most this many work-groups: the update streams more
// slowly and the forward's small GEMMs, which wait on HBM behind it, less so (same step, ms:
// 256 work-groups 8.16, 384 7.94-8.06, 512 8.02; the former order: uncapped 8.24, 768 8.39,
// 512 8.08-8.19, 384 7.97, 256 8.18).  Four float4 of each stream per thread instead of two
// measured the same (8.02).
constexpr int UPD_MAX_GROUPS = 384;
// Profiling (NE_PROF_ADAM) records one event pair around the whole pass on st2, whose chunks
// run back to back there: one pair per launch added 0.22 ms to the 256-token step.
struct UpdateQueue {
  ne_ctx *c;
  int next = -1;  // next chunk: -1 the gains, l < L the layer l, L the embedding
  hipEvent_t e0 = nullptr;
  int chunk(long off, long n, long n_decay) {
    AdamArgs ch = c->upd;
    ch.p = c->P + off; ch.g = c->G + off; ch.m = c->M + off; ch.v = c->Vm + off; ch.pb = c->Pb + off;
    ch.n = n; ch.n_decay = n_decay;
    ch.max_groups = UPD_MAX_GROUPS;
    return launch_adam(c->dt, ch, c->st2);
  }
  // enqueue the chunks up to and including chunk l (l = L: everything)
  int upto(int l) {
    const int L = c->L;
    for (; next <= std::min(l, L); next++) {
      if (next == -1) {
        c->adam_pending = true;
        NE_CHECK(tl_mark(c, c->tl.upd0, c->st2));
        prof_begin(c, NE_PROF_ADAM, &e0, c->st2);
        NE_CHECK(chunk(c->n_decay, c->n_params - c->n_decay, 0));
        NE_HIP(hipEventRecord(c->ev_adam[0], c->st2));
      } else if (next < L) {
        NE_CHECK(chunk(c->lo[next].wqkv, layer_params(c), layer_params(c)));
        NE_HIP(hipEventRecord(c->ev_adam[1 + next], c->st2));
      } else {
        NE_HIP(hipStreamWaitEvent(c->st2, c->ev_lookup, 0));
        for (size_t p = 0; p + 1 < c->ce_cut.size(); p++) {
          const long r0 = c->ce_cut[p], n = (long)(c->ce_cut[p + 1] - r0) * c->D;
          NE_CHECK(chunk(c->off_E + r0 * c->D, n, n));
          if (p + 2 < c->ce_cut.size()) NE_HIP(hipEventRecord(c->ev_adam[L + 1 + p], c->st2));
        }
        prof_end(c, NE_PROF_ADAM, e0, c->st2);
        NE_HIP(hipEventRecord(c->ev_adam.back(), c->st2));
        NE_CHECK(tl_mark(c, c->tl.upd1, c->st2));
        c->tl.opt_ok = c->tl.on;
      }
    }
    return 0;
  }
};

// Enqueue one forward+backward on c->st with token ids already in c->tok_in/tok_tgt.
// Free of host synchronisation and memsets, so it can be captured into a HIP graph.
static int train_step_enqueue(ne_ctx *c, float loss_scale, bool fresh, bool two, bool upd = false) {
  const int T = c->T, S = c->S, D = c->D, H = c->H, Q = c->Q, KV = c->KV, QKV = c->QKV, V = c->V;
  const float alpha = c->c.res_alpha, eps = c->c.norm_eps;
  const h16_t *Pb = c->Pb;
  const float *P = c->P;
  float *G = c->G;
  AttnArgs at = {};
  at.B = c->B; at.S = S; at.NH = c->NH; at.NKV = c->NKV; at.HD = c->HD;
  at.scale = 1.0f / sqrtf((float)c->HD);

  // The backward runs at an internal power-of-two scale gs (dlogits = (p - onehot) * gs) that
  // keeps 16-bit gradients in range; fp32 sinks (weight / gain / embedding grads) take
  // u = (loss_scale / T) / gs, so G accumulates d(loss * loss_scale)/dw exactly as the
  // reference's loss_scale convention (TD/train.m:180, TD/cpu_ops.h:348-382).
  const int dt = c->dt;
  const float u = loss_scale / (float)T / c->gs;
  int *ovf = c->ovf;  // + OVF_* site index
  // The first micro-step after an optimizer step (or zero_grads) writes the weight
  // gradients instead of accumulating (no zeroing pass, no read of G); only the gains,
  // which accumulate through atomics, are cleared.
  const int EPI_DW = fresh ? EPI_F32 : EPI_F32_ACC;
  // With upd, the deferred optimizer update (UpdateQueue) runs on st2 beside the forward:
  // the lookup applies it to the rows it reads, then the step waits for chunk 0 (the gains,
  // whose gradients the fresh fill below clears), chunk 1 + l before layer l and the last
  // embedding piece before the classifier, all before the backward, the first writer of G.
  auto wait_update = [&](int k) -> int {
    if (upd) NE_HIP(hipStreamWaitEvent(c->st, c->ev_adam[k], 0));
    return 0;
  };
  UpdateQueue uq{c};
  NE_CHECK(tl_mark(c, c->tl.start));
  // ---------------- forward ----------------
  {
    ProfScope ps(c, NE_PROF_EMBED);
    if (upd) {
      NE_HIP(hipEventRecord(c->ev_fork, c->st));
      NE_HIP(hipStreamWaitEvent(c->st2, c->ev_fork, 0));
      NE_CHECK(uq.upto(-1));  // the gains
      NE_CHECK(launch_embed_fwd_adam(P + c->off_E, G + c->off_E, c->M + c->off_E, c->Vm + c->off_E, c->tok_in,
                                     c->act[0].x_in, T, D, c->upd, c->st));
      NE_HIP(hipEventRecord(c->ev_lookup, c->st));
      NE_CHECK(uq.upto(UPD_AHEAD - 1));
    } else {
      NE_CHECK(launch_embed_fwd(P + c->off_E, c->tok_in, c->act[0].x_in, T, D, c->st));
    }
  }
  NE_CHECK(wait_update(0));
  NE_CHECK(tl_mark(c, c->tl.lookup));
  if (fresh) NE_CHECK(launch_fill_f32(G + c->n_decay, 0.f, c->n_params - c->n_decay, c->st));

  // The residual-producing GEMMs (Wo, W2) leave their split-K partials to the RMSNorm that
  // reads their output; sp_x describes the pending partials of the next norm's input.
  SplitIn sp_x;
  for (int l = 0; l < c->L; l++) {
    LayerAct &a = c->act[l];
    const LayerOff &o = c->lo[l];
    float *x_next = (l + 1 < c->L) ? c->act[l + 1].x_in : c->xL;
    if (upd) NE_CHECK(uq.upto(l + UPD_AHEAD));
    NE_CHECK(wait_update(1 + l));
    {
      ProfScope ps(c, NE_PROF_NORM);
      NE_CHECK(launch_rmsnorm_fwd(dt, a.x_in, P + o.g_att, a.xn, a.r1, T, D, eps, ovf + OVF_NORM_FWD, c->st, sp_x));
    }
    // QKV, W1|W3 and (backward) dO GEMMs leave their split-K partials to the kernel that
    // reads their output first (QK-prep, SwiGLU, the attention delta)
    SplitIn sp_h;
    NE_CHECK(gemm_split(c, NE_PROF_GEMM_FWD, GEMM_NT, EPI_H16, T, QKV, D, a.xn, D, Pb + o.wqkv, D, a.qkv, &sp_h,
                        nullptr, 1.f, ovf + OVF_QKV));
    {
      ProfScope ps(c, NE_PROF_ATTN_FWD);
      NE_CHECK(launch_qk_prep_fwd(dt, a.qkv, QKV, c->cosb, c->sinb, c->c.qk_norm ? P + o.gq : nullptr,
                                  c->c.qk_norm ? P + o.gk : nullptr, a.qr, a.kr, a.rq, a.rk, T, S, c->NH, c->NKV,
                                  c->HD, eps, c->st, sp_h, ovf + OVF_QKV));
      at.q = a.qr; at.ldq = Q; at.k = a.kr; at.ldk = KV; at.v = a.qkv + Q + KV; at.ldv = QKV;
      at.o = a.attn; at.ldo = Q; at.lse = a.lse;
      NE_CHECK(launch_attn_fwd(dt, at, c->st));
    }
    NE_CHECK(gemm_split(c, NE_PROF_GEMM_FWD, GEMM_NT, EPI_RESID, T, D, Q, a.attn, Q, Pb + o.wo, Q, a.x2, &sp_x,
                        a.x_in, alpha));
    {
      ProfScope ps(c, NE_PROF_NORM);
      NE_CHECK(launch_rmsnorm_fwd(dt, a.x2, P + o.g_ffn, a.x2n, a.r2, T, D, eps, ovf + OVF_NORM_FWD, c->st, sp_x));
    }
    if (swiglu_in_gemm(c)) {
      NE_CHECK(gemm_swiglu_fwd(c, a.x2n, Pb + o.w13, a.h13, a.gate));
    } else {
      NE_CHECK(gemm_split(c, NE_PROF_GEMM_FWD, GEMM_NT, EPI_H16, T, 2 * H, D, a.x2n, D, Pb + o.w13, D, a.h13, &sp_h,
                          nullptr, 1.f, ovf + OVF_H13));
      ProfScope ps(c, NE_PROF_NORM);
      NE_CHECK(launch_swiglu_fwd(dt, a.h13, a.gate, T, H, ovf + OVF_SWIGLU, c->st, sp_h, ovf + OVF_H13));
    }
    NE_CHECK(gemm_split(c, NE_PROF_GEMM_FWD, GEMM_NT, EPI_RESID, T, D, H, a.gate, H, Pb + o.w2, H, x_next, &sp_x,
                        a.x2, alpha));
    NE_CHECK(tl_mark(c, c->tl.fwd_l[l]));
  }
  {
    ProfScope ps(c, NE_PROF_NORM);
    NE_CHECK(launch_rmsnorm_fwd(dt, c->xL, P + c->off_gfinal, c->xf, c->rf, T, D, eps, ovf + OVF_NORM_FWD, c->st,
                                sp_x));
  }
  NE_CHECK(tl_mark(c, c->tl.fwd));
  if (upd) NE_CHECK(uq.upto(c->L));
  // classifier: the tied embedding, or its compact rows (vocabulary compaction; padding
  // columns cv..cvp are masked out of the softmax).  The full vocabulary's logits GEMM runs in
  // the pieces of ce_cut, each right after the update of its embedding rows: the last pieces
  // of the update overlap the first pieces of the GEMM.
  const bool compact = c->cv > 0;
  const int Vc = compact ? c->cvp : V, Vvalid = compact ? c->cv : V;
  const h16_t *Ecls = compact ? c->cE : Pb + c->off_E;
  {
    ProfScope ps(c, NE_PROF_CE);
    if (compact) {
      NE_CHECK(wait_update((int)c->ev_adam.size() - 1));
      NE_CHECK(launch_gather_rows16(Pb + c->off_E, c->cids, c->cE, c->cvp, D, c->st));
      NE_CHECK(ce_forward_grad(dt, c->xf, Ecls, c->tok_tgt, T, D, Vc, Vvalid, c->ce_part, c->ce_tgt, c->ce_lse,
                               c->ce_rows, c->loss, c->gs, c->dlogits, ovf + OVF_DLOGITS, c->st));
    } else {
      for (size_t p = 0; p + 1 < c->ce_cut.size(); p++) {
        NE_CHECK(wait_update(c->L + 1 + (int)p));
        NE_CHECK(ce_forward_piece(dt, c->xf, Ecls, c->tok_tgt, T, D, V, V, c->ce_cut[p], c->ce_cut[p + 1],
                                  c->ce_part, c->ce_tgt, c->dlogits, c->st));
      }
      // the loss's mean is taken below, off the backward's chain
      NE_CHECK(ce_forward_finish(dt, c->tok_tgt, T, D, V, V, c->ce_part, c->ce_tgt, c->ce_lse, c->ce_rows, nullptr,
                                 c->gs, c->dlogits, ovf + OVF_DLOGITS, c->st));
    }
  }

  // ---------------- backward (gradients at scale gs until the fp32 sinks) ----------------
  // The dX GEMMs feeding an RMSNorm backward leave their split-K partials to it (sp_d).  The
  // weight-gradient GEMMs run on st2, forked after the kernel producing their dY: what they
  // read (dlogits, the saved activations, the per-layer dbf / dh13 / dqkv) is not written
  // again in this step, so st never waits for them until the join before the gain sums.
  WgradQueue wq{c, two, {}};
  const size_t TD = (size_t)T * D;
  SplitIn sp_d;
  if (compact) {
    // compact embedding gradient, then added to its rows (TD/cpu_ops.h:425-431); the rows
    // outside the compact vocabulary get only the input-embedding gradient
    NE_CHECK(wq.add(NE_PROF_CE, EPI_F32, Vc, D, T, c->dlogits, Vc, c->xf, D, c->gcE, u));
    NE_CHECK(wq.flush());  // the fill and scatter below follow it on the same stream
    ProfScope ps(c, NE_PROF_CE);
    hipStream_t sd = wq.on ? c->st2 : c->st;
    if (fresh) NE_CHECK(launch_fill_f32(G + c->off_E, 0.f, (long)V * D, sd));
    NE_CHECK(launch_scatter_add_rows(G + c->off_E, c->gcE, c->cids, c->cv, D, sd));
    // the embedding gradient as it stands before the input-embedding scatter (which reports
    // its change per row)
    NE_CHECK(wq.sumsq(G + c->off_E, (long)V * D, gn_embed(c), (int)c->gn_emb));
  }
  // The embedding gradient's GEMM (row block p of de_pieces; compaction: none), whose tiles
  // leave the embedding gradient's sum of squares as it stands before the input-embedding
  // scatter (which reports its change per row).
  long de_slot = gn_embed(c);
  auto add_de = [&](int p) -> int {
    if (compact || p >= c->de_pieces) return 0;
    const int r0 = c->de_rows[p], r1 = c->de_rows[p + 1];
    const long ns = gemm_sq_parts(EPI_F32, r1 - r0, D, T, c->ws_elems);
    NE_CHECK(wq.add(NE_PROF_CE, EPI_DW, r1 - r0, D, T, c->dlogits + r0, V, c->xf, D, G + c->off_E + (long)r0 * D, u,
                    c->gn_part + de_slot, ns));
    de_slot += ns;
    return 0;
  };
  if (c->de_pieces == 1) NE_CHECK(add_de(0));
  NE_CHECK(wq.flush());
  if (!compact) {  // the loss's mean, beside the backward on two streams (the join waits for it)
    ProfScope ps(c, NE_PROF_CE);
    hipStream_t sm = c->st;
    if (wq.on) {  // after the row losses (the flush above forks only when it had jobs)
      NE_HIP(hipEventRecord(c->ev_fork, c->st));
      NE_HIP(hipStreamWaitEvent(c->st2, c->ev_fork, 0));
      sm = c->st2;
    }
    NE_CHECK(launch_ce_mean(c->ce_rows, c->loss, T, sm));
  }
  NE_CHECK(gemm_split(c, NE_PROF_CE, GEMM_NN, EPI_F32, T, D, Vc, c->dlogits, Vc, Ecls, D, c->dtmp, &sp_d));
  {
    ProfScope ps(c, NE_PROF_NORM);
    NE_CHECK(launch_rmsnorm_bwd(dt, c->dtmp, c->xL, P + c->off_gfinal, c->rf, nullptr, c->dx,
                                c->dbf + 2 * (size_t)(c->L - 1) * TD, alpha, G + c->off_gfinal, u, T, D,
                                ovf + OVF_NORM_BWD, norm_part(c, 0), c->st, sp_d, true, c->rms_bwd_ref));
  }
  NE_CHECK(tl_mark(c, c->tl.cls));
  for (int l = c->L - 1; l >= 0; l--) {
    LayerAct &a = c->act[l];
    const LayerOff &o = c->lo[l];
    h16_t *dbf_ffn = c->dbf + 2 * (size_t)l * TD, *dbf_att = dbf_ffn + TD;
    h16_t *dh13 = c->dh13 + (size_t)l * T * 2 * H, *dqkv = c->dqkv + (size_t)l * T * QKV;
    // FFN: dbf_ffn = alpha * dx
    NE_CHECK(gemm(c, NE_PROF_GEMM_BWD, OVF_DH13, GEMM_NN, EPI_SWIGLU_BWD, T, H, D, dbf_ffn, D, Pb + o.w2, H, dh13,
                  2 * H, a.h13, 2 * H));
    NE_CHECK(wq.add(NE_PROF_GEMM_BWD, EPI_DW, D, H, T, dbf_ffn, D, a.gate, H, G + o.w2, u,
                    c->gn_part + gn_job(c, l, GN_W2), c->gn_n[GN_W2]));
    NE_CHECK(wq.add(NE_PROF_GEMM_BWD, EPI_DW, 2 * H, D, T, dh13, 2 * H, a.x2n, D, G + o.w13, u,
                    c->gn_part + gn_job(c, l, GN_W13), c->gn_n[GN_W13]));
    NE_CHECK(gemm_split(c, NE_PROF_GEMM_BWD, GEMM_NN, EPI_F32, T, D, 2 * H, dh13, 2 * H, Pb + o.w13, D, c->dtmp,
                        &sp_d));
    {
      ProfScope ps(c, NE_PROF_NORM);
      NE_CHECK(launch_rmsnorm_bwd(dt, c->dtmp, a.x2, P + o.g_ffn, a.r2, c->dx, c->dx2, dbf_att, alpha, G + o.g_ffn,
                                  u, T, D, ovf + OVF_NORM_BWD, norm_part(c, 1 + 2 * l), c->st, sp_d, true, c->rms_bwd_ref));
    }
    // attention: dbf_att = alpha * dx2
    SplitIn sp_o;
    NE_CHECK(gemm_split(c, NE_PROF_GEMM_BWD, GEMM_NN, EPI_H16, T, Q, D, dbf_att, D, Pb + o.wo, Q, c->dattn, &sp_o,
                        nullptr, 1.f, ovf + OVF_DATTN));
    {
      ProfScope ps(c, NE_PROF_ATTN_BWD);
      at.dsp = sp_o;
      at.ovf_dout = ovf + OVF_DATTN;
      at.q = a.qr; at.ldq = Q; at.k = a.kr; at.ldk = KV; at.v = a.qkv + Q + KV; at.ldv = QKV;
      at.o = a.attn; at.ldo = Q; at.lse = a.lse;
      at.dout = c->dattn; at.lddo = Q; at.delta = c->delta;
      at.dq = c->dq; at.lddq = Q; at.dk = c->dk; at.lddk = KV; at.dv = dqkv + Q + KV; at.lddv = QKV;
      at.part = c->attn_split ? c->attn_part : nullptr;
      at.defer_gqa = at.part != nullptr;  // the QK-prep backward sums the per-query-head dK/dV
      at.ovf = ovf + OVF_DV;
      NE_CHECK(launch_attn_bwd(dt, at, c->st));
      NE_CHECK(launch_qk_prep_bwd(dt, c->dq, c->dk, a.qkv, QKV, c->cosb, c->sinb, c->c.qk_norm ? P + o.gq : nullptr,
                                  c->c.qk_norm ? P + o.gk : nullptr, a.rq, a.rk, dqkv,
                                  c->c.qk_norm ? G + o.gq : nullptr, c->c.qk_norm ? G + o.gk : nullptr, u, T, S,
                                  c->NH, c->NKV, c->HD, ovf + OVF_DQKV, c->c.qk_norm ? qk_part(c, l) : nullptr,
                                  c->st, true, at.part, ovf + OVF_DV));
    }
    NE_CHECK(wq.add(NE_PROF_GEMM_BWD, EPI_DW, D, Q, T, dbf_att, D, a.attn, Q, G + o.wo, u,
                    c->gn_part + gn_job(c, l, GN_WO), c->gn_n[GN_WO]));
    NE_CHECK(wq.add(NE_PROF_GEMM_BWD, EPI_DW, QKV, D, T, dqkv, QKV, a.xn, D, G + o.wqkv, u,
                    c->gn_part + gn_job(c, l, GN_WQKV), c->gn_n[GN_WQKV]));
    if (c->de_pieces > 1) NE_CHECK(add_de(c->L - 1 - l));
    NE_CHECK(wq.flush());  // one hand-over per layer
    NE_CHECK(gemm_split(c, NE_PROF_GEMM_BWD, GEMM_NN, EPI_F32, T, D, QKV, dqkv, QKV, Pb + o.wqkv, D, c->dtmp, &sp_d));
    {
      ProfScope ps(c, NE_PROF_NORM);
      // the bottom layer needs no 16-bit copy (the embedding scatter reads the fp32 dx)
      NE_CHECK(launch_rmsnorm_bwd(dt, c->dtmp, a.x_in, P + o.g_att, a.r1, c->dx2, c->dx,
                                  l > 0 ? c->dbf + 2 * (size_t)(l - 1) * TD : nullptr, alpha, G + o.g_att, u, T, D,
                                  ovf + OVF_NORM_BWD, norm_part(c, 2 + 2 * l), c->st, sp_d, true, c->rms_bwd_ref));
    }
    NE_CHECK(tl_mark(c, c->tl.bwd_l[l]));
  }
  NE_CHECK(tl_mark(c, c->tl.bwd));
  NE_CHECK(wq.join());
  NE_CHECK(tl_mark(c, c->tl.join));
  {
    ProfScope ps(c, NE_PROF_NORM);
    NE_CHECK(launch_colsum_batch(c->cs_jobs, c->cs_njobs, std::max(c->D, c->HD), c->st));
    NE_CHECK(launch_sumsq(G + c->n_decay, c->n_params - c->n_decay, c->gn_part + gn_gains(c), GN_GAINS, c->st));
  }
  {
    ProfScope ps(c, NE_PROF_EMBED);
    NE_CHECK(launch_embed_bwd_chain(G + c->off_E, c->tok_in, c->tok_nxt, c->tok_first, c->dx, u, T, D, c->st,
                                    c->gn_part + gn_rows(c)));
  }
  NE_CHECK(tl_mark(c, c->tl.end));
  return 0;
}

// Graph cache: one captured step per (fresh, loss scale, internal gradient scale).
static int train_step_graph(ne_ctx *c, float loss_scale, bool fresh, bool two) {
  for (auto &e : c->graphs)
    if (e.fresh == fresh && e.loss_scale == loss_scale && e.gs == c->gs) {
      NE_HIP(hipGraphLaunch(e.exec, c->st));
      return 0;
    }
  hipGraph_t graph = nullptr;
  NE_HIP(hipStreamBeginCapture(c->st, hipStreamCaptureModeThreadLocal));
  const int rc = train_step_enqueue(c, loss_scale, fresh, two);
  const hipError_t ec = hipStreamEndCapture(c->st, &graph);
  if (rc) {
    if (graph) (void)hipGraphDestroy(graph);
    return rc;
  }
  NE_HIP(ec);
  hipGraphExec_t exec = nullptr;
  const hipError_t ei = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  NE_HIP(ei);
  if (c->graphs.size() >= 8) {  // bounded: drop the oldest
    (void)hipGraphExecDestroy(c->graphs.front().exec);
    c->graphs.erase(c->graphs.begin());
  }
  c->graphs.push_back({fresh, loss_scale, c->gs, exec});
  NE_HIP(hipGraphLaunch(exec, c->st));
  return 0;
}

extern "C" int ne_train_step(ne_ctx *c, const int32_t *tokens, float loss_scale, float *loss_out) {
  if (!c || !tokens) return ne_fail(NE_ERR_ARG, "null argument");
  const int T = c->T, S = c->S, V = c->V;
  // double-buffered pinned staging: wait until the copy issued two calls ago has finished
  const int slot = c->tok_slot;
  c->tok_slot ^= 1;
  NE_HIP(hipEventSynchronize(c->tok_ev[slot]));
  int32_t *h = c->h_tok + (size_t)slot * 4 * T;
  for (int b = 0; b < c->B; b++)
    for (int s = 0; s < S; s++) {
      const int32_t ti = tokens[(long)b * (S + 1) + s], tt = tokens[(long)b * (S + 1) + s + 1];
      if (ti < 0 || ti >= V || tt < 0 || tt >= V) return ne_fail(NE_ERR_ARG, "token id out of [0, %d)", V);
      h[(long)b * S + s] = ti;
      h[T + (long)b * S + s] = c->cv ? c->f2c[tt] : tt;
      if (c->cv && c->f2c[tt] < 0) return ne_fail(NE_ERR_ARG, "target id %d is not in the compact vocabulary", tt);
    }
  // per-id chains of input rows in token order, for the deterministic embedding scatter
  int32_t *nxt = h + 2 * T, *first = h + 3 * T;
  for (int t = 0; t < T; t++) {
    int32_t &last = c->tok_last[h[t]];
    first[t] = last < 0;
    if (last >= 0) nxt[last] = t;
    nxt[t] = -1;
    last = t;
  }
  for (int t = 0; t < T; t++) c->tok_last[h[t]] = -1;
  NE_HIP(hipMemcpyAsync(c->tok_in, h, 4 * (size_t)T * 4, hipMemcpyHostToDevice, c->st));
  NE_HIP(hipEventRecord(c->tok_ev[slot], c->st));
  const bool fresh = c->grads_fresh;
  c->grads_fresh = false;
  // event timing of kernels inside the step needs eager launches; optimizer families don't
  const int step_fams = c->prof.mask & ~((1 << NE_PROF_ADAM) | (1 << NE_PROF_GNORM));
  const bool profiled = c->prof.on && step_fams;
  // per-family event timing needs every kernel of the step on st.  The two-stream step is
  // launched eagerly: replaying it from a graph measured slower than in order on one stream
  // (the branches' hand-overs cost more in a graph than between eager launches).
  const bool two = c->overlap_wgrad && !profiled;
  // a deferred update: the two-stream step runs it beside its forward (UpdateQueue)
  const bool upd = c->upd_deferred && two;
  if (upd) c->upd_deferred = false;
  else NE_CHECK(adam_join(c));
  c->gn_ready = c->gn_parts_ok = false;
  c->last_u = loss_scale / (float)T / c->gs;  // the factor train_step_enqueue gives the fp32 sinks
  // the timeline's events need eager launches too
  if (c->use_graphs && !profiled && !two && !c->tl.on) NE_CHECK(train_step_graph(c, loss_scale, fresh, false));
  else NE_CHECK(train_step_enqueue(c, loss_scale, fresh, two, upd));
  c->tl.step_ok = c->tl.on;
  c->adam_pending = false;  // the forward waited for the last chunk before the backward
  c->gn_ready = true;  // the step refreshed every sum-of-squares partial of G
  c->stats_ok = true;
  if (loss_out) {
    NE_HIP(hipMemcpyAsync(c->h_scalar, c->loss, 4, hipMemcpyDeviceToHost, c->st));
    NE_HIP(hipStreamSynchronize(c->st));
    *loss_out = c->h_scalar[0];
  }
  return 0;
}

extern "C" int ne_use_graphs(ne_ctx *c, int on) {
  if (!c) return ne_fail(NE_ERR_ARG, "null context");
  c->use_graphs = on != 0;
  return 0;
}

extern "C" int ne_overlap_weight_grads(ne_ctx *c, int on) {
  if (!c) return ne_fail(NE_ERR_ARG, "null context");
  if (c->overlap_wgrad == (on != 0)) return 0;
  NE_CHECK(adam_join(c));
  NE_HIP(hipStreamSynchronize(c->st));
  // the captured steps bake the stream layout in
  for (auto &e : c->graphs) (void)hipGraphExecDestroy(e.exec);
  c->graphs.clear();
  c->overlap_wgrad = on != 0;
  return 0;
}

extern "C" int ne_rmsnorm_bwd_formula(ne_ctx *c, int ref) {
  if (!c) return ne_fail(NE_ERR_ARG, "null context");
  if (c->rms_bwd_ref == (ref != 0)) return 0;
  NE_CHECK(adam_join(c));
  NE_HIP(hipStreamSynchronize(c->st));
  // the captured steps bake the kernel choice in
  for (auto &e : c->graphs) (void)hipGraphExecDestroy(e.exec);
  c->graphs.clear();
  c->rms_bwd_ref = ref != 0;
  return 0;
}

extern "C" int ne_set_vocab_map(ne_ctx *c, const int32_t *ids, int cv) {
  if (!c) return ne_fail(NE_ERR_ARG, "null context");
  NE_CHECK(adam_join(c));
  if (cv < 0 || cv > c->V || (cv > 0 && !ids)) return ne_fail(NE_ERR_ARG, "vocab map: %d ids of %d", cv, c->V);
  if (!c->grads_fresh) return ne_fail(NE_ERR_STATE, "vocab map: change it between accumulation windows");
  std::vector<int32_t> f2c(cv ? c->V : 0, -1);
  for (int i = 0; i < cv; i++) {
    if (ids[i] < 0 || ids[i] >= c->V) return ne_fail(NE_ERR_ARG, "vocab map: id %d out of [0, %d)", ids[i], c->V);
    if (f2c[ids[i]] >= 0) return ne_fail(NE_ERR_ARG, "vocab map: id %d repeated", ids[i]);
    f2c[ids[i]] = i;
  }
  NE_HIP(hipStreamSynchronize(c->st));
  // the captured steps bake the classifier in
  for (auto &e : c->graphs) (void)hipGraphExecDestroy(e.exec);
  c->graphs.clear();
  if (c->cids) (void)hipFree(c->cids);
  if (c->cE) (void)hipFree(c->cE);
  if (c->gcE) (void)hipFree(c->gcE);
  c->cids = nullptr; c->cE = nullptr; c->gcE = nullptr;
  c->cv = c->cvp = 0;
  c->f2c.clear();
  if (cv == 0) return 0;
  const int cvp = (cv + 63) / 64 * 64;
  std::vector<int32_t> padded(ids, ids + cv);
  padded.resize(cvp, ids[0]);
  NE_HIP(hipMalloc((void **)&c->cids, (size_t)cvp * sizeof(int32_t)));
  NE_HIP(hipMalloc((void **)&c->cE, (size_t)cvp * c->D * sizeof(h16_t)));
  NE_HIP(hipMalloc((void **)&c->gcE, (size_t)cvp * c->D * sizeof(float)));
  NE_HIP(hipMemcpy(c->cids, padded.data(), (size_t)cvp * sizeof(int32_t), hipMemcpyHostToDevice));
  c->cv = cv;
  c->cvp = cvp;
  c->f2c.swap(f2c);
  return 0;
}

extern "C" int ne_zero_grads(ne_ctx *c) {
  if (!c) return ne_fail(NE_ERR_ARG, "null context");
  NE_CHECK(adam_join(c));
  NE_HIP(hipMemsetAsync(c->ovf, 0, OVF_COUNT * sizeof(int), c->st));
  NE_HIP(hipStreamSynchronize(c->st));
  c->grads_fresh = true;
  c->gn_parts_ok = false;
  return 0;
}

extern "C" int ne_optimizer_step(ne_ctx *c, float lr, float b1, float b2, float eps, float wd, float grad_scale,
                                 float clip, float *gnorm_out) {
  if (!c) return ne_fail(NE_ERR_ARG, "null context");
  NE_CHECK(adam_join(c));
  // overflow check of the accumulation window (dynamic gradient scaling)
  NE_HIP(hipMemcpyAsync(c->h_ovf, c->ovf, OVF_COUNT * sizeof(int), hipMemcpyDeviceToHost, c->st));
  NE_HIP(hipStreamSynchronize(c->st));
  int32_t sites = 0;
  for (int i = 0; i < OVF_COUNT; i++)
    if (c->h_ovf[i]) sites |= 1 << i;
  if (sites) {
    c->last_ovf_sites = sites;
    c->grads_fresh = true;
    NE_HIP(hipMemsetAsync(c->ovf, 0, OVF_COUNT * sizeof(int), c->st));
    NE_HIP(hipStreamSynchronize(c->st));
    c->gs = c->gs * 0.5f;
    c->skipped += 1;
    c->gn_parts_ok = false;
    c->good_steps = 0;
    if (gnorm_out) *gnorm_out = NAN;
    return 1;
  }
  NE_CHECK(tl_mark(c, c->tl.opt0));
  {
    ProfScope ps(c, NE_PROF_GNORM);
    // the last micro-step left the partials of G as it is now; otherwise (G written through
    // ne_set_tensor, or no micro-step since the last update) sum it here
    if (c->gn_ready && !c->grads_fresh) {
      NE_CHECK(launch_clip_finalize(c->gn_part, (int)gn_slots(c), grad_scale, clip, c->gscale, c->gnorm, c->st));
    } else {
      if (c->grads_fresh) NE_CHECK(launch_fill_f32(c->G, 0.f, c->n_params, c->st));
      NE_CHECK(gn_sum_all(c));
      NE_CHECK(launch_clip_finalize(c->gn_part, (int)gn_slots(c), grad_scale, clip, c->gscale, c->gnorm, c->st));
    }
  }
  NE_CHECK(tl_mark(c, c->tl.opt1));
  c->gn_parts_ok = true;
  c->gn_gsc = grad_scale;
  c->state.adam_t += 1;
  const int t = c->state.adam_t;
  AdamArgs a = {};
  a.p = c->P; a.g = c->G; a.m = c->M; a.v = c->Vm; a.pb = c->Pb;
  a.n = c->n_params; a.n_decay = c->n_decay;
  a.lr = lr; a.b1 = b1; a.b2 = b2; a.eps = eps; a.wd = wd;
  a.bc1 = 1.f - powf(b1, (float)t);
  a.bc2 = 1.f - powf(b2, (float)t);
  a.gscale = c->gscale; a.zero_grad = 0;
  if (c->overlap_wgrad) {
    // left to the next training step, which runs it beside its forward (UpdateQueue)
    c->upd = a;
    c->upd_deferred = true;
  } else {
    NE_CHECK(tl_mark(c, c->tl.upd0));
    {
      ProfScope ps(c, NE_PROF_ADAM);
      NE_CHECK(launch_adam(c->dt, a, c->st));
    }
    NE_CHECK(tl_mark(c, c->tl.upd1));
    c->tl.opt_ok = c->tl.on;
  }
  c->grads_fresh = true;
  c->state.lr = lr;
  // grow the internal scale after a long overflow-free run (bounded)
  if (++c->good_steps >= 1000 && c->gs < 65536.f) {
    c->gs *= 2.f;
    c->good_steps = 0;
  }
  if (gnorm_out) {
    NE_HIP(hipMemcpyAsync(c->h_scalar + 1, c->gnorm, 4, hipMemcpyDeviceToHost, c->st));
    NE_HIP(hipStreamSynchronize(c->st));
    *gnorm_out = c->h_scalar[1];
  }
  return 0;
}

extern "C" int ne_grad_scale_info(const ne_ctx *c, float *scale, int32_t *skipped, int32_t *sites) {
  if (!c) return ne_fail(NE_ERR_ARG, "null context");
  if (scale) *scale = c->gs;
  if (skipped) *skipped = c->skipped;
  if (sites) *sites = c->last_ovf_sites;
  return 0;
}

extern "C" int ne_grad_norm_parts(ne_ctx *c, float *out) {
  if (!c || !out) return ne_fail(NE_ERR_ARG, "null argument");
  if (!c->gn_parts_ok) return ne_fail(NE_ERR_STATE, "grad norm parts: no optimizer update since the gradients last changed");
  std::vector<double> h(gn_slots(c));
  NE_HIP(hipMemcpyAsync(h.data(), c->gn_part, h.size() * sizeof(double), hipMemcpyDeviceToHost, c->st));
  NE_HIP(hipStreamSynchronize(c->st));
  double attn = 0, ffn = 0, embed = 0, total = 0;
  for (int l = 0; l < c->L; l++)
    for (long k = 0; k < c->gn_lay; k++) (k < gn_attn_n(c) ? attn : ffn) += h[gn_layer(c, l) + k];
  for (long k = gn_embed(c); k < gn_gains(c); k++) embed += h[k];
  for (long k = gn_rows(c); k < gn_slots(c); k++) embed += h[k];
  for (double v : h) total += v;
  const double sc = c->gn_gsc;
  out[0] = (float)(sqrt(fmax(total, 0.0)) * sc);
  out[1] = (float)(sqrt(fmax(attn, 0.0)) * sc);
  out[2] = (float)(sqrt(fmax(ffn, 0.0)) * sc);
  out[3] = (float)(sqrt(fmax(embed, 0.0)) * sc);
  return 0;
}

extern "C" int ne_step_stats(ne_ctx *c, float *out) {
  if (!c || !out) return ne_fail(NE_ERR_ARG, "null argument");
  if (!c->stats_ok) return ne_fail(NE_ERR_STATE, "step stats: no training step has run");
  const long n = (long)c->T * c->D;
  NE_CHECK(launch_minmax(c->xL, n, c->stats_part, NE_STATS_BLOCKS, c->st));
  NE_CHECK(launch_minmax(c->dx, n, c->stats_part + 2 * NE_STATS_BLOCKS, NE_STATS_BLOCKS, c->st));
  std::vector<float> h(4 * NE_STATS_BLOCKS);
  NE_HIP(hipMemcpyAsync(h.data(), c->stats_part, h.size() * sizeof(float), hipMemcpyDeviceToHost, c->st));
  NE_HIP(hipStreamSynchronize(c->st));
  // a NaN anywhere (a block's NaN partials) makes both ends of that range NaN
  float v[4] = {INFINITY, -INFINITY, INFINITY, -INFINITY};
  for (int k = 0; k < 2; k++)
    for (int b = 0; b < NE_STATS_BLOCKS; b++) {
      const float lo = h[(size_t)(k * NE_STATS_BLOCKS + b) * 2], hi = h[(size_t)(k * NE_STATS_BLOCKS + b) * 2 + 1];
      if (lo != lo || hi != hi || v[2 * k] != v[2 * k]) {
        v[2 * k] = v[2 * k + 1] = NAN;
        continue;
      }
      v[2 * k] = fminf(v[2 * k], lo);
      v[2 * k + 1] = fmaxf(v[2 * k + 1], hi);
    }
  // dx holds the gradient at the internal scale; u > 0 maps it to the reference's scale
  out[0] = v[0];
  out[1] = v[1];
  out[2] = v[2] * c->last_u;
  out[3] = v[3] * c->last_u;
  return 0;
}

// ------------------------------------------------------------------------ profiling ----

extern "C" int ne_timeline(ne_ctx *c, int on) {
  if (!c) return ne_fail(NE_ERR_ARG, "null context");
  Timeline &t = c->tl;
  if (on && !t.start) {
    std::vector<hipEvent_t *> evs = {&t.start, &t.lookup, &t.fwd, &t.cls, &t.bwd, &t.join, &t.end,
                                     &t.opt0,  &t.opt1,   &t.upd0, &t.upd1};
    for (auto &e : t.fwd_l) evs.push_back(&e);
    for (auto &e : t.bwd_l) evs.push_back(&e);
    for (hipEvent_t *e : evs) NE_HIP(hipEventCreate(e));
  }
  t.on = on != 0;
  t.step_ok = t.opt_ok = false;
  return 0;
}

extern "C" int ne_update_launches(const ne_ctx *c) {
  if (!c) return ne_fail(NE_ERR_ARG, "null context");
  return 1 + c->L + (int)c->ce_cut.size() - 1;
}

extern "C" int ne_step_timeline(ne_ctx *c, float *out, float *layer_fwd, float *layer_bwd) {
  if (!c || !out) return ne_fail(NE_ERR_ARG, "null argument");
  const Timeline &t = c->tl;
  if (!t.step_ok) return ne_fail(NE_ERR_STATE, "step timeline: no training step has run with the timeline on");
  NE_HIP(hipEventSynchronize(t.end));
  auto ms = [](hipEvent_t a, hipEvent_t b) -> float {
    float v = 0.f;
    return hipEventElapsedTime(&v, a, b) == hipSuccess ? v : NAN;
  };
  for (int i = 0; i < NE_TL_COUNT; i++) out[i] = NAN;
  out[NE_TL_WAIT] = ms(t.start, t.lookup);
  out[NE_TL_FWD] = ms(t.lookup, t.fwd);
  out[NE_TL_CLS] = ms(t.fwd, t.cls);
  out[NE_TL_BWD] = ms(t.cls, t.bwd);
  out[NE_TL_DWAIT] = ms(t.bwd, t.join);
  out[NE_TL_TAIL] = ms(t.join, t.end);
  out[NE_TL_STEP] = ms(t.start, t.end);
  if (t.opt_ok) {
    NE_HIP(hipEventSynchronize(t.upd1));
    out[NE_TL_OPT] = ms(t.opt0, t.opt1);
    out[NE_TL_UPDATE] = ms(t.upd0, t.upd1);
  }
  for (int l = 0; l < c->L; l++) {
    if (layer_fwd) layer_fwd[l] = ms(l ? t.fwd_l[l - 1] : t.lookup, t.fwd_l[l]);
    if (layer_bwd) layer_bwd[l] = ms(l + 1 < c->L ? t.bwd_l[l + 1] : t.cls, t.bwd_l[l]);
  }
  return 0;
}

extern "C" int ne_prof_enable(ne_ctx *c, int mask) {
  const int on = mask;
  if (!c) return ne_fail(NE_ERR_ARG, "null context");
  NE_CHECK(prof_collect(c));
  c->prof.on = on != 0;
  c->prof.mask = on;
  return 0;
}

extern "C" int ne_prof_reset(ne_ctx *c) {
  if (!c) return ne_fail(NE_ERR_ARG, "null context");
  NE_CHECK(prof_collect(c));
  for (int i = 0; i < NE_PROF_COUNT; i++) {
    c->prof.ms[i] = 0;
    c->prof.cnt[i] = 0;
  }
  return 0;
}

extern "C" int ne_prof_get(ne_ctx *c, int fam, double *ms, int64_t *count) {
  if (!c || fam < 0 || fam >= NE_PROF_COUNT) return ne_fail(NE_ERR_ARG, "bad profiling family");
  NE_CHECK(prof_collect(c));
  if (ms) *ms = c->prof.ms[fam];
  if (count) *count = c->prof.cnt[fam];
  return 0;
}

// ---------------------------------------------------------------------- checkpoints ----

namespace {

size_t ckpt_size(const ne_ctx *c, bool with_qkn) {
  const size_t D = c->D, H = c->H, Q = c->Q, KV = c->KV, V = c->V;
  const size_t per_layer = Q * D + 2 * KV * D + D * Q + 3 * H * D + 2 * D;
  size_t n = c->L * per_layer + D + V * D;
  size_t sz = sizeof(CkptHdr) + 3 * 4 * n;
  if (with_qkn) sz += 12 + (size_t)c->L * 6 * c->HD * 4;
  return sz;
}

int io_tensor(ne_ctx *c, FILE *f, int id, int kind, bool rd, std::vector<float> &buf) {
  const size_t n = c->t_numel[id];
  buf.resize(n);
  float *dev = kind_base(c, kind) + c->t_off[id];
  if (rd) {
    if (fread(buf.data(), 4, n, f) != n) return ne_fail(NE_ERR_FORMAT, "checkpoint truncated at tensor %d", id);
    NE_HIP(hipMemcpy(dev, buf.data(), n * 4, hipMemcpyHostToDevice));
  } else {
    NE_HIP(hipMemcpy(buf.data(), dev, n * 4, hipMemcpyDeviceToHost));
    if (fwrite(buf.data(), 4, n, f) != n) return ne_fail(NE_ERR_IO, "checkpoint write failed at tensor %d", id);
  }
  return 0;
}

// v4 body order: per layer 9 tensors then their (m, v); rms_final, m, v; embed, m, v.
int io_body(ne_ctx *c, FILE *f, bool rd, bool qkn) {
  std::vector<float> buf;
  for (int l = 0; l < c->L; l++) {
    for (int j = 0; j < 9; j++) NE_CHECK(io_tensor(c, f, 9 * l + j, NE_PARAM, rd, buf));
    for (int j = 0; j < 9; j++) {
      NE_CHECK(io_tensor(c, f, 9 * l + j, NE_ADAM_M, rd, buf));
      NE_CHECK(io_tensor(c, f, 9 * l + j, NE_ADAM_V, rd, buf));
    }
  }
  for (int id : {9 * c->L, 9 * c->L + 1})
    for (int kind : {NE_PARAM, NE_ADAM_M, NE_ADAM_V}) NE_CHECK(io_tensor(c, f, id, kind, rd, buf));
  if (qkn) {
    int32_t tag[3] = {QKN_TAG, c->L, c->HD};
    if (rd) {
      if (fread(tag, 4, 3, f) != 3 || tag[0] != QKN_TAG || tag[1] != c->L || tag[2] != c->HD)
        return ne_fail(NE_ERR_FORMAT, "checkpoint QK-norm trailer mismatch");
    } else if (fwrite(tag, 4, 3, f) != 3) {
      return ne_fail(NE_ERR_IO, "checkpoint write failed");
    }
    for (int l = 0; l < c->L; l++)
      for (int j = 0; j < 2; j++)
        for (int kind : {NE_PARAM, NE_ADAM_M, NE_ADAM_V})
          NE_CHECK(io_tensor(c, f, 9 * c->L + 2 + 2 * l + j, kind, rd, buf));
  }
  return 0;
}

}  // namespace

extern "C" int ne_load_ckpt_v4(ne_ctx *c, const char *path, ne_train_state *st) {
  if (!c || !path) return ne_fail(NE_ERR_ARG, "null argument");
  NE_CHECK(adam_join(c));
  NE_HIP(hipStreamSynchronize(c->st));
  FILE *f = fopen(path, "rb");
  if (!f) return ne_fail(NE_ERR_IO, "cannot open %s", path);
  CkptHdr h;
  int rc = 0;
  if (fread(&h, sizeof h, 1, f) != 1) rc = ne_fail(NE_ERR_FORMAT, "%s: short header", path);
  else if (h.magic != CKPT_MAGIC || h.version != 4) rc = ne_fail(NE_ERR_FORMAT, "%s: not a v4 checkpoint", path);
  else if (h.n_layers != c->L || h.vocab_size != c->V || h.dim != c->D || h.hidden_dim != c->H ||
           h.n_heads != c->NH || h.kv_heads != c->NKV || h.head_dim != c->HD || h.q_dim != c->Q)
    rc = ne_fail(NE_ERR_FORMAT, "%s: model dims do not match the context", path);
  if (!rc) {
    fseek(f, 0, SEEK_END);
    const size_t sz = (size_t)ftell(f);
    fseek(f, sizeof h, SEEK_SET);
    const bool qkn = c->c.qk_norm && sz == ckpt_size(c, true);
    if (sz != ckpt_size(c, false) && !qkn)
      rc = ne_fail(NE_ERR_FORMAT, "%s: size %zu, expected %zu", path, sz, ckpt_size(c, c->c.qk_norm));
    else
      rc = io_body(c, f, true, qkn);
  }
  fclose(f);
  if (rc) return rc;
  NE_CHECK(launch_f32_to_h16(c->dt, c->P, c->Pb, c->n_params, c->st));
  NE_HIP(hipStreamSynchronize(c->st));
  c->state.step = h.step; c->state.total_steps = h.total_steps; c->state.lr = h.lr; c->state.loss = h.loss;
  c->state.cum_compile = h.cum_compile; c->state.cum_train = h.cum_train; c->state.cum_wall = h.cum_wall;
  c->state.cum_steps = h.cum_steps; c->state.cum_batches = h.cum_batches; c->state.adam_t = h.adam_t;
  if (st) *st = c->state;
  return 0;
}

extern "C" int ne_save_ckpt_v4(ne_ctx *c, const char *path, const ne_train_state *st) {
  if (!c || !path) return ne_fail(NE_ERR_ARG, "null argument");
  NE_CHECK(adam_join(c));
  NE_HIP(hipStreamSynchronize(c->st));
  const ne_train_state &s = st ? *st : c->state;
  CkptHdr h = {};
  h.magic = CKPT_MAGIC; h.version = 4; h.step = s.step; h.total_steps = s.total_steps;
  h.n_layers = c->L; h.vocab_size = c->V; h.dim = c->D; h.hidden_dim = c->H; h.n_heads = c->NH; h.seq_len = c->S;
  h.lr = s.lr; h.loss = s.loss;
  h.cum_compile = s.cum_compile; h.cum_train = s.cum_train; h.cum_wall = s.cum_wall;
  h.cum_steps = s.cum_steps; h.cum_batches = s.cum_batches; h.adam_t = s.adam_t;
  h.kv_heads = c->NKV; h.head_dim = c->HD; h.q_dim = c->Q;
  FILE *f = fopen(path, "wb");
  if (!f) return ne_fail(NE_ERR_IO, "cannot create %s", path);
  int rc = 0;
  if (fwrite(&h, sizeof h, 1, f) != 1) rc = ne_fail(NE_ERR_IO, "%s: header write failed", path);
  if (!rc) rc = io_body(c, f, false, c->c.qk_norm != 0);
  if (fclose(f) != 0 && !rc) rc = ne_fail(NE_ERR_IO, "%s: close failed", path);
  return rc;
}

namespace {

// MT19937 (Matsumoto & Nishimura 1998, "Mersenne Twister: a 623-dimensionally equidistributed
// uniform pseudo-random number generator"): 624-word state, initialised from a 32-bit seed by
// the published recurrence x[i] = 1812433253 * (x[i-1] ^ (x[i-1] >> 30)) + i, and the 53-bit
// double of two draws, (a >> 5) * 2^26 + (b >> 6) over 2^53 -- what numpy's legacy
// RandomState(seed).random_sample() returns for an integer seed, and so the draw of
// np.random.choice in TD/tools/generate.py:215 after np.random.seed(seed) (generate.py:248-249).
struct MT19937 {
  uint32_t x[624];
  int i = 624;
  explicit MT19937(uint32_t seed) {
    x[0] = seed;
    for (int k = 1; k < 624; k++) x[k] = 1812433253u * (x[k - 1] ^ (x[k - 1] >> 30)) + (uint32_t)k;
  }
  uint32_t next() {
    if (i >= 624) {
      for (int k = 0; k < 624; k++) {
        const uint32_t y = (x[k] & 0x80000000u) | (x[(k + 1) % 624] & 0x7fffffffu);
        x[k] = x[(k + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
      }
      i = 0;
    }
    uint32_t y = x[i++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
  }
  double uniform() {
    const uint32_t a = next() >> 5, b = next() >> 6;
    return (a * 67108864.0 + b) / 9007199254740992.0;
  }
};

}  // namespace

extern "C" int ne_mt19937_uniforms(uint64_t seed, int64_t n, double *out) {
  if (!out || n < 0) return ne_fail(NE_ERR_ARG, "mt19937: null output or negative count");
  if (seed > 0xffffffffull) return ne_fail(NE_ERR_ARG, "mt19937: seed must be in [0, 2^32)");
  MT19937 mt((uint32_t)seed);
  for (int64_t k = 0; k < n; k++) out[k] = mt.uniform();
  return 0;
}

extern "C" int ne_decode_seeded(ne_ctx *c, const int32_t *prompt, int B, int P, int n_new, float temperature,
                                float top_p, uint64_t seed, int32_t *out_tokens) {
  if (!c || !prompt || !out_tokens) return ne_fail(NE_ERR_ARG, "null argument");
  if (B <= 0 || n_new <= 0) return ne_fail(NE_ERR_ARG, "decode: B=%d n_new=%d", B, n_new);
  if (temperature < 1e-6f) return ne_decode(c, prompt, B, P, n_new, temperature, top_p, nullptr, out_tokens);
  // one draw per sampled token, position by position, the sequences of a position in order
  std::vector<double> s((size_t)B * n_new), u((size_t)B * n_new);
  NE_CHECK(ne_mt19937_uniforms(seed, (int64_t)s.size(), s.data()));
  for (int j = 0; j < n_new; j++)
    for (int b = 0; b < B; b++) u[(size_t)b * n_new + j] = s[(size_t)j * B + b];
  return ne_decode(c, prompt, B, P, n_new, temperature, top_p, u.data(), out_tokens);
}

extern "C" int ne_decode(ne_ctx *c, const int32_t *prompt, int B, int P, int n_new, float temperature, float top_p,
                         const double *uniforms, int32_t *out_tokens) {
  if (!c || !prompt || !out_tokens) return ne_fail(NE_ERR_ARG, "null argument");
  NE_CHECK(adam_join(c));
  return decode_run(c, prompt, B, P, n_new, temperature, top_p, uniforms, out_tokens);
}
