// The context object shared by the orchestrator (ne_host.hip) and the token loop
// (k_decode.hip).
#pragma once
#include <vector>

#include "../../include/ne.h"
#include "ne_internal.h"

struct Prof {
  bool on = false;
  int mask = 0;  // families with event pairs
  std::vector<hipEvent_t> pool;
  struct Rec { int fam; hipEvent_t a, b; };
  std::vector<Rec> pending;
  double ms[NE_PROF_COUNT] = {};
  int64_t cnt[NE_PROF_COUNT] = {};
  hipEvent_t get() {
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    hipEvent_t e;
    hipEventCreate(&e);
    return e;
  }
};

// 16-bit conversion sites with an overflow flag each
enum {
  OVF_NORM_FWD = 0, OVF_QKV, OVF_H13, OVF_SWIGLU, OVF_DLOGITS, OVF_NORM_BWD, OVF_DH13, OVF_DATTN,
  OVF_DV, OVF_DQKV, OVF_COUNT
};

constexpr int NE_STATS_BLOCKS = 256;

// Phase timeline (ne_timeline): timing events recorded at the phase boundaries of the step on
// st and around the optimizer's update, without changing the schedule (the two-stream step
// stays two-stream; only the captured single-stream graph is replaced by eager launches).
struct Timeline {
  bool on = false;
  bool step_ok = false, opt_ok = false;  // the last step / optimizer call recorded its events
  hipEvent_t start = nullptr, lookup = nullptr, fwd = nullptr, cls = nullptr, bwd = nullptr, join = nullptr,
             end = nullptr;
  hipEvent_t opt0 = nullptr, opt1 = nullptr, upd0 = nullptr, upd1 = nullptr;
  std::vector<hipEvent_t> fwd_l, bwd_l;  // end of layer l's forward / backward on st
};

struct LayerAct {
  float *x_in, *r1, *x2, *r2, *rq, *rk, *lse;
  h16_t *xn, *qkv, *qr, *kr, *attn, *x2n, *h13, *gate;
};

struct LayerOff {
  long wqkv, wo, w13, w2, g_att, g_ffn, gq, gk;
};

struct ne_ctx {
  ne_config c;
  int D, H, NH, NKV, HD, L, V, S, B, T, Q, KV, QKV;
  int dt;                 // 16-bit format (NE_BF16 / NE_FP16)
  float gs = 256.f;       // internal gradient scale: dlogits = (p - onehot) * gs
  int32_t skipped = 0;    // optimizer steps skipped after a 16-bit overflow
  int good_steps = 0;     // consecutive non-overflowing optimizer steps
  hipStream_t st = nullptr;
  // weight-gradient GEMMs run on st2 beside the dX chain on st: forked after the GEMM that
  // produces each dY, joined once before the end of the backward
  hipStream_t st2 = nullptr;
  hipEvent_t ev_fork = nullptr, ev_join = nullptr;
  // Two-stream schedule: ne_optimizer_step leaves its AdamW pass (upd, after the norm and
  // clip on st) to the next training step, which enqueues it on st2 in chunks, each marked by
  // ev_adam[k] (0: the gains, 1 + l: layer l, L + 1 + p: the embedding rows of classifier piece
  // p), and waits for chunk k just before it reads what the chunk writes; its lookup computes
  // the updated rows itself, and the embedding's pieces start after it (ev_lookup).
  // upd_deferred: such a pass has not been enqueued yet (any other entry point that touches
  // the parameters runs it on st first); adam_pending: enqueued, not yet waited for by st.
  std::vector<hipEvent_t> ev_adam;
  // The classifier's vocabulary pieces (gemm_ce_pieces of the T x V x D logits GEMM): columns
  // [ce_cut[p], ce_cut[p + 1]), each run after the AdamW chunk of its embedding rows.
  std::vector<int> ce_cut;
  hipEvent_t ev_lookup = nullptr;
  AdamArgs upd = {};
  bool upd_deferred = false;
  bool adam_pending = false;
  long n_params = 0, n_decay = 0;
  float *P = nullptr, *G = nullptr, *M = nullptr, *Vm = nullptr;
  h16_t *Pb = nullptr;
  std::vector<LayerOff> lo;
  long off_E = 0, off_gfinal = 0;
  std::vector<long> t_off, t_numel;  // per tensor id
  void *arena = nullptr;
  std::vector<LayerAct> act;
  float *xL, *rf;
  h16_t *xf;
  float *dx, *dx2, *dtmp, *dq, *dk, *delta, *attn_part;
  bool attn_split = false;  // GQA attention backward through per-query-head partials (attn_part)
  // per layer (the weight-gradient GEMMs on st2 read them while st moves on): dbf [2L][T, D]
  // (alpha * dx into the FFN of layer l at 2l, into its attention at 2l + 1), dh13 [L][T, 2H],
  // dqkv [L][T, QKV]
  h16_t *dbf, *dh13, *dattn, *dqkv, *dlogits;
  float *ce_part, *ce_tgt, *ce_lse, *ce_rows, *loss;
  int32_t *tok_in, *tok_tgt, *tok_nxt, *tok_first;  // [T] each, one staging copy
  std::vector<int32_t> tok_last;                     // host scratch [V] for the id chains
  float *cosb, *sinb;
  // sum-of-squares partials of the gradient, in a fixed reduction order: gn_slots() slots.
  // The step fills them as each part of G becomes final (see gn_layer etc. in ne_host.hip);
  // gn_ready: they describe G as it is now (else the optimizer sums G itself)
  double *gn_part;
  // slots per layer of its Wqkv, Wo, W13, W2 weight-gradient GEMMs (one per tile, the tiling
  // the launches take, fixed by the shapes) and of the embedding gradient's GEMM
  long gn_n[4] = {0, 0, 0, 0};
  long gn_lay = 0, gn_emb = 0;
  // the embedding gradient's GEMM in de_pieces row blocks (de_rows[p], p <= de_pieces), piece
  // p queued with the weight gradients of the (p+1)-th layer the backward reaches
  int de_pieces = 1;
  std::vector<int> de_rows;
  bool gn_grouped = false;  // a layer's weight gradients run as one grouped launch
  bool gn_ready = false;
  // the last non-skipped optimizer step summed gn_part over G as it then was, at grad_scale
  // gn_gsc (ne_grad_norm_parts reads the groups back until the next step or gradient write)
  bool gn_parts_ok = false;
  float gn_gsc = 1.f;
  float *stats_part;      // device [2][2 * NE_STATS_BLOCKS] min/max partials (ne_step_stats)
  float last_u = 0.f;     // fp32-sink factor of the last step: reference-scale dx = dx * last_u
  bool stats_ok = false;  // a step has run since the context was created
  float *gscale, *gnorm;
  int *ovf;               // device flags [32], one per conversion site (OVF_*): a 16-bit value
                          // of this accumulation window was not finite
  int32_t last_ovf_sites = 0;  // bit mask of the sites that flagged the last skipped step
  bool grads_fresh = true;     // G holds no accumulation yet: the next step overwrites it
  float *ws = nullptr;         // split-K workspace (st)
  float *ws2 = nullptr;        // split-K workspace of the weight-gradient GEMMs (st2)
  long ws_elems = 0;           // capacity of each, floats
  float *gpart = nullptr;      // per-block gain-gradient partials: one slab per norm site
  long rms_slab = 0, qk_slab = 0;  // floats per RMSNorm / QK-norm site
  ColsumJob *cs_jobs = nullptr;    // device table: every site's ordered partial sum, one launch
  int cs_njobs = 0;
  int32_t *h_tok = nullptr;  // pinned [2][4T] (double-buffered token staging)
  hipEvent_t tok_ev[2] = {nullptr, nullptr};
  int tok_slot = 0;
  // captured training steps (HIP graphs), keyed by what changes kernel arguments
  struct GraphEntry { bool fresh; float loss_scale; float gs; hipGraphExec_t exec; };
  std::vector<GraphEntry> graphs;
  bool use_graphs = true;
  bool overlap_wgrad = true;  // weight-gradient GEMMs on st2 (ne_overlap_weight_grads)
  bool rms_bwd_ref = false;   // the reference's RMSNorm backward formula (ne_rmsnorm_bwd_formula)
  float *h_scalar = nullptr; // pinned [4]
  int *h_ovf = nullptr;      // pinned [32]
  ne_train_state state = {};
  Prof prof;
  Timeline tl;
  // vocabulary compaction: the classifier covers cv embedding rows (cvp = cv rounded up to
  // 64, the padding columns masked out of the softmax)
  int cv = 0, cvp = 0;
  int32_t *cids = nullptr;   // device [cvp] full ids of the compact rows (padding repeats ids[0])
  h16_t *cE = nullptr;       // device [cvp, D] 16-bit compact embedding, gathered each step
  float *gcE = nullptr;      // device [cvp, D] compact embedding gradient
  std::vector<int32_t> f2c;  // host [V] full -> compact id, -1 outside
  // token loop (k_decode.hip)
  void *dec = nullptr;
};

