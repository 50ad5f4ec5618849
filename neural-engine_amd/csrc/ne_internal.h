// Internal host-side declarations shared by the kernel files and the orchestrator.
// `dt` selects the 16-bit format (0 bf16, 1 fp16); `ovf` (nullable) is a device int set
// to 1 when a 16-bit result is not finite.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

typedef uint16_t h16_t;

// ---- error plumbing (thread-local last error, negative status codes) ----
int ne_fail(int code, const char *fmt, ...);
int ne_hip_status(hipError_t e, const char *what);
#define NE_HIP(call)                                       \
  do {                                                     \
    hipError_t _e = (call);                                \
    if (_e != hipSuccess) return ne_hip_status(_e, #call); \
  } while (0)
#define NE_CHECK(call)      \
  do {                      \
    int _r = (call);        \
    if (_r != 0) return _r; \
  } while (0)

enum {
  NE_ERR_ARG = -1,     // invalid argument / unsupported shape
  NE_ERR_STATE = -2,   // call not valid in the current context state
  NE_ERR_IO = -3,      // file open/read/write failure
  NE_ERR_FORMAT = -4,  // checkpoint magic/version/dims/size mismatch
  NE_ERR_NOMEM = -5,
};

// ---- GEMM: C[M,N] = epilogue(alpha * A[M,K] . B[K,N]) on 16-bit MFMA (k_gemm.hip) ----
// layout bit 0: A stored M-contiguous ([K,M]); bit 1: B stored N-contiguous ([K,N]).
enum { GEMM_NT = 0, GEMM_NN = 2, GEMM_TN = 3 };
enum {
  EPI_H16 = 0,         // C 16-bit
  EPI_F32 = 1,         // C fp32
  EPI_F32_ACC = 2,     // C fp32 += result
  EPI_RESID = 3,       // C fp32 = R fp32 + result
  EPI_SWIGLU_BWD = 4,  // result is dgate [M,N]; R = h13 16-bit [M,2N]; C = dh13 16-bit [M,2N]
  EPI_CE_FWD = 5,      // result is logits; writes per-(row, N-tile) max/sumexp + target logit
  EPI_CE_BWD = 6,      // C 16-bit = (exp(logit - lse) - onehot) * scale
  EPI_SWIGLU_FWD = 7,  // B = [W1; W3] [N,K] (layout NT); C = h13 16-bit [M,N]; C2 = gate 16-bit [M,N/2]
};

struct GemmArgs {
  int M, N, K;
  const void *A; long lda;
  const void *B; long ldb;
  void *C; long ldc;
  const void *R; long ldr;   // EPI_RESID: fp32 residual; EPI_SWIGLU_BWD: 16-bit h13
  float alpha;
  float scale;               // EPI_CE_BWD gradient scale
  const int32_t *targets;    // [M] (CE epilogues)
  const float *lse;          // [M] (EPI_CE_BWD)
  float *part;               // [M, n_tiles, 2] (EPI_CE_FWD): tile max, tile sum exp
  float *tgt_logit;          // [M] (EPI_CE_FWD)
  int *ovf;                  // 16-bit outputs: overflow flag (nullable)
  void *C2; long ldc2;       // EPI_SWIGLU_FWD: the gate silu(h1) * h3
  int *ovf2;                 // EPI_SWIGLU_FWD: the gate's overflow flag (nullable)
  float *ws;                 // split-K workspace (nullable: no split)
  long ws_elems;             // its capacity in floats
  int n_tiles;               // set by the launcher: N / BN
  int split;                 // set by the launcher: K splits (grid.z)
  int defer_reduce;          // with K splits, leave the fp32 partials in ws for the consumer
  int n_valid;               // CE epilogues: columns >= n_valid are outside the softmax (0: N)
  int col0;                  // CE epilogues: the full output's column of this launch's column 0
  int tile0;                 // EPI_CE_FWD: the partial slot of this launch's first N tile
  int part_ld;               // EPI_CE_FWD: partial slots per row (0: N / BN)
  double *sq;                // EPI_F32 / EPI_F32_ACC (nullable): sums of squares of C as stored,
                             // one slot per output tile (mt * N/BN + nt) or, with split-K, per
                             // block of the ordered reduction; gemm_sq_parts slots in all
};

// Up to GEMM_GROUP_MAX GEMMs run as one launch (gemm_group_launch): problem p's tiles are
// the work-groups [first[p], first[p + 1]).
constexpr int GEMM_GROUP_MAX = 4;
struct GemmGroup {
  GemmArgs g[GEMM_GROUP_MAX];
  int first[GEMM_GROUP_MAX + 1];
  int n;
};

// Split-K partials of a GEMM whose reduction is folded into its consumer: element e of the
// result is base[e] + alpha * sum_{z < n} part[z * slice + e] (z ascending, the order of the
// GEMM's own reduction).  n = 0: no partials.
struct SplitIn {
  const float *part = nullptr;
  int n = 0;
  long slice = 0;
  const float *base = nullptr;  // nullable
  float alpha = 1.f;
};

// *split_out (nullable) receives the K splits used; with a.defer_reduce and more than one
// split, C is not written and the partials stay in a.ws (M*N floats per split).
int gemm_launch(int dt, int layout, int epi, GemmArgs a, hipStream_t s, int *split_out = nullptr);
int gemm_ce_tiles(int M, int N, int K);  // EPI_CE_FWD: the partial slots per row it writes
// EPI_CE_FWD's column tiling: columns [0, main_cols) in tiles of w_main, the rest in tiles of
// w_rest; partial slot of column c: c < main_cols ? c / w_main : main_cols / w_main +
// (c - main_cols) / w_rest.
void gemm_ce_layout(int M, int N, int K, int *main_cols, int *w_main, int *w_rest);
// Column pieces of EPI_CE_FWD's M x N x K GEMM that run with the whole shape's tiles: cut[0] = 0
// < cut[1] < ... < cut[np] = N on its tile boundaries, each piece as many tiles as run at once
// on the device (the last takes the remainder).  Returns np (<= max_pieces; 1 when the shape is
// ragged or a piece would plan another tile).
int gemm_ce_pieces(int M, int N, int K, int max_pieces, int *cut);
// Whether columns [c0, c1) are such a piece (or the whole).
bool gemm_ce_piece_ok(int M, int N, int K, int c0, int c1);
// K splits gemm_launch would use for this shape with a workspace of ws_elems floats (1: none).
int gemm_splits(int epi, int M, int N, int K, long ws_elems);
// Sum-of-squares slots (GemmArgs::sq) gemm_launch writes for this shape (EPI_F32 /
// EPI_F32_ACC, no deferred reduction), ws_elems as for gemm_splits; with gemm_group_launch
// a problem writes (M / 256) * (N / 256).
long gemm_sq_parts(int epi, int M, int N, int K, long ws_elems);
// Weight-gradient GEMMs (layout TN, fp32 out: EPI_F32 or EPI_F32_ACC, one epilogue for all)
// of n <= GEMM_GROUP_MAX problems as one launch of 256x256 tiles, each over its whole K range
// (no split-K, no workspace).  gemm_group_fits: whether a set of shapes takes this path (every
// M and N a multiple of 256, K >= 8192, and at least 192 tiles in all: a long reduction into
// outputs that alone would need split-K to fill the CUs).
bool gemm_group_fits(const GemmArgs *g, int n);
int gemm_group_launch(int dt, int epi, const GemmArgs *g, int n, hipStream_t s);
// Measurement kernel: MFMA chains without memory traffic (shape 0 = 32x32x16, 1 = 16x16x32).
int launch_mfma_ceiling(int dt, int shape, int blocks, int iters, float *out, hipStream_t s);

// ---- embedding / normalisation / elementwise (k_norm.hip) ----
int launch_embed_fwd(const float *E, const int32_t *tok, float *x, int T, int D, hipStream_t s);
int launch_embed_bwd(float *gE, const int32_t *tok, const float *dx, float scale, int T, int D,
                     hipStream_t s);
// Deterministic scatter over per-id row chains (nxt / first arrays built on the host).
// dsq (nullable, [T] doubles): per row, the change of the sum of squares of the gE row it
// updated (0 for rows that are not the first of their id).
int launch_embed_bwd_chain(float *gE, const int32_t *tok, const int32_t *nxt, const int32_t *first,
                           const float *dx, float scale, int T, int D, hipStream_t s, double *dsq = nullptr);
// With sp.n > 0, x is formed from split-K partials (SplitIn) and written to x before use.
int launch_rmsnorm_fwd(int dt, const float *x, const float *g, h16_t *y, float *r, int T, int D,
                       float eps, int *ovf, hipStream_t s, const SplitIn &sp = SplitIn());
// Gain gradients: with `part` (scratch of *_part_elems floats) per-block partials are summed
// in a second, ordered pass (deterministic); without it blocks add atomically.
long rmsnorm_bwd_part_elems(int T, int D);
long qk_prep_bwd_part_elems(int T, int NH, int NKV, int HD);
// With sp.n > 0, dy is formed from split-K partials (SplitIn) instead of read.  With
// defer_colsum the partials are left for one colsum_batch launch (ColsumJob) later.  With
// ref_formula dx follows the reference's formula (gain factor on the projection term too).
int launch_rmsnorm_bwd(int dt, const float *dy, const float *x, const float *g, const float *r,
                       const float *resid, float *dx, h16_t *dxb, float bscale, float *dg,
                       float dg_scale, int T, int D, int *ovf, float *part, hipStream_t s,
                       const SplitIn &sp = SplitIn(), bool defer_colsum = false, bool ref_formula = false);
// Ordered column sums of per-block partial rows: out[j] += sum_r part[r * n + j], r ascending
// in the fixed grouping of colsum_kernel, for several independent jobs in one launch.
struct ColsumJob {
  const float *part;
  float *out;
  int rows, n;
};
int rmsnorm_bwd_part_rows(int T);                              // partial rows of one rmsnorm_bwd
void qk_prep_bwd_part_rows(int T, int NH, int NKV, int HD, int *rows_q, int *rows_k);
int launch_colsum_batch(const ColsumJob *jobs_dev, int njobs, int max_n, hipStream_t s);
// With sp.n > 0 the 16-bit input (h13 / qkv, the GEMM's output) is formed from split-K
// partials and written before use; ovf_h13 / ovf_qkv take the GEMM's overflow flag.
int launch_swiglu_fwd(int dt, const h16_t *h13, h16_t *gate, int T, int H, int *ovf, hipStream_t s,
                      const SplitIn &sp = SplitIn(), int *ovf_h13 = nullptr);
int launch_qk_prep_fwd(int dt, const h16_t *qkv, long ld, const float *cosb, const float *sinb,
                       const float *gq, const float *gk, h16_t *qr, h16_t *kr, float *rq, float *rk,
                       int T, int S, int NH, int NKV, int HD, float eps, hipStream_t s,
                       const SplitIn &sp = SplitIn(), int *ovf_qkv = nullptr);
int launch_qk_prep_bwd(int dt, const float *dq, const float *dk, const h16_t *qkv, long ld,
                       const float *cosb, const float *sinb, const float *gq, const float *gk,
                       const float *rq, const float *rk, h16_t *dqkv, float *dgq, float *dgk,
                       float dg_scale, int T, int S, int NH, int NKV, int HD, int *ovf, float *part,
                       hipStream_t s, bool defer_colsum = false, const float *kvpart = nullptr,
                       int *ovf_v = nullptr);

// ---- attention (k_attn.hip): causal, GQA kv head = q head / (NH/NKV) ----
struct AttnArgs {
  const h16_t *q; long ldq;   // [T, NH*HD] rows of the batch-major token index t = b*S + s
  const h16_t *k; long ldk;   // [T, NKV*HD]
  const h16_t *v; long ldv;   // [T, NKV*HD]
  h16_t *o; long ldo;         // [T, NH*HD]
  float *lse;                 // [T, NH] natural-log sum exp of scaled scores
  // backward
  const h16_t *dout; long lddo;  // [T, NH*HD]
  float *delta;                  // [T, NH] rowsum(dO * O) (scratch)
  float *dq; long lddq;          // [T, NH*HD] fp32
  float *dk; long lddk;          // [T, NKV*HD] fp32
  h16_t *dv; long lddv;          // [T, NKV*HD] 16-bit
  float *part;                   // nullable: [2][T, NH*HD] fp32 per-query-head dK/dV partials
                                 // (GQA only: one block per query head, then a head-order sum)
  bool defer_gqa;                // with part: leave the per-query-head dK/dV partials in part
                                 // (launch_qk_prep_bwd with kvpart sums them; dk, dv unwritten)
  SplitIn dsp;                   // split-K partials of dout (its GEMM's reduction, done by the
                                 // delta kernel, which writes dout); dsp.n = 0: dout is written
  int *ovf_dout;                 // overflow flag of dout's 16-bit rounding (with dsp)
  int *ovf;
  int B, S, NH, NKV, HD;
  float scale;
};
int launch_attn_fwd(int dt, const AttnArgs &a, hipStream_t s);
int launch_attn_bwd(int dt, const AttnArgs &a, hipStream_t s);
// Whether the backward at this shape should take per-query-head dK/dV partials (AttnArgs::part)
// with GQA: yes when the KV heads alone give too few dK/dV blocks to fill the device.
bool attn_bwd_split_heads(int B, int S, int NH, int NKV);

// ---- cross-entropy (k_ce.hip over the EPI_CE_* GEMM epilogues) ----
// The row log-sum-exp and loss of the logits GEMM's tile partials (launch_ce_rows), and the
// mean of the row losses (launch_ce_mean); launch_ce_reduce runs both.
int launch_ce_rows(const float *part, int n_tiles, const float *tgt_logit, float *lse, float *loss_rows, int T,
                   hipStream_t s);
int launch_ce_mean(const float *loss_rows, float *loss, int T, hipStream_t s);
int launch_ce_reduce(const float *part, int n_tiles, const float *tgt_logit, float *lse,
                     float *loss_rows, float *loss, int T, hipStream_t s);
// V columns of which the first n_valid take part in the softmax (n_valid <= V; the rest
// are padding: no probability, zero gradient).
int ce_forward(int dt, const void *x, const void *E, const int32_t *targets, int T, int D, int V,
               int n_valid, float *part, float *tgt_logit, float *lse, float *loss_rows, float *loss,
               hipStream_t s);
int ce_backward(int dt, const void *x, const void *E, const int32_t *targets, const float *lse,
                int T, int D, int V, int n_valid, float scale, void *dlogits, int *ovf, hipStream_t s);
// The forward with its gradient: the logits GEMM also stores e = exp(logit - tile max) in
// dlogits (16-bit [T, V]), and after the row reduction one streaming pass turns it in place
// into (softmax - onehot) * scale (no second logits GEMM).  ovf: the gradient's overflow flag.
int ce_forward_grad(int dt, const void *x, const void *E, const int32_t *targets, int T, int D, int V,
                    int n_valid, float *part, float *tgt_logit, float *lse, float *loss_rows, float *loss,
                    float scale, void *dlogits, int *ovf, hipStream_t s);
// The same in parts: ce_forward_piece runs the logits GEMM over vocabulary columns [c0, c1)
// (boundaries from gemm_ce_pieces(T, V, D, ...)) against E rows [c0, c1); once every piece has
// run, ce_forward_finish reduces the rows and forms the gradient (loss null: the mean of the row
// losses is left to the caller, launch_ce_mean).  The pieces give the same bits as the whole.
int ce_forward_piece(int dt, const void *x, const void *E, const int32_t *targets, int T, int D, int V,
                     int n_valid, int c0, int c1, float *part, float *tgt_logit, void *dlogits, hipStream_t s);
int ce_forward_finish(int dt, const int32_t *targets, int T, int D, int V, int n_valid, float *part,
                      float *tgt_logit, float *lse, float *loss_rows, float *loss, float scale, void *dlogits,
                      int *ovf, hipStream_t s);
int launch_ce_grad(int dt, h16_t *dl, int T, int V, int n_valid, const float *part, int n_tiles, int main_cols,
                   int w_main, int w_rest, const float *lse, const float *tgt_logit, const int32_t *targets,
                   float scale, int *ovf, hipStream_t s);
// Vocabulary compaction: dst[r] = src[ids[r]] (16-bit rows of D); G[ids[r]] += src[r] for
// r < n (fp32 rows of D; the ids are distinct).
int launch_gather_rows16(const h16_t *src, const int32_t *ids, h16_t *dst, int n, int D, hipStream_t s);
int launch_scatter_add_rows(float *G, const float *src, const int32_t *ids, int n, int D, hipStream_t s);

// ---- optimizer (k_optim.hip) ----
struct AdamArgs {
  float *p, *g, *m, *v;
  h16_t *pb;            // 16-bit shadow of p (may be null)
  long n, n_decay;      // elements [0, n_decay) get weight decay
  float lr, b1, b2, eps, wd, bc1, bc2;
  const float *gscale;  // device scalar: grad_scale * clip factor
  const int *skip;      // device flag: when set, leave p/m/v untouched (overflowed step)
  int zero_grad;        // write g = 0 after the update
  int max_groups;       // work-group cap of the launch (0: the streaming default)
};
int launch_sumsq(const float *g, long n, double *partials, int nparts, hipStream_t s);
// Embedding lookup x[t] = E[tok[t]] with the AdamW update a (weight decay on; its gscale on
// the device) applied to the rows read, as adam_kernel would leave them; writes only x.
int launch_embed_fwd_adam(const float *E, const float *G, const float *M, const float *V, const int32_t *tok,
                          float *x, int T, int D, const AdamArgs &a, hipStream_t s);
int launch_clip_finalize(const double *partials, int nparts, float grad_scale, float clip,
                         float *gscale_out, float *gnorm_out, hipStream_t s);
int launch_adam(int dt, const AdamArgs &a, hipStream_t s);
int launch_f32_to_h16(int dt, const float *src, h16_t *dst, long n, hipStream_t s);
int launch_fill_f32(float *dst, float v, long n, hipStream_t s);
// Per-block minimum and maximum of a[0, n): out[2*b] = min, out[2*b + 1] = max over the
// elements of block b (nblocks blocks, grid-strided; a block with no element writes +inf, -inf).
int launch_minmax(const float *a, long n, float *out, int nblocks, hipStream_t s);
