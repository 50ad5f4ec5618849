// Error plumbing and the kernel-level C-ABI entry points (device pointers).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "../../include/ne.h"
#include "ne_internal.h"

static thread_local char g_err[512] = "";

int ne_fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int ne_hip_status(hipError_t e, const char *what) {
  if (e == hipSuccess) return 0;
  snprintf(g_err, sizeof g_err, "%s: %s", what, hipGetErrorString(e));
  return -1000 - (int)e;
}

extern "C" const char *ne_last_error(void) { return g_err; }

#define S(stream) ((hipStream_t)(stream))
#define CHECK_DT(dt) \
  if ((dt) != NE_BF16 && (dt) != NE_FP16) return ne_fail(NE_ERR_ARG, "unknown 16-bit format %d", (dt))

extern "C" int ne_k_rmsnorm_fwd(int dtype, const float *x, const float *g, void *y, float *r, int T, int D,
                                float eps, void *stream) {
  CHECK_DT(dtype);
  return launch_rmsnorm_fwd(dtype, x, g, (h16_t *)y, r, T, D, eps, nullptr, S(stream));
}

extern "C" int ne_k_rmsnorm_bwd(int dtype, const float *dy, const float *x, const float *g, const float *r,
                                const float *resid, float *dx, void *dxb, float bscale, float *dg,
                                float dg_scale, int T, int D, void *stream) {
  CHECK_DT(dtype);
  return launch_rmsnorm_bwd(dtype, dy, x, g, r, resid, dx, (h16_t *)dxb, bscale, dg, dg_scale, T, D, nullptr,
                            nullptr, S(stream));
}

extern "C" int ne_k_gemm(int dtype, int layout, int epi, int M, int N, int K, const void *A, int64_t lda,
                         const void *B, int64_t ldb, void *C, int64_t ldc, const void *R, int64_t ldr,
                         float alpha, void *stream) {
  CHECK_DT(dtype);
  if (epi == EPI_CE_FWD || epi == EPI_CE_BWD || epi < 0 || epi > EPI_SWIGLU_FWD)
    return ne_fail(NE_ERR_ARG, "ne_k_gemm: epilogue %d not available here (use ne_k_ce_*)", epi);
  GemmArgs g = {};
  g.M = M; g.N = N; g.K = K;
  g.A = A; g.lda = lda; g.B = B; g.ldb = ldb; g.C = C; g.ldc = ldc; g.R = R; g.ldr = ldr;
  g.alpha = alpha;
  if (epi == EPI_SWIGLU_FWD) {  // R is the gate output
    g.C2 = const_cast<void *>(R);
    g.ldc2 = ldr;
    g.R = nullptr;
    g.ldr = 0;
  }
  return gemm_launch(dtype, layout, epi, g, S(stream));
}

extern "C" int ne_k_gemm_wgrad_group(int dtype, int n, const int *M, const int *N, int K, const void *const *A,
                                     const int64_t *lda, const void *const *B, const int64_t *ldb,
                                     float *const *C, int accumulate, float alpha, void *stream) {
  CHECK_DT(dtype);
  if (n < 1 || n > GEMM_GROUP_MAX || !M || !N || !A || !lda || !B || !ldb || !C)
    return ne_fail(NE_ERR_ARG, "ne_k_gemm_wgrad_group: n = %d (1..%d) or a NULL array", n, GEMM_GROUP_MAX);
  GemmArgs g[GEMM_GROUP_MAX] = {};
  for (int i = 0; i < n; i++) {
    g[i].M = M[i]; g[i].N = N[i]; g[i].K = K;
    g[i].A = A[i]; g[i].lda = lda[i]; g[i].B = B[i]; g[i].ldb = ldb[i]; g[i].C = C[i]; g[i].ldc = N[i];
    g[i].alpha = alpha;
  }
  return gemm_group_launch(dtype, accumulate ? EPI_F32_ACC : EPI_F32, g, n, S(stream));
}

extern "C" int ne_k_qk_prep_fwd(int dtype, const void *qkv, int64_t ld, const float *cosb, const float *sinb,
                                const float *gq, const float *gk, void *qr, void *kr, float *rq, float *rk,
                                int T, int S, int NH, int NKV, int HD, float eps, void *stream) {
  CHECK_DT(dtype);
  return launch_qk_prep_fwd(dtype, (const h16_t *)qkv, ld, cosb, sinb, gq, gk, (h16_t *)qr, (h16_t *)kr, rq, rk,
                            T, S, NH, NKV, HD, eps, S(stream));
}

extern "C" int ne_k_qk_prep_bwd(int dtype, const float *dq, const float *dk, const void *qkv, int64_t ld,
                                const float *cosb, const float *sinb, const float *gq, const float *gk,
                                const float *rq, const float *rk, void *dqkv, float *dgq, float *dgk,
                                float dg_scale, int T, int S, int NH, int NKV, int HD, void *stream) {
  CHECK_DT(dtype);
  return launch_qk_prep_bwd(dtype, dq, dk, (const h16_t *)qkv, ld, cosb, sinb, gq, gk, rq, rk, (h16_t *)dqkv,
                            dgq, dgk, dg_scale, T, S, NH, NKV, HD, nullptr, nullptr, S(stream));
}

static AttnArgs attn_args(const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v, int64_t ldv,
                          int B, int S, int NH, int NKV, int HD, float scale) {
  AttnArgs a = {};
  a.q = (const h16_t *)q; a.ldq = ldq;
  a.k = (const h16_t *)k; a.ldk = ldk;
  a.v = (const h16_t *)v; a.ldv = ldv;
  a.B = B; a.S = S; a.NH = NH; a.NKV = NKV; a.HD = HD; a.scale = scale;
  return a;
}

extern "C" int ne_k_attn_fwd(int dtype, const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v,
                             int64_t ldv, void *o, int64_t ldo, float *lse, int B, int S, int NH, int NKV,
                             int HD, float scale, void *stream) {
  CHECK_DT(dtype);
  AttnArgs a = attn_args(q, ldq, k, ldk, v, ldv, B, S, NH, NKV, HD, scale);
  a.o = (h16_t *)o; a.ldo = ldo; a.lse = lse;
  return launch_attn_fwd(dtype, a, S(stream));
}

extern "C" int ne_k_attn_bwd(int dtype, const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v,
                             int64_t ldv, const void *o, int64_t ldo, const float *lse, const void *dout,
                             int64_t lddo, float *delta, float *dq, int64_t lddq, float *dk, int64_t lddk,
                             void *dv, int64_t lddv, int B, int S, int NH, int NKV, int HD, float scale,
                             void *stream) {
  CHECK_DT(dtype);
  AttnArgs a = attn_args(q, ldq, k, ldk, v, ldv, B, S, NH, NKV, HD, scale);
  a.o = (h16_t *)o; a.ldo = ldo; a.lse = (float *)lse;
  a.dout = (const h16_t *)dout; a.lddo = lddo; a.delta = delta;
  a.dq = dq; a.lddq = lddq; a.dk = dk; a.lddk = lddk; a.dv = (h16_t *)dv; a.lddv = lddv;
  return launch_attn_bwd(dtype, a, S(stream));
}

// ---- ne_k_attn_bwd_noalloc: the attention backward with its delta scratch in a fixed
// device array instead of a caller buffer (no allocation on any call) ----

// delta [B*S, NH] of the backward (rowsum(dO * O)); each GPU holds its own copy, kept until
// the process ends
constexpr long NE_ATTN_SCRATCH_FLOATS = 1L << 20;  // 4 MiB
static __device__ __align__(256) float scratch[NE_ATTN_SCRATCH_FLOATS];

// The device address of `scratch` on each GPU, looked up once per device on the first call
// there (in host code the array's name is not a device address).
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[64];

static int scratch_ptr(float **out) {
  int dev = 0;
  NE_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return ne_fail(NE_ERR_ARG, "device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    NE_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    g_scratch_ptr[dev] = p;
  }
  *out = (float *)g_scratch_ptr[dev];
  return 0;
}

extern "C" int ne_k_attn_bwd_noalloc(int dtype, const void *q, int64_t ldq, const void *k, int64_t ldk,
                                     const void *v, int64_t ldv, const void *o, int64_t ldo, const float *lse,
                                     const void *dout, int64_t lddo, float *dq, int64_t lddq, float *dk,
                                     int64_t lddk, void *dv, int64_t lddv, int B, int S, int NH, int NKV, int HD,
                                     float scale, void *stream) {
  CHECK_DT(dtype);
  if (B <= 0 || S <= 0 || NH <= 0)
    return ne_fail(NE_ERR_ARG, "attn_bwd_noalloc: B=%d S=%d NH=%d must be positive", B, S, NH);
  if ((long)B * S * NH > NE_ATTN_SCRATCH_FLOATS)
    return ne_fail(NE_ERR_ARG, "attn_bwd_noalloc: B*S*NH = %ld exceeds the fixed scratch of %ld rows x heads",
                   (long)B * S * NH, NE_ATTN_SCRATCH_FLOATS);
  float *delta = nullptr;
  NE_CHECK(scratch_ptr(&delta));
  // the delta kernel writes every element of delta before the backward reads it: nothing in
  // the scratch needs clearing between calls
  AttnArgs a = attn_args(q, ldq, k, ldk, v, ldv, B, S, NH, NKV, HD, scale);
  a.o = (h16_t *)o; a.ldo = ldo; a.lse = (float *)lse;
  a.dout = (const h16_t *)dout; a.lddo = lddo; a.delta = delta;
  a.dq = dq; a.lddq = lddq; a.dk = dk; a.lddk = lddk; a.dv = (h16_t *)dv; a.lddv = lddv;
  return launch_attn_bwd(dtype, a, S(stream));
}

int ce_forward(int dt, const void *x, const void *E, const int32_t *targets, int T, int D, int V, int n_valid,
               float *part, float *tgt_logit, float *lse, float *loss_rows, float *loss, hipStream_t s) {
  if (n_valid <= 0 || n_valid > V) return ne_fail(NE_ERR_ARG, "ce: %d valid columns of %d", n_valid, V);
  GemmArgs g = {};
  g.M = T; g.N = V; g.K = D;
  g.A = x; g.lda = D; g.B = E; g.ldb = D;
  g.alpha = 1.f;
  g.targets = targets; g.part = part; g.tgt_logit = tgt_logit;
  g.n_valid = n_valid;
  NE_CHECK(gemm_launch(dt, GEMM_NT, EPI_CE_FWD, g, s));
  return launch_ce_reduce(part, gemm_ce_tiles(T, V, D), tgt_logit, lse, loss_rows, loss, T, s);
}

int ce_backward(int dt, const void *x, const void *E, const int32_t *targets, const float *lse, int T, int D,
                int V, int n_valid, float scale, void *dlogits, int *ovf, hipStream_t s) {
  if (n_valid <= 0 || n_valid > V) return ne_fail(NE_ERR_ARG, "ce: %d valid columns of %d", n_valid, V);
  GemmArgs g = {};
  g.M = T; g.N = V; g.K = D;
  g.A = x; g.lda = D; g.B = E; g.ldb = D;
  g.C = dlogits; g.ldc = V;
  g.alpha = 1.f; g.scale = scale;
  g.targets = targets; g.lse = lse; g.ovf = ovf;
  g.n_valid = n_valid;
  return gemm_launch(dt, GEMM_NT, EPI_CE_BWD, g, s);
}

int ce_forward_piece(int dt, const void *x, const void *E, const int32_t *targets, int T, int D, int V, int n_valid,
                     int c0, int c1, float *part, float *tgt_logit, void *dlogits, hipStream_t s) {
  if (n_valid <= 0 || n_valid > V) return ne_fail(NE_ERR_ARG, "ce: %d valid columns of %d", n_valid, V);
  if (!dlogits || ((uintptr_t)dlogits & 15)) return ne_fail(NE_ERR_ARG, "ce: dlogits must be 16-byte aligned");
  GemmArgs g = {};
  g.M = T; g.N = V; g.K = D;
  g.A = x; g.lda = D; g.B = E; g.ldb = D;
  g.C = dlogits; g.ldc = V;
  g.alpha = 1.f;
  g.targets = targets; g.part = part; g.tgt_logit = tgt_logit;
  g.n_valid = n_valid;
  if (!gemm_ce_piece_ok(T, V, D, c0, c1))
    return ne_fail(NE_ERR_ARG, "ce: columns [%d, %d) are not a piece of the %d x %d x %d classifier", c0, c1, T, V, D);
  if (c0 != 0 || c1 != V) {  // a piece: its own tiles of the whole shape's tiling
    int mc, wm, wr;
    gemm_ce_layout(T, V, D, &mc, &wm, &wr);
    g.N = c1 - c0;
    g.B = (const h16_t *)E + (long)c0 * D;
    g.C = (h16_t *)dlogits + c0;
    g.col0 = c0;
    g.part_ld = gemm_ce_tiles(T, V, D);
    g.tile0 = c0 / wm;
  }
  return gemm_launch(dt, GEMM_NT, EPI_CE_FWD, g, s);
}

int ce_forward_finish(int dt, const int32_t *targets, int T, int D, int V, int n_valid, float *part,
                      float *tgt_logit, float *lse, float *loss_rows, float *loss, float scale, void *dlogits,
                      int *ovf, hipStream_t s) {
  const int n_tiles = gemm_ce_tiles(T, V, D);
  NE_CHECK(launch_ce_rows(part, n_tiles, tgt_logit, lse, loss_rows, T, s));
  if (loss) NE_CHECK(launch_ce_mean(loss_rows, loss, T, s));
  int mc, wm, wr;
  gemm_ce_layout(T, V, D, &mc, &wm, &wr);
  return launch_ce_grad(dt, (h16_t *)dlogits, T, V, n_valid, part, n_tiles, mc, wm, wr, lse, tgt_logit, targets,
                        scale, ovf, s);
}

int ce_forward_grad(int dt, const void *x, const void *E, const int32_t *targets, int T, int D, int V, int n_valid,
                    float *part, float *tgt_logit, float *lse, float *loss_rows, float *loss, float scale,
                    void *dlogits, int *ovf, hipStream_t s) {
  NE_CHECK(ce_forward_piece(dt, x, E, targets, T, D, V, n_valid, 0, V, part, tgt_logit, dlogits, s));
  return ce_forward_finish(dt, targets, T, D, V, n_valid, part, tgt_logit, lse, loss_rows, loss, scale, dlogits, ovf,
                           s);
}

extern "C" int ne_k_ce_fwd(int dtype, const void *x, const void *E, const int32_t *targets, int T, int D, int V,
                           float *part, float *tgt_logit, float *lse, float *loss_rows, float *loss,
                           void *stream) {
  CHECK_DT(dtype);
  return ce_forward(dtype, x, E, targets, T, D, V, V, part, tgt_logit, lse, loss_rows, loss, S(stream));
}

extern "C" int ne_k_ce_bwd(int dtype, const void *x, const void *E, const int32_t *targets, const float *lse,
                           int T, int D, int V, float scale, void *dlogits, void *stream) {
  CHECK_DT(dtype);
  return ce_backward(dtype, x, E, targets, lse, T, D, V, V, scale, dlogits, nullptr, S(stream));
}

extern "C" int ne_k_ce_fwd_grad(int dtype, const void *x, const void *E, const int32_t *targets, int T, int D,
                                int V, float *part, float *tgt_logit, float *lse, float *loss_rows, float *loss,
                                float scale, void *dlogits, void *stream) {
  CHECK_DT(dtype);
  return ce_forward_grad(dtype, x, E, targets, T, D, V, V, part, tgt_logit, lse, loss_rows, loss, scale, dlogits,
                         nullptr, S(stream));
}

extern "C" int ne_k_adam(int dtype, float *p, float *g, float *m, float *v, void *pb, int64_t n,
                         int64_t n_decay, float lr, float b1, float b2, float eps, float wd, int t,
                         const float *gscale, int zero_grad, void *stream) {
  CHECK_DT(dtype);
  if (t < 1) return ne_fail(NE_ERR_ARG, "adam: step t=%d must be >= 1", t);
  AdamArgs a = {};
  a.p = p; a.g = g; a.m = m; a.v = v; a.pb = (h16_t *)pb;
  a.n = n; a.n_decay = n_decay;
  a.lr = lr; a.b1 = b1; a.b2 = b2; a.eps = eps; a.wd = wd;
  a.bc1 = 1.f - powf(b1, (float)t);
  a.bc2 = 1.f - powf(b2, (float)t);
  a.gscale = gscale; a.zero_grad = zero_grad;
  return launch_adam(dtype, a, S(stream));
}

extern "C" int ne_k_grad_norm(const float *g, int64_t n, float grad_scale, float clip, double *partials,
                              float *gscale, float *gnorm, void *stream) {
  NE_CHECK(launch_sumsq(g, n, partials, 1024, S(stream)));
  return launch_clip_finalize(partials, 1024, grad_scale, clip, gscale, gnorm, S(stream));
}

extern "C" int ne_k_embed_fwd(const float *E, const int32_t *tok, float *x, int T, int D, void *stream) {
  return launch_embed_fwd(E, tok, x, T, D, S(stream));
}

extern "C" int ne_k_embed_bwd(float *gE, const int32_t *tok, const float *dx, float scale, int T, int D,
                              void *stream) {
  return launch_embed_bwd(gE, tok, dx, scale, T, D, S(stream));
}

extern "C" int ne_k_swiglu_fwd(int dtype, const void *h13, void *gate, int T, int H, void *stream) {
  CHECK_DT(dtype);
  return launch_swiglu_fwd(dtype, (const h16_t *)h13, (h16_t *)gate, T, H, nullptr, S(stream));
}

extern "C" int ne_k_mfma_ceiling(int dtype, int shape, int blocks, int iters, float *out, void *stream) {
  CHECK_DT(dtype);
  return launch_mfma_ceiling(dtype, shape, blocks, iters, out, S(stream));
}
