// Cross-entropy reduction over the vocab tiles written by the logits GEMM epilogue.
//
// The LM-head GEMM (k_gemm.hip, EPI_CE_FWD) leaves per (row, vocab tile) the tile max and
// sum of exp, plus the target logit.  This kernel merges the tiles into the row's
// log-sum-exp and the per-row loss -log(p_tgt + 1e-10) of TD/cpu_ops.h:348-382, and a
// second single-block pass averages the rows (mean over the T tokens of the step).
// Logits are never materialised in HBM.
#include "common.h"
#include "ne_internal.h"

namespace {

// One 256-thread block per row: each thread takes every 256th tile of the row, the (max, sum)
// pairs of up to CE_ROW_REG tiles held in registers between the max and the sum (a 256-token
// Qwen3-0.6B step has 1187 tiles a row: one wave per row took 11 us, two dependent passes of 19
// loads per lane).
constexpr int CE_ROW_REG = 8;
__global__ __launch_bounds__(256) void ce_rows_kernel(const float *__restrict__ part, int n_tiles,
                                                      const float *__restrict__ tgt, float *__restrict__ lse,
                                                      float *__restrict__ loss_rows, int T) {
  __shared__ float red[2][4];
  const int row = blockIdx.x, t = threadIdx.x;
  const float2 *p = (const float2 *)(part + (long)row * n_tiles * 2);
  float2 v[CE_ROW_REG];
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < CE_ROW_REG; k++) {
    const int i = t + k * 256;
    v[k] = i < n_tiles ? p[i] : make_float2(-INFINITY, 0.f);
    mx = fmaxf(mx, v[k].x);
  }
  for (int i = t + CE_ROW_REG * 256; i < n_tiles; i += 256) mx = fmaxf(mx, p[i].x);
  mx = wave_max(mx);
  if ((t & 63) == 0) red[0][t >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < CE_ROW_REG; k++)
    if (t + k * 256 < n_tiles) s += v[k].y * __expf(v[k].x - mx);
  for (int i = t + CE_ROW_REG * 256; i < n_tiles; i += 256) {
    const float2 q = p[i];
    s += q.y * __expf(q.x - mx);
  }
  s = wave_sum(s);
  if ((t & 63) == 0) red[1][t >> 6] = s;
  __syncthreads();
  if (t == 0) {
    const float l = mx + logf((red[1][0] + red[1][1]) + (red[1][2] + red[1][3]));
    lse[row] = l;
    loss_rows[row] = -logf(expf(tgt[row] - l) + 1e-10f);
  }
}

__global__ void mean_kernel(const float *__restrict__ x, int n, float *__restrict__ out) {
  __shared__ double red[16];
  double s = 0.0;
  for (int i = threadIdx.x; i < n; i += blockDim.x) s += x[i];
  s = wave_sum_d(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) t += red[w];
    out[0] = (float)(t / n);
  }
}

// dst[r, :] = src[ids[r], :], 16-bit rows of D (D % 8 == 0): one block per row.
__global__ void gather_rows16_kernel(const h16_t *__restrict__ src, const int32_t *__restrict__ ids,
                                     h16_t *__restrict__ dst, int D) {
  const long r = blockIdx.x;
  const u16x8 *s8 = (const u16x8 *)(src + (long)ids[r] * D);
  u16x8 *d8 = (u16x8 *)(dst + r * D);
  for (int i = threadIdx.x; i < D / 8; i += blockDim.x) d8[i] = s8[i];
}

// G[ids[r], :] += src[r, :], fp32 rows of D (D % 4 == 0): one block per row; the ids are
// distinct, so no two blocks touch the same row.
__global__ void scatter_add_rows_kernel(float *__restrict__ G, const float *__restrict__ src,
                                        const int32_t *__restrict__ ids, int D) {
  const long r = blockIdx.x;
  float4 *g4 = (float4 *)(G + (long)ids[r] * D);
  const float4 *s4 = (const float4 *)(src + r * D);
  for (int i = threadIdx.x; i < D / 4; i += blockDim.x) {
    float4 a = g4[i];
    const float4 b = s4[i];
    a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
    g4[i] = a;
  }
}

// The cross-entropy gradient in place over e = exp(logit - tile max), the 16-bit values the
// LM-head GEMM's forward epilogue stored: dl = (softmax - onehot) * scale with softmax =
// e * exp(tile max - lse) (TD/cpu_ops.h:373-378: p - 1 at the target, times the loss
// scale); at the target the probability is formed from its fp32 logit, exp(tgt - lse), as
// the loss is; padding columns (>= n_valid) are 0.  Eight consecutive columns per thread,
// which never straddle a tile (tile widths are multiples of 64).
template <typename HT>
__global__ __launch_bounds__(256) void ce_grad_kernel(h16_t *__restrict__ dl, int V, int n_valid,
                                                      const float *__restrict__ part, int n_tiles, int main_cols,
                                                      int w_main, int w_rest, const float *__restrict__ lse,
                                                      const float *__restrict__ tgt_logit,
                                                      const int32_t *__restrict__ targets, float scale,
                                                      int *__restrict__ ovf) {
  const long row = blockIdx.y;
  const int c0 = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (c0 >= V) return;
  const int slot = c0 < main_cols ? c0 / w_main : main_cols / w_main + (c0 - main_cols) / w_rest;
  const float l = lse[row];
  const float f = __expf(part[(row * n_tiles + slot) * 2] - l) * scale;
  const int tc = targets[row] - c0;
  u16x8 *p8 = (u16x8 *)(dl + row * V + c0);
  const u16x8 ev = *p8;
  u16x8 o;
  bool bad = false;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    float v = c0 + k < n_valid ? HT::f(ev[k]) * f : 0.f;
    if (k == tc) v = (__expf(tgt_logit[row] - l) - 1.f) * scale;
    o[k] = HT::h(v);
    bad |= HT::bad(o[k]);
  }
  *p8 = o;
  flag_overflow(ovf, bad);
}

}  // namespace

int launch_ce_grad(int dt, h16_t *dl, int T, int V, int n_valid, const float *part, int n_tiles, int main_cols,
                   int w_main, int w_rest, const float *lse, const float *tgt_logit, const int32_t *targets,
                   float scale, int *ovf, hipStream_t s) {
  if (V % 64 || (((uintptr_t)dl) & 15)) return ne_fail(NE_ERR_ARG, "ce_grad: V %% 64 and 16-byte aligned rows");
  const dim3 grid((V / 8 + 255) / 256, T);
  return DISPATCH_H16(dt, [&] {
    hipLaunchKernelGGL(ce_grad_kernel<HT>, grid, dim3(256), 0, s, dl, V, n_valid, part, n_tiles, main_cols, w_main,
                       w_rest, lse, tgt_logit, targets, scale, ovf);
    return ne_hip_status(hipGetLastError(), "ce_grad");
  }());
}

int launch_gather_rows16(const h16_t *src, const int32_t *ids, h16_t *dst, int n, int D, hipStream_t s) {
  if (D % 8) return ne_fail(NE_ERR_ARG, "gather_rows16: D=%d must be a multiple of 8", D);
  if (n <= 0) return 0;
  hipLaunchKernelGGL(gather_rows16_kernel, dim3(n), dim3(128), 0, s, src, ids, dst, D);
  return ne_hip_status(hipGetLastError(), "gather_rows16");
}

int launch_scatter_add_rows(float *G, const float *src, const int32_t *ids, int n, int D, hipStream_t s) {
  if (D % 4) return ne_fail(NE_ERR_ARG, "scatter_add_rows: D=%d must be a multiple of 4", D);
  if (n <= 0) return 0;
  hipLaunchKernelGGL(scatter_add_rows_kernel, dim3(n), dim3(256), 0, s, G, src, ids, D);
  return ne_hip_status(hipGetLastError(), "scatter_add_rows");
}

int launch_ce_rows(const float *part, int n_tiles, const float *tgt_logit, float *lse, float *loss_rows, int T,
                   hipStream_t s) {
  if (T <= 0) return 0;
  hipLaunchKernelGGL(ce_rows_kernel, dim3(T), dim3(256), 0, s, part, n_tiles, tgt_logit, lse, loss_rows, T);
  return ne_hip_status(hipGetLastError(), "ce_rows");
}

int launch_ce_mean(const float *loss_rows, float *loss, int T, hipStream_t s) {
  hipLaunchKernelGGL(mean_kernel, dim3(1), dim3(1024), 0, s, loss_rows, T, loss);
  return ne_hip_status(hipGetLastError(), "ce_mean");
}

int launch_ce_reduce(const float *part, int n_tiles, const float *tgt_logit, float *lse,
                     float *loss_rows, float *loss, int T, hipStream_t s) {
  NE_CHECK(launch_ce_rows(part, n_tiles, tgt_logit, lse, loss_rows, T, s));
  return launch_ce_mean(loss_rows, loss, T, s);
}
