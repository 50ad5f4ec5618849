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

__global__ void ce_rows_kernel(const float *__restrict__ part, int n_tiles, const float *__restrict__ tgt,
                               float *__restrict__ lse, float *__restrict__ loss_rows, int T) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= T) return;
  const float *p = part + (long)row * n_tiles * 2;
  float mx = -INFINITY;
  for (int i = lane; i < n_tiles; i += 64) mx = fmaxf(mx, p[2 * i]);
  mx = wave_max(mx);
  float s = 0.f;
  for (int i = lane; i < n_tiles; i += 64) s += p[2 * i + 1] * __expf(p[2 * i] - mx);
  s = wave_sum(s);
  if (lane == 0) {
    const float l = mx + logf(s);
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

}  // namespace

int launch_ce_reduce(const float *part, int n_tiles, const float *tgt_logit, float *lse,
                     float *loss_rows, float *loss, int T, hipStream_t s) {
  hipLaunchKernelGGL(ce_rows_kernel, dim3((T + 3) / 4), dim3(256), 0, s, part, n_tiles, tgt_logit, lse,
                     loss_rows, T);
  NE_HIP(hipGetLastError());
  hipLaunchKernelGGL(mean_kernel, dim3(1), dim3(1024), 0, s, loss_rows, T, loss);
  return ne_hip_status(hipGetLastError(), "ce_reduce");
}
