// Gradient norm / clip and the single-pass fused AdamW over the flat parameter buffer.
//
// Replaces TD/train.m:782-849 (grad scale, global L2 norm, clip) and
// TD/cpu_ops.h:266-303 adam_update called per tensor (TD/train.m:861-897), plus the
// fp16 weight restaging of TD/train.m:872-895: here the update writes the 16-bit shadow
// the GEMMs read, in the same pass.  Per element: read p, g, m, v (16 B), write
// p, m, v (12 B), 16-bit shadow (2 B) = 30 B (+4 B when it also zeroes g).  A step whose backward
// overflowed the 16-bit range (device flag) leaves p, m, v untouched and only zeroes g.
#include "common.h"
#include "ne_internal.h"

namespace {

// Sum of squares of g[0, n) over nb blocks (block b of them is `b`): partials[b].
__device__ __forceinline__ void sumsq_block(const float *__restrict__ g, long n, int b, int nb,
                                            double *__restrict__ partials) {
  __shared__ float red[4];
  const long n4 = n / 4;
  float acc = 0.f;
  const float4 *g4 = (const float4 *)g;
  for (long i = b * 256L + threadIdx.x; i < n4; i += (long)nb * 256) {
    const float4 v = g4[i];
    acc += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  if (b == 0)
    for (long i = n4 * 4 + threadIdx.x; i < n; i += 256) acc += g[i] * g[i];
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) partials[b] = (double)red[0] + red[1] + red[2] + red[3];
}

__global__ __launch_bounds__(256) void sumsq_kernel(const float *__restrict__ g, long n,
                                                    double *__restrict__ partials) {
  sumsq_block(g, n, blockIdx.x, gridDim.x, partials);
}

// norm = grad_scale * sqrt(sum partials); factor = grad_scale * (clip / norm if norm > clip).
// One block of 1024 threads (it sits between the backward and the update, so its latency is
// on the step's critical path; the partials are the weight-gradient GEMMs' per-tile sums, tens
// of thousands): each thread sums a strided subset, CL loads issued before the adds, then
// the 16 wave sums in order.  Fixed order throughout (deterministic).
__global__ __launch_bounds__(1024) void clip_finalize_kernel(const double *__restrict__ partials, int nparts,
                                                             float grad_scale, float clip, float *__restrict__ gscale,
                                                             float *__restrict__ gnorm) {
  constexpr int NT = 1024, CL = 8;
  __shared__ double red[NT / 64];
  double s = 0.0;
  for (int i0 = threadIdx.x; i0 < nparts; i0 += CL * NT) {
    double v[CL];
#pragma unroll
    for (int u = 0; u < CL; u++) v[u] = i0 + u * NT < nparts ? partials[i0 + u * NT] : 0.0;
#pragma unroll
    for (int u = 0; u < CL; u++) s += v[u];
  }
  s = wave_sum_d(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    s = 0.0;
#pragma unroll
    for (int w = 0; w < NT / 64; w++) s += red[w];
    // the partials may include signed row changes (embedding scatter): never below 0
    const float norm = (float)(sqrt(fmax(s, 0.0)) * (double)grad_scale);
    float f = grad_scale;
    if (clip > 0.f && norm > clip) f *= clip / norm;
    gscale[0] = f;
    gnorm[0] = norm;
  }
}

// Two float4 of each stream per thread per iteration, non-temporal loads and stores (each
// byte is touched once): measured at the streaming-copy ceiling of the device.
template <typename HT, bool SHADOW>
__global__ __launch_bounds__(256) void adam_kernel(AdamArgs a) {
  const AdamConst k(a.gscale, a.b1, a.b2, a.bc1, a.bc2, a.lr, a.eps);
  const bool skip = a.skip && a.skip[0];
  const long n4 = a.n / 4;
  const long stride = (long)gridDim.x * 256;
  f32x4 *p4 = (f32x4 *)a.p, *g4 = (f32x4 *)a.g, *m4 = (f32x4 *)a.m, *v4 = (f32x4 *)a.v;
  for (long i0 = blockIdx.x * 256L + threadIdx.x; i0 < n4; i0 += 2 * stride) {
    f32x4 P[2], G[2], M[2], V[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const long i = i0 + u * stride;
      if (i < n4) {
        G[u] = __builtin_nontemporal_load(g4 + i);
        if (!skip) {
          P[u] = __builtin_nontemporal_load(p4 + i);
          M[u] = __builtin_nontemporal_load(m4 + i);
          V[u] = __builtin_nontemporal_load(v4 + i);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const long i = i0 + u * stride;
      if (i >= n4) break;
      if (skip) {
        if (a.zero_grad) __builtin_nontemporal_store(f32x4{0.f, 0.f, 0.f, 0.f}, g4 + i);
        continue;
      }
      const float wd = (i * 4 < a.n_decay) ? a.wd : 0.f;
      u16x4 b;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        float pj = P[u][j], mj = M[u][j], vj = V[u][j];
        adam_elem(k, pj, G[u][j], mj, vj, wd);
        P[u][j] = pj; M[u][j] = mj; V[u][j] = vj;
        b[j] = HT::h(pj);
      }
      __builtin_nontemporal_store(P[u], p4 + i);
      __builtin_nontemporal_store(M[u], m4 + i);
      __builtin_nontemporal_store(V[u], v4 + i);
      if (a.zero_grad) __builtin_nontemporal_store(f32x4{0.f, 0.f, 0.f, 0.f}, g4 + i);
      if (SHADOW) __builtin_nontemporal_store(b, (u16x4 *)a.pb + i);
    }
  }
}

template <typename HT>
__global__ void f32_to_h16_kernel(const float *__restrict__ src, h16_t *__restrict__ dst, long n) {
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256) dst[i] = HT::h(src[i]);
}

__global__ void fill_f32_kernel(float *__restrict__ dst, float v, long n) {
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256) dst[i] = v;
}

// A block that meets a NaN writes NaN for both (fminf / fmaxf alone would skip it and report
// a finite range for a diverged run).
__global__ __launch_bounds__(256) void minmax_kernel(const float *__restrict__ a, long n, float *__restrict__ out) {
  __shared__ float rmn[4], rmx[4];
  __shared__ int rnan[4];
  float mn = INFINITY, mx = -INFINITY;
  int nan = 0;
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
    const float v = a[i];
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
    nan |= v != v;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    mn = fminf(mn, __shfl_xor(mn, o, 64));
    mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    nan |= __shfl_xor(nan, o, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    rmn[threadIdx.x >> 6] = mn;
    rmx[threadIdx.x >> 6] = mx;
    rnan[threadIdx.x >> 6] = nan;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const bool any = rnan[0] | rnan[1] | rnan[2] | rnan[3];
    out[2 * blockIdx.x] = any ? NAN : fminf(fminf(rmn[0], rmn[1]), fminf(rmn[2], rmn[3]));
    out[2 * blockIdx.x + 1] = any ? NAN : fmaxf(fmaxf(rmx[0], rmx[1]), fmaxf(rmx[2], rmx[3]));
  }
}

int grid_for(long n) { return (int)std::max<long>(1, std::min<long>((n + 255) / 256, 256L * 32)); }

}  // namespace

int launch_sumsq(const float *g, long n, double *partials, int nparts, hipStream_t s) {
  hipLaunchKernelGGL(sumsq_kernel, dim3(nparts), dim3(256), 0, s, g, n, partials);
  return ne_hip_status(hipGetLastError(), "sumsq");
}

int launch_clip_finalize(const double *partials, int nparts, float grad_scale, float clip,
                         float *gscale_out, float *gnorm_out, hipStream_t s) {
  hipLaunchKernelGGL(clip_finalize_kernel, dim3(1), dim3(1024), 0, s, partials, nparts, grad_scale, clip,
                     gscale_out, gnorm_out);
  return ne_hip_status(hipGetLastError(), "clip_finalize");
}

int launch_adam(int dt, const AdamArgs &a, hipStream_t s) {
  if (a.n % 4 || a.n_decay % 4) return ne_fail(NE_ERR_ARG, "adam: sizes must be multiples of 4");
  // 64K work-groups: measured at the streaming ceiling of the device for this read/write mix
  const long cap = a.max_groups > 0 ? a.max_groups : 65536;
  const int grid = (int)std::max<long>(1, std::min<long>((a.n / 4 + 511) / 512, cap));
  return DISPATCH_H16(dt, [&] {
    if (a.pb) hipLaunchKernelGGL((adam_kernel<HT, true>), dim3(grid), dim3(256), 0, s, a);
    else hipLaunchKernelGGL((adam_kernel<HT, false>), dim3(grid), dim3(256), 0, s, a);
    return ne_hip_status(hipGetLastError(), "adam");
  }());
}

int launch_f32_to_h16(int dt, const float *src, h16_t *dst, long n, hipStream_t s) {
  return DISPATCH_H16(dt, [&] {
    hipLaunchKernelGGL(f32_to_h16_kernel<HT>, dim3(grid_for(n)), dim3(256), 0, s, src, dst, n);
    return ne_hip_status(hipGetLastError(), "f32_to_h16");
  }());
}

int launch_minmax(const float *a, long n, float *out, int nblocks, hipStream_t s) {
  hipLaunchKernelGGL(minmax_kernel, dim3(nblocks), dim3(256), 0, s, a, n, out);
  return ne_hip_status(hipGetLastError(), "minmax");
}

int launch_fill_f32(float *dst, float v, long n, hipStream_t s) {
  hipLaunchKernelGGL(fill_f32_kernel, dim3(grid_for(n)), dim3(256), 0, s, dst, v, n);
  return ne_hip_status(hipGetLastError(), "fill_f32");
}
