// Embedding gather/scatter, RMSNorm fwd/bwd, SwiGLU gate, and the RoPE + QK-RMSNorm
// prologue/epilogue of attention.  All HBM-bound: one wavefront per token row,
// float4 / 8-byte vector accesses, fp32 arithmetic, 16-bit (fp16/bf16) GEMM operands out.
#include "common.h"
#include "ne_internal.h"

namespace {

// x[t, :] = E[tok[t], :]   (TD/cpu_ops.h:433-439 embed_lookup; token-major here)
__global__ void embed_fwd_kernel(const float *__restrict__ E, const int32_t *__restrict__ tok,
                                 float *__restrict__ x, int T, int D) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= T) return;
  const float4 *src = (const float4 *)(E + (long)tok[row] * D);
  float4 *dst = (float4 *)(x + (long)row * D);
  for (int i = lane; i < D / 4; i += 64) dst[i] = src[i];
}

// The lookup of a step whose preceding AdamW update of E has not run yet: x[t] = the row
// E[tok[t]] as the update will leave it, computed from E, G, M, V with the update's element
// arithmetic (adam_elem, weight decay on) and nothing written back; the update itself runs
// later, beside the forward, and gives the same values bit for bit.
__global__ void embed_fwd_adam_kernel(const float *__restrict__ E, const float *__restrict__ G,
                                      const float *__restrict__ M, const float *__restrict__ V,
                                      const int32_t *__restrict__ tok, float *__restrict__ x, int T, int D,
                                      AdamArgs a) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= T) return;
  const AdamConst k(a.gscale, a.b1, a.b2, a.bc1, a.bc2, a.lr, a.eps);
  const long off = (long)tok[row] * D;
  float *dst = x + (long)row * D;
  for (int i = lane; i < D; i += 64) {
    float p = E[off + i], m = M[off + i], v = V[off + i];
    adam_elem(k, p, G[off + i], m, v, a.wd);
    dst[i] = p;
  }
}

// gE[tok[t], :] += scale * dx[t, :]   (TD/cpu_ops.h:441-447 embed_backward)
__global__ void embed_bwd_kernel(float *__restrict__ gE, const int32_t *__restrict__ tok,
                                 const float *__restrict__ dx, float scale, int T, int D) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= T) return;
  float *dst = gE + (long)tok[row] * D;
  const float *src = dx + (long)row * D;
  for (int i = lane; i < D; i += 64) atomicAdd(dst + i, scale * src[i]);
}

// Deterministic form of embed_bwd_kernel: the rows of one token id are chained in token
// order (nxt[t]: next row with the same id, -1 at the end; first[t]: t is the id's first
// row), and the wave of the first row sums the chain in that order and adds it to gE once.
// No atomics, so the result does not depend on scheduling.  With dsq, slot t receives the
// change of the sum of squares of the gE row the wave of row t updated (0 for the other rows),
// so a sum of squares of gE taken before this kernel can be brought up to date.
constexpr int EMB_MAXV = 8;  // float4 per lane: D <= 2048
__global__ __launch_bounds__(256) void embed_bwd_chain_kernel(float *__restrict__ gE, const int32_t *__restrict__ tok,
                                                              const int32_t *__restrict__ nxt,
                                                              const int32_t *__restrict__ first,
                                                              const float *__restrict__ dx, float scale, int T,
                                                              int D, double *__restrict__ dsq) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= T) return;
  if (!first[row]) {
    if (dsq && lane == 0) dsq[row] = 0.0;
    return;
  }
  const int D4 = D / 4;
  float4 acc[EMB_MAXV];
#pragma unroll
  for (int j = 0; j < EMB_MAXV; j++) acc[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int t = row; t >= 0; t = nxt[t]) {
    const float4 *src = (const float4 *)(dx + (long)t * D);
#pragma unroll
    for (int j = 0; j < EMB_MAXV; j++) {
      const int i = lane + 64 * j;
      if (i < D4) {
        const float4 v = src[i];
        acc[j].x += v.x; acc[j].y += v.y; acc[j].z += v.z; acc[j].w += v.w;
      }
    }
  }
  float4 *dst = (float4 *)(gE + (long)tok[row] * D);
  double d = 0.0;
#pragma unroll
  for (int j = 0; j < EMB_MAXV; j++) {
    const int i = lane + 64 * j;
    if (i < D4) {
      float4 g = dst[i];
      const float o = g.x * g.x + g.y * g.y + g.z * g.z + g.w * g.w;
      g.x += scale * acc[j].x; g.y += scale * acc[j].y; g.z += scale * acc[j].z; g.w += scale * acc[j].w;
      dst[i] = g;
      d += (double)(g.x * g.x + g.y * g.y + g.z * g.z + g.w * g.w) - (double)o;
    }
  }
  if (dsq) {
    d = wave_sum_d(d);
    if (lane == 0) dsq[row] = d;
  }
}

// One 256-thread block per row (in flight), each thread owning float4 columns t and t + 256:
// rows of D <= 2048 floats.  Per-row sums go through a fixed-order block reduction.
constexpr int RMS_NT = 256, RMS_VPT = 2;

// Sum over the block of one value per thread: wave sums, then the 4 wave totals in wave order.
// `red` alternates between two slots by row parity so consecutive rows need one barrier each.
__device__ __forceinline__ float block_sum_row(float v, float (*red)[RMS_NT / 64], int slot) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[slot][threadIdx.x >> 6] = v;
  lds_barrier();  // waits for the LDS writes only: global loads issued earlier stay in flight
  return red[slot][0] + red[slot][1] + red[slot][2] + red[slot][3];
}

// Row `row` of a split-K result, columns t and t + 256 (as float4): base + alpha * sum_z part[z].
// The partials are added in z order (the GEMM's own reduction order) with the loads of four
// consecutive z issued together.
__device__ __forceinline__ void split_row(const SplitIn &sp, long row, int D, float4 (&o)[RMS_VPT]) {
  const int D4 = D / 4, t = threadIdx.x;
  const float4 *p = (const float4 *)(sp.part + row * D);
  const long sl = sp.slice / 4;
#pragma unroll
  for (int j = 0; j < RMS_VPT; j++) o[j] = t + RMS_NT * j < D4 ? p[t + RMS_NT * j] : make_float4(0.f, 0.f, 0.f, 0.f);
  int z = 1;
  for (; z + 3 < sp.n; z += 4) {
    float4 q[4][RMS_VPT];
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
      for (int j = 0; j < RMS_VPT; j++)
        q[u][j] = t + RMS_NT * j < D4 ? p[(z + u) * sl + t + RMS_NT * j] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
      for (int j = 0; j < RMS_VPT; j++) {
        o[j].x += q[u][j].x; o[j].y += q[u][j].y; o[j].z += q[u][j].z; o[j].w += q[u][j].w;
      }
  }
  for (; z < sp.n; z++)
#pragma unroll
    for (int j = 0; j < RMS_VPT; j++)
      if (t + RMS_NT * j < D4) {
        const float4 q = p[z * sl + t + RMS_NT * j];
        o[j].x += q.x; o[j].y += q.y; o[j].z += q.z; o[j].w += q.w;
      }
  const float4 *b = sp.base ? (const float4 *)(sp.base + row * D) : nullptr;
#pragma unroll
  for (int j = 0; j < RMS_VPT; j++) {
    const float a = sp.alpha;
    float4 v = make_float4(a * o[j].x, a * o[j].y, a * o[j].z, a * o[j].w);
    if (b && t + RMS_NT * j < D4) {
      const float4 q = b[t + RMS_NT * j];
      v.x = q.x + v.x; v.y = q.y + v.y; v.z = q.z + v.z; v.w = q.w + v.w;
    }
    o[j] = v;
  }
}

// y = x * r * g, r = (mean(x^2) + eps)^-1/2   (TD/cpu_ops.h:20-60 rmsnorm).  With split-K
// partials (sp.n > 0) the row x is formed from them and written to x first.
template <typename HT>
__global__ __launch_bounds__(RMS_NT) void rmsnorm_fwd_kernel(float *__restrict__ x, const float *__restrict__ g,
                                                             h16_t *__restrict__ y, float *__restrict__ rr, int D,
                                                             float eps, int *ovf, SplitIn sp) {
  __shared__ float red[1][RMS_NT / 64];
  const long row = blockIdx.x;
  const int t = threadIdx.x, D4 = D / 4;
  float4 *xr = (float4 *)(x + row * D);
  float4 xv[RMS_VPT];
  if (sp.n > 0) {
    split_row(sp, row, D, xv);
#pragma unroll
    for (int j = 0; j < RMS_VPT; j++)
      if (t + RMS_NT * j < D4) xr[t + RMS_NT * j] = xv[j];
  } else {
#pragma unroll
    for (int j = 0; j < RMS_VPT; j++)
      xv[j] = t + RMS_NT * j < D4 ? xr[t + RMS_NT * j] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < RMS_VPT; j++) ss += xv[j].x * xv[j].x + xv[j].y * xv[j].y + xv[j].z * xv[j].z + xv[j].w * xv[j].w;
  ss = block_sum_row(ss, red, 0);
  const float r = 1.0f / sqrtf(ss / (float)D + eps);
  if (t == 0) rr[row] = r;
  u16x4 *yr = (u16x4 *)(y + row * D);
  const float4 *gv = (const float4 *)g;
  bool bad = false;
#pragma unroll
  for (int j = 0; j < RMS_VPT; j++) {
    const int i = t + RMS_NT * j;
    if (i < D4) {
      const float4 v = xv[j], w = gv[i];
      u16x4 o;
      o[0] = HT::h(v.x * r * w.x);
      o[1] = HT::h(v.y * r * w.y);
      o[2] = HT::h(v.z * r * w.z);
      o[3] = HT::h(v.w * r * w.w);
      bad |= HT::bad(o[0]) | HT::bad(o[1]) | HT::bad(o[2]) | HT::bad(o[3]);
      yr[i] = o;
    }
  }
  flag_overflow(ovf, bad);
}

// Exact RMSNorm backward with fused residual add and gain-gradient accumulation:
//   dx = r*g*dy - x*r^3*sum(dy*x*g)/D (+ resid);  dg += sum_t dy*x*r
//   dxb = 16-bit(bscale * dx)  (the alpha-scaled operand of the next GEMM); the gain
//   gradient is accumulated times dg_scale (removes the backward's internal scale)
// Replaces TD/cpu_ops.h:108-261 (rmsnorm_bwd / rmsnorm_bwd_add).  With REF the
// reference's own formula is used instead, dx = (dy - x*r^2*sum(dy*x*g)/D)*r*g
// (TD/cpu_ops.h:146-153, 188-189, 255-256), whose projection term carries one more
// factor g than the exact gradient; both agree while every gain is 1.  A block walks
// rows_per_block rows; each thread keeps the gain-gradient sums of its own columns and
// writes them as the block's partial row (or adds them atomically without `part`).  With
// split-K partials (sp.n > 0) dy is formed from them.
template <typename HT, bool REF>
__global__ __launch_bounds__(RMS_NT) void rmsnorm_bwd_kernel(
    const float *__restrict__ dy, const float *__restrict__ x, const float *__restrict__ g,
    const float *__restrict__ rr, const float *__restrict__ resid, float *__restrict__ dx,
    h16_t *__restrict__ dxb, float bscale, float *__restrict__ dg, float dg_scale, int T, int D,
    int rows_per_block, int *ovf, float *__restrict__ part, SplitIn sp) {
  __shared__ float red[2][RMS_NT / 64];
  const int t = threadIdx.x, D4 = D / 4;
  float4 acc[RMS_VPT], gw[RMS_VPT];
  const float4 *gv = (const float4 *)g;
#pragma unroll
  for (int j = 0; j < RMS_VPT; j++) {
    acc[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    gw[j] = t + RMS_NT * j < D4 ? gv[t + RMS_NT * j] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const float invD = 1.0f / (float)D;
  const int r0 = blockIdx.x * rows_per_block;
  const int r1 = min(T, r0 + rows_per_block);
  bool bad = false;
  // Row loads (dy, x, the residual and r) are issued one row ahead: the next row's loads are in
  // flight during this row's block reduction and stores.
  float4 dyv[RMS_VPT], xv[RMS_VPT], rsv[RMS_VPT];
  float r = 0.f;
  auto load_row = [&](int row, float4 (&dyo)[RMS_VPT], float4 (&xo)[RMS_VPT], float4 (&rso)[RMS_VPT], float &ro) {
    if (sp.n > 0) {
      split_row(sp, row, D, dyo);
    } else {
      const float4 *dyr = (const float4 *)(dy + (long)row * D);
#pragma unroll
      for (int j = 0; j < RMS_VPT; j++)
        dyo[j] = t + RMS_NT * j < D4 ? dyr[t + RMS_NT * j] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float4 *xr = (const float4 *)(x + (long)row * D);
    const float4 *rsr = resid ? (const float4 *)(resid + (long)row * D) : nullptr;
#pragma unroll
    for (int j = 0; j < RMS_VPT; j++) {
      xo[j] = t + RMS_NT * j < D4 ? xr[t + RMS_NT * j] : make_float4(0.f, 0.f, 0.f, 0.f);
      rso[j] = rsr && t + RMS_NT * j < D4 ? rsr[t + RMS_NT * j] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    ro = rr[row];
  };
  if (r0 < r1) load_row(r0, dyv, xv, rsv, r);
  for (int row = r0; row < r1; row++) {
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < RMS_VPT; j++)
      dot += dyv[j].x * xv[j].x * gw[j].x + dyv[j].y * xv[j].y * gw[j].y + dyv[j].z * xv[j].z * gw[j].z +
             dyv[j].w * xv[j].w * gw[j].w;
    float4 dyn[RMS_VPT], xn[RMS_VPT], rsn[RMS_VPT];
    float rn = 0.f;
    if (row + 1 < r1) load_row(row + 1, dyn, xn, rsn, rn);
    dot = block_sum_row(dot, red, row & 1);
    const float c = REF ? r * r * dot * invD : r * r * r * dot * invD;
    float4 *dxr = (float4 *)(dx + (long)row * D);
    u16x4 *dbr = dxb ? (u16x4 *)(dxb + (long)row * D) : nullptr;
#pragma unroll
    for (int j = 0; j < RMS_VPT; j++) {
      const int i = t + RMS_NT * j;
      if (i < D4) {
        const float4 w = gw[j];
        float4 o;
        if (REF) {
          o.x = (dyv[j].x - xv[j].x * c) * r * w.x;
          o.y = (dyv[j].y - xv[j].y * c) * r * w.y;
          o.z = (dyv[j].z - xv[j].z * c) * r * w.z;
          o.w = (dyv[j].w - xv[j].w * c) * r * w.w;
        } else {
          o.x = r * w.x * dyv[j].x - xv[j].x * c;
          o.y = r * w.y * dyv[j].y - xv[j].y * c;
          o.z = r * w.z * dyv[j].z - xv[j].z * c;
          o.w = r * w.w * dyv[j].w - xv[j].w * c;
        }
        if (resid) {
          o.x += rsv[j].x; o.y += rsv[j].y; o.z += rsv[j].z; o.w += rsv[j].w;
        }
        dxr[i] = o;
        if (dbr) {
          u16x4 b;
          b[0] = HT::h(o.x * bscale);
          b[1] = HT::h(o.y * bscale);
          b[2] = HT::h(o.z * bscale);
          b[3] = HT::h(o.w * bscale);
          bad |= HT::bad(b[0]) | HT::bad(b[1]) | HT::bad(b[2]) | HT::bad(b[3]);
          dbr[i] = b;
        }
        acc[j].x += dyv[j].x * xv[j].x * r;
        acc[j].y += dyv[j].y * xv[j].y * r;
        acc[j].z += dyv[j].z * xv[j].z * r;
        acc[j].w += dyv[j].w * xv[j].w * r;
      }
    }
    if (row + 1 < r1) {
#pragma unroll
      for (int j = 0; j < RMS_VPT; j++) {
        dyv[j] = dyn[j];
        xv[j] = xn[j];
        rsv[j] = rsn[j];
      }
      r = rn;
    }
  }
  flag_overflow(ovf, bad);
#pragma unroll
  for (int j = 0; j < RMS_VPT; j++) {
    const int i = t + RMS_NT * j;
    if (i < D4) {
      const float4 v = make_float4(dg_scale * acc[j].x, dg_scale * acc[j].y, dg_scale * acc[j].z, dg_scale * acc[j].w);
      if (part) {
        *(float4 *)(part + (long)blockIdx.x * D + 4 * i) = v;  // reduced in block order by colsum_kernel
      } else {
        atomicAdd(dg + 4 * i, v.x);
        atomicAdd(dg + 4 * i + 1, v.y);
        atomicAdd(dg + 4 * i + 2, v.z);
        atomicAdd(dg + 4 * i + 3, v.w);
      }
    }
  }
}

// out[j] += sum_r part[r * n + j] for r in [0, rows): the deterministic second pass of the
// per-block gain-gradient partials.  Block = 64 columns x 16 row groups; row group g sums
// rows g, g+16, ... in order, then the 16 group sums are added in group order, so the
// result does not depend on scheduling.  grid.y selects one of two (part, rows, out) sets.
constexpr int CS_COLS = 64, CS_GROUPS = 16;
__global__ __launch_bounds__(CS_COLS * CS_GROUPS) void colsum_kernel(const float *__restrict__ part0, int rows0,
                                                                     float *__restrict__ out0,
                                                                     const float *__restrict__ part1, int rows1,
                                                                     float *__restrict__ out1, int n) {
  __shared__ float red[CS_GROUPS][CS_COLS];
  const float *part = blockIdx.y ? part1 : part0;
  const int rows = blockIdx.y ? rows1 : rows0;
  float *out = blockIdx.y ? out1 : out0;
  const int c = threadIdx.x % CS_COLS, grp = threadIdx.x / CS_COLS;
  const int j = blockIdx.x * CS_COLS + c;
  float s = 0.f;
  if (j < n) {
    int r = grp;
    for (; r + 3 * CS_GROUPS < rows; r += 4 * CS_GROUPS) {
      const float a = part[(long)r * n + j], b = part[(long)(r + CS_GROUPS) * n + j];
      const float d = part[(long)(r + 2 * CS_GROUPS) * n + j], e = part[(long)(r + 3 * CS_GROUPS) * n + j];
      s += a;
      s += b;
      s += d;
      s += e;
    }
    for (; r < rows; r += CS_GROUPS) s += part[(long)r * n + j];
  }
  red[grp][c] = s;
  __syncthreads();
  if (grp == 0 && j < n) {
    float t = red[0][c];
#pragma unroll
    for (int g = 1; g < CS_GROUPS; g++) t += red[g][c];
    out[j] += t;
  }
}

// colsum_kernel over a table of jobs (blockIdx.y = job), the same summation order.
__global__ __launch_bounds__(CS_COLS * CS_GROUPS) void colsum_batch_kernel(const ColsumJob *__restrict__ jobs) {
  __shared__ float red[CS_GROUPS][CS_COLS];
  const ColsumJob jb = jobs[blockIdx.y];
  const float *part = jb.part;
  const int rows = jb.rows, n = jb.n;
  const int c = threadIdx.x % CS_COLS, grp = threadIdx.x / CS_COLS;
  const int j = blockIdx.x * CS_COLS + c;
  if (blockIdx.x * CS_COLS >= n) return;  // uniform: this job has fewer columns
  float s = 0.f;
  if (j < n) {
    int r = grp;
    for (; r + 3 * CS_GROUPS < rows; r += 4 * CS_GROUPS) {
      const float a = part[(long)r * n + j], b = part[(long)(r + CS_GROUPS) * n + j];
      const float d = part[(long)(r + 2 * CS_GROUPS) * n + j], e = part[(long)(r + 3 * CS_GROUPS) * n + j];
      s += a;
      s += b;
      s += d;
      s += e;
    }
    for (; r < rows; r += CS_GROUPS) s += part[(long)r * n + j];
  }
  red[grp][c] = s;
  __syncthreads();
  if (grp == 0 && j < n) {
    float t = red[0][c];
#pragma unroll
    for (int g = 1; g < CS_GROUPS; g++) t += red[g][c];
    jb.out[j] += t;
  }
}

// gate = silu(h1) * h3, h13 = [h1 | h3] per row   (TD/mil_dynamic.h:276-281)
// With split-K partials of the W1|W3 GEMM (sp.n > 0) h1 and h3 are summed in split order,
// scaled, rounded to 16 bits and written to h13 (read by the backward) before use.
template <typename HT>
__global__ void swiglu_fwd_kernel(h16_t *__restrict__ h13, h16_t *__restrict__ gate, int T,
                                  int H, int *ovf, SplitIn sp, int *ovf_h13) {
  bool bad = false, bad13 = false;
  const long n4 = (long)T * H / 4;
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n4; i += (long)gridDim.x * blockDim.x) {
    const long e = i * 4;
    const long t = e / H, c = e % H;
    u16x4 a, b;
    if (sp.n > 0) {
      const float *p = sp.part + t * 2 * H + c;
      float4 s1 = *(const float4 *)p, s3 = *(const float4 *)(p + H);
      for (int z = 1; z < sp.n; z++) {
        const float4 q1 = *(const float4 *)(p + z * sp.slice), q3 = *(const float4 *)(p + z * sp.slice + H);
        s1.x += q1.x; s1.y += q1.y; s1.z += q1.z; s1.w += q1.w;
        s3.x += q3.x; s3.y += q3.y; s3.z += q3.z; s3.w += q3.w;
      }
      a[0] = HT::h(s1.x * sp.alpha); a[1] = HT::h(s1.y * sp.alpha);
      a[2] = HT::h(s1.z * sp.alpha); a[3] = HT::h(s1.w * sp.alpha);
      b[0] = HT::h(s3.x * sp.alpha); b[1] = HT::h(s3.y * sp.alpha);
      b[2] = HT::h(s3.z * sp.alpha); b[3] = HT::h(s3.w * sp.alpha);
#pragma unroll
      for (int j = 0; j < 4; j++) bad13 |= HT::bad(a[j]) | HT::bad(b[j]);
      *(u16x4 *)(h13 + t * 2 * H + c) = a;
      *(u16x4 *)(h13 + t * 2 * H + H + c) = b;
    } else {
      a = *(const u16x4 *)(h13 + t * 2 * H + c);
      b = *(const u16x4 *)(h13 + t * 2 * H + H + c);
    }
    u16x4 o;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      o[j] = swiglu_gate<HT>(a[j], b[j]);
      bad |= HT::bad(o[j]);
    }
    *(u16x4 *)(gate + e) = o;
  }
  flag_overflow(ovf, bad);
  flag_overflow(ovf_h13, bad13);
}

// Per (token, head): optional per-head RMSNorm with gain g[HD], then interleaved RoPE on the
// pairs (2i, 2i+1) at position t % S with fp32 tables cos/sin [S, HD/2].  One block per token;
// each head slot is HD/8 consecutive lanes owning 8 elements (4 pairs) each, so every access
// is 16 bytes.  Head slots 0..NH-1 are q heads (qkv columns h*HD), NH..NH+NKV-1 are k heads
// (columns NH*HD + (h-NH)*HD).  Replaces the RoPE of gen_sdpa_fwd_dynamic
// (TD/mil_dynamic.h:133-169).
// With split-K partials of the QKV GEMM (sp.n > 0, qkv row pitch ld = q|k|v width) the
// threads also cover the v heads: each element is summed in split order, scaled, rounded to
// 16 bits and written to qkv (the GEMM's own output, read by attention and the backward), and
// the q/k elements continue from the rounded values.
template <typename HT, bool QKN, int HD>
__global__ __launch_bounds__(256) void qk_prep_fwd_kernel(h16_t *__restrict__ qkv, long ld,
                                                          const float *__restrict__ cosb,
                                                          const float *__restrict__ sinb,
                                                          const float *__restrict__ gq,
                                                          const float *__restrict__ gk, h16_t *__restrict__ qr,
                                                          h16_t *__restrict__ kr, float *__restrict__ rq,
                                                          float *__restrict__ rk, int S, int NH, int NKV,
                                                          float eps, SplitIn sp, int *ovf_qkv) {
  constexpr int TPH = HD / 8, HALF = HD / 2;  // lanes per head slot (a divisor of 64)
  const long t = blockIdx.x;
  const int slots = sp.n > 0 ? NH + 2 * NKV : NH + NKV;
  const int pos = (int)(t % S);
  bool bad = false;
  // whole head slots are active or idle together, so the shuffles below stay within a slot
  for (int w = threadIdx.x; w < slots * TPH; w += 256) {
    const int h = w / TPH, j = w % TPH;
    const bool isq = h < NH, isv = h >= NH + NKV;
    const int hh = isq ? h : isv ? h - NH - NKV : h - NH;
    const long col = (isq ? 0 : isv ? (long)(NH + NKV) * HD : (long)NH * HD) + (long)hh * HD + 8 * j;
    u16x8 pr;
    if (sp.n > 0) {
      const float *p = sp.part + t * ld + col;
      float4 s0 = *(const float4 *)p, s1 = *(const float4 *)(p + 4);
      for (int z = 1; z < sp.n; z++) {
        const float4 a0 = *(const float4 *)(p + z * sp.slice), a1 = *(const float4 *)(p + z * sp.slice + 4);
        s0.x += a0.x; s0.y += a0.y; s0.z += a0.z; s0.w += a0.w;
        s1.x += a1.x; s1.y += a1.y; s1.z += a1.z; s1.w += a1.w;
      }
      const float v[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
      for (int e = 0; e < 8; e++) {
        pr[e] = HT::h(v[e] * sp.alpha);
        bad |= HT::bad(pr[e]);
      }
      *(u16x8 *)(qkv + t * ld + col) = pr;
      if (isv) continue;  // uniform per head slot
    } else {
      pr = *(const u16x8 *)(qkv + t * ld + col);
    }
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; e++) x[e] = HT::f(pr[e]);
    if (QKN) {
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; e++) ss += x[e] * x[e];
      ss = group_sum<TPH>(ss);
      const float r = 1.0f / sqrtf(ss / (float)HD + eps);
      const float *gg = (isq ? gq : gk) + 8 * j;
      const float4 g0 = *(const float4 *)gg, g1 = *(const float4 *)(gg + 4);
      const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
      for (int e = 0; e < 8; e++) x[e] = x[e] * r * gv[e];
      if (j == 0) {
        if (isq) rq[t * NH + hh] = r;
        else rk[t * NKV + hh] = r;
      }
    }
    const float4 c4 = *(const float4 *)(cosb + (long)pos * HALF + 4 * j);
    const float4 s4 = *(const float4 *)(sinb + (long)pos * HALF + 4 * j);
    const float cv[4] = {c4.x, c4.y, c4.z, c4.w}, sv[4] = {s4.x, s4.y, s4.z, s4.w};
    u16x8 o;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const float x0 = x[2 * q], x1 = x[2 * q + 1];
      o[2 * q] = HT::h(x0 * cv[q] - x1 * sv[q]);
      o[2 * q + 1] = HT::h(x0 * sv[q] + x1 * cv[q]);
    }
    if (isq) *(u16x8 *)(qr + t * (long)NH * HD + (long)hh * HD + 8 * j) = o;
    else *(u16x8 *)(kr + t * (long)NKV * HD + (long)hh * HD + 8 * j) = o;
  }
  flag_overflow(ovf_qkv, bad);
}

// Backward of qk_prep: inverse rotation (TD/cpu_ops.h:510-537), then the exact
// per-head RMSNorm backward; gain gradients reduced per block, one atomic per channel.
// Block = 256 threads = 256/(HD/2) token rows of one head slot; grid.y = head slot.
template <typename HT, bool QKN>
__global__ __launch_bounds__(256) void qk_prep_bwd_kernel(
    const float *__restrict__ dq, const float *__restrict__ dk, const h16_t *__restrict__ qkv, long ld,
    const float *__restrict__ cosb, const float *__restrict__ sinb, const float *__restrict__ gq,
    const float *__restrict__ gk, const float *__restrict__ rq, const float *__restrict__ rk,
    h16_t *__restrict__ dqkv, float *__restrict__ dgq, float *__restrict__ dgk, float dg_scale, int T,
    int S, int NH, int NKV, int HD, int tok_per_block, int *ovf, float *__restrict__ part,
    const float *__restrict__ kvpart, int *ovf_v) {
  bool bad = false;
  __shared__ float red[256 * 2];
  const int half = HD / 2;
  const int i = threadIdx.x % half;
  const int sub = threadIdx.x / half, nsub = 256 / half;
  const int h = blockIdx.y;
  const int ratio = NH / NKV;
  if (h >= NH + NKV) {
    // dV of kv head h - NH - NKV: the head-order sum of its query heads' partials (kvpart's
    // second half), rounded to 16 bits into dqkv's v columns
    const int kvh = h - NH - NKV;
    const float *pv = kvpart + (long)T * NH * HD;
    const long t0 = (long)blockIdx.x * tok_per_block, t1 = min((long)T, t0 + tok_per_block);
    for (long t = t0 + sub; t < t1; t += nsub) {
      float2 sv = make_float2(0.f, 0.f);
      for (int r = 0; r < ratio; r++) {
        const float2 y = *(const float2 *)(pv + t * NH * HD + (long)(kvh * ratio + r) * HD + 2 * i);
        sv.x += y.x; sv.y += y.y;
      }
      const h16_t o0 = HT::h(sv.x), o1 = HT::h(sv.y);
      bad |= HT::bad(o0) | HT::bad(o1);
      *(uint32_t *)(dqkv + t * ld + (long)(NH + NKV) * HD + (long)kvh * HD + 2 * i) = (uint32_t)o0 | ((uint32_t)o1 << 16);
    }
    flag_overflow(ovf_v, bad);
    return;
  }
  const bool isq = h < NH;
  const int hh = isq ? h : h - NH;
  const long col = (isq ? 0 : (long)NH * HD) + (long)hh * HD + 2 * i;
  const float *gg = isq ? gq : gk;
  float g0 = 0.f, g1 = 0.f;
  if (QKN) {
    g0 = gg[2 * i];
    g1 = gg[2 * i + 1];
  }
  float a0 = 0.f, a1 = 0.f;
  const long t0 = (long)blockIdx.x * tok_per_block;
  const long t1 = min((long)T, t0 + tok_per_block);
  for (long t = t0 + sub; t < t1; t += nsub) {
    float2 dd;
    if (isq) {
      dd = *(const float2 *)(dq + t * (long)NH * HD + (long)hh * HD + 2 * i);
    } else if (kvpart) {  // dK: the head-order sum of the query heads' partials
      dd = make_float2(0.f, 0.f);
      for (int r = 0; r < ratio; r++) {
        const float2 y = *(const float2 *)(kvpart + t * (long)NH * HD + (long)(hh * ratio + r) * HD + 2 * i);
        dd.x += y.x; dd.y += y.y;
      }
    } else {
      dd = *(const float2 *)(dk + t * (long)NKV * HD + (long)hh * HD + 2 * i);
    }
    const int pos = t % S;
    const float c = cosb[pos * half + i], s = sinb[pos * half + i];
    float d0 = dd.x * c + dd.y * s;
    float d1 = dd.y * c - dd.x * s;
    if (QKN) {
      const uint32_t pr = *(const uint32_t *)(qkv + t * ld + col);
      const float x0 = HT::f((h16_t)(pr & 0xFFFF)), x1 = HT::f((h16_t)(pr >> 16));
      const float r = isq ? rq[t * NH + hh] : rk[t * NKV + hh];
      float dot = d0 * x0 * g0 + d1 * x1 * g1;
      dot = half == 64 ? group_sum<64>(dot) : group_sum<32>(dot);  // HD = 128 or 64
      const float cc = r * r * r * dot / (float)HD;
      a0 += d0 * x0 * r;
      a1 += d1 * x1 * r;
      d0 = r * g0 * d0 - x0 * cc;
      d1 = r * g1 * d1 - x1 * cc;
    }
    const h16_t o0 = HT::h(d0), o1 = HT::h(d1);
    bad |= HT::bad(o0) | HT::bad(o1);
    *(uint32_t *)(dqkv + t * ld + col) = (uint32_t)o0 | ((uint32_t)o1 << 16);
  }
  flag_overflow(ovf, bad);
  if (QKN) {
    red[threadIdx.x * 2] = a0;
    red[threadIdx.x * 2 + 1] = a1;
    __syncthreads();
    if (sub == 0) {
      float s0 = 0.f, s1 = 0.f;
      for (int k = 0; k < nsub; k++) {
        s0 += red[(k * half + i) * 2];
        s1 += red[(k * half + i) * 2 + 1];
      }
      if (part) {  // layout [head slot][token block][HD], reduced by colsum_kernel
        float *pp = part + ((long)h * gridDim.x + blockIdx.x) * HD;
        pp[2 * i] = dg_scale * s0;
        pp[2 * i + 1] = dg_scale * s1;
      } else {
        float *dg = isq ? dgq : dgk;
        atomicAdd(dg + 2 * i, dg_scale * s0);
        atomicAdd(dg + 2 * i + 1, dg_scale * s1);
      }
    }
  }
}

}  // namespace

int launch_embed_fwd(const float *E, const int32_t *tok, float *x, int T, int D, hipStream_t s) {
  if (D % 4) return ne_fail(NE_ERR_ARG, "embed: D %% 4 != 0");
  hipLaunchKernelGGL(embed_fwd_kernel, dim3((T + 3) / 4), dim3(256), 0, s, E, tok, x, T, D);
  return ne_hip_status(hipGetLastError(), "embed_fwd");
}

int launch_embed_fwd_adam(const float *E, const float *G, const float *M, const float *V, const int32_t *tok,
                          float *x, int T, int D, const AdamArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(embed_fwd_adam_kernel, dim3((T + 3) / 4), dim3(256), 0, s, E, G, M, V, tok, x, T, D, a);
  return ne_hip_status(hipGetLastError(), "embed_fwd_adam");
}

int launch_embed_bwd(float *gE, const int32_t *tok, const float *dx, float scale, int T, int D, hipStream_t s) {
  hipLaunchKernelGGL(embed_bwd_kernel, dim3((T + 3) / 4), dim3(256), 0, s, gE, tok, dx, scale, T, D);
  return ne_hip_status(hipGetLastError(), "embed_bwd");
}

int launch_embed_bwd_chain(float *gE, const int32_t *tok, const int32_t *nxt, const int32_t *first,
                           const float *dx, float scale, int T, int D, hipStream_t s, double *dsq) {
  if (D % 4 || D > 4 * 64 * EMB_MAXV) return ne_fail(NE_ERR_ARG, "embed_bwd: D must be a multiple of 4, <= 2048");
  hipLaunchKernelGGL(embed_bwd_chain_kernel, dim3((T + 3) / 4), dim3(256), 0, s, gE, tok, nxt, first, dx, scale, T, D,
                     dsq);
  return ne_hip_status(hipGetLastError(), "embed_bwd_chain");
}

int launch_rmsnorm_fwd(int dt, const float *x, const float *g, h16_t *y, float *r, int T, int D, float eps,
                       int *ovf, hipStream_t s, const SplitIn &sp) {
  if (D % 4 || D > 4 * RMS_NT * RMS_VPT)
    return ne_fail(NE_ERR_ARG, "rmsnorm: D=%d must be a multiple of 4 <= 2048", D);
  if (T <= 0) return 0;
  return DISPATCH_H16(dt, [&] {
    hipLaunchKernelGGL(rmsnorm_fwd_kernel<HT>, dim3(T), dim3(RMS_NT), 0, s, (float *)x, g, y, r, D, eps, ovf, sp);
    return ne_hip_status(hipGetLastError(), "rmsnorm_fwd");
  }());
}

namespace {
int rms_rows(int T) { return std::max(1, (T + 1023) / 1024); }  // rows per block: <= 1024 blocks
// Tokens per block of the QK-prep backward: on short steps one per thread group (HD/2 threads a
// token), so a block runs one pass and there are 4x-8x more blocks (256 tokens: 10.3 us with
// 16 tokens a block, four passes of dependent loads); 128 on long steps.
int qk_tpb(int T, int HD) { return T <= 4096 ? 512 / HD : 128; }
}  // namespace

long rmsnorm_bwd_part_elems(int T, int D) { return (long)((T + rms_rows(T) - 1) / rms_rows(T)) * D; }
int rmsnorm_bwd_part_rows(int T) { return (T + rms_rows(T) - 1) / rms_rows(T); }
void qk_prep_bwd_part_rows(int T, int NH, int NKV, int HD, int *rows_q, int *rows_k) {
  const int nbx = (T + qk_tpb(T, HD) - 1) / qk_tpb(T, HD);
  *rows_q = NH * nbx;
  *rows_k = NKV * nbx;
}

int launch_colsum_batch(const ColsumJob *jobs_dev, int njobs, int max_n, hipStream_t s) {
  if (njobs <= 0) return 0;
  hipLaunchKernelGGL(colsum_batch_kernel, dim3((max_n + CS_COLS - 1) / CS_COLS, njobs), dim3(CS_COLS * CS_GROUPS), 0,
                     s, jobs_dev);
  return ne_hip_status(hipGetLastError(), "colsum_batch");
}
long qk_prep_bwd_part_elems(int T, int NH, int NKV, int HD) {
  return (long)((T + qk_tpb(T, HD) - 1) / qk_tpb(T, HD)) * (NH + NKV) * HD;
}

int launch_rmsnorm_bwd(int dt, const float *dy, const float *x, const float *g, const float *r,
                       const float *resid, float *dx, h16_t *dxb, float bscale, float *dg, float dg_scale, int T,
                       int D, int *ovf, float *part, hipStream_t s, const SplitIn &sp, bool defer_colsum,
                       bool ref_formula) {
  if (D % 4 || D > 4 * RMS_NT * RMS_VPT)
    return ne_fail(NE_ERR_ARG, "rmsnorm_bwd: D=%d must be a multiple of 4 <= 2048", D);
  if (T <= 0) return 0;
  const int rows = rms_rows(T);
  const int nb = (T + rows - 1) / rows;
  NE_CHECK(DISPATCH_H16(dt, [&] {
    auto kernel = ref_formula ? rmsnorm_bwd_kernel<HT, true> : rmsnorm_bwd_kernel<HT, false>;
    hipLaunchKernelGGL(kernel, dim3(nb), dim3(RMS_NT), 0, s, dy, x, g, r, resid, dx, dxb, bscale, dg, dg_scale, T, D,
                       rows, ovf, part, sp);
    return ne_hip_status(hipGetLastError(), "rmsnorm_bwd");
  }()));
  if (part && !defer_colsum) {
    hipLaunchKernelGGL(colsum_kernel, dim3((D + CS_COLS - 1) / CS_COLS, 1), dim3(CS_COLS * CS_GROUPS), 0, s, part, nb,
                       dg, part, nb, dg, D);
    NE_HIP(hipGetLastError());
  }
  return 0;
}

int launch_swiglu_fwd(int dt, const h16_t *h13, h16_t *gate, int T, int H, int *ovf, hipStream_t s,
                      const SplitIn &sp, int *ovf_h13) {
  if (H % 4) return ne_fail(NE_ERR_ARG, "swiglu: H %% 4 != 0");
  const long n4 = (long)T * H / 4;
  const int blocks = (int)std::min<long>((n4 + 255) / 256, 8192);
  return DISPATCH_H16(dt, [&] {
    hipLaunchKernelGGL(swiglu_fwd_kernel<HT>, dim3(blocks), dim3(256), 0, s, (h16_t *)h13, gate, T, H, ovf, sp,
                       ovf_h13);
    return ne_hip_status(hipGetLastError(), "swiglu_fwd");
  }());
}

int launch_qk_prep_fwd(int dt, const h16_t *qkv, long ld, const float *cosb, const float *sinb,
                       const float *gq, const float *gk, h16_t *qr, h16_t *kr, float *rq,
                       float *rk, int T, int S, int NH, int NKV, int HD, float eps, hipStream_t s,
                       const SplitIn &sp, int *ovf_qkv) {
  if (HD != 64 && HD != 128) return ne_fail(NE_ERR_ARG, "qk_prep: head_dim %d not in {64,128}", HD);
  if (sp.n > 0 && ld != (long)(NH + 2 * NKV) * HD) return ne_fail(NE_ERR_ARG, "qk_prep: split input needs a dense qkv");
  if (ld % 8 || ((uintptr_t)qkv & 15)) return ne_fail(NE_ERR_ARG, "qk_prep: qkv rows must be 16-byte aligned (ld %% 8 == 0)");
  h16_t *q = (h16_t *)qkv;
  return DISPATCH_H16(dt, [&] {
    auto go = [&](auto kernel) {
      hipLaunchKernelGGL(kernel, dim3(T), dim3(256), 0, s, q, ld, cosb, sinb, gq, gk, qr, kr, rq, rk, S, NH, NKV, eps,
                         sp, ovf_qkv);
    };
    if (HD == 128) {
      if (gq) go(qk_prep_fwd_kernel<HT, true, 128>);
      else go(qk_prep_fwd_kernel<HT, false, 128>);
    } else {
      if (gq) go(qk_prep_fwd_kernel<HT, true, 64>);
      else go(qk_prep_fwd_kernel<HT, false, 64>);
    }
    return ne_hip_status(hipGetLastError(), "qk_prep_fwd");
  }());
}

int launch_qk_prep_bwd(int dt, const float *dq, const float *dk, const h16_t *qkv, long ld,
                       const float *cosb, const float *sinb, const float *gq, const float *gk,
                       const float *rq, const float *rk, h16_t *dqkv, float *dgq, float *dgk, float dg_scale,
                       int T, int S, int NH, int NKV, int HD, int *ovf, float *part, hipStream_t s,
                       bool defer_colsum, const float *kvpart, int *ovf_v) {
  if (HD != 64 && HD != 128) return ne_fail(NE_ERR_ARG, "qk_prep: head_dim %d not in {64,128}", HD);
  if (kvpart && (ld % 2 || NH % NKV)) return ne_fail(NE_ERR_ARG, "qk_prep: bad layout for the dK/dV partials");
  const int tpb = qk_tpb(T, HD);
  const int nbx = (T + tpb - 1) / tpb;
  dim3 grid(nbx, NH + NKV + (kvpart ? NKV : 0));
  NE_CHECK(DISPATCH_H16(dt, [&] {
    if (gq) hipLaunchKernelGGL((qk_prep_bwd_kernel<HT, true>), grid, dim3(256), 0, s, dq, dk, qkv, ld, cosb, sinb, gq, gk, rq, rk, dqkv, dgq, dgk, dg_scale, T, S, NH, NKV, HD, tpb, ovf, part, kvpart, ovf_v);
    else hipLaunchKernelGGL((qk_prep_bwd_kernel<HT, false>), grid, dim3(256), 0, s, dq, dk, qkv, ld, cosb, sinb, gq, gk, rq, rk, dqkv, dgq, dgk, dg_scale, T, S, NH, NKV, HD, tpb, ovf, part, kvpart, ovf_v);
    return ne_hip_status(hipGetLastError(), "qk_prep_bwd");
  }()));
  if (gq && part && !defer_colsum) {
    hipLaunchKernelGGL(colsum_kernel, dim3((HD + CS_COLS - 1) / CS_COLS, 2), dim3(CS_COLS * CS_GROUPS), 0, s, part,
                       NH * nbx, dgq, part + (long)NH * nbx * HD, NKV * nbx, dgk, HD);
    NE_HIP(hipGetLastError());
  }
  return 0;
}
