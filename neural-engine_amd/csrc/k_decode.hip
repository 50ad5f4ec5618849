// KV-cached token loop: the MI355X form of generate() in TD/tools/generate.py:113-228.
//
// Per generated position every layer runs: RMSNorm -> fused QKV GEMV -> (QK-norm) RoPE +
// KV-cache append -> GQA attention over the cache -> Wo GEMV + residual -> RMSNorm ->
// W1|W3 GEMV -> SwiGLU -> W2 GEMV + residual; then the final norm, the tied LM-head GEMV
// and greedy / temperature / top-p sampling on device.  Weights are the 16-bit shadow;
// activations, the KV cache and all accumulation are fp32.
//
// The GEMVs run on v_mfma_f32_16x16x4_f32: a wave multiplies 16 weight rows by up to 16
// (or 32) sequences, each lane loading 8 consecutive 16-bit weights per 32-wide K chunk, so
// every weight byte is read once per step whatever the batch.  The four waves of a block
// split K and reduce through LDS (deterministic).
#include <math.h>

#include "common.h"
#include "ne_ctx.h"

namespace {

struct Dec {
  int Bp;                 // padded batch (16 or 32)
  int ctx;                // max positions
  float *kc, *vc;         // [L][Bp][NKV][ctx][HD]
  float *x, *xn, *qkv, *q, *att, *h13, *gate, *logits;  // [Bp, *]
  int32_t *tok;           // [Bp] current token
  int32_t *out;           // [Bp, ctx] generated tokens
  double *unif;           // [Bp, ctx]
  float *cosb, *sinb;     // [ctx, HD/2]
  void *arena;
};

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, const f32x4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// out[b, n] = (resid ? resid[b,n] : 0) + alpha * sum_k W[n,k] x[b,k]
template <typename HT, int NB>
__global__ __launch_bounds__(256) void gemv_kernel(const h16_t *__restrict__ W, long ldw,
                                                   const float *__restrict__ x, int K,
                                                   float *out, long ldo, const float *resid, float alpha) {
  __shared__ f32x4 red[4][NB][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const long row = (long)blockIdx.x * 16 + r;
  const int ks = K / 4;
  const int kbeg = w * ks;
  f32x4 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; nb++) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  const h16_t *wr = W + row * ldw;
  for (int k0 = kbeg; k0 < kbeg + ks; k0 += 32) {
    const u16x8 wv = *(const u16x8 *)(wr + k0 + g * 8);
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
      const float4 *xr = (const float4 *)(x + (long)(nb * 16 + r) * K + k0 + g * 8);
      const float4 xa = xr[0], xb = xr[1];
      const float xs[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
      for (int j = 0; j < 8; j++) acc[nb] = mfma_f32(HT::f(wv[j]), xs[j], acc[nb]);
    }
  }
#pragma unroll
  for (int nb = 0; nb < NB; nb++) red[w][nb][lane] = acc[nb];
  __syncthreads();
  if (w == 0) {
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
      f32x4 s = red[0][nb][lane] + red[1][nb][lane] + red[2][nb][lane] + red[3][nb][lane];
      // s[i] = out[batch nb*16 + r][row block*16 + 4g + i]
      const long b = nb * 16 + r;
      const long n = (long)blockIdx.x * 16 + g * 4;
      float4 o = make_float4(alpha * s[0], alpha * s[1], alpha * s[2], alpha * s[3]);
      if (resid) {
        const float4 q = *(const float4 *)(resid + b * ldo + n);
        o.x += q.x; o.y += q.y; o.z += q.z; o.w += q.w;
      }
      *(float4 *)(out + b * ldo + n) = o;
    }
  }
}

template <typename HT>
__global__ void dec_embed_kernel(const h16_t *__restrict__ E, const int32_t *__restrict__ tok, float *x, int D,
                                 int B) {
  const int b = blockIdx.x;
  for (int i = threadIdx.x; i < D; i += blockDim.x)
    x[(long)b * D + i] = (b < B) ? HT::f(E[(long)tok[b] * D + i]) : 0.f;
}

// generate.py:81-84: (x / rms) * w, rms = sqrt(mean(x^2) + eps); one block per sequence
__global__ void dec_rmsnorm_kernel(const float *__restrict__ x, const float *__restrict__ g, float *y, int D,
                                   float eps) {
  __shared__ float red[4];
  const int b = blockIdx.x;
  const float *xr = x + (long)b * D;
  float ss = 0.f;
  for (int i = threadIdx.x; i < D; i += 256) ss += xr[i] * xr[i];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = red[0] + red[1] + red[2] + red[3];
  const float rms = sqrtf(tot / (float)D + eps);
  for (int i = threadIdx.x; i < D; i += 256) y[(long)b * D + i] = xr[i] / rms * g[i];
}

// One block per (sequence, head slot): optional per-head RMSNorm, RoPE at position pos,
// q -> qbuf, k/v -> cache[l][b][kvh][pos].  HD/2 threads, one pair each.
__global__ void dec_qk_kernel(const float *__restrict__ qkv, int QKV, const float *__restrict__ gq,
                              const float *__restrict__ gk, const float *__restrict__ cosb,
                              const float *__restrict__ sinb, float *q, float *kc, float *vc, int NH, int NKV,
                              int HD, int ctx, int pos, float eps, int B) {
  const int b = blockIdx.x, h = blockIdx.y;
  const int i = threadIdx.x, half = HD / 2;
  if (b >= B) return;
  const bool isq = h < NH;
  const int hh = isq ? h : h - NH;
  const float *src = qkv + (long)b * QKV + (isq ? 0 : NH * HD) + hh * HD;
  float x0 = src[2 * i], x1 = src[2 * i + 1];
  const float *gg = isq ? gq : gk;
  if (gg) {
    float ss = x0 * x0 + x1 * x1;
    for (int o = 1; o < half; o <<= 1) ss += __shfl_xor(ss, o, 64);
    const float rms = sqrtf(ss / (float)HD + eps);
    x0 = x0 / rms * gg[2 * i];
    x1 = x1 / rms * gg[2 * i + 1];
  }
  const float c = cosb[pos * half + i], s = sinb[pos * half + i];
  const float y0 = x0 * c - x1 * s, y1 = x0 * s + x1 * c;
  if (isq) {
    q[(long)b * NH * HD + hh * HD + 2 * i] = y0;
    q[(long)b * NH * HD + hh * HD + 2 * i + 1] = y1;
  } else {
    const long base = (((long)b * NKV + hh) * ctx + pos) * HD;
    kc[base + 2 * i] = y0;
    kc[base + 2 * i + 1] = y1;
    const float *vs = qkv + (long)b * QKV + (NH + NKV) * HD + hh * HD;
    vc[base + 2 * i] = vs[2 * i];
    vc[base + 2 * i + 1] = vs[2 * i + 1];
  }
}

// One block per (sequence, q head): softmax(q.K^T * scale) V over positions 0..pos
// (generate.py:164-181).  256 threads; npos <= ctx.
__global__ __launch_bounds__(256) void dec_attn_kernel(const float *__restrict__ q, const float *__restrict__ kc,
                                                       const float *__restrict__ vc, float *att, int NH, int NKV,
                                                       int HD, int ctx, int npos, double scale, int B) {
  extern __shared__ float sm[];
  float *qs = sm;          // [HD]
  float *sc = sm + HD;     // [npos]
  __shared__ float red[8];
  const int b = blockIdx.x, h = blockIdx.y;
  if (b >= B) return;
  const int kvh = h / (NH / NKV);
  for (int d = threadIdx.x; d < HD; d += 256) qs[d] = q[(long)b * NH * HD + h * HD + d];
  __syncthreads();
  const float *K = kc + ((long)b * NKV + kvh) * ctx * HD;
  const float *V = vc + ((long)b * NKV + kvh) * ctx * HD;
  float mx = -INFINITY;
  for (int t = threadIdx.x; t < npos; t += 256) {
    const float4 *kr = (const float4 *)(K + (long)t * HD);
    float s = 0.f;
    for (int d4 = 0; d4 < HD / 4; d4++) {
      const float4 kv = kr[d4];
      s += qs[4 * d4] * kv.x + qs[4 * d4 + 1] * kv.y + qs[4 * d4 + 2] * kv.z + qs[4 * d4 + 3] * kv.w;
    }
    s = (float)((double)s * scale);
    sc[t] = s;
    mx = fmaxf(mx, s);
  }
  mx = wave_max(mx);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sum = 0.f;
  for (int t = threadIdx.x; t < npos; t += 256) {
    const float e = __expf(sc[t] - mx);
    sc[t] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  if ((threadIdx.x & 63) == 0) red[4 + (threadIdx.x >> 6)] = sum;
  __syncthreads();
  const float inv = 1.f / (red[4] + red[5] + red[6] + red[7]);
  for (int d = threadIdx.x; d < HD; d += 256) {
    float o = 0.f;
    for (int t = 0; t < npos; t++) o += sc[t] * inv * V[(long)t * HD + d];
    att[(long)b * NH * HD + h * HD + d] = o;
  }
}

__global__ void dec_swiglu_kernel(const float *__restrict__ h13, float *gate, int H, int B) {
  const int b = blockIdx.y;
  for (int j = blockIdx.x * 256 + threadIdx.x; j < H; j += gridDim.x * 256) {
    const float h1 = h13[(long)b * 2 * H + j], h3 = h13[(long)b * 2 * H + H + j];
    gate[(long)b * H + j] = h1 * (1.f / (1.f + expf(-h1))) * h3;
  }
}

// Block-wide helpers for the sampler (1024 threads).
__device__ float block_max(float v, float *red) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float m = red[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); i++) m = fmaxf(m, red[i]);
  return m;
}
__device__ double block_sum_d(double v, double *red) {
  v = wave_sum_d(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double s = 0.0;
  for (int i = 0; i < (int)(blockDim.x >> 6); i++) s += red[i];
  return s;
}

// Greedy: first index of the maximum logit (np.argmax).  Sampling: p = softmax(logits/T)
// in fp32, optional top-p mask, then the first index whose fp64 cumulative mass exceeds
// u * total (np.random.choice: cdf.searchsorted(u, side='right')).  One block / sequence.
__global__ __launch_bounds__(1024) void dec_sample_kernel(float *logits, int V, float temp, float top_p,
                                                          const double *__restrict__ unif, int ctx, int step,
                                                          int32_t *tok, int32_t *out) {
  __shared__ float redf[16];
  __shared__ double redd[16];
  __shared__ int redi[16];
  __shared__ double wsum[16];
  const int b = blockIdx.x;
  float *lg = logits + (long)b * V;
  const int tid = threadIdx.x, nt = blockDim.x;
  if (temp < 1e-6f) {
    float best = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = tid; i < V; i += nt) {
      const float v = lg[i];
      if (v > best) { best = v; bi = i; }
    }
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(best, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
    }
    if ((tid & 63) == 0) { redf[tid >> 6] = best; redi[tid >> 6] = bi; }
    __syncthreads();
    if (tid == 0) {
      float bv = redf[0];
      int bj = redi[0];
      for (int w = 1; w < nt / 64; w++)
        if (redf[w] > bv || (redf[w] == bv && redi[w] < bj)) { bv = redf[w]; bj = redi[w]; }
      tok[b] = bj;
      out[(long)b * ctx + step] = bj;
    }
    return;
  }
  // p_i = exp(x_i - max) / sum, x_i = logit_i / temp  (generate.py:201-202, softmax 87-90)
  float mx = -INFINITY;
  for (int i = tid; i < V; i += nt) mx = fmaxf(mx, lg[i] / temp);
  mx = block_max(mx, redf);
  double zs = 0.0;
  for (int i = tid; i < V; i += nt) zs += (double)expf(lg[i] / temp - mx);
  const float Z = (float)block_sum_d(zs, redd);
  for (int i = tid; i < V; i += nt) lg[i] = expf(lg[i] / temp - mx) / Z;
  __syncthreads();
  float thr = 0.f;  // keep p >= thr
  if (top_p < 1.f) {
    // thr = largest probability value v with mass(p >= v) >= top_p (generate.py:205-213):
    // bisection on the float bit pattern (monotone for positive floats).
    uint32_t lo = 0, hi = 0x3f800001u;  // mass(p >= bits(lo)) >= top_p holds at lo = 0
    while (hi - lo > 1) {
      const uint32_t mid = lo + (hi - lo) / 2;
      const float v = __uint_as_float(mid);
      double m = 0.0;
      for (int i = tid; i < V; i += nt) m += lg[i] >= v ? (double)lg[i] : 0.0;
      m = block_sum_d(m, redd);
      if (m >= (double)top_p) lo = mid; else hi = mid;
    }
    thr = __uint_as_float(lo);
  }
  // cumulative mass in vocabulary order, then the first index with cdf > u * total.
  // Thread i owns the contiguous chunk [i0, i1) and the mass interval [start[i], start[i+1]).
  __shared__ double start[1025];
  const int chunk = (V + nt - 1) / nt;
  const int i0 = min(V, tid * chunk), i1 = min(V, i0 + chunk);
  double local = 0.0;
  for (int i = i0; i < i1; i++) local += lg[i] >= thr ? (double)lg[i] : 0.0;
  double incl = local;
  for (int o = 1; o < 64; o <<= 1) {
    const double n = __shfl_up(incl, o, 64);
    if ((tid & 63) >= o) incl += n;
  }
  if ((tid & 63) == 63) wsum[tid >> 6] = incl;
  __syncthreads();
  double before = 0.0, total = 0.0;
  for (int w = 0; w < nt / 64; w++) {
    if (w < (tid >> 6)) before += wsum[w];
    total += wsum[w];
  }
  double prev = __shfl_up(incl, 1, 64);
  if ((tid & 63) == 0) prev = 0.0;
  start[tid] = before + prev;
  if (tid == 0) start[nt] = total;
  __syncthreads();
  const double u = unif[(long)b * ctx + step] * total;
  const bool last = tid == nt - 1;
  if ((start[tid] <= u && u < start[tid + 1]) || (last && u >= start[nt])) {
    double c = start[tid];
    int pick = -1;
    for (int i = i0; i < i1; i++) {
      const double p = lg[i] >= thr ? (double)lg[i] : 0.0;
      if (p > 0.0) pick = i;
      c += p;
      if (p > 0.0 && c > u) break;
    }
    if (pick < 0) {  // empty chunk (rounding at a boundary): last kept index before it
      pick = i0 - 1;
      while (pick > 0 && !(lg[pick] >= thr && lg[pick] > 0.f)) pick--;
      if (pick < 0) pick = 0;
    }
    tok[b] = pick;
    out[(long)b * ctx + step] = pick;
  }
}

__global__ void set_tokens_kernel(const int32_t *__restrict__ prompt, int P, int pos, int32_t *tok, int B) {
  const int b = threadIdx.x;
  if (b < B) tok[b] = prompt[(long)b * P + pos];
}

int gemv(ne_ctx *c, const h16_t *W, int N, int K, const float *x, float *out, const float *resid, float alpha) {
  Dec *d = (Dec *)c->dec;
  if (N % 16 || K % 128) return ne_fail(NE_ERR_ARG, "decode gemv: N=%d K=%d (need N%%16, K%%128)", N, K);
  return DISPATCH_H16(c->dt, [&] {
    if (d->Bp == 16) hipLaunchKernelGGL((gemv_kernel<HT, 1>), dim3(N / 16), dim3(256), 0, c->st, W, (long)K, x, K, out, (long)N, resid, alpha);
    else hipLaunchKernelGGL((gemv_kernel<HT, 2>), dim3(N / 16), dim3(256), 0, c->st, W, (long)K, x, K, out, (long)N, resid, alpha);
    return ne_hip_status(hipGetLastError(), "decode gemv");
  }());
}

}  // namespace

int decode_alloc(ne_ctx *c) {
  Dec *d = new Dec();
  c->dec = d;
  if (c->c.decode_batch > 32) return ne_fail(NE_ERR_ARG, "decode_batch %d > 32", c->c.decode_batch);
  d->Bp = c->c.decode_batch <= 16 ? 16 : 32;
  d->ctx = c->c.decode_ctx;
  const size_t Bp = d->Bp, ctx = d->ctx, L = c->L, D = c->D, H = c->H, Q = c->Q, NKV = c->NKV, HD = c->HD;
  const size_t kv = L * Bp * NKV * ctx * HD;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += (bytes + 255) & ~(size_t)255; return o; };
  const size_t o_kc = take(kv * 4), o_vc = take(kv * 4), o_x = take(Bp * D * 4), o_xn = take(Bp * D * 4);
  const size_t o_qkv = take(Bp * (Q + 2 * NKV * HD) * 4), o_q = take(Bp * Q * 4), o_att = take(Bp * Q * 4);
  const size_t o_h13 = take(Bp * 2 * H * 4), o_gate = take(Bp * H * 4), o_lg = take(Bp * (size_t)c->V * 4);
  const size_t o_tok = take(Bp * 4), o_out = take(Bp * ctx * 4), o_u = take(Bp * ctx * 8);
  const size_t o_cos = take(ctx * HD / 2 * 4), o_sin = take(ctx * HD / 2 * 4);
  NE_HIP(hipMalloc(&d->arena, off));
  char *base = (char *)d->arena;
  d->kc = (float *)(base + o_kc); d->vc = (float *)(base + o_vc);
  d->x = (float *)(base + o_x); d->xn = (float *)(base + o_xn);
  d->qkv = (float *)(base + o_qkv); d->q = (float *)(base + o_q); d->att = (float *)(base + o_att);
  d->h13 = (float *)(base + o_h13); d->gate = (float *)(base + o_gate); d->logits = (float *)(base + o_lg);
  d->tok = (int32_t *)(base + o_tok); d->out = (int32_t *)(base + o_out); d->unif = (double *)(base + o_u);
  d->cosb = (float *)(base + o_cos); d->sinb = (float *)(base + o_sin);
  NE_HIP(hipMemset(d->arena, 0, off));
  // RoPE tables for decode positions: float64 angles rounded to fp32 (generate.py:101-105)
  const int half = c->HD / 2;
  std::vector<float> cs(ctx * half), sn(ctx * half);
  for (size_t p = 0; p < ctx; p++)
    for (int i = 0; i < half; i++) {
      const double ang = (double)p * (1.0 / pow((double)c->c.rope_theta, 2.0 * i / c->HD));
      cs[p * half + i] = (float)cos(ang);
      sn[p * half + i] = (float)sin(ang);
    }
  NE_HIP(hipMemcpy(d->cosb, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
  NE_HIP(hipMemcpy(d->sinb, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
  return 0;
}

void decode_free(ne_ctx *c) {
  Dec *d = (Dec *)c->dec;
  if (!d) return;
  if (d->arena) hipFree(d->arena);
  delete d;
  c->dec = nullptr;
}

int decode_run(ne_ctx *c, const int32_t *prompt, int B, int P, int n_new, float temp, float top_p,
               const double *uniforms, int32_t *out) {
  Dec *d = (Dec *)c->dec;
  if (!d) return ne_fail(NE_ERR_STATE, "context created without decode buffers (decode_batch/decode_ctx)");
  if (B <= 0 || B > c->c.decode_batch || P <= 0 || n_new <= 0 || P + n_new > d->ctx)
    return ne_fail(NE_ERR_ARG, "decode: B=%d P=%d n_new=%d exceed decode_batch=%d / decode_ctx=%d", B, P, n_new,
                   c->c.decode_batch, d->ctx);
  if (temp >= 1e-6f && !uniforms) return ne_fail(NE_ERR_ARG, "decode: sampling needs uniforms");
  for (long i = 0; i < (long)B * P; i++)
    if (prompt[i] < 0 || prompt[i] >= c->V) return ne_fail(NE_ERR_ARG, "decode: prompt id out of range");
  const int D = c->D, H = c->H, Q = c->Q, NH = c->NH, NKV = c->NKV, HD = c->HD, QKV = c->QKV, V = c->V;
  const float eps = c->c.norm_eps, alpha = c->c.res_alpha;
  const double scale = 1.0 / sqrt((double)HD);
  int32_t *dprompt = nullptr;
  NE_HIP(hipMalloc((void **)&dprompt, (size_t)B * P * 4));
  NE_HIP(hipMemcpyAsync(dprompt, prompt, (size_t)B * P * 4, hipMemcpyHostToDevice, c->st));
  if (uniforms) {
    std::vector<double> u((size_t)d->Bp * d->ctx, 0.0);
    for (int b = 0; b < B; b++)
      for (int j = 0; j < n_new; j++) u[(size_t)b * d->ctx + j] = uniforms[(size_t)b * n_new + j];
    NE_HIP(hipMemcpyAsync(d->unif, u.data(), u.size() * 8, hipMemcpyHostToDevice, c->st));
    NE_HIP(hipStreamSynchronize(c->st));
  }
  const h16_t *Pb = c->Pb;
  const float *Pf = c->P;
  int rc = 0;
  int step = 0;
  for (int pos = 0; pos < P + n_new - 1 && !rc; pos++) {
    if (pos < P) hipLaunchKernelGGL(set_tokens_kernel, dim3(1), dim3(64), 0, c->st, dprompt, P, pos, d->tok, B);
    if (c->dt == NE_FP16) hipLaunchKernelGGL(dec_embed_kernel<H16F>, dim3(d->Bp), dim3(256), 0, c->st, Pb + c->off_E, d->tok, d->x, D, B);
    else hipLaunchKernelGGL(dec_embed_kernel<H16B>, dim3(d->Bp), dim3(256), 0, c->st, Pb + c->off_E, d->tok, d->x, D, B);
    for (int l = 0; l < c->L && !rc; l++) {
      const LayerOff &o = c->lo[l];
      const size_t kvl = (size_t)l * d->Bp * NKV * d->ctx * HD;
      hipLaunchKernelGGL(dec_rmsnorm_kernel, dim3(B), dim3(256), 0, c->st, d->x, Pf + o.g_att, d->xn, D, eps);
      if ((rc = gemv(c, Pb + o.wqkv, QKV, D, d->xn, d->qkv, nullptr, 1.f))) break;
      hipLaunchKernelGGL(dec_qk_kernel, dim3(B, NH + NKV), dim3(HD / 2), 0, c->st, d->qkv, QKV,
                         c->c.qk_norm ? Pf + o.gq : nullptr, c->c.qk_norm ? Pf + o.gk : nullptr, d->cosb, d->sinb,
                         d->q, d->kc + kvl, d->vc + kvl, NH, NKV, HD, d->ctx, pos, eps, B);
      hipLaunchKernelGGL(dec_attn_kernel, dim3(B, NH), dim3(256), (HD + d->ctx) * sizeof(float), c->st, d->q,
                         d->kc + kvl, d->vc + kvl, d->att, NH, NKV, HD, d->ctx, pos + 1, scale, B);
      if ((rc = gemv(c, Pb + o.wo, D, Q, d->att, d->x, d->x, alpha))) break;
      hipLaunchKernelGGL(dec_rmsnorm_kernel, dim3(B), dim3(256), 0, c->st, d->x, Pf + o.g_ffn, d->xn, D, eps);
      if ((rc = gemv(c, Pb + o.w13, 2 * H, D, d->xn, d->h13, nullptr, 1.f))) break;
      hipLaunchKernelGGL(dec_swiglu_kernel, dim3((H + 255) / 256, B), dim3(256), 0, c->st, d->h13, d->gate, H, B);
      if ((rc = gemv(c, Pb + o.w2, D, H, d->gate, d->x, d->x, alpha))) break;
    }
    if (rc) break;
    hipLaunchKernelGGL(dec_rmsnorm_kernel, dim3(B), dim3(256), 0, c->st, d->x, Pf + c->off_gfinal, d->xn, D, eps);
    if (pos >= P - 1) {
      if ((rc = gemv(c, Pb + c->off_E, V, D, d->xn, d->logits, nullptr, 1.f))) break;
      hipLaunchKernelGGL(dec_sample_kernel, dim3(B), dim3(1024), 0, c->st, d->logits, V, temp, top_p, d->unif,
                         d->ctx, step, d->tok, d->out);
      step++;
    }
    if ((rc = ne_hip_status(hipGetLastError(), "decode step"))) break;
  }
  if (!rc) {
    std::vector<int32_t> o((size_t)d->Bp * d->ctx);
    rc = ne_hip_status(hipMemcpyAsync(o.data(), d->out, o.size() * 4, hipMemcpyDeviceToHost, c->st), "decode out");
    if (!rc) rc = ne_hip_status(hipStreamSynchronize(c->st), "decode sync");
    if (!rc)
      for (int b = 0; b < B; b++)
        for (int j = 0; j < n_new; j++) out[(size_t)b * n_new + j] = o[(size_t)b * d->ctx + j];
  }
  hipStreamSynchronize(c->st);
  hipFree(dprompt);
  return rc;
}
