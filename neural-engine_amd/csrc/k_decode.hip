// KV-cached token loop: the MI355X form of generate() in TD/tools/generate.py:113-228.
//
// Per position every layer runs: RMSNorm -> fused QKV GEMV -> (QK-norm) RoPE + KV-cache
// append -> GQA attention over the cache -> Wo GEMV + residual -> RMSNorm -> W1|W3 GEMV ->
// SwiGLU -> W2 GEMV + residual; then the final norm, the tied LM-head GEMV and greedy /
// temperature / top-p sampling on the device.  Weights are the 16-bit shadow; activations,
// the KV cache and all accumulation are fp32.
//
// Every kernel reads the position from device memory (DecState), so the launch sequence of
// one position does not depend on it: it is captured once as a HIP graph (one for prompt
// positions, one for generated positions) and replayed per position.
//
// GEMVs are HBM-bound (each weight byte is read once per position whatever the batch):
//  * batch <= 4: VALU kernel.  The block stages its input rows in LDS (fusing the RMSNorm or
//    the SwiGLU gate into that prologue), each wave streams 1-4 weight rows with 16-byte
//    loads (8 weights per lane, two chunks of 512 in flight), wave reductions.  The LM-head
//    launch also writes per-block (max, first index) partials for greedy argmax.
//  * batch 5..32: v_mfma_f32_16x16x4_f32, 16 weight rows x 16 sequences per MFMA tile,
//    K split over the 4 waves of a block and over grid.y (fp32 partials, ordered reduction).
#include <math.h>

#include "common.h"
#include "ne_ctx.h"

namespace {

struct DecState {
  int pos;      // position being processed
  int P;        // prompt length
  float temp;   // < 1e-6: greedy
  float top_p;
};

constexpr int VB = 4;            // largest batch of the VALU GEMV path
constexpr int BIG_ARGMAX = 256;  // argmax partials per sequence on the MFMA path

struct Dec {
  int Bmax;               // decode_batch
  int Bp;                 // MFMA path: batch padded to 16 or 32
  int ctx;                // max positions
  float *kc, *vc;         // [L][Bmax][NKV] of V [ctx][HD] and K [ctx][HD] (batch <= 4: [HD/4][ctx] float4 pieces)
  float *x, *xn, *qkv, *att, *logits;  // [Bp, *]
  float *ws;              // MFMA split-K partials
  long ws_elems;
  float *gate;            // [Bp, H] SwiGLU gate (batch 5..32)
  float *amv;             // argmax partials [Bmax][nblk]
  int32_t *ami;
  int lm_nblk;
  int32_t *tok;           // [Bp] current token
  int32_t *out;           // [Bp, ctx] generated tokens
  int32_t *prompt;        // [Bp, ctx]
  double *unif;           // [Bp, ctx]
  float *cosb, *sinb;     // [ctx, HD/2]
  DecState *st;
  void *arena;
  struct Graph { int B; bool greedy; hipGraphExec_t pre, gen; };
  std::vector<Graph> graphs;
};

// ------------------------------------------------------------------ GEMV, batch <= 4 ----

enum { PRO_NONE = 0, PRO_RMSNORM = 1, PRO_SWIGLU = 2 };

// out[b, n] = alpha * sum_k W[n, k] * in'(b, k) + (resid ? resid[b, n] : 0), rows n of this
// block = (blockIdx.x * 4 + wave) * RPW + r.  in' = in (PRO_NONE), in / rms(in) * g
// (PRO_RMSNORM, generate.py:81-84) or silu(h1) * h3 with in = [h1 | h3] rows of 2K
// (PRO_SWIGLU).  resid may alias out (each element is read, then written, by one lane).
// AMX: also write the block's (max, first row) of each sequence to amv/ami [b][blockIdx.x].
// Every global load (input rows, gains, residual, then the wave's weights: KC chunks of 512
// per row, K <= 512*KC) is issued before the first wait, so the block pays one HBM latency,
// not one per load: with loads behind branches or in a load-store loop each waited for the
// one before, which doubled the time of a batch-1 GEMV.
// GATE (W1|W3 rows [2*gate_n, K]): the wave's rows are j..j+RPW/2-1 of W1 and the same j of
// W3 (rows gate_n + j), and it writes gate[b, j] = silu(h1) * h3 (generate.py:190) instead of h1, h3.
template <typename HT, int NB, int RPW, int KC, int PRO, bool AMX, bool GATE>
__global__ __launch_bounds__(256) void gemv_valu_kernel(const h16_t *__restrict__ W, int K,
                                                        const float *__restrict__ in, long ldi,
                                                        const float *__restrict__ g, float eps, float *out, long ldo,
                                                        const float *resid, float alpha, int B, float *amv,
                                                        int32_t *ami, int nblk, long gate_n) {
  extern __shared__ float xs[];  // [NB][K]
  __shared__ float red[4][NB];
  __shared__ float bmv[NB][4 * RPW];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  constexpr int HALF = GATE ? RPW / 2 : RPW;
  const long row0 = ((long)blockIdx.x * 4 + w) * HALF;
  auto wrow = [&](int r) -> long { return GATE && r >= HALF ? gate_n + row0 + (r - HALF) : row0 + r; };
  // Every global load of the block is issued before the first wait: the input rows (16 bytes
  // per lane, XI per row), the gains, the residual and then the weights.  Addresses past the
  // end of a row are clamped into it (no branches around loads, so none waits for another);
  // the values they bring are not used.
  constexpr int XI = (KC + 1) / 2;  // 1024 * XI >= 512 * KC >= K
  float4 xa[NB][XI], xb[PRO == PRO_SWIGLU ? NB : 1][XI], gv[XI];
#pragma unroll
  for (int i = 0; i < XI; i++) {
    const int k = (i * 256 + tid) * 4, kc = k < K ? k : K - 4;
#pragma unroll
    for (int b = 0; b < NB; b++) {
      const float *src = in + (long)(b < B ? b : B - 1) * ldi;
      xa[b][i] = *(const float4 *)(src + kc);
      if (PRO == PRO_SWIGLU) xb[b][i] = *(const float4 *)(src + K + kc);
    }
    if (PRO == PRO_RMSNORM) gv[i] = *(const float4 *)(g + kc);
  }
  // residual of this lane's output (written by the same lane below; resid may alias out)
  const int rl = lane < RPW * NB ? lane / NB : 0, bl = lane < RPW * NB ? lane % NB : 0;
  const float res_v = !GATE && resid && lane < RPW * NB && bl < B ? resid[(long)bl * ldo + row0 + rl] : 0.f;
  u16x8 wv[RPW][KC];
#pragma unroll
  for (int c = 0; c < KC; c++) {
    const int k = c * 512 + lane * 8, kc = k < K ? k : K - 8;
#pragma unroll
    for (int r = 0; r < RPW; r++) wv[r][c] = __builtin_nontemporal_load((const u16x8 *)(W + wrow(r) * K + kc));
  }
  float rms[NB];
  if (PRO == PRO_RMSNORM) {
    float ss[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
      ss[b] = 0.f;
#pragma unroll
      for (int i = 0; i < XI; i++)
        if ((i * 256 + tid) * 4 < K) {
          const float4 v = xa[b][i];
          ss[b] += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
      ss[b] = wave_sum(ss[b]);
    }
    if (lane == 0)
#pragma unroll
      for (int b = 0; b < NB; b++) red[w][b] = ss[b];
    __syncthreads();
#pragma unroll
    for (int b = 0; b < NB; b++) rms[b] = sqrtf((red[0][b] + red[1][b] + red[2][b] + red[3][b]) / (float)K + eps);
  }
#pragma unroll
  for (int i = 0; i < XI; i++) {
    const int k = (i * 256 + tid) * 4;
    if (k < K) {
#pragma unroll
      for (int b = 0; b < NB; b++) {
        float4 v = xa[b][i];
        if (PRO == PRO_SWIGLU) {
          const float4 h3 = xb[b][i];
          v.x = v.x * (1.f / (1.f + expf(-v.x))) * h3.x;
          v.y = v.y * (1.f / (1.f + expf(-v.y))) * h3.y;
          v.z = v.z * (1.f / (1.f + expf(-v.z))) * h3.z;
          v.w = v.w * (1.f / (1.f + expf(-v.w))) * h3.w;
        } else if (PRO == PRO_RMSNORM) {
          v.x = v.x / rms[b] * gv[i].x;
          v.y = v.y / rms[b] * gv[i].y;
          v.z = v.z / rms[b] * gv[i].z;
          v.w = v.w / rms[b] * gv[i].w;
        }
        if (b >= B) v = make_float4(0.f, 0.f, 0.f, 0.f);
        *(float4 *)(xs + b * K + k) = v;
      }
    }
  }
  __syncthreads();

  float acc[RPW][NB];
#pragma unroll
  for (int r = 0; r < RPW; r++)
#pragma unroll
    for (int b = 0; b < NB; b++) acc[r][b] = 0.f;
#pragma unroll
  for (int c = 0; c < KC; c++) {
    const int k = c * 512 + lane * 8;
    if (k < K) {
#pragma unroll
      for (int b = 0; b < NB; b++) {
        const float4 x0 = *(const float4 *)(xs + b * K + k), x1 = *(const float4 *)(xs + b * K + k + 4);
        const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int r = 0; r < RPW; r++)
#pragma unroll
          for (int j = 0; j < 8; j++) acc[r][b] = fmaf(HT::f(wv[r][c][j]), xv[j], acc[r][b]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; r++)
#pragma unroll
    for (int b = 0; b < NB; b++) acc[r][b] = wave_sum(acc[r][b]);
  if (GATE) {
    if (lane < HALF * NB) {
      const int r = lane / NB, b = lane % NB;
      float h1 = 0.f, h3 = 0.f;
#pragma unroll
      for (int rr = 0; rr < HALF; rr++)
#pragma unroll
        for (int bb = 0; bb < NB; bb++)
          if (rr == r && bb == b) {
            h1 = acc[rr][bb];
            h3 = acc[rr + HALF][bb];
          }
      if (b < B) out[(long)b * ldo + row0 + r] = h1 * (1.f / (1.f + expf(-h1))) * h3;
    }
    return;
  }
  if (lane < RPW * NB) {
    const int r = lane / NB, b = lane % NB;
    float v = 0.f;
#pragma unroll
    for (int rr = 0; rr < RPW; rr++)
#pragma unroll
      for (int bb = 0; bb < NB; bb++)
        if (rr == r && bb == b) v = acc[rr][bb];
    if (b < B) {
      const long n = row0 + r;
      float o = alpha * v;
      if (resid) o += res_v;
      out[(long)b * ldo + n] = o;
      if (AMX) bmv[b][w * RPW + r] = o;
    }
  }
  if (AMX) {
    __syncthreads();
    if (tid < NB && tid < B) {
      float best = bmv[tid][0];
      int bi = 0;
      for (int i = 1; i < 4 * RPW; i++)
        if (bmv[tid][i] > best) { best = bmv[tid][i]; bi = i; }  // first maximum
      amv[(long)tid * nblk + blockIdx.x] = best;
      ami[(long)tid * nblk + blockIdx.x] = (int32_t)(blockIdx.x * 4 * RPW + bi);
    }
  }
}

// ------------------------------------------------------------------ GEMV, batch 5..32 ----

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, const f32x4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Products of 16 weight rows (blockIdx.x) with x rows [Bp, K] (fp32, row stride ldx) over the
// K range of split blockIdx.y, for NT tiles of 16 sequences; the 4 waves split that range.
// With a workspace ws, split z's products go to slice z of ws [ksplit][Bp, N] (one split's
// slice is laid out as the output rows); without (one split), out = alpha * products + resid.
// GATE (one split; W = [W1; W3], gate_n rows each): the block's rows are j0..j0+7 of W1 and
// the same of W3 (j0 = 8 * blockIdx.x), and it writes out[b, j] = silu(h1) * h3
// (generate.py:190).  WV waves per block split the K range; each loads up to 8 weight chunks
// ahead of their use.
template <typename HT, int NT, bool GATE, int WV = 4>
__global__ __launch_bounds__(WV * 64) void gemv_mfma_kernel(const h16_t *__restrict__ W, long ldw,
                                                        const float *__restrict__ x, long ldx, int K, int ksplit,
                                                        float *out, long ldo, const float *resid, float alpha,
                                                        float *ws, int N, int B, long gate_n) {
  __shared__ f32x4 red[WV][NT][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const long row = GATE ? (r < 8 ? (long)blockIdx.x * 8 + r : gate_n + (long)blockIdx.x * 8 + r - 8)
                        : (long)blockIdx.x * 16 + r;
  const int kc = K / ksplit, ks = kc / WV;
  const int kbeg = blockIdx.y * kc + w * ks, kend = kbeg + ks;
  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const h16_t *wr = W + row * ldw;
  for (int base = kbeg; base < kend; base += 8 * 32) {
    u16x8 wv[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
      if (base + i * 32 < kend) wv[i] = __builtin_nontemporal_load((const u16x8 *)(wr + base + i * 32 + g * 8));
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int k0 = base + i * 32;
      if (k0 < kend) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
          const float *xr = x + (long)(t * 16 + r) * ldx + k0 + g * 8;
          const float4 a0 = *(const float4 *)xr, a1 = *(const float4 *)(xr + 4);
          const float xv[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
          for (int j = 0; j < 8; j++) acc[t] = mfma_f32(HT::f(wv[i][j]), xv[j], acc[t]);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < NT; t++) red[w][t][lane] = acc[t];
  __syncthreads();
  if (w == 0) {
#pragma unroll
    for (int t = 0; t < NT; t++) {
      f32x4 s = red[0][t][lane];
#pragma unroll
      for (int v = 1; v < WV; v++) s += red[v][t][lane];
      // s[i] = sum for sequence t*16 + r, weight row blockIdx.x*16 + 4g + i
      const int b = t * 16 + r;
      const long n = (long)blockIdx.x * 16 + g * 4;
      if (GATE) {
        // lanes g = 0, 1 hold h1 of gate outputs j0 + 4g + i; lanes g + 2 hold their h3
        f32x4 h3;
#pragma unroll
        for (int i = 0; i < 4; i++) h3[i] = __shfl(s[i], (lane + 32) & 63, 64);
        if (g < 2 && b < B) {
          float4 o;
          float *op = &o.x;
#pragma unroll
          for (int i = 0; i < 4; i++) op[i] = s[i] * (1.f / (1.f + expf(-s[i]))) * h3[i];
          *(float4 *)(out + b * ldo + (long)blockIdx.x * 8 + g * 4) = o;
        }
      } else if (ws) {
        *(f32x4 *)(ws + ((long)blockIdx.y * NT * 16 + b) * N + n) = s;
      } else if (b < B) {
        float4 o = make_float4(alpha * s[0], alpha * s[1], alpha * s[2], alpha * s[3]);
        if (resid) {
          const float4 q = *(const float4 *)(resid + b * ldo + n);
          o.x += q.x; o.y += q.y; o.z += q.z; o.w += q.w;
        }
        *(float4 *)(out + b * ldo + n) = o;
      }
    }
  }
}

// ------------------------------------------- GEMV, batch 5..32, bf16 weights, exact ----

// x = hi + mid + lo, three bf16 values obtained by truncation: hi keeps the top 8 significant
// bits of x, mid the next 8 of the remainder x - hi, lo what is left, so the sum is exact and
// each product of a bf16 weight with a part is exact in fp32.
__device__ __forceinline__ void split3(float x, uint16_t &hi, uint16_t &mid, uint16_t &lo) {
  const uint32_t u = __float_as_uint(x) & 0xFFFF0000u;
  const float r1 = x - __uint_as_float(u);
  const uint32_t u1 = __float_as_uint(r1) & 0xFFFF0000u;
  const float r2 = r1 - __uint_as_float(u1);
  hi = (uint16_t)(u >> 16);
  mid = (uint16_t)(u1 >> 16);
  lo = (uint16_t)(__float_as_uint(r2) >> 16);
}

enum { BF3_WS = 0, BF3_GATE = 1, BF3_PLAIN = 2 };

// Products of bf16 weight rows W [N, K] with fp32 x rows [Bp, K] (row stride ldx) on
// v_mfma_f32_16x16x32_bf16: each x value is split into three bf16 parts (split3) and every
// weight fragment meets the three, so the sums are of the exact products (fp32 accumulation,
// as the fp32-MFMA GEMV).  A block has 4 * NTW waves: wave w takes batch tile w / 4 (16
// sequences) and K slice w % 4 of the block's K range (KS steps of 32), holds that slice of x
// as bf16 parts in registers for all its RT row tiles of 16 weight rows, and the four K
// slices are summed in LDS in slice order.  x is read once per block for RT * 16 rows
// (the 16-row fp32-MFMA GEMV reads it once per 16 rows, 4x its weight bytes at batch 32).
//  BF3_WS:    split blockIdx.y's sums to ws slice [blockIdx.y][Bp, N] (every sequence row);
//  BF3_GATE:  W = [W1; W3] (gate_n rows each), one split: row tiles 0..RT/2-1 are W1 rows
//             j0 + 16 rt.., the rest the same rows of W3; writes out[b, j] = silu(h1) * h3
//             (generate.py:190) for b < B;
//  BF3_PLAIN: one split, out[b, n] = sums for b < B (the LM head's logits).
template <int NTW, int RT, int KS, int MODE>
__global__ __launch_bounds__(NTW * 256) void gemv_bf3_kernel(const h16_t *__restrict__ W, long ldw,
                                                             const float *__restrict__ x, long ldx,
                                                             float *__restrict__ out, long ldo, int N, int B,
                                                             int Bp, long gate_n) {
  __shared__ f32x4 red[3][NTW][RT][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int ksl = w & 3, t = w >> 2;
  const int r16 = lane & 15, g = lane >> 4;
  const int kb = (blockIdx.y * 4 + ksl) * KS * 32 + g * 8;  // this lane's k in step 0
  constexpr int HALF = RT / 2;
  auto wrow = [&](int rt) -> long {
    if constexpr (MODE == BF3_GATE) {
      const long j = (long)blockIdx.x * 16 * HALF + (rt % HALF) * 16 + r16;
      return rt < HALF ? j : gate_n + j;
    } else {
      return (long)blockIdx.x * 16 * RT + rt * 16 + r16;
    }
  };
  // the weight stream first: every fragment of the wave in flight at once
  u16x8 wf[RT][KS];
#pragma unroll
  for (int rt = 0; rt < RT; rt++) {
    const h16_t *wr = W + wrow(rt) * ldw + kb;
#pragma unroll
    for (int ks = 0; ks < KS; ks++) wf[rt][ks] = __builtin_nontemporal_load((const u16x8 *)(wr + ks * 32));
  }
  const int b = t * 16 + r16;
  u16x8 xh[KS], xm[KS], xl[KS];
  {
    const float *xr = x + (long)b * ldx + kb;
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
      const float4 a0 = *(const float4 *)(xr + ks * 32), a1 = *(const float4 *)(xr + ks * 32 + 4);
      const float v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
      for (int e = 0; e < 8; e++) {
        uint16_t h, m, l;
        split3(v[e], h, m, l);
        xh[ks][e] = h; xm[ks][e] = m; xl[ks][e] = l;
      }
    }
  }
  f32x4 acc[RT];
#pragma unroll
  for (int rt = 0; rt < RT; rt++) {
    acc[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
      const bf16x8 a = H16B::op(wf[rt][ks]);
      acc[rt] = H16B::mfma16(a, H16B::op(xh[ks]), acc[rt]);
      acc[rt] = H16B::mfma16(a, H16B::op(xm[ks]), acc[rt]);
      acc[rt] = H16B::mfma16(a, H16B::op(xl[ks]), acc[rt]);
    }
  }
  // acc[rt][i] = sum over this K slice for weight row (tile rt) 4g + i, sequence b
  if (ksl > 0) {
#pragma unroll
    for (int rt = 0; rt < RT; rt++) red[ksl - 1][t][rt][lane] = acc[rt];
  }
  __syncthreads();
  if (ksl != 0) return;
#pragma unroll
  for (int rt = 0; rt < RT; rt++) {
#pragma unroll
    for (int q = 0; q < 3; q++) acc[rt] += red[q][t][rt][lane];
  }
  if constexpr (MODE == BF3_WS) {
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
      const long n = (long)blockIdx.x * 16 * RT + rt * 16 + g * 4;
      *(f32x4 *)(out + ((long)blockIdx.y * Bp + b) * N + n) = acc[rt];
    }
  } else if constexpr (MODE == BF3_GATE) {
    if (b < B) {
#pragma unroll
      for (int rt = 0; rt < HALF; rt++) {
        float4 o;
        float *op = &o.x;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float h1 = acc[rt][i], h3 = acc[rt + HALF][i];
          op[i] = h1 * (1.f / (1.f + expf(-h1))) * h3;
        }
        *(float4 *)(out + (long)b * ldo + (long)blockIdx.x * 16 * HALF + rt * 16 + g * 4) = o;
      }
    }
  } else {
    if (b < B) {
#pragma unroll
      for (int rt = 0; rt < RT; rt++)
        *(f32x4 *)(out + (long)b * ldo + (long)blockIdx.x * 16 * RT + rt * 16 + g * 4) = acc[rt];
    }
  }
}

// One block per sequence b: out[b, :] = alpha * (ordered sum of the split-K partials, split 0
// first) + resid[b, :], and (gn != null) xn[b, :] = out[b, :] / rms * gn, the RMSNorm of the
// new row (generate.py:81-84, rms = sqrt(mean(out^2) + eps)) that the next GEMV reads.
// KS > 0 (the split count, rows of at most 1024): every partial and residual load of a thread
// is issued before the first add.
template <int KS>
__global__ __launch_bounds__(256) void gemv_reduce_rows_kernel(const float *__restrict__ ws, int ksplit, int Bp, int N,
                                                               float *out, long ldo, const float *resid, float alpha,
                                                               const float *gn, float *xn, float eps) {
  __shared__ float red[4];
  const int b = blockIdx.x, tid = threadIdx.x;
  float ss = 0.f;
  float rv[4];  // KS path: the thread's residual inputs, then its outputs
  if constexpr (KS > 0) {
    float v[4 * (KS > 0 ? KS : 1)];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int n = min(tid + 256 * e, N - 1);  // rows shorter than 1024: clamped, unused
#pragma unroll
      for (int z = 0; z < KS; z++) v[e * KS + z] = ws[((long)z * Bp + b) * N + n];
      rv[e] = resid ? resid[(long)b * ldo + n] : 0.f;
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int n = tid + 256 * e;
      if (n < N) {
        float s = 0.f;
#pragma unroll
        for (int z = 0; z < KS; z++) s += v[e * KS + z];
        float o = alpha * s;
        if (resid) o += rv[e];
        out[(long)b * ldo + n] = o;
        ss += o * o;
        rv[e] = o;
      }
    }
  } else {
    for (int n = tid; n < N; n += 256) {
      float s = 0.f;
      for (int z = 0; z < ksplit; z++) s += ws[((long)z * Bp + b) * N + n];
      float o = alpha * s;
      if (resid) o += resid[(long)b * ldo + n];
      out[(long)b * ldo + n] = o;
      ss += o * o;
    }
  }
  if (!gn) return;
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float rms = sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)N + eps);
  if constexpr (KS > 0) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int n = tid + 256 * e;
      if (n < N) xn[(long)b * N + n] = rv[e] / rms * gn[n];
    }
  } else {  // read back what this thread wrote
    for (int n = tid; n < N; n += 256) xn[(long)b * N + n] = out[(long)b * ldo + n] / rms * gn[n];
  }
}

// ------------------------------------------------------------- elementwise / attention ----

// Token of this position (prompt id while pos < P, else the last sampled id) and its
// embedding row.  One block per sequence.
template <typename HT>
__global__ void dec_token_kernel(const int32_t *__restrict__ prompt, int ctx, const DecState *__restrict__ st,
                                 int32_t *tok, const h16_t *__restrict__ E, float *x, int D, int B,
                                 const float *__restrict__ gn, float *xn, float eps) {
  __shared__ float red[4];
  const int b = blockIdx.x;
  const int pos = st->pos;
  const int t = pos < st->P ? prompt[(long)b * ctx + pos] : tok[b];
  float ss = 0.f;
  for (int i = threadIdx.x; i < D; i += blockDim.x) {
    const float v = b < B ? HT::f(E[(long)t * D + i]) : 0.f;
    x[(long)b * D + i] = v;
    ss += v * v;
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  if (threadIdx.x == 0) tok[b] = t;
  if (gn) {  // the RMSNorm of the row (generate.py:81-84), read by the batch-5..32 QKV GEMV
    const float rms = sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)D + eps);
    for (int i = threadIdx.x; i < D; i += blockDim.x) xn[(long)b * D + i] = x[(long)b * D + i] / rms * gn[i];
  }
}

// KCOL (batch <= 4, one block per KV head): the K cache holds float4 d4 of position t at
// K4[d4 * ctx + t], so that the score loop's lanes (one position each) read consecutive 16-byte
// pieces; else row-major like V ([ctx][HD]), which measured faster at batch 32.
template <int HD, int RATIO, bool KCOL>
__global__ __launch_bounds__(256) void dec_attn_kernel(const float *__restrict__ qkv, int QKV,
                                                       const float *__restrict__ gq, const float *__restrict__ gk,
                                                       const float *__restrict__ cosb, const float *__restrict__ sinb,
                                                       float *kc, float *vc, float *att, int NH, int NKV, int ctx,
                                                       const DecState *__restrict__ st, float eps, double scale,
                                                       const float *__restrict__ qws, int qnz, int Bp) {
  extern __shared__ float sc[];  // [RATIO][ctx]
  constexpr int C4 = HD / 4, NG = 256 / C4, HALF = HD / 2;
  __shared__ float4 qs[RATIO][C4];
  __shared__ float4 vn[C4];
  __shared__ float4 part[NG][RATIO][C4];
  __shared__ float red[RATIO][8];
  // block y: query heads qh0 .. qh0 + RATIO - 1 of KV head kvh (RATIO may be a part of the
  // model's NH / NKV query heads per KV head: the blocks of one KV head then append the same
  // K and V values)
  const int b = blockIdx.x, qh0 = blockIdx.y * RATIO, kvh = qh0 / (NH / NKV), tid = threadIdx.x;
  const int pos = st->pos, npos = pos + 1;
  float *K = kc + ((long)b * NKV + kvh) * ctx * HD;
  float *V = vc + ((long)b * NKV + kvh) * ctx * HD;
  const float *row = qkv + (long)b * QKV;
  // element col of this sequence's q|k|v row: the row itself, or (qnz > 1) the ordered sum of
  // the QKV GEMV's split-K partial slices [qnz][Bp, QKV]
  auto qval = [&](int col) -> float {
    if (qnz <= 1) return row[col];
    float s = 0.f;
    for (int z = 0; z < qnz; z++) s += qws[((long)z * Bp + b) * QKV + col];
    return s;
  };
  // slots 0..RATIO-1: q heads qh0 + slot; RATIO: k head kvh; RATIO+1: v head kvh
  for (int i = tid; i < (RATIO + 2) * HALF; i += 256) {
    const int slot = i / HALF, p = i % HALF;
    float *q2 = (float *)qs, *v2 = (float *)vn;
    if (slot == RATIO + 1) {
      const int c0 = (NH + NKV) * HD + kvh * HD;
      const float y0 = qval(c0 + 2 * p), y1 = qval(c0 + 2 * p + 1);
      v2[2 * p] = y0; v2[2 * p + 1] = y1;
      V[(long)pos * HD + 2 * p] = y0;
      V[(long)pos * HD + 2 * p + 1] = y1;
      continue;
    }
    const bool isq = slot < RATIO;
    const int c0 = isq ? (qh0 + slot) * HD : NH * HD + kvh * HD;
    float x0 = qval(c0 + 2 * p), x1 = qval(c0 + 2 * p + 1);
    const float *gg = isq ? gq : gk;
    if (gg) {  // uniform per block: every lane of the slot's (half-)wave takes part
      float ss = x0 * x0 + x1 * x1;
      ss = HALF == 64 ? wave_sum(ss) : half_wave_sum(ss);
      const float rms = sqrtf(ss / (float)HD + eps);
      x0 = x0 / rms * gg[2 * p];
      x1 = x1 / rms * gg[2 * p + 1];
    }
    const float c = cosb[pos * HALF + p], s = sinb[pos * HALF + p];
    const float y0 = x0 * c - x1 * s, y1 = x0 * s + x1 * c;
    if (isq) {
      q2[slot * HD + 2 * p] = y0;
      q2[slot * HD + 2 * p + 1] = y1;
    } else {
      if (KCOL) {
        *(float2 *)(K + ((long)(p >> 1) * ctx + pos) * 4 + 2 * (p & 1)) = make_float2(y0, y1);
      } else {
        K[(long)pos * HD + 2 * p] = y0;
        K[(long)pos * HD + 2 * p + 1] = y1;
      }
    }
  }
  __syncthreads();
  float mx[RATIO];
#pragma unroll
  for (int r = 0; r < RATIO; r++) mx[r] = -INFINITY;
  const float4 *K4 = (const float4 *)K;
  for (int t = tid; t < npos; t += 256) {
    // position pos was written by this block above; the barrier made it visible
    float s[RATIO];
#pragma unroll
    for (int r = 0; r < RATIO; r++) s[r] = 0.f;
#pragma unroll 8
    for (int d4 = 0; d4 < C4; d4++) {
      const float4 kv = KCOL ? K4[(long)d4 * ctx + t] : K4[(long)t * C4 + d4];
#pragma unroll
      for (int r = 0; r < RATIO; r++) {
        const float4 qv = qs[r][d4];
        s[r] += qv.x * kv.x + qv.y * kv.y + qv.z * kv.z + qv.w * kv.w;
      }
    }
#pragma unroll
    for (int r = 0; r < RATIO; r++) {
      const float v = (float)((double)s[r] * scale);
      sc[r * ctx + t] = v;
      mx[r] = fmaxf(mx[r], v);
    }
  }
#pragma unroll
  for (int r = 0; r < RATIO; r++) {
    mx[r] = wave_max(mx[r]);
    if ((tid & 63) == 0) red[r][tid >> 6] = mx[r];
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < RATIO; r++) mx[r] = fmaxf(fmaxf(red[r][0], red[r][1]), fmaxf(red[r][2], red[r][3]));
  float sum[RATIO];
#pragma unroll
  for (int r = 0; r < RATIO; r++) sum[r] = 0.f;
  for (int t = tid; t < npos; t += 256)
#pragma unroll
    for (int r = 0; r < RATIO; r++) {
      const float e = __expf(sc[r * ctx + t] - mx[r]);
      sc[r * ctx + t] = e;
      sum[r] += e;
    }
#pragma unroll
  for (int r = 0; r < RATIO; r++) {
    sum[r] = wave_sum(sum[r]);
    if ((tid & 63) == 0) red[r][4 + (tid >> 6)] = sum[r];
  }
  __syncthreads();
  const int c = tid % C4, grp = tid / C4;
  float4 acc[RATIO];
#pragma unroll
  for (int r = 0; r < RATIO; r++) acc[r] = make_float4(0.f, 0.f, 0.f, 0.f);
  // four positions per iteration: their V loads are in flight together
  int t = grp;
  for (; t + 3 * NG < npos; t += 4 * NG) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int tu = t + u * NG;
      v[u] = tu == pos ? vn[c] : *(const float4 *)(V + (long)tu * HD + c * 4);
    }
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
      for (int r = 0; r < RATIO; r++) {
        const float p = sc[r * ctx + t + u * NG];
        acc[r].x += p * v[u].x; acc[r].y += p * v[u].y; acc[r].z += p * v[u].z; acc[r].w += p * v[u].w;
      }
  }
  for (; t < npos; t += NG) {
    const float4 v = t == pos ? vn[c] : *(const float4 *)(V + (long)t * HD + c * 4);
#pragma unroll
    for (int r = 0; r < RATIO; r++) {
      const float p = sc[r * ctx + t];
      acc[r].x += p * v.x; acc[r].y += p * v.y; acc[r].z += p * v.z; acc[r].w += p * v.w;
    }
  }
#pragma unroll
  for (int r = 0; r < RATIO; r++) part[grp][r][c] = acc[r];
  __syncthreads();
  if (grp < RATIO) {
    const int r = grp;
    const float inv = 1.f / (red[r][4] + red[r][5] + red[r][6] + red[r][7]);
    float4 o = part[0][r][c];
    for (int gi = 1; gi < NG; gi++) {
      const float4 p = part[gi][r][c];
      o.x += p.x; o.y += p.y; o.z += p.z; o.w += p.w;
    }
    o.x *= inv; o.y *= inv; o.z *= inv; o.w *= inv;
    *(float4 *)(att + (long)b * NH * HD + (long)(qh0 + r) * HD + c * 4) = o;
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

__device__ __forceinline__ int gen_step(const DecState *st) { return st->pos - (st->P - 1); }

// Greedy from per-block partials: first index of the maximum logit (np.argmax).  One block
// (1024 threads) per sequence.
__global__ __launch_bounds__(1024) void dec_argmax_kernel(const float *__restrict__ amv, const int32_t *__restrict__ ami,
                                                          int nblk, const DecState *__restrict__ st, int ctx,
                                                          int32_t *tok, int32_t *out) {
  __shared__ float rv[16];
  __shared__ int ri[16];
  const int b = blockIdx.x, tid = threadIdx.x;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = tid; i < nblk; i += 1024) {
    const float v = amv[(long)b * nblk + i];
    const int j = ami[(long)b * nblk + i];
    if (v > best || (v == best && j < bi)) { best = v; bi = j; }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
  }
  if ((tid & 63) == 0) { rv[tid >> 6] = best; ri[tid >> 6] = bi; }
  __syncthreads();
  if (tid == 0) {
    best = rv[0]; bi = ri[0];
    for (int w = 1; w < 16; w++)
      if (rv[w] > best || (rv[w] == best && ri[w] < bi)) { best = rv[w]; bi = ri[w]; }
    // no logit above -inf (all NaN or -inf): token 0, so the next lookup stays in the table
    if (bi == 0x7fffffff) bi = 0;
    tok[b] = bi;
    out[(long)b * ctx + gen_step(st)] = bi;
  }
}

// Greedy over full logits rows (batch > 4): per-block partials of 4096-wide chunks.
__global__ __launch_bounds__(256) void dec_argmax_part_kernel(const float *__restrict__ logits, int V, int nblk,
                                                              float *amv, int32_t *ami) {
  __shared__ float rv[4];
  __shared__ int ri[4];
  const int b = blockIdx.y, tid = threadIdx.x;
  const int chunk = (V + nblk - 1) / nblk;
  const int i0 = blockIdx.x * chunk, i1 = min(V, i0 + chunk);
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = i0 + tid; i < i1; i += 256) {
    const float v = logits[(long)b * V + i];
    if (v > best) { best = v; bi = i; }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
  }
  if ((tid & 63) == 0) { rv[tid >> 6] = best; ri[tid >> 6] = bi; }
  __syncthreads();
  if (tid == 0) {
    best = rv[0]; bi = ri[0];
    for (int w = 1; w < 4; w++)
      if (rv[w] > best || (rv[w] == best && ri[w] < bi)) { best = rv[w]; bi = ri[w]; }
    amv[(long)b * nblk + blockIdx.x] = best;
    ami[(long)b * nblk + blockIdx.x] = bi;
  }
}

// Sampling: p = softmax(logits/T) in fp32, optional top-p mask, then the first index whose
// fp64 cumulative mass exceeds u * total (np.random.choice: cdf.searchsorted(u,
// side='right')).  One block (1024 threads) per sequence.
__global__ __launch_bounds__(1024) void dec_sample_kernel(float *logits, int V, const DecState *__restrict__ st,
                                                          const double *__restrict__ unif, int ctx, int32_t *tok,
                                                          int32_t *out) {
  __shared__ float redf[16];
  __shared__ double redd[16];
  __shared__ double wsum[16];
  const int b = blockIdx.x;
  const float temp = st->temp, top_p = st->top_p;
  const int step = gen_step(st);
  float *lg = logits + (long)b * V;
  const int tid = threadIdx.x, nt = blockDim.x;
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

__global__ void dec_advance_kernel(DecState *st) {
  if (threadIdx.x == 0) st->pos += 1;
}

// ----------------------------------------------------------------------- launchers ----

int pick_rpw(int N) {
  for (int rpw : {4, 2}) if (N % (4 * rpw) == 0 && N / (4 * rpw) >= 512) return rpw;
  return 1;
}

template <typename HT, int NB, int RPW, int PRO, bool AMX, bool GATE>
int gemv_valu_kc(const h16_t *W, int N, int K, const float *in, long ldi, const float *g, float eps, float *out,
                 long ldo, const float *resid, float alpha, int B, float *amv, int32_t *ami, hipStream_t s) {
  // GATE: N counts gate outputs, each from two weight rows
  const int nblk = GATE ? N / (4 * RPW / 2) : N / (4 * RPW);
  const size_t sh = (size_t)NB * K * sizeof(float);
  const long gate_n = N;
  if (K <= 1024)
    hipLaunchKernelGGL((gemv_valu_kernel<HT, NB, RPW, 2, PRO, AMX, GATE>), dim3(nblk), dim3(256), sh, s, W, K, in,
                       ldi, g, eps, out, ldo, resid, alpha, B, amv, ami, nblk, gate_n);
  else if (K <= 2048)
    hipLaunchKernelGGL((gemv_valu_kernel<HT, NB, RPW, 4, PRO, AMX, GATE>), dim3(nblk), dim3(256), sh, s, W, K, in,
                       ldi, g, eps, out, ldo, resid, alpha, B, amv, ami, nblk, gate_n);
  else
    hipLaunchKernelGGL((gemv_valu_kernel<HT, NB, RPW, 6, PRO, AMX, GATE>), dim3(nblk), dim3(256), sh, s, W, K, in,
                       ldi, g, eps, out, ldo, resid, alpha, B, amv, ami, nblk, gate_n);
  return ne_hip_status(hipGetLastError(), "decode gemv");
}

template <typename HT, int NB, int PRO, bool AMX, bool GATE = false>
int gemv_valu_nb(const h16_t *W, int N, int K, const float *in, long ldi, const float *g, float eps, float *out,
                 long ldo, const float *resid, float alpha, int B, float *amv, int32_t *ami, hipStream_t s) {
  if (GATE) {  // two weight rows (W1 j, W3 j) per gate output; 2 outputs per wave
    if (N % 8) return ne_fail(NE_ERR_ARG, "decode gate gemv: hidden %d not a multiple of 8", N);
    return gemv_valu_kc<HT, NB, 4, PRO, AMX, true>(W, N, K, in, ldi, g, eps, out, ldo, resid, alpha, B, amv, ami, s);
  }
  const int rpw = pick_rpw(N);
  if (rpw == 4) return gemv_valu_kc<HT, NB, 4, PRO, AMX, false>(W, N, K, in, ldi, g, eps, out, ldo, resid, alpha, B, amv, ami, s);
  if (rpw == 2) return gemv_valu_kc<HT, NB, 2, PRO, AMX, false>(W, N, K, in, ldi, g, eps, out, ldo, resid, alpha, B, amv, ami, s);
  return gemv_valu_kc<HT, NB, 1, PRO, AMX, false>(W, N, K, in, ldi, g, eps, out, ldo, resid, alpha, B, amv, ami, s);
}

template <typename HT, int PRO, bool AMX, bool GATE = false>
int gemv_valu_pro(int B, const h16_t *W, int N, int K, const float *in, long ldi, const float *g, float eps,
                  float *out, long ldo, const float *resid, float alpha, float *amv, int32_t *ami, hipStream_t s) {
  if (B == 1) return gemv_valu_nb<HT, 1, PRO, AMX, GATE>(W, N, K, in, ldi, g, eps, out, ldo, resid, alpha, B, amv, ami, s);
  if (B == 2) return gemv_valu_nb<HT, 2, PRO, AMX, GATE>(W, N, K, in, ldi, g, eps, out, ldo, resid, alpha, B, amv, ami, s);
  return gemv_valu_nb<HT, 4, PRO, AMX, GATE>(W, N, K, in, ldi, g, eps, out, ldo, resid, alpha, B, amv, ami, s);
}

// Batch <= 4: out = alpha * W . pro(in) + resid.  Requires N % 4 == 0, K % 8 == 0.
int gemv_small(ne_ctx *c, int B, int pro, bool amx, const h16_t *W, int N, int K, const float *in, long ldi,
               const float *g, float *out, long ldo, const float *resid, float alpha, bool gate = false) {
  Dec *d = (Dec *)c->dec;
  if (N % 4 || K % 8 || K > 3072)
    return ne_fail(NE_ERR_ARG, "decode gemv: N=%d K=%d (need N%%4, K%%8, K <= 3072)", N, K);
  if ((((uintptr_t)in | (uintptr_t)(g ? g : in)) & 15) || ldi % 4)
    return ne_fail(NE_ERR_ARG, "decode gemv: input rows and gains must be 16-byte aligned");
  const float eps = c->c.norm_eps;
  return DISPATCH_H16(c->dt, [&] {
    if (pro == PRO_RMSNORM && gate)
      return gemv_valu_pro<HT, PRO_RMSNORM, false, true>(B, W, N, K, in, ldi, g, eps, out, ldo, nullptr, 1.f, nullptr, nullptr, c->st);
    if (pro == PRO_RMSNORM) {
      if (amx) return gemv_valu_pro<HT, PRO_RMSNORM, true>(B, W, N, K, in, ldi, g, eps, out, ldo, resid, alpha, d->amv, d->ami, c->st);
      return gemv_valu_pro<HT, PRO_RMSNORM, false>(B, W, N, K, in, ldi, g, eps, out, ldo, resid, alpha, nullptr, nullptr, c->st);
    }
    if (pro == PRO_SWIGLU)
      return gemv_valu_pro<HT, PRO_SWIGLU, false>(B, W, N, K, in, ldi, g, eps, out, ldo, resid, alpha, nullptr, nullptr, c->st);
    return gemv_valu_pro<HT, PRO_NONE, false>(B, W, N, K, in, ldi, g, eps, out, ldo, resid, alpha, nullptr, nullptr, c->st);
  }());
}

// Batch 5..32: the products of W [N, K] with x rows [Bp, K] (row stride ldx).  wsp
// (nullable): a workspace of cap floats for the split-K partials.
//  * nz_out != null: the partials stay in wsp for the consumer (*nz_out slices of [Bp, N]);
//  * else, with wsp: out = alpha * (their ordered sum) + resid, one block per sequence, and
//    with gn also xn = RMSNorm(out) * gn (the next GEMV's input);
//  * without wsp: one split, out = alpha * products (+ resid) directly;
//  * gate: W = [W1; W3] (2N rows), out [Bp, N] = silu(W1.x) * (W3.x), one split.
// Requires N % 16 (gate: N % 8), K % 128.
int gemv_big(ne_ctx *c, int B, const h16_t *W, int N, int K, const float *x, long ldx, float *wsp, long cap,
             float *out, long ldo, const float *resid, float alpha, int *nz_out, const float *gn = nullptr,
             float *xn = nullptr, bool gate = false) {
  Dec *d = (Dec *)c->dec;
  if ((gate ? N % 8 : N % 16) || K % 128)
    return ne_fail(NE_ERR_ARG, "decode gemv: N=%d K=%d (need N%%16 (gate: %%8), K%%128)", N, K);
  if (gate && wsp) return ne_fail(NE_ERR_ARG, "decode gemv: the gate form has one split");
  int ks = 1;
  if (wsp)
    while ((N / 16) * ks < 512 && K % (128 * ks * 2) == 0 && (long)ks * 2 * d->Bp * N <= cap) ks *= 2;
  if (wsp && (long)ks * d->Bp * N > cap) return ne_fail(NE_ERR_ARG, "decode gemv: workspace too small");
  const dim3 grid(gate ? N / 8 : N / 16, ks);
  // the gate form has one split: 8 waves per block shorten each wave's K range instead
  // (K % 256 then; else 4 waves)
  const bool wide = gate && K % 256 == 0;
  NE_CHECK(DISPATCH_H16(c->dt, [&] {
    auto go = [&](auto kernel, int threads) {
      hipLaunchKernelGGL(kernel, grid, dim3(threads), 0, c->st, W, (long)K, x, ldx, K, ks, out, ldo, resid, alpha,
                         wsp, N, B, (long)N);
    };
    if (d->Bp == 16) {
      if (wide) go(gemv_mfma_kernel<HT, 1, true, 8>, 512);
      else if (gate) go(gemv_mfma_kernel<HT, 1, true>, 256);
      else go(gemv_mfma_kernel<HT, 1, false>, 256);
    } else {
      if (wide) go(gemv_mfma_kernel<HT, 2, true, 8>, 512);
      else if (gate) go(gemv_mfma_kernel<HT, 2, true>, 256);
      else go(gemv_mfma_kernel<HT, 2, false>, 256);
    }
    return ne_hip_status(hipGetLastError(), "decode gemv");
  }()));
  if (nz_out) {
    *nz_out = ks;
    return 0;
  }
  if (wsp) {
    auto go = [&](auto kernel) {
      hipLaunchKernelGGL(kernel, dim3(B), dim3(256), 0, c->st, wsp, ks, d->Bp, N, out, ldo, resid, alpha, gn, xn,
                         c->c.norm_eps);
    };
    if (N > 1024) go(gemv_reduce_rows_kernel<0>);
    else if (ks == 1) go(gemv_reduce_rows_kernel<1>);
    else if (ks == 2) go(gemv_reduce_rows_kernel<2>);
    else if (ks == 4) go(gemv_reduce_rows_kernel<4>);
    else if (ks == 8) go(gemv_reduce_rows_kernel<8>);
    else go(gemv_reduce_rows_kernel<0>);
    NE_HIP(hipGetLastError());
  }
  return 0;
}

// Batch 5..32 with bf16 weights: the GEMV on gemv_bf3_kernel when its shape allows (returns
// 1 after launching; 0: not applicable, nothing launched).  mode BF3_WS: the split-K partials
// go to d->ws and *nz receives the split count; BF3_GATE: W = [W1; W3] (N rows each), gate
// [Bp, N] -> out; BF3_PLAIN: out [Bp, ldo] = products.
int gemv_bf3(ne_ctx *c, int B, const h16_t *W, int N, int K, const float *x, long ldx, int mode, float *out,
             long ldo, int *nz) {
  Dec *d = (Dec *)c->dec;
  if (c->dt != NE_BF16 || K % 128) return 0;
  int ks = 0, rt = 2, ksplit = 1;
  if (mode == BF3_WS) {
    for (int cand : {2, 3, 1})
      if (K % (128 * cand) == 0 && K / (128 * cand) <= 8) {
        ks = cand;
        break;
      }
    if (!ks) return 0;
    ksplit = K / (128 * ks);
    rt = (N % 64 == 0 && (N / 64) * ksplit >= 192) ? 4 : 2;
    if (N % (16 * rt) || (long)ksplit * d->Bp * N > d->ws_elems) return 0;
  } else {
    ks = K / 128;
    if (ks != 1 && ks != 6 && ks != 8) return 0;
    if (N % (mode == BF3_GATE ? 16 : 32)) return 0;
    // the LM head: 128 rows per block (x read once per 128 rows: 1.61 -> 1.57 ms per batch-32
    // position against 32)
    if (mode == BF3_PLAIN && N % 128 == 0) rt = 8;
  }
  const int ntw = d->Bp / 16;
  const dim3 grid(mode == BF3_GATE ? N / 16 : N / (16 * rt), ksplit);
  float *dst = mode == BF3_WS ? d->ws : out;
  const long ldd = mode == BF3_WS ? N : ldo;
  bool done = false;
  auto go = [&](auto kernel, int nt) {
    hipLaunchKernelGGL(kernel, grid, dim3(nt * 256), 0, c->st, W, (long)K, x, ldx, dst, ldd, N, B, d->Bp, (long)N);
    done = true;
  };
#define NE_BF3(NTW_)                                                                                 \
  if (mode == BF3_WS) {                                                                              \
    if (rt == 4 && ks == 2) go(gemv_bf3_kernel<NTW_, 4, 2, BF3_WS>, NTW_);                           \
    else if (rt == 4 && ks == 3) go(gemv_bf3_kernel<NTW_, 4, 3, BF3_WS>, NTW_);                      \
    else if (rt == 4 && ks == 1) go(gemv_bf3_kernel<NTW_, 4, 1, BF3_WS>, NTW_);                      \
    else if (rt == 2 && ks == 2) go(gemv_bf3_kernel<NTW_, 2, 2, BF3_WS>, NTW_);                      \
    else if (rt == 2 && ks == 3) go(gemv_bf3_kernel<NTW_, 2, 3, BF3_WS>, NTW_);                      \
    else if (rt == 2 && ks == 1) go(gemv_bf3_kernel<NTW_, 2, 1, BF3_WS>, NTW_);                      \
  } else if (mode == BF3_GATE) {                                                                     \
    if (ks == 8) go(gemv_bf3_kernel<NTW_, 2, 8, BF3_GATE>, NTW_);                                    \
    else if (ks == 6) go(gemv_bf3_kernel<NTW_, 2, 6, BF3_GATE>, NTW_);                               \
    else go(gemv_bf3_kernel<NTW_, 2, 1, BF3_GATE>, NTW_);                                            \
  } else if (rt == 8) {                                                                              \
    if (ks == 8) go(gemv_bf3_kernel<NTW_, 8, 8, BF3_PLAIN>, NTW_);                                   \
    else if (ks == 6) go(gemv_bf3_kernel<NTW_, 8, 6, BF3_PLAIN>, NTW_);                              \
    else go(gemv_bf3_kernel<NTW_, 8, 1, BF3_PLAIN>, NTW_);                                           \
  } else {                                                                                           \
    if (ks == 8) go(gemv_bf3_kernel<NTW_, 2, 8, BF3_PLAIN>, NTW_);                                   \
    else if (ks == 6) go(gemv_bf3_kernel<NTW_, 2, 6, BF3_PLAIN>, NTW_);                              \
    else go(gemv_bf3_kernel<NTW_, 2, 1, BF3_PLAIN>, NTW_);                                           \
  }
  if (ntw == 1) {
    NE_BF3(1)
  } else {
    NE_BF3(2)
  }
#undef NE_BF3
  if (!done) return 0;
  NE_CHECK(ne_hip_status(hipGetLastError(), "decode gemv (bf16 parts)"));
  if (nz) *nz = ksplit;
  return 1;
}

// Wo / W2 on gemv_bf3_kernel with the split-K sum, residual and RMSNorm of gemv_big's
// workspace form (gemv_reduce_rows_kernel); returns 0 when not applicable.
int gemv_bf3_resid(ne_ctx *c, int B, const h16_t *W, int N, int K, const float *x, long ldx, float *out, long ldo,
                   const float *resid, float alpha, const float *gn, float *xn) {
  Dec *d = (Dec *)c->dec;
  int ks = 0;
  const int rc = gemv_bf3(c, B, W, N, K, x, ldx, BF3_WS, nullptr, 0, &ks);
  if (rc <= 0) return rc;
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(B), dim3(256), 0, c->st, d->ws, ks, d->Bp, N, out, ldo, resid, alpha, gn, xn,
                       c->c.norm_eps);
  };
  if (N > 1024) go(gemv_reduce_rows_kernel<0>);
  else if (ks == 1) go(gemv_reduce_rows_kernel<1>);
  else if (ks == 2) go(gemv_reduce_rows_kernel<2>);
  else if (ks == 4) go(gemv_reduce_rows_kernel<4>);
  else if (ks == 8) go(gemv_reduce_rows_kernel<8>);
  else go(gemv_reduce_rows_kernel<0>);
  NE_CHECK(ne_hip_status(hipGetLastError(), "decode gemv reduce"));
  return 1;
}

// qkv: the q|k|v rows [Bp, QKV], or (qnz > 1) qnz split-K partial slices of them.
int launch_attn(ne_ctx *c, int B, const LayerOff &o, float *kc, float *vc, const float *qkv, int qnz, bool kcol) {
  Dec *d = (Dec *)c->dec;
  const int ratio = c->NH / c->NKV;
  // query heads per block: at batch <= 4 one (the blocks of a KV head share its K/V reads
  // through L2, and twice the blocks run), else all of the KV head's
  const int qpb = kcol ? 1 : ratio;
  const size_t sh = (size_t)qpb * d->ctx * sizeof(float);
  const double scale = 1.0 / sqrt((double)c->HD);
  const float *gq = c->c.qk_norm ? c->P + o.gq : nullptr, *gk = c->c.qk_norm ? c->P + o.gk : nullptr;
  const dim3 grid(B, c->NH / qpb);
#define NE_DEC_ATTN(HDV, R)                                                                                     \
  if (kcol)                                                                                                     \
    hipLaunchKernelGGL((dec_attn_kernel<HDV, R, true>), grid, dim3(256), sh, c->st, qkv, c->QKV, gq, gk,        \
                       d->cosb, d->sinb, kc, vc, d->att, c->NH, c->NKV, d->ctx, d->st, c->c.norm_eps, scale,   \
                       qkv, qnz, d->Bp);                                                                        \
  else                                                                                                          \
    hipLaunchKernelGGL((dec_attn_kernel<HDV, R, false>), grid, dim3(256), sh, c->st, qkv, c->QKV, gq, gk,       \
                       d->cosb, d->sinb, kc, vc, d->att, c->NH, c->NKV, d->ctx, d->st, c->c.norm_eps, scale,   \
                       qkv, qnz, d->Bp)
  if (c->HD == 128) {
    if (qpb == 1) NE_DEC_ATTN(128, 1);
    else if (qpb == 2) NE_DEC_ATTN(128, 2);
    else NE_DEC_ATTN(128, 4);
  } else {
    if (qpb == 1) NE_DEC_ATTN(64, 1);
    else if (qpb == 2) NE_DEC_ATTN(64, 2);
    else NE_DEC_ATTN(64, 4);
  }
#undef NE_DEC_ATTN
  return ne_hip_status(hipGetLastError(), "decode attention");
}

// Enqueue the kernels of one position for B sequences.  gen: also the final norm, LM head
// and token choice.  Position-independent (everything position-dependent is read from
// d->st), so it can be captured once and replayed.
int enqueue_position(ne_ctx *c, int B, bool gen, bool greedy) {
  Dec *d = (Dec *)c->dec;
  const int D = c->D, H = c->H, Q = c->Q, NKV = c->NKV, HD = c->HD, QKV = c->QKV, V = c->V;
  const float eps = c->c.norm_eps, alpha = c->c.res_alpha;
  const h16_t *Pb = c->Pb;
  const float *Pf = c->P;
  const bool small = B <= VB;
  // batch 5..32: the kernels that write x (the token lookup, the Wo / W2 split-K reductions)
  // also write its RMSNorm with the next gain into xn; the QKV GEMV's partials are summed by
  // the attention kernel
  const long cap = d->ws_elems;
  const float *g0 = small ? nullptr : Pf + c->lo[0].g_att;
  if (c->dt == NE_FP16)
    hipLaunchKernelGGL(dec_token_kernel<H16F>, dim3(B), dim3(256), 0, c->st, d->prompt, d->ctx, d->st, d->tok,
                       Pb + c->off_E, d->x, D, B, g0, d->xn, eps);
  else
    hipLaunchKernelGGL(dec_token_kernel<H16B>, dim3(B), dim3(256), 0, c->st, d->prompt, d->ctx, d->st, d->tok,
                       Pb + c->off_E, d->x, D, B, g0, d->xn, eps);
  NE_HIP(hipGetLastError());
  for (int l = 0; l < c->L; l++) {
    const LayerOff &o = c->lo[l];
    const size_t kvl = (size_t)l * d->Bmax * NKV * d->ctx * HD;
    if (small) {
      NE_CHECK(gemv_small(c, B, PRO_RMSNORM, false, Pb + o.wqkv, QKV, D, d->x, D, Pf + o.g_att, d->qkv, QKV, nullptr, 1.f));
      NE_CHECK(launch_attn(c, B, o, d->kc + kvl, d->vc + kvl, d->qkv, 1, true));
    } else {
      int qnz = 0;
      int rc = gemv_bf3(c, B, Pb + o.wqkv, QKV, D, d->xn, D, BF3_WS, nullptr, 0, &qnz);
      if (rc < 0) return rc;
      if (!rc) NE_CHECK(gemv_big(c, B, Pb + o.wqkv, QKV, D, d->xn, D, d->ws, cap, nullptr, 0, nullptr, 1.f, &qnz));
      NE_CHECK(launch_attn(c, B, o, d->kc + kvl, d->vc + kvl, d->ws, qnz, false));
    }
    if (small) {
      NE_CHECK(gemv_small(c, B, PRO_NONE, false, Pb + o.wo, D, Q, d->att, Q, nullptr, d->x, D, d->x, alpha));
      // W1|W3 with the SwiGLU gate in its epilogue (gate -> xn), then W2 + residual
      NE_CHECK(gemv_small(c, B, PRO_RMSNORM, false, Pb + o.w13, H, D, d->x, D, Pf + o.g_ffn, d->xn, H, nullptr, 1.f,
                          true));
      NE_CHECK(gemv_small(c, B, PRO_NONE, false, Pb + o.w2, D, H, d->xn, H, nullptr, d->x, D, d->x, alpha));
    } else {
      const float *g_next = l + 1 < c->L ? Pf + c->lo[l + 1].g_att : Pf + c->off_gfinal;
      int rc = gemv_bf3_resid(c, B, Pb + o.wo, D, Q, d->att, Q, d->x, D, d->x, alpha, Pf + o.g_ffn, d->xn);
      if (rc < 0) return rc;
      if (!rc)
        NE_CHECK(gemv_big(c, B, Pb + o.wo, D, Q, d->att, Q, d->ws, cap, d->x, D, d->x, alpha, nullptr, Pf + o.g_ffn,
                          d->xn));
      rc = gemv_bf3(c, B, Pb + o.w13, H, D, d->xn, D, BF3_GATE, d->gate, H, nullptr);
      if (rc < 0) return rc;
      if (!rc)
        NE_CHECK(gemv_big(c, B, Pb + o.w13, H, D, d->xn, D, nullptr, 0, d->gate, H, nullptr, 1.f, nullptr, nullptr,
                          nullptr, true));
      rc = gemv_bf3_resid(c, B, Pb + o.w2, D, H, d->gate, H, d->x, D, d->x, alpha, g_next, d->xn);
      if (rc < 0) return rc;
      if (!rc)
        NE_CHECK(gemv_big(c, B, Pb + o.w2, D, H, d->gate, H, d->ws, cap, d->x, D, d->x, alpha, nullptr, g_next, d->xn));
    }
  }
  if (gen) {
    if (small) {
      NE_CHECK(gemv_small(c, B, PRO_RMSNORM, greedy, Pb + c->off_E, V, D, d->x, D, Pf + c->off_gfinal, d->logits, V,
                          nullptr, 1.f));
      if (greedy)
        hipLaunchKernelGGL(dec_argmax_kernel, dim3(B), dim3(1024), 0, c->st, d->amv, d->ami, V / (4 * pick_rpw(V)),
                           d->st, d->ctx, d->tok, d->out);
    } else {
      const int rc = gemv_bf3(c, B, Pb + c->off_E, V, D, d->xn, D, BF3_PLAIN, d->logits, V, nullptr);
      if (rc < 0) return rc;
      if (!rc) NE_CHECK(gemv_big(c, B, Pb + c->off_E, V, D, d->xn, D, nullptr, 0, d->logits, V, nullptr, 1.f, nullptr));
      if (greedy) {
        hipLaunchKernelGGL(dec_argmax_part_kernel, dim3(BIG_ARGMAX, B), dim3(256), 0, c->st, d->logits, V, BIG_ARGMAX,
                           d->amv, d->ami);
        hipLaunchKernelGGL(dec_argmax_kernel, dim3(B), dim3(1024), 0, c->st, d->amv, d->ami, BIG_ARGMAX, d->st, d->ctx,
                           d->tok, d->out);
      }
    }
    if (!greedy)
      hipLaunchKernelGGL(dec_sample_kernel, dim3(B), dim3(1024), 0, c->st, d->logits, V, d->st, d->unif, d->ctx,
                         d->tok, d->out);
  }
  hipLaunchKernelGGL(dec_advance_kernel, dim3(1), dim3(64), 0, c->st, d->st);
  return ne_hip_status(hipGetLastError(), "decode position");
}

int capture(ne_ctx *c, int B, bool gen, bool greedy, hipGraphExec_t *exec) {
  hipGraph_t graph = nullptr;
  NE_HIP(hipStreamBeginCapture(c->st, hipStreamCaptureModeThreadLocal));
  const int rc = enqueue_position(c, B, gen, greedy);
  const hipError_t ec = hipStreamEndCapture(c->st, &graph);
  if (rc) {
    if (graph) (void)hipGraphDestroy(graph);
    return rc;
  }
  NE_HIP(ec);
  const hipError_t ei = hipGraphInstantiate(exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  NE_HIP(ei);
  return 0;
}

}  // namespace

int decode_alloc(ne_ctx *c) {
  Dec *d = new Dec();
  c->dec = d;
  if (c->c.decode_batch > 32) return ne_fail(NE_ERR_ARG, "decode_batch %d > 32", c->c.decode_batch);
  if (c->NH / c->NKV != 1 && c->NH / c->NKV != 2 && c->NH / c->NKV != 4)
    return ne_fail(NE_ERR_ARG, "decode: %d query heads per KV head (1, 2 or 4)", c->NH / c->NKV);
  if (c->D % 128 || c->H % 128 || c->Q % 128)
    return ne_fail(NE_ERR_ARG, "decode: dim, hidden and q_dim must be multiples of 128");
  d->Bmax = c->c.decode_batch;
  d->Bp = d->Bmax <= 16 ? 16 : 32;
  d->ctx = c->c.decode_ctx;
  const size_t Bp = d->Bp, Bm = d->Bmax, ctx = d->ctx, L = c->L, D = c->D, H = c->H, Q = c->Q, NKV = c->NKV,
               HD = c->HD, V = c->V;
  const size_t kv = L * Bm * NKV * ctx * HD;
  d->lm_nblk = std::max<int>(c->V / (4 * pick_rpw(c->V)), BIG_ARGMAX);
  d->ws_elems = (long)8 * Bp * std::max<size_t>(2 * H, Q + 2 * NKV * HD);
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += (bytes + 255) & ~(size_t)255; return o; };
  const size_t o_kc = take(kv * 4), o_vc = take(kv * 4), o_x = take(Bp * D * 4);
  const size_t o_xn = take(Bp * std::max(D, H) * 4);
  const size_t o_qkv = take(Bp * (Q + 2 * NKV * HD) * 4), o_att = take(Bp * Q * 4);
  const size_t o_lg = take(Bp * V * 4);
  const size_t o_ws = take((size_t)d->ws_elems * 4), o_gate = take(Bp * H * 4);
  const size_t o_amv = take(Bp * (size_t)d->lm_nblk * 4), o_ami = take(Bp * (size_t)d->lm_nblk * 4);
  const size_t o_tok = take(Bp * 4), o_out = take(Bp * ctx * 4), o_pr = take(Bp * ctx * 4), o_u = take(Bp * ctx * 8);
  const size_t o_cos = take(ctx * HD / 2 * 4), o_sin = take(ctx * HD / 2 * 4), o_st = take(sizeof(DecState));
  NE_HIP(hipMalloc(&d->arena, off));
  char *base = (char *)d->arena;
  d->kc = (float *)(base + o_kc); d->vc = (float *)(base + o_vc);
  d->x = (float *)(base + o_x); d->xn = (float *)(base + o_xn);
  d->qkv = (float *)(base + o_qkv); d->att = (float *)(base + o_att);
  d->logits = (float *)(base + o_lg);
  d->ws = (float *)(base + o_ws);
  d->gate = (float *)(base + o_gate);
  d->amv = (float *)(base + o_amv); d->ami = (int32_t *)(base + o_ami);
  d->tok = (int32_t *)(base + o_tok); d->out = (int32_t *)(base + o_out); d->prompt = (int32_t *)(base + o_pr);
  d->unif = (double *)(base + o_u);
  d->cosb = (float *)(base + o_cos); d->sinb = (float *)(base + o_sin);
  d->st = (DecState *)(base + o_st);
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
  for (auto &g : d->graphs) {
    if (g.pre) hipGraphExecDestroy(g.pre);
    if (g.gen) hipGraphExecDestroy(g.gen);
  }
  if (d->arena) hipFree(d->arena);
  delete d;
  c->dec = nullptr;
}

namespace {
int replay(ne_ctx *c, int B, int P, int n_new, bool greedy);
}

int decode_run(ne_ctx *c, const int32_t *prompt, int B, int P, int n_new, float temp, float top_p,
               const double *uniforms, int32_t *out) {
  Dec *d = (Dec *)c->dec;
  if (!d) return ne_fail(NE_ERR_STATE, "context created without decode buffers (decode_batch/decode_ctx)");
  if (B <= 0 || B > c->c.decode_batch || P <= 0 || n_new <= 0 || P + n_new > d->ctx)
    return ne_fail(NE_ERR_ARG, "decode: B=%d P=%d n_new=%d exceed decode_batch=%d / decode_ctx=%d", B, P, n_new,
                   c->c.decode_batch, d->ctx);
  const bool greedy = temp < 1e-6f;
  if (!greedy && !uniforms) return ne_fail(NE_ERR_ARG, "decode: sampling needs uniforms");
  for (long i = 0; i < (long)B * P; i++)
    if (prompt[i] < 0 || prompt[i] >= c->V) return ne_fail(NE_ERR_ARG, "decode: prompt id out of range");
  // Every call runs its prompt from position 0 and rebuilds the KV cache, so the cache layout
  // may follow this call's batch size (K column-major at B <= 4, row-major above,
  // dec_attn_kernel); a cache kept across calls would have to keep one layout for both.
  // per-call inputs: prompt rows, uniforms, state (outside the captured graphs)
  std::vector<int32_t> pr((size_t)d->Bp * d->ctx, 0);
  for (int b = 0; b < B; b++)
    for (int j = 0; j < P; j++) pr[(size_t)b * d->ctx + j] = prompt[(size_t)b * P + j];
  NE_HIP(hipMemcpyAsync(d->prompt, pr.data(), pr.size() * 4, hipMemcpyHostToDevice, c->st));
  std::vector<double> u;
  if (!greedy) {
    u.assign((size_t)d->Bp * d->ctx, 0.0);
    for (int b = 0; b < B; b++)
      for (int j = 0; j < n_new; j++) u[(size_t)b * d->ctx + j] = uniforms[(size_t)b * n_new + j];
    NE_HIP(hipMemcpyAsync(d->unif, u.data(), u.size() * 8, hipMemcpyHostToDevice, c->st));
  }
  const DecState s0 = {0, P, temp, top_p};
  NE_HIP(hipMemcpyAsync(d->st, &s0, sizeof s0, hipMemcpyHostToDevice, c->st));
  NE_HIP(hipStreamSynchronize(c->st));  // host staging vectors are released at return

  if (!c->use_graphs) {  // eager launches (tracers that do not follow graph launches)
    for (int pos = 0; pos < P + n_new - 1; pos++) NE_CHECK(enqueue_position(c, B, pos >= P - 1, greedy));
  } else {
    NE_CHECK(replay(c, B, P, n_new, greedy));
  }
  std::vector<int32_t> o((size_t)d->Bp * d->ctx);
  NE_HIP(hipMemcpyAsync(o.data(), d->out, o.size() * 4, hipMemcpyDeviceToHost, c->st));
  NE_HIP(hipStreamSynchronize(c->st));
  for (int b = 0; b < B; b++)
    for (int j = 0; j < n_new; j++) out[(size_t)b * n_new + j] = o[(size_t)b * d->ctx + j];
  return 0;
}

namespace {

// Replay the captured position graphs (captured on first use per batch size and mode).
int replay(ne_ctx *c, int B, int P, int n_new, bool greedy) {
  Dec *d = (Dec *)c->dec;
  Dec::Graph *gr = nullptr;
  for (auto &g : d->graphs)
    if (g.B == B && g.greedy == greedy) gr = &g;
  if (!gr) {
    Dec::Graph g = {B, greedy, nullptr, nullptr};
    int rc = capture(c, B, false, greedy, &g.pre);
    if (!rc) rc = capture(c, B, true, greedy, &g.gen);
    if (rc) {
      if (g.pre) hipGraphExecDestroy(g.pre);
      return rc;
    }
    d->graphs.push_back(g);
    gr = &d->graphs.back();
  }
  for (int pos = 0; pos < P - 1; pos++) NE_HIP(hipGraphLaunch(gr->pre, c->st));
  for (int j = 0; j < n_new; j++) NE_HIP(hipGraphLaunch(gr->gen, c->st));
  return 0;
}

}  // namespace
