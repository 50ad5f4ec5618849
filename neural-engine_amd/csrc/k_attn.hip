// Causal flash attention forward / backward on 16-bit MFMA (v_mfma_f32_16x16x32_{f16,bf16}).
//
// Replaces the score/softmax/PV part of gen_sdpa_fwd_dynamic (TD/mil_dynamic.h:171-223,
// full S x S scores plus a -65504 mask blob, TD/mil_dynamic.h:716-725) and the two
// backward programs gen_sdpa_bwd1_noweight / gen_sdpa_bwd2 (TD/mil_dynamic.h:583-707)
// together with the GQA tile/reduce of TD/io.h:423-430 and TD/cpu_ops.h:585-605.
// Nothing O(S^2) is stored: the forward keeps the row log-sum-exp, the backward
// recomputes P per tile.  GQA: kv head = q head / (NH/NKV); the dK/dV kernel loops over
// the query heads of its kv head, so the reduction happens in registers.
//
// Score tiles are computed transposed where that lets the fp32 accumulator registers be
// reused directly as the next MFMA's operand: a 16x16 accumulator gives lane l the rows
// 4*(l/16)+i of column l%16, i.e. 4 values along the row index, which is what an
// operand needs along K.  Two 16-row blocks give the 8 K-values of a 32-deep MFMA; the
// other operand is read from LDS with the same K permutation.
#include "common.h"
#include "ne_internal.h"

namespace {

constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr int BLK = 64;  // queries per q tile and keys per kv tile

template <typename HT>
__device__ __forceinline__ typename HT::v8 ld8(const h16_t *p) { return HT::op(*(const u16x8 *)p); }

// 8 K-values from a transposed LDS tile: columns c0..c0+3 and c1..c1+3 of one row.
template <typename HT>
__device__ __forceinline__ typename HT::v8 ld_pair4(const h16_t *row, int c0, int c1) {
  const u16x4 x = *(const u16x4 *)(row + c0);
  const u16x4 y = *(const u16x4 *)(row + c1);
  u16x8 r;
  r[0] = x[0]; r[1] = x[1]; r[2] = x[2]; r[3] = x[3];
  r[4] = y[0]; r[5] = y[1]; r[6] = y[2]; r[7] = y[3];
  return HT::op(r);
}

template <typename HT>
__device__ __forceinline__ typename HT::v8 pack_acc(const f32x4 &x, const f32x4 &y) {
  u16x8 r;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    r[i] = HT::h(x[i]);
    r[4 + i] = HT::h(y[i]);
  }
  return HT::op(r);
}

// Stage a 64-row x HD tile of rows t0.. (column offset col) into LDS row-major
// (pitch RP) and/or transposed (pitch TP).
template <int HD, int RP, int TP, bool ROW, bool TRN, int NT>
__device__ __forceinline__ void stage_tile(const h16_t *__restrict__ src, long ld, long t0, int col,
                                           h16_t *rows, h16_t *trn) {
  for (int c = threadIdx.x; c < BLK * HD / 8; c += NT) {
    const int r = c / (HD / 8), d8 = c % (HD / 8);
    const u16x8 v = *(const u16x8 *)(src + (t0 + r) * ld + col + d8 * 8);
    if (ROW) *(u16x8 *)(rows + r * RP + d8 * 8) = v;
    if (TRN) {
#pragma unroll
      for (int j = 0; j < 8; j++) trn[(d8 * 8 + j) * TP + r] = v[j];
    }
  }
}

// NW waves per block, 16 queries per wave; key tiles of 64.
template <typename HT, int HD, int NW>
__global__ __launch_bounds__(NW * 64) void attn_fwd_kernel(AttnArgs a) {
  constexpr int RP = HD + 8, TP = BLK + 4, NK = HD / 32, ND = HD / 16;
  __shared__ __attribute__((aligned(16))) h16_t Ks[BLK * RP];
  __shared__ __attribute__((aligned(16))) h16_t Vt[HD * TP];
  const int q0 = (gridDim.x - 1 - blockIdx.x) * NW * 16;  // longest rows first
  const int kb_last = (q0 + NW * 16 - 1) / BLK;
  const int h = blockIdx.y, b = blockIdx.z;
  const int kvh = h / (a.NH / a.NKV);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const long tb = (long)b * a.S;
  const int qi = q0 + w * 16 + c16;  // this lane's query (position in sequence)
  const long tq = tb + qi;
  typename HT::v8 qf[NK];
#pragma unroll
  for (int kk = 0; kk < NK; kk++) qf[kk] = ld8<HT>(a.q + tq * a.ldq + h * HD + kk * 32 + g * 8);
  f32x4 acc[ND];
#pragma unroll
  for (int d = 0; d < ND; d++) acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_i = -INFINITY, l_i = 0.f;
  const float sl2 = a.scale * LOG2E;

  for (int kb = 0; kb <= kb_last; kb++) {
    __syncthreads();
    stage_tile<HD, RP, TP, true, false, NW * 64>(a.k, a.ldk, tb + kb * BLK, kvh * HD, Ks, nullptr);
    stage_tile<HD, RP, TP, false, true, NW * 64>(a.v, a.ldv, tb + kb * BLK, kvh * HD, nullptr, Vt);
    __syncthreads();
    f32x4 s[4];
#pragma unroll
    for (int nb = 0; nb < 4; nb++) {
      s[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < NK; kk++)
        s[nb] = HT::mfma16(ld8<HT>(Ks + (nb * 16 + c16) * RP + kk * 32 + g * 8), qf[kk], s[nb]);
    }
    // s[nb][i] = score(key kb*64 + nb*16 + 4g + i, query qi)
    float mx = -INFINITY;
#pragma unroll
    for (int nb = 0; nb < 4; nb++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        float v = s[nb][i] * sl2;
        if (kb == kb_last && kb * BLK + nb * 16 + g * 4 + i > qi) v = -INFINITY;
        s[nb][i] = v;
        mx = fmaxf(mx, v);
      }
    mx = quad16_max(mx);
    const float m_new = fmaxf(m_i, mx);
    const float alpha = exp2f(m_i - m_new);
    m_i = m_new;
    float ls = 0.f;
#pragma unroll
    for (int nb = 0; nb < 4; nb++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float p = exp2f(s[nb][i] - m_new);
        s[nb][i] = p;
        ls += p;
      }
    l_i = l_i * alpha + ls;
#pragma unroll
    for (int d = 0; d < ND; d++) acc[d] *= alpha;
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const typename HT::v8 pb = pack_acc<HT>(s[2 * c], s[2 * c + 1]);
#pragma unroll
      for (int d = 0; d < ND; d++)
        acc[d] = HT::mfma16(ld_pair4<HT>(Vt + (d * 16 + c16) * TP, 2 * c * 16 + g * 4, (2 * c + 1) * 16 + g * 4), pb, acc[d]);
    }
  }
  const float l_tot = quad16_sum(l_i);
  const float inv = 1.f / l_tot;
#pragma unroll
  for (int d = 0; d < ND; d++) {
    u16x4 o;
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = HT::h(acc[d][i] * inv);
    *(u16x4 *)(a.o + tq * a.ldo + h * HD + d * 16 + g * 4) = o;
  }
  if (g == 0) a.lse[tq * a.NH + h] = (m_i + log2f(l_tot)) * LN2;
}

// delta[t, h] = sum_d dO[t,h,d] * O[t,h,d]
template <typename HT, int HD>
__global__ void attn_delta_kernel(AttnArgs a, long rows) {
  constexpr int L = HD / 8;  // lanes per row
  const long gid = blockIdx.x * 256L + threadIdx.x;
  const long row = gid / L;
  const int j = gid % L;
  float s = 0.f;
  if (row < rows) {
    const long t = row / a.NH;
    const int h = row % a.NH;
    const u16x8 o = *(const u16x8 *)(a.o + t * a.ldo + h * HD + j * 8);
    const u16x8 d = *(const u16x8 *)(a.dout + t * a.lddo + h * HD + j * 8);
#pragma unroll
    for (int e = 0; e < 8; e++) s += HT::f(o[e]) * HT::f(d[e]);
  }
#pragma unroll
  for (int off = 1; off < L; off <<= 1) s += __shfl_xor(s, off, 64);
  if (row < rows && j == 0) a.delta[row] = s;
}

// NW waves per block, 16 keys per wave; query tiles of 64 from the diagonal on.
template <typename HT, int HD, int NW>
__global__ __launch_bounds__(NW * 64) void attn_bwd_dkdv_kernel(AttnArgs a) {
  constexpr int RP = HD + 8, TP = BLK + 4, NK = HD / 32, ND = HD / 16;
  __shared__ __attribute__((aligned(16))) h16_t Qs[BLK * RP];
  __shared__ __attribute__((aligned(16))) h16_t dOs[BLK * RP];
  __shared__ __attribute__((aligned(16))) h16_t Qt[HD * TP];
  __shared__ __attribute__((aligned(16))) h16_t dOt[HD * TP];
  __shared__ float lse_s[BLK], dl_s[BLK];
  const int nqb = a.S / BLK;
  const int k0 = blockIdx.x * NW * 16;  // smallest keys have the most query tiles: launched first
  const int qb_first = k0 / BLK;
  const int kvh = blockIdx.y, b = blockIdx.z;
  const int ratio = a.NH / a.NKV;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const long tb = (long)b * a.S;
  const int ki = k0 + w * 16 + c16;  // this lane's key (as MFMA column)
  const long tk = tb + ki;
  typename HT::v8 kf[NK], vf[NK];
#pragma unroll
  for (int kk = 0; kk < NK; kk++) {
    kf[kk] = ld8<HT>(a.k + tk * a.ldk + kvh * HD + kk * 32 + g * 8);
    vf[kk] = ld8<HT>(a.v + tk * a.ldv + kvh * HD + kk * 32 + g * 8);
  }
  f32x4 dk[ND], dv[ND];
#pragma unroll
  for (int d = 0; d < ND; d++) dk[d] = dv[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float sl2 = a.scale * LOG2E;

  for (int hq = 0; hq < ratio; hq++) {
    const int h = kvh * ratio + hq;
    for (int qb = qb_first; qb < nqb; qb++) {
      __syncthreads();
      stage_tile<HD, RP, TP, true, true, NW * 64>(a.q, a.ldq, tb + qb * BLK, h * HD, Qs, Qt);
      stage_tile<HD, RP, TP, true, true, NW * 64>(a.dout, a.lddo, tb + qb * BLK, h * HD, dOs, dOt);
      if (threadIdx.x < BLK) {
        const long t = tb + qb * BLK + threadIdx.x;
        lse_s[threadIdx.x] = a.lse[t * a.NH + h] * LOG2E;
        dl_s[threadIdx.x] = a.delta[t * a.NH + h];
      }
      __syncthreads();
      f32x4 sp[4], dp[4];
#pragma unroll
      for (int mb = 0; mb < 4; mb++) {
        sp[mb] = dp[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NK; kk++) {
          sp[mb] = HT::mfma16(ld8<HT>(Qs + (mb * 16 + c16) * RP + kk * 32 + g * 8), kf[kk], sp[mb]);
          dp[mb] = HT::mfma16(ld8<HT>(dOs + (mb * 16 + c16) * RP + kk * 32 + g * 8), vf[kk], dp[mb]);
        }
      }
      // sp[mb][i] = score(query qb*64 + mb*16 + 4g + i, key ki)
#pragma unroll
      for (int mb = 0; mb < 4; mb++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int ql = mb * 16 + g * 4 + i;
          float p = exp2f(sp[mb][i] * sl2 - lse_s[ql]);
          if (qb == qb_first && ki > qb * BLK + ql) p = 0.f;
          sp[mb][i] = p;
          dp[mb][i] = p * (dp[mb][i] - dl_s[ql]);
        }
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const typename HT::v8 pb = pack_acc<HT>(sp[2 * c], sp[2 * c + 1]);
        const typename HT::v8 sb = pack_acc<HT>(dp[2 * c], dp[2 * c + 1]);
        const int c0 = 2 * c * 16 + g * 4, c1 = (2 * c + 1) * 16 + g * 4;
#pragma unroll
        for (int d = 0; d < ND; d++) {
          dv[d] = HT::mfma16(ld_pair4<HT>(dOt + (d * 16 + c16) * TP, c0, c1), pb, dv[d]);
          dk[d] = HT::mfma16(ld_pair4<HT>(Qt + (d * 16 + c16) * TP, c0, c1), sb, dk[d]);
        }
      }
    }
  }
  // dv[d][i] = dV[key ki][dim d*16 + 4g + i]
  bool bad = false;
#pragma unroll
  for (int d = 0; d < ND; d++) {
    *(float4 *)(a.dk + tk * a.lddk + kvh * HD + d * 16 + g * 4) =
        make_float4(dk[d][0] * a.scale, dk[d][1] * a.scale, dk[d][2] * a.scale, dk[d][3] * a.scale);
    u16x4 o;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      o[i] = HT::h(dv[d][i]);
      bad |= HT::bad(o[i]);
    }
    *(u16x4 *)(a.dv + tk * a.lddv + kvh * HD + d * 16 + g * 4) = o;
  }
  flag_overflow(a.ovf, bad);
}

// NW waves per block, 16 queries per wave; key tiles of 64 up to the diagonal.
template <typename HT, int HD, int NW>
__global__ __launch_bounds__(NW * 64) void attn_bwd_dq_kernel(AttnArgs a) {
  constexpr int RP = HD + 8, TP = BLK + 4, NK = HD / 32, ND = HD / 16;
  __shared__ __attribute__((aligned(16))) h16_t Ks[BLK * RP];
  __shared__ __attribute__((aligned(16))) h16_t Vs[BLK * RP];
  __shared__ __attribute__((aligned(16))) h16_t Kt[HD * TP];
  const int q0 = (gridDim.x - 1 - blockIdx.x) * NW * 16;  // longest rows first
  const int kb_last = (q0 + NW * 16 - 1) / BLK;
  const int h = blockIdx.y, b = blockIdx.z;
  const int kvh = h / (a.NH / a.NKV);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const long tb = (long)b * a.S;
  const int qi = q0 + w * 16 + c16;
  const long tq = tb + qi;
  typename HT::v8 qf[NK], df[NK];
#pragma unroll
  for (int kk = 0; kk < NK; kk++) {
    qf[kk] = ld8<HT>(a.q + tq * a.ldq + h * HD + kk * 32 + g * 8);
    df[kk] = ld8<HT>(a.dout + tq * a.lddo + h * HD + kk * 32 + g * 8);
  }
  const float lse2 = a.lse[tq * a.NH + h] * LOG2E;
  const float dl = a.delta[tq * a.NH + h];
  f32x4 dq[ND];
#pragma unroll
  for (int d = 0; d < ND; d++) dq[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float sl2 = a.scale * LOG2E;

  for (int kb = 0; kb <= kb_last; kb++) {
    __syncthreads();
    stage_tile<HD, RP, TP, true, true, NW * 64>(a.k, a.ldk, tb + kb * BLK, kvh * HD, Ks, Kt);
    stage_tile<HD, RP, TP, true, false, NW * 64>(a.v, a.ldv, tb + kb * BLK, kvh * HD, Vs, nullptr);
    __syncthreads();
    f32x4 sp[4], dp[4];
#pragma unroll
    for (int nb = 0; nb < 4; nb++) {
      sp[nb] = dp[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < NK; kk++) {
        sp[nb] = HT::mfma16(ld8<HT>(Ks + (nb * 16 + c16) * RP + kk * 32 + g * 8), qf[kk], sp[nb]);
        dp[nb] = HT::mfma16(ld8<HT>(Vs + (nb * 16 + c16) * RP + kk * 32 + g * 8), df[kk], dp[nb]);
      }
    }
    // sp[nb][i] = score(key kb*64 + nb*16 + 4g + i, query qi)
#pragma unroll
    for (int nb = 0; nb < 4; nb++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        float p = exp2f(sp[nb][i] * sl2 - lse2);
        if (kb == kb_last && kb * BLK + nb * 16 + g * 4 + i > qi) p = 0.f;
        dp[nb][i] = p * (dp[nb][i] - dl);
      }
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const typename HT::v8 sb = pack_acc<HT>(dp[2 * c], dp[2 * c + 1]);
      const int c0 = 2 * c * 16 + g * 4, c1 = (2 * c + 1) * 16 + g * 4;
#pragma unroll
      for (int d = 0; d < ND; d++) dq[d] = HT::mfma16(ld_pair4<HT>(Kt + (d * 16 + c16) * TP, c0, c1), sb, dq[d]);
    }
  }
  // dq[d][i] = dQ[query qi][dim d*16 + 4g + i]
#pragma unroll
  for (int d = 0; d < ND; d++)
    *(float4 *)(a.dq + tq * a.lddq + h * HD + d * 16 + g * 4) =
        make_float4(dq[d][0] * a.scale, dq[d][1] * a.scale, dq[d][2] * a.scale, dq[d][3] * a.scale);
}

int check(const AttnArgs &a) {
  if (a.HD != 64 && a.HD != 128) return ne_fail(NE_ERR_ARG, "attention: head_dim %d not in {64,128}", a.HD);
  if (a.S % BLK) return ne_fail(NE_ERR_ARG, "attention: seq %d must be a multiple of %d", a.S, BLK);
  if (a.NKV <= 0 || a.NH % a.NKV) return ne_fail(NE_ERR_ARG, "attention: heads %d not a multiple of kv heads %d", a.NH, a.NKV);
  return 0;
}

}  // namespace

namespace {

// Single-wave blocks (NW=1) stage the same tiles with a quarter of the threads; measured
// slower than 4-wave blocks even on short sequences, so 4 waves are used throughout.
bool small_grid(const AttnArgs &a) { (void)a; return false; }

template <typename HT, int HD, int NW>
int fwd_hd(const AttnArgs &a, hipStream_t s) {
  dim3 grid(a.S / (16 * NW), a.NH, a.B);
  hipLaunchKernelGGL((attn_fwd_kernel<HT, HD, NW>), grid, dim3(NW * 64), 0, s, a);
  return ne_hip_status(hipGetLastError(), "attn_fwd");
}

template <typename HT>
int fwd_t(const AttnArgs &a, hipStream_t s) {
  const bool sm = small_grid(a);
  if (a.HD == 128) return sm ? fwd_hd<HT, 128, 1>(a, s) : fwd_hd<HT, 128, 4>(a, s);
  return sm ? fwd_hd<HT, 64, 1>(a, s) : fwd_hd<HT, 64, 4>(a, s);
}

template <typename HT, int HD, int NW>
int bwd_hd(const AttnArgs &a, hipStream_t s) {
  dim3 gkv(a.S / (16 * NW), a.NKV, a.B), gq(a.S / (16 * NW), a.NH, a.B);
  hipLaunchKernelGGL((attn_bwd_dkdv_kernel<HT, HD, NW>), gkv, dim3(NW * 64), 0, s, a);
  hipLaunchKernelGGL((attn_bwd_dq_kernel<HT, HD, NW>), gq, dim3(NW * 64), 0, s, a);
  return ne_hip_status(hipGetLastError(), "attn_bwd");
}

template <typename HT>
int bwd_t(const AttnArgs &a, hipStream_t s) {
  const long rows = (long)a.B * a.S * a.NH;
  const long thr = rows * (a.HD / 8);
  if (a.HD == 128) hipLaunchKernelGGL((attn_delta_kernel<HT, 128>), dim3((thr + 255) / 256), dim3(256), 0, s, a, rows);
  else hipLaunchKernelGGL((attn_delta_kernel<HT, 64>), dim3((thr + 255) / 256), dim3(256), 0, s, a, rows);
  NE_HIP(hipGetLastError());
  const bool sm = small_grid(a);
  if (a.HD == 128) return sm ? bwd_hd<HT, 128, 1>(a, s) : bwd_hd<HT, 128, 4>(a, s);
  return sm ? bwd_hd<HT, 64, 1>(a, s) : bwd_hd<HT, 64, 4>(a, s);
}

}  // namespace

int launch_attn_fwd(int dt, const AttnArgs &a, hipStream_t s) {
  NE_CHECK(check(a));
  return DISPATCH_H16(dt, fwd_t<HT>(a, s));
}

int launch_attn_bwd(int dt, const AttnArgs &a, hipStream_t s) {
  NE_CHECK(check(a));
  return DISPATCH_H16(dt, bwd_t<HT>(a, s));
}
