// Causal flash attention forward / backward on 16-bit MFMA (v_mfma_f32_16x16x32_{f16,bf16}).
//
// Replaces the score/softmax/PV part of gen_sdpa_fwd_dynamic (TD/mil_dynamic.h:171-223,
// full S x S scores plus a -65504 mask blob, TD/mil_dynamic.h:716-725) and the two
// backward programs gen_sdpa_bwd1_noweight / gen_sdpa_bwd2 (TD/mil_dynamic.h:583-707)
// together with the GQA tile/reduce of TD/io.h:423-430 and TD/cpu_ops.h:585-605.
// Nothing O(S^2) is stored: the forward keeps the row log-sum-exp, the backward
// recomputes P per tile.  GQA: kv head = q head / (NH/NKV).
//
// Tiles of 64 keys (or queries) are staged row-major in LDS (16-byte copies, double
// buffered through registers, one barrier per tile; the forward loads its K/V tiles two
// steps ahead and waits only on LDS at the barrier).  A wave owns 16 or 32 rows (one or two
// groups of 16 sharing every LDS operand read).  Operands that are needed transposed
// (V^T for P.V, Q^T and dO^T for dK/dV, K^T for dQ) are read from the same row-major tiles
// with gfx950's LDS transpose read (ds_read_b64_tr_b16): the 16 lanes of a group each give
// the address of 4 consecutive elements, and lane i receives column i of the 4 rows.
//
// Score tiles are computed transposed so the fp32 accumulator of a 16x16 MFMA (lane l holds
// rows 4*(l/16)+i of column l%16, 4 values along the row index) is re-packed in registers
// as the next MFMA's K operand; the transposed reads use the same K permutation.
#include "common.h"
#include "ne_internal.h"

namespace {

constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr int BLK = 64;  // keys per kv tile, queries per q tile

// A compile-time flag passed to a generic lambda (one instance per value).
template <bool V>
struct Bool {
  static constexpr bool value = V;
};

typedef short s16x4 __attribute__((ext_vector_type(4)));

template <typename HT>
__device__ __forceinline__ typename HT::v8 ld8(const h16_t *p) { return HT::op(*(const u16x8 *)p); }

// Lane i of each 16-lane group receives tile[row0 + k][col0 + i], k = 0..3 (row pitch RP);
// row0 / col0 may differ between the 4 groups of the wave.
template <int RP>
__device__ __forceinline__ u16x4 tr4(const h16_t *tile, int row0, int col0) {
  const int m = threadIdx.x & 15;
  const h16_t *p = tile + (row0 + (m >> 2)) * RP + col0 + 4 * (m & 3);
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)p);
  return __builtin_bit_cast(u16x4, r);
}

// MFMA K operand of a transposed tile: rows (keys/queries) {32c + 4g + 0..3} then
// {32c + 16 + 4g + 0..3} (the order pack_acc gives), column col0 + lane%16.
template <typename HT, int RP>
__device__ __forceinline__ typename HT::v8 tr8(const h16_t *tile, int c, int col0) {
  const int g = (threadIdx.x & 63) >> 4;
  const u16x4 lo = tr4<RP>(tile, 32 * c + 4 * g, col0);
  const u16x4 hi = tr4<RP>(tile, 32 * c + 16 + 4 * g, col0);
  u16x8 r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return HT::op(r);
}

// 2^x by v_exp_f32 alone.  Every argument here is a score minus a running max or the row
// log-sum-exp (<= 8, or -inf for masked keys): results below 2^-126 may flush to zero, which
// is below the resolution of the 16-bit P and of the fp32 row sums they join.
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

// The forward's running row max moves only when a tile's max exceeds it by more than this
// (log2 units), so P <= 2^8 and the accumulator rescale is rare.
constexpr float RESCALE_SLACK = 8.f;

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

// Register-staged copy of 64-row x HD tiles (row-major, pitch RP) of up to two sources.
// Thread t copies the 16-byte chunks of rows t/CPR + i*RSTEP at column (t%CPR)*8: its
// offset within a tile is fixed, and the tile's origin is a uniform (scalar) address.
template <int HD, int NT, int NSRC>
struct TileCopy {
  static constexpr int CPR = HD / 8;      // 16-byte chunks per row
  static constexpr int CH = BLK * CPR;    // chunks per tile
  static constexpr int PER = CH / NT;     // chunks per thread
  static constexpr int RSTEP = NT / CPR;  // rows between a thread's chunks
  static_assert(NT % CPR == 0 && CH % NT == 0, "tile copy: threads must tile the 64 x HD tile");
  u16x8 v[NSRC][PER];
  __device__ __forceinline__ void load(int s, const h16_t *__restrict__ src, long ld, long t0, int col) {
    const h16_t *b = src + t0 * ld + col;
    const long off = (long)(threadIdx.x / CPR) * ld + (threadIdx.x % CPR) * 8;
#pragma unroll
    for (int i = 0; i < PER; i++) v[s][i] = *(const u16x8 *)(b + off + (long)i * RSTEP * ld);
  }
  template <int RP>
  __device__ __forceinline__ void store(int s, h16_t *dst) {
    h16_t *d = dst + (threadIdx.x / CPR) * RP + (threadIdx.x % CPR) * 8;
#pragma unroll
    for (int i = 0; i < PER; i++) *(u16x8 *)(d + i * RSTEP * RP) = v[s][i];
  }
};

// ---------------------------------------------------------------------------- forward ----

// Block (bx, by, bz) that this work-group runs.  Work-groups go to the 8 XCDs round-robin in
// launch order (x fastest) and each XCD has its own L2: each XCD takes one contiguous stretch
// of that order instead, so that the blocks of one (head, sequence), which read the same
// Q / K / V / dO rows, share an L2 (with consecutive blocks on different XCDs every XCD
// fetched every tile: the backward read 3.0 GB per layer at batch 8 x seq 2048).
__device__ __forceinline__ void xcd_block(int &bx, int &by, int &bz) {
  const int gx = gridDim.x, gy = gridDim.y;
  const int n = gx * gy * gridDim.z;
  const int pid = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const int x = pid % 8, q = n / 8, rem = n % 8;
  const int u = x * q + min(x, rem) + pid / 8;  // a bijection of [0, n)
  bx = u % gx;
  by = (u / gx) % gy;
  bz = u / (gx * gy);
}

// NW waves per block, RG groups of 16 queries per wave (the K/V fragments read from LDS
// serve every group: RG = 2 halves LDS traffic per MFMA); key tiles of 64.
template <typename HT, int HD, int NW, int RG>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2))) void attn_fwd_kernel(AttnArgs a) {
  constexpr int RP = HD + 16, NK = HD / 32, ND = HD / 16, NT = NW * 64, TILE = BLK * RP;
  constexpr int ROWS = NW * 16 * RG;  // queries per block
  // [K tile, V tile] per buffer; two named buffers so the compiler sees that the stores into
  // one and the reads from the other do not alias
  __shared__ __attribute__((aligned(16))) h16_t lds0[2 * TILE];
  __shared__ __attribute__((aligned(16))) h16_t lds1[2 * TILE];
  int bx, by, bz;
  xcd_block(bx, by, bz);
  const int q0 = (gridDim.x - 1 - bx) * ROWS;  // longest rows first
  const int kb_last = (q0 + ROWS - 1) / BLK;
  const int h = by, b = bz;
  const int kvh = h / (a.NH / a.NKV);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const long tb = (long)b * a.S;
  const int qw = q0 + w * 16 * RG;  // first query of this wave
  int qi[RG];
  typename HT::v8 qf[RG][NK];
  f32x4 acc[RG][ND];
  float m_i[RG], l_i[RG];
#pragma unroll
  for (int r = 0; r < RG; r++) {
    qi[r] = qw + r * 16 + c16;
#pragma unroll
    for (int kk = 0; kk < NK; kk++) qf[r][kk] = ld8<HT>(a.q + (tb + qi[r]) * a.ldq + h * HD + kk * 32 + g * 8);
#pragma unroll
    for (int d = 0; d < ND; d++) acc[r][d] = f32x4{0.f, 0.f, 0.f, 0.f};
    m_i[r] = -INFINITY;
    l_i[r] = 0.f;
  }
  const float sl2 = a.scale * LOG2E;

  // K/V tiles are loaded two steps ahead into alternating register sets; each step writes the
  // next tile (loaded during the previous step) into the other LDS buffer right after its
  // QK^T MFMAs, and the LDS-only barrier lets the loads in flight cross the step boundary.
  // Loads past the last tile repeat it (valid memory, never used), so the loop has no tail.
  typedef TileCopy<HD, NT, 2> TC;
  TC cp0, cp1;
  auto tload = [&](TC &cp, int kb) {
    const int kc = min(kb, kb_last);
    cp.load(0, a.k, a.ldk, tb + kc * BLK, kvh * HD);
    cp.load(1, a.v, a.ldv, tb + kc * BLK, kvh * HD);
  };
  auto tstore = [&](TC &cp, h16_t *L) {
    cp.template store<RP>(0, L);
    cp.template store<RP>(1, L + TILE);
  };
  auto step = [&](int kb, const h16_t *L, TC &nxt, h16_t *Ln) {
    if (kb * BLK <= qw + 16 * RG - 1) {  // tiles wholly above this wave's queries add nothing
      const h16_t *Ks = L, *Vs = L + TILE;
      f32x4 s[RG][4];
#pragma unroll
      for (int nb = 0; nb < 4; nb++)
#pragma unroll
        for (int r = 0; r < RG; r++) s[r][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
      // four independent accumulator chains per K step
#pragma unroll
      for (int kk = 0; kk < NK; kk++)
#pragma unroll
        for (int nb = 0; nb < 4; nb++) {
          const typename HT::v8 kfrag = ld8<HT>(Ks + (nb * 16 + c16) * RP + kk * 32 + g * 8);
#pragma unroll
          for (int r = 0; r < RG; r++) s[r][nb] = HT::mfma16(kfrag, qf[r][kk], s[r][nb]);
        }
      tstore(nxt, Ln);  // the next tile, while the softmax and P.V run
      // s[r][nb][i] = score(key kb*64 + nb*16 + 4g + i, query qi[r]); keys above a query are
      // masked on the tiles that cross this wave's diagonal only
      const bool diag = kb * BLK + BLK - 1 > qw;
      typename HT::v8 pb[RG][2];
#pragma unroll
      for (int r = 0; r < RG; r++) {
        if (diag) {
#pragma unroll
          for (int nb = 0; nb < 4; nb++)
#pragma unroll
            for (int i = 0; i < 4; i++)
              if (kb * BLK + nb * 16 + g * 4 + i > qi[r]) s[r][nb][i] = -INFINITY;
        }
        float mx = -INFINITY;
#pragma unroll
        for (int nb = 0; nb < 4; nb++)
#pragma unroll
          for (int i = 0; i < 4; i++) mx = fmaxf(mx, s[r][nb][i]);
        mx = quad16_max(mx) * sl2;
        // every processed tile holds key kb*64 <= some query of the group's earlier tiles or
        // key 0 (kb = 0), so the reference max is finite after the first tile
        if (__any(mx > m_i[r] + RESCALE_SLACK)) {
          const float m_new = fmaxf(m_i[r], mx);
          const float alpha = fexp2(m_i[r] - m_new);
          m_i[r] = m_new;
          l_i[r] *= alpha;
#pragma unroll
          for (int d = 0; d < ND; d++) acc[r][d] *= alpha;
        }
        const float nm = -m_i[r];
        float ls = 0.f;
#pragma unroll
        for (int nb = 0; nb < 4; nb++)
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float p = fexp2(fmaf(s[r][nb][i], sl2, nm));
            s[r][nb][i] = p;
            ls += p;
          }
        l_i[r] += ls;
        pb[r][0] = pack_acc<HT>(s[r][0], s[r][1]);
        pb[r][1] = pack_acc<HT>(s[r][2], s[r][3]);
      }
#pragma unroll
      for (int c = 0; c < 2; c++)
#pragma unroll
        for (int d = 0; d < ND; d++) {
          const typename HT::v8 vfrag = tr8<HT, RP>(Vs, c, d * 16);
#pragma unroll
          for (int r = 0; r < RG; r++) acc[r][d] = HT::mfma16(vfrag, pb[r][c], acc[r][d]);
        }
    } else {
      tstore(nxt, Ln);
    }
  };
  tload(cp0, 0);
  tstore(cp0, lds0);
  tload(cp0, 1);
  lds_barrier();
  const int nkb = kb_last + 1;
  for (int kb = 0; kb + 1 < nkb; kb += 2) {
    tload(cp1, kb + 2);
    step(kb, lds0, cp0, lds1);
    lds_barrier();
    tload(cp0, kb + 3);
    step(kb + 1, lds1, cp1, lds0);
    lds_barrier();
  }
  if (nkb & 1) step(nkb - 1, lds0, cp1, lds1);  // stores an unused tile into the idle buffer
#pragma unroll
  for (int r = 0; r < RG; r++) {
    const long tq = tb + qi[r];
    const float l_tot = quad16_sum(l_i[r]);
    const float inv = 1.f / l_tot;
#pragma unroll
    for (int d = 0; d < ND; d++) {
      u16x4 o;
#pragma unroll
      for (int i = 0; i < 4; i++) o[i] = HT::h(acc[r][d][i] * inv);
      *(u16x4 *)(a.o + tq * a.ldo + h * HD + d * 16 + g * 4) = o;
    }
    if (g == 0) a.lse[tq * a.NH + h] = (m_i[r] + log2f(l_tot)) * LN2;
  }
}

// --------------------------------------------------------------------------- backward ----

// delta[t, h] = sum_d dO[t,h,d] * O[t,h,d].  With split-K partials of dO (a.dsp.n > 0, dO of
// row pitch lddo = NH*HD) dO is summed in split order, scaled, rounded to 16 bits and written
// (the dK/dV and dQ kernels read it) before use.
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
    u16x8 d;
    if (a.dsp.n > 0) {
      const float *p = a.dsp.part + t * a.lddo + h * HD + j * 8;
      float4 lo = *(const float4 *)p, hi = *(const float4 *)(p + 4);
      for (int z = 1; z < a.dsp.n; z++) {
        const float4 ql = *(const float4 *)(p + z * a.dsp.slice), qh = *(const float4 *)(p + z * a.dsp.slice + 4);
        lo.x += ql.x; lo.y += ql.y; lo.z += ql.z; lo.w += ql.w;
        hi.x += qh.x; hi.y += qh.y; hi.z += qh.z; hi.w += qh.w;
      }
      const float al = a.dsp.alpha;
      d[0] = HT::h(lo.x * al); d[1] = HT::h(lo.y * al); d[2] = HT::h(lo.z * al); d[3] = HT::h(lo.w * al);
      d[4] = HT::h(hi.x * al); d[5] = HT::h(hi.y * al); d[6] = HT::h(hi.z * al); d[7] = HT::h(hi.w * al);
      bool bad = false;
#pragma unroll
      for (int e = 0; e < 8; e++) bad |= HT::bad(d[e]);
      flag_overflow(a.ovf_dout, bad);
      *(u16x8 *)((h16_t *)a.dout + t * a.lddo + h * HD + j * 8) = d;
    } else {
      d = *(const u16x8 *)(a.dout + t * a.lddo + h * HD + j * 8);
    }
#pragma unroll
    for (int e = 0; e < 8; e++) s += HT::f(o[e]) * HT::f(d[e]);
  }
  s = group_sum<L>(s);
  if (row < rows && j == 0) a.delta[row] = s;
}

// dK / dV of NW*16*RG keys (RG groups of 16 per wave) of one kv head.  SPLIT: the block
// handles one query head (block row by) and writes fp32 per-query-head partials to a.part
// (reduced by gqa_reduce_kernel); otherwise it loops over the query heads of its kv head
// (block row by) and writes dK (fp32) and dV (16-bit) directly.  Query tiles of 64 from the
// block's diagonal on.
// Block (bx, by, bz) of the dK / dV grid; lds: [buffer][Q tile, dO tile].
template <typename HT, int HD, int NW, int RG, bool SPLIT>
__device__ __forceinline__ void dkdv_block(const AttnArgs &a, int bx, int by, int bz, h16_t (*lds)[2 * BLK * (HD + 16)],
                                           float (*lse_s)[BLK], float (*ndl_s)[BLK]) {
  constexpr int RP = HD + 16, NK = HD / 32, ND = HD / 16, NT = NW * 64, TILE = BLK * RP;
  constexpr int ROWS = NW * 16 * RG;  // keys per block
  const int nqb = a.S / BLK;
  const int k0 = bx * ROWS;  // smallest keys have the most query tiles: launched first
  const int qb_first = k0 / BLK;
  const int ratio = a.NH / a.NKV;
  const int kvh = SPLIT ? by / ratio : by, b = bz;
  const int h_begin = SPLIT ? by : kvh * ratio, h_end = SPLIT ? by + 1 : (kvh + 1) * ratio;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const long tb = (long)b * a.S;
  const int kw = k0 + w * 16 * RG;  // first key of this wave
  int ki[RG];
  typename HT::v8 kf[RG][NK], vf[RG][NK];
  f32x4 dk[RG][ND], dv[RG][ND];
#pragma unroll
  for (int r = 0; r < RG; r++) {
    ki[r] = kw + r * 16 + c16;
    const long tk = tb + ki[r];
#pragma unroll
    for (int kk = 0; kk < NK; kk++) {
      kf[r][kk] = ld8<HT>(a.k + tk * a.ldk + kvh * HD + kk * 32 + g * 8);
      vf[r][kk] = ld8<HT>(a.v + tk * a.ldv + kvh * HD + kk * 32 + g * 8);
    }
#pragma unroll
    for (int d = 0; d < ND; d++) dk[r][d] = dv[r][d] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float sl2 = a.scale * LOG2E;

  // flattened (head, query tile) iteration with a one-tile register prefetch
  const int per_head = nqb - qb_first;
  const int n_it = (h_end - h_begin) * per_head;
  TileCopy<HD, NT, 2> cp;
  float lse_r = 0.f, dl_r = 0.f;
  auto fetch = [&](int it) {
    const int h = h_begin + it / per_head, qb = qb_first + it % per_head;
    cp.load(0, a.q, a.ldq, tb + qb * BLK, h * HD);
    cp.load(1, a.dout, a.lddo, tb + qb * BLK, h * HD);
    if (threadIdx.x < BLK) {
      const long t = tb + qb * BLK + threadIdx.x;
      lse_r = a.lse[t * a.NH + h] * LOG2E;
      dl_r = a.delta[t * a.NH + h];
    }
  };
  auto put = [&](int buf) {
    cp.template store<RP>(0, lds[buf]);
    cp.template store<RP>(1, lds[buf] + TILE);
    if (threadIdx.x < BLK) {
      lse_s[buf][threadIdx.x] = lse_r;
      ndl_s[buf][threadIdx.x] = -dl_r;
    }
  };
  fetch(0);
  put(0);
  __syncthreads();
  for (int it = 0; it < n_it; it++) {
    const int cur = it & 1;
    const int qb = qb_first + it % per_head;
    if (it + 1 < n_it) fetch(it + 1);
    if (qb * BLK + BLK - 1 >= kw) {  // tiles wholly below this wave's keys add nothing
      const h16_t *Qs = lds[cur], *dOs = lds[cur] + TILE;
      f32x4 sp[RG][4], dp[RG][4];
#pragma unroll
      for (int mb = 0; mb < 4; mb++) {
        // dP starts from -delta of its query rows, so the MFMAs leave dP - delta
        const f32x4 nd = *(const f32x4 *)&ndl_s[cur][mb * 16 + g * 4];
#pragma unroll
        for (int r = 0; r < RG; r++) {
          sp[r][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
          dp[r][mb] = nd;
        }
      }
#pragma unroll
      for (int kk = 0; kk < NK; kk++)
#pragma unroll
        for (int mb = 0; mb < 4; mb++) {
          const typename HT::v8 qfrag = ld8<HT>(Qs + (mb * 16 + c16) * RP + kk * 32 + g * 8);
          const typename HT::v8 ofrag = ld8<HT>(dOs + (mb * 16 + c16) * RP + kk * 32 + g * 8);
#pragma unroll
          for (int r = 0; r < RG; r++) {
            sp[r][mb] = HT::mfma16(qfrag, kf[r][kk], sp[r][mb]);
            dp[r][mb] = HT::mfma16(ofrag, vf[r][kk], dp[r][mb]);
          }
        }
      // sp[r][mb][i] = score(query qb*64 + mb*16 + 4g + i, key ki[r])
      // Only the first query tile of a head crosses this wave's keys: the others skip the mask.
      const bool diag = kw + 16 * RG - 1 > qb * BLK;  // some key of this wave above some query
      typename HT::v8 pb[RG][2], sb[RG][2];
      auto elem = [&](auto masked) {
#pragma unroll
        for (int r = 0; r < RG; r++) {
#pragma unroll
          for (int mb = 0; mb < 4; mb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const int ql = mb * 16 + g * 4 + i;
              float p = fexp2(fmaf(sp[r][mb][i], sl2, -lse_s[cur][ql]));
              if (decltype(masked)::value && ki[r] > qb * BLK + ql) p = 0.f;
              sp[r][mb][i] = p;
              dp[r][mb][i] = p * dp[r][mb][i];
            }
#pragma unroll
          for (int c = 0; c < 2; c++) {
            pb[r][c] = pack_acc<HT>(sp[r][2 * c], sp[r][2 * c + 1]);
            sb[r][c] = pack_acc<HT>(dp[r][2 * c], dp[r][2 * c + 1]);
          }
        }
      };
      if (diag) elem(Bool<true>{});
      else elem(Bool<false>{});
#pragma unroll
      for (int c = 0; c < 2; c++)
#pragma unroll
        for (int d = 0; d < ND; d++) {
          const typename HT::v8 ot = tr8<HT, RP>(dOs, c, d * 16), qt = tr8<HT, RP>(Qs, c, d * 16);
#pragma unroll
          for (int r = 0; r < RG; r++) {
            dv[r][d] = HT::mfma16(ot, pb[r][c], dv[r][d]);
            dk[r][d] = HT::mfma16(qt, sb[r][c], dk[r][d]);
          }
        }
    }
    if (it + 1 < n_it) put(cur ^ 1);
    __syncthreads();
  }
  // dv[r][d][i] = dV[key ki[r]][dim d*16 + 4g + i]
  bool bad = false;
#pragma unroll
  for (int r = 0; r < RG; r++) {
    const long tk = tb + ki[r];
    if (SPLIT) {
      const int h = by;
      float *pk = a.part, *pv = a.part + (long)a.B * a.S * a.NH * HD;
#pragma unroll
      for (int d = 0; d < ND; d++) {
        const long o = tk * a.NH * HD + h * HD + d * 16 + g * 4;
        *(float4 *)(pk + o) = make_float4(dk[r][d][0] * a.scale, dk[r][d][1] * a.scale, dk[r][d][2] * a.scale,
                                          dk[r][d][3] * a.scale);
        *(float4 *)(pv + o) = make_float4(dv[r][d][0], dv[r][d][1], dv[r][d][2], dv[r][d][3]);
      }
    } else {
#pragma unroll
      for (int d = 0; d < ND; d++) {
        *(float4 *)(a.dk + tk * a.lddk + kvh * HD + d * 16 + g * 4) =
            make_float4(dk[r][d][0] * a.scale, dk[r][d][1] * a.scale, dk[r][d][2] * a.scale, dk[r][d][3] * a.scale);
        u16x4 o;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          o[i] = HT::h(dv[r][d][i]);
          bad |= HT::bad(o[i]);
        }
        *(u16x4 *)(a.dv + tk * a.lddv + kvh * HD + d * 16 + g * 4) = o;
      }
    }
  }
  if (!SPLIT) flag_overflow(a.ovf, bad);
}

// Sum of the per-query-head dK / dV partials of each kv head, in head order: dK fp32,
// dV 16-bit.  One thread per 4 elements of [T, NKV*HD].
template <typename HT>
__global__ void gqa_reduce_kernel(AttnArgs a) {
  const long n4 = (long)a.B * a.S * a.NKV * a.HD / 4;
  const int ratio = a.NH / a.NKV;
  const float *pk = a.part, *pv = a.part + (long)a.B * a.S * a.NH * a.HD;
  bool bad = false;
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n4; i += (long)gridDim.x * 256) {
    const long e = i * 4;
    const long t = e / ((long)a.NKV * a.HD);
    const int col = (int)(e % ((long)a.NKV * a.HD));  // kvh * HD + d
    const int kvh = col / a.HD, d = col % a.HD;
    float4 sk = make_float4(0.f, 0.f, 0.f, 0.f), sv = sk;
    for (int r = 0; r < ratio; r++) {
      const long o = t * a.NH * a.HD + (long)(kvh * ratio + r) * a.HD + d;
      const float4 x = *(const float4 *)(pk + o), y = *(const float4 *)(pv + o);
      sk.x += x.x; sk.y += x.y; sk.z += x.z; sk.w += x.w;
      sv.x += y.x; sv.y += y.y; sv.z += y.z; sv.w += y.w;
    }
    *(float4 *)(a.dk + t * a.lddk + col) = sk;
    u16x4 o;
    o[0] = HT::h(sv.x); o[1] = HT::h(sv.y); o[2] = HT::h(sv.z); o[3] = HT::h(sv.w);
    bad |= HT::bad(o[0]) | HT::bad(o[1]) | HT::bad(o[2]) | HT::bad(o[3]);
    *(u16x4 *)(a.dv + t * a.lddv + col) = o;
  }
  flag_overflow(a.ovf, bad);
}

// NW waves per block, RG groups of 16 queries per wave; key tiles of 64 up to the diagonal.
// Block (bx, by, bz) of a dQ grid nbx blocks wide; lds: [buffer][K tile, V tile].
template <typename HT, int HD, int NW, int RG>
__device__ __forceinline__ void dq_block(const AttnArgs &a, int bx, int by, int bz, int nbx,
                                         h16_t (*lds)[2 * BLK * (HD + 16)]) {
  constexpr int RP = HD + 16, NK = HD / 32, ND = HD / 16, NT = NW * 64, TILE = BLK * RP;
  constexpr int ROWS = NW * 16 * RG;  // queries per block
  const int q0 = (nbx - 1 - bx) * ROWS;  // longest rows first
  const int kb_last = (q0 + ROWS - 1) / BLK;
  const int h = by, b = bz;
  const int kvh = h / (a.NH / a.NKV);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const long tb = (long)b * a.S;
  const int qw = q0 + w * 16 * RG;
  int qi[RG];
  typename HT::v8 qf[RG][NK], df[RG][NK];
  float lse2[RG], dl[RG];
  f32x4 dq[RG][ND];
#pragma unroll
  for (int r = 0; r < RG; r++) {
    qi[r] = qw + r * 16 + c16;
    const long tq = tb + qi[r];
#pragma unroll
    for (int kk = 0; kk < NK; kk++) {
      qf[r][kk] = ld8<HT>(a.q + tq * a.ldq + h * HD + kk * 32 + g * 8);
      df[r][kk] = ld8<HT>(a.dout + tq * a.lddo + h * HD + kk * 32 + g * 8);
    }
    lse2[r] = a.lse[tq * a.NH + h] * LOG2E;
    dl[r] = a.delta[tq * a.NH + h];
#pragma unroll
    for (int d = 0; d < ND; d++) dq[r][d] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float sl2 = a.scale * LOG2E;

  TileCopy<HD, NT, 2> cp;
  cp.load(0, a.k, a.ldk, tb, kvh * HD);
  cp.load(1, a.v, a.ldv, tb, kvh * HD);
  cp.template store<RP>(0, lds[0]);
  cp.template store<RP>(1, lds[0] + TILE);
  __syncthreads();
  for (int kb = 0; kb <= kb_last; kb++) {
    const int cur = kb & 1;
    if (kb < kb_last) {
      cp.load(0, a.k, a.ldk, tb + (kb + 1) * BLK, kvh * HD);
      cp.load(1, a.v, a.ldv, tb + (kb + 1) * BLK, kvh * HD);
    }
    if (kb * BLK <= qw + 16 * RG - 1) {
      const h16_t *Ks = lds[cur], *Vs = lds[cur] + TILE;
      f32x4 sp[RG][4], dp[RG][4];
#pragma unroll
      for (int nb = 0; nb < 4; nb++)
#pragma unroll
        for (int r = 0; r < RG; r++) {
          sp[r][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
          dp[r][nb] = f32x4{-dl[r], -dl[r], -dl[r], -dl[r]};  // the MFMAs leave dP - delta
        }
#pragma unroll
      for (int kk = 0; kk < NK; kk++)
#pragma unroll
        for (int nb = 0; nb < 4; nb++) {
          const typename HT::v8 kfrag = ld8<HT>(Ks + (nb * 16 + c16) * RP + kk * 32 + g * 8);
          const typename HT::v8 vfrag = ld8<HT>(Vs + (nb * 16 + c16) * RP + kk * 32 + g * 8);
#pragma unroll
          for (int r = 0; r < RG; r++) {
            sp[r][nb] = HT::mfma16(kfrag, qf[r][kk], sp[r][nb]);
            dp[r][nb] = HT::mfma16(vfrag, df[r][kk], dp[r][nb]);
          }
        }
      // sp[r][nb][i] = score(key kb*64 + nb*16 + 4g + i, query qi[r])
      // Only the last key tile crosses this wave's queries: the others skip the mask.
      const bool diag = kb * BLK + BLK - 1 > qw;  // some key of the tile above some query
      typename HT::v8 sb[RG][2];
      auto elem = [&](auto masked) {
#pragma unroll
        for (int r = 0; r < RG; r++) {
#pragma unroll
          for (int nb = 0; nb < 4; nb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
              float p = fexp2(fmaf(sp[r][nb][i], sl2, -lse2[r]));
              if (decltype(masked)::value && kb * BLK + nb * 16 + g * 4 + i > qi[r]) p = 0.f;
              dp[r][nb][i] = p * dp[r][nb][i];
            }
          sb[r][0] = pack_acc<HT>(dp[r][0], dp[r][1]);
          sb[r][1] = pack_acc<HT>(dp[r][2], dp[r][3]);
        }
      };
      if (diag) elem(Bool<true>{});
      else elem(Bool<false>{});
#pragma unroll
      for (int c = 0; c < 2; c++)
#pragma unroll
        for (int d = 0; d < ND; d++) {
          const typename HT::v8 kt = tr8<HT, RP>(Ks, c, d * 16);
#pragma unroll
          for (int r = 0; r < RG; r++) dq[r][d] = HT::mfma16(kt, sb[r][c], dq[r][d]);
        }
    }
    if (kb < kb_last) {
      cp.template store<RP>(0, lds[cur ^ 1]);
      cp.template store<RP>(1, lds[cur ^ 1] + TILE);
    }
    __syncthreads();
  }
  // dq[r][d][i] = dQ[query qi[r]][dim d*16 + 4g + i]
#pragma unroll
  for (int r = 0; r < RG; r++)
#pragma unroll
    for (int d = 0; d < ND; d++)
      *(float4 *)(a.dq + (tb + qi[r]) * a.lddq + h * HD + d * 16 + g * 4) =
          make_float4(dq[r][d][0] * a.scale, dq[r][d][1] * a.scale, dq[r][d][2] * a.scale, dq[r][d][3] * a.scale);
}

int check(const AttnArgs &a) {
  if (a.dsp.n > 0 && a.lddo != (long)a.NH * a.HD)
    return ne_fail(NE_ERR_ARG, "attention: split-K dout needs a dense [T, NH*HD] layout");
  if (a.HD != 64 && a.HD != 128) return ne_fail(NE_ERR_ARG, "attention: head_dim %d not in {64,128}", a.HD);
  if (a.S % BLK) return ne_fail(NE_ERR_ARG, "attention: seq %d must be a multiple of %d", a.S, BLK);
  if (a.NKV <= 0 || a.NH % a.NKV) return ne_fail(NE_ERR_ARG, "attention: heads %d not a multiple of kv heads %d", a.NH, a.NKV);
  return 0;
}

// Block shape (waves NW, 16-row groups per wave RG) by the work-group count it gives.
// Two row groups per wave halve the LDS reads per MFMA and double the accumulators: the
// forward still fits two waves per SIMD with them (used for long sequences); the dK/dV and
// dQ kernels would drop to one, which costs more than the LDS traffic saves, so they keep
// one group.  4 waves while 64-row blocks give 256 work-groups, else 2 (short sequences
// would leave most CUs idle).
enum { SHAPE_2x1 = 0, SHAPE_4x1 = 1, SHAPE_4x2 = 2 };
int pick_shape(const AttnArgs &a) {
  const long units64 = (long)(a.S / BLK) * a.NH * a.B;
  if (a.S % 128 == 0 && units64 / 2 >= 512) return SHAPE_4x2;
  if (units64 >= 256) return SHAPE_4x1;
  return SHAPE_2x1;
}

template <typename HT, int HD, int NW, int RG>
int fwd_hd(const AttnArgs &a, hipStream_t s) {
  dim3 grid(a.S / (16 * NW * RG), a.NH, a.B);
  hipLaunchKernelGGL((attn_fwd_kernel<HT, HD, NW, RG>), grid, dim3(NW * 64), 0, s, a);
  return ne_hip_status(hipGetLastError(), "attn_fwd");
}

template <typename HT, int HD>
int fwd_shape(const AttnArgs &a, hipStream_t s) {
  switch (pick_shape(a)) {
    case SHAPE_4x2: return fwd_hd<HT, HD, 4, 2>(a, s);
    case SHAPE_4x1: return fwd_hd<HT, HD, 4, 1>(a, s);
    default: return fwd_hd<HT, HD, 2, 1>(a, s);
  }
}

template <typename HT>
int fwd_t(const AttnArgs &a, hipStream_t s) {
  if (a.HD == 128) return fwd_shape<HT, 128>(a, s);
  return fwd_shape<HT, 64>(a, s);
}

// dK / dV and dQ in one launch: blocks x < nkv are dK / dV key blocks (grid.y rows >= nky
// idle: without the per-query-head split there is one block row per KV head), the rest dQ
// query blocks.  The two kinds depend only on delta (computed before), so they run side by
// side: at short sequences each alone leaves half the CUs idle.
template <typename HT, int HD, int NW, int RG, bool SPLIT>
__global__ __launch_bounds__(NW * 64) void attn_bwd_kernel(AttnArgs a, int nkv, int nky) {
  __shared__ __attribute__((aligned(16))) h16_t lds[2][2 * BLK * (HD + 16)];
  __shared__ __attribute__((aligned(16))) float lse_s[2][BLK], ndl_s[2][BLK];
  int bx, by, bz;
  xcd_block(bx, by, bz);
  if (bx < nkv) {
    if (by < nky) dkdv_block<HT, HD, NW, RG, SPLIT>(a, bx, by, bz, lds, lse_s, ndl_s);
  } else {
    dq_block<HT, HD, NW, RG>(a, bx - nkv, by, bz, gridDim.x - nkv, lds);
  }
}

template <typename HT, int HD, int NW, int RG>
int bwd_hd(const AttnArgs &a, hipStream_t s) {
  const int nblk = a.S / (16 * NW * RG);  // key blocks of dK / dV = query blocks of dQ
  const dim3 grid(2 * nblk, a.NH, a.B);
  if (a.part && a.NH != a.NKV) {
    hipLaunchKernelGGL((attn_bwd_kernel<HT, HD, NW, RG, true>), grid, dim3(NW * 64), 0, s, a, nblk, a.NH);
    NE_HIP(hipGetLastError());
    if (!a.defer_gqa) {
      const long n4 = (long)a.B * a.S * a.NKV * HD / 4;
      hipLaunchKernelGGL(gqa_reduce_kernel<HT>, dim3((int)std::min<long>((n4 + 255) / 256, 4096)), dim3(256), 0, s, a);
    }
  } else {
    hipLaunchKernelGGL((attn_bwd_kernel<HT, HD, NW, RG, false>), grid, dim3(NW * 64), 0, s, a, nblk, a.NKV);
  }
  return ne_hip_status(hipGetLastError(), "attn_bwd");
}

template <typename HT, int HD>
int bwd_shape(const AttnArgs &a, hipStream_t s) {
  if (pick_shape(a) != SHAPE_2x1) return bwd_hd<HT, HD, 4, 1>(a, s);
  return bwd_hd<HT, HD, 2, 1>(a, s);
}

template <typename HT>
int bwd_t(const AttnArgs &a, hipStream_t s) {
  const long rows = (long)a.B * a.S * a.NH;
  const long thr = rows * (a.HD / 8);
  if (a.HD == 128) hipLaunchKernelGGL((attn_delta_kernel<HT, 128>), dim3((thr + 255) / 256), dim3(256), 0, s, a, rows);
  else hipLaunchKernelGGL((attn_delta_kernel<HT, 64>), dim3((thr + 255) / 256), dim3(256), 0, s, a, rows);
  NE_HIP(hipGetLastError());
  if (a.HD == 128) return bwd_shape<HT, 128>(a, s);
  return bwd_shape<HT, 64>(a, s);
}

}  // namespace

// With GQA the dK/dV blocks either take one query head each and leave fp32 partials that the
// QK-prep backward sums (twice the blocks: a 256-token Qwen3-0.6B step has 64 dK/dV blocks
// per layer without them, 7.37 vs 7.52-7.57 ms per step), or loop over the query heads of
// their KV head and write dK and dV directly (no partials to write and read back: 268 MB
// per layer less of each at batch 8 x 2048, 103.2-103.4 vs 101.6-102.1 ms per step).  The
// split is taken below two dK/dV blocks per CU.
bool attn_bwd_split_heads(int B, int S, int NH, int NKV) {
  if (NH == NKV || S % BLK) return false;
  AttnArgs a = {};
  a.B = B; a.S = S; a.NH = NH; a.NKV = NKV;
  const int rows = pick_shape(a) == SHAPE_2x1 ? 32 : 64;  // keys per dK/dV block (RG = 1)
  return (long)(S / rows) * NKV * B < 512;
}

int launch_attn_fwd(int dt, const AttnArgs &a, hipStream_t s) {
  NE_CHECK(check(a));
  return DISPATCH_H16(dt, fwd_t<HT>(a, s));
}

int launch_attn_bwd(int dt, const AttnArgs &a, hipStream_t s) {
  NE_CHECK(check(a));
  return DISPATCH_H16(dt, bwd_t<HT>(a, s));
}
