// 16-bit MFMA GEMM for gfx950 with LDS-staged tiles, split-K and fused epilogues.
//
// C[M,N] = epi(alpha * sum_k A[m,k] B[k,n]).  Operands are 16-bit (fp16 or bf16) with fp32
// accumulation on v_mfma_f32_32x32x16_{f16,bf16}.  Each operand may be K-contiguous
// (activation rows, weight rows [N,K]) or M/N-contiguous (the dY^T and X of a
// weight-gradient GEMM, the weights of a dX GEMM); either is staged into LDS as it lies in
// memory (16-byte loads and stores), and an MFMA operand is one 16-byte LDS read
// (K-contiguous) or two gfx950 transpose reads (M/N-contiguous).  Double-buffered LDS, one
// LDS-only barrier per K step, global loads two steps ahead, memory instructions interleaved
// with the MFMAs.  Block tiles: 256x256 or 256x128 with 8 waves (64x128 / 64x64 each) for
// large shapes, 128x128 or 64x64 with 4 waves (64x64 / 32x32) otherwise.
//
// Small-M shapes (a 256-token step) leave too few output tiles to fill 256 CUs, so the
// launcher splits K over grid.z: each split writes its fp32 partial tile to a workspace
// and an ordered reduction (deterministic) applies the epilogue.
//
// Replaces the ANE matmuls of TD/mil_dynamic.h (gen_sdpa_fwd_dynamic QKV/Wo,
// gen_ffn_fused_dynamic W1/W3/W2, gen_ffn_bwd_full_dynamic, gen_wot_dynamic,
// gen_qkv_bwd_dynamic) and the cblas_sgemm weight-gradient / classifier calls of
// TD/train.m:500-524, 554-557, 594-597, 654-655, 733-738.
#include <type_traits>

#include "common.h"
#include "ne_internal.h"

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));

// gfx950 LDS transpose read: lane i of each 16-lane group receives tile[row0 + j][col0 + i],
// j = 0..3 (row pitch P); row0 / col0 may differ between the 4 groups of the wave.
template <int P>
__device__ __forceinline__ u16x4 tr4(const h16_t *tile, int row0, int col0) {
  const int m = threadIdx.x & 15;
  const h16_t *p = tile + (row0 + (m >> 2)) * P + col0 + 4 * (m & 3);
  return __builtin_bit_cast(u16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)p));
}

// One operand's K-step tile: R rows (M or N) by BK columns (K), staged into LDS as it lies
// in memory, 16 bytes per global load and per LDS store.
//  KC (K-contiguous, element (r, k) at p[r*ld + k]): LDS [R][BK + 8]; an MFMA operand (8
//    consecutive k of one row) is one 16-byte LDS read.
//  MN-contiguous (element at p[k*ld + r]): LDS [BK][R + 32]; the operand is two transpose
//    reads (ds_read_b64_tr_b16) of 4 k rows each.  The 64-byte row pad puts the 4 rows a
//    16-lane group reads on distinct banks.
template <int NT, int R, int BK, bool KC>
struct Stage {
  static constexpr int PITCH = KC ? BK + 8 : R + 32;
  static constexpr int ELEMS = KC ? R * PITCH : BK * PITCH;
  static constexpr int NCH = R * BK / 8;  // 16-byte chunks
  static constexpr int PER = (NCH + NT - 1) / NT;
  static constexpr int FRAG_READS = KC ? 1 : 2;  // LDS reads per MFMA operand
  u16x8 v[PER];

  // chunk c -> (row of the LDS tile, 8-element column block); consecutive threads take
  // consecutive 16-byte pieces of one memory row
  __device__ __forceinline__ static void idx(int c, int &row, int &col8) {
    constexpr int CPR = KC ? BK / 8 : R / 8;  // chunks per memory row
    row = c / CPR;
    col8 = c % CPR;
  }

  __device__ __forceinline__ void load(const h16_t *p, long ld, int r0, int k0, int tid) {
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int c = tid + i * NT;
      if (NCH % NT == 0 || c < NCH) {
        int row, col8;
        idx(c, row, col8);
        v[i] = KC ? *(const u16x8 *)(p + (long)(r0 + row) * ld + k0 + col8 * 8)
                  : *(const u16x8 *)(p + (long)(k0 + row) * ld + r0 + col8 * 8);
      }
    }
  }

  // K-contiguous rows from two places: tile rows [0, half) at lo + row * ld, the rest at
  // hi + row * ld (lo and hi already offset to this tile's rows)
  __device__ __forceinline__ void load_split(const h16_t *lo, const h16_t *hi, long ld, int half, int k0, int tid) {
    static_assert(KC, "load_split: K-contiguous operand");
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int c = tid + i * NT;
      if (NCH % NT == 0 || c < NCH) {
        int row, col8;
        idx(c, row, col8);
        v[i] = *(const u16x8 *)((row < half ? lo : hi) + (long)row * ld + k0 + col8 * 8);
      }
    }
  }

  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < PER; i++) v[i] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
  }

  __device__ __forceinline__ void store(h16_t *lds, int tid) {
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int c = tid + i * NT;
      if (NCH % NT == 0 || c < NCH) {
        int row, col8;
        idx(c, row, col8);
        *(u16x8 *)(lds + row * PITCH + col8 * 8) = v[i];
      }
    }
  }

  // MFMA 32x32x16 operand of rows rb + (lane & 31), k = 16 kk + 8 (lane >> 5) + 0..7
  __device__ __forceinline__ static u16x8 frag(const h16_t *lds, int rb, int kk, int lane) {
    if constexpr (KC) {
      return *(const u16x8 *)(lds + (rb + (lane & 31)) * PITCH + kk * 16 + (lane >> 5) * 8);
    } else {
      const int g = lane >> 4;
      const int col = rb + 16 * (g & 1), k = kk * 16 + 8 * (g >> 1);
      const u16x4 lo = tr4<PITCH>(lds, k, col), hi = tr4<PITCH>(lds, k + 4, col);
      return u16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  }
};

__device__ __forceinline__ float fast_sigmoid(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Instruction order of one K step, for the scheduler: G groups, each [MFMA, fragment reads,
// global load, MFMA, LDS store], the counts spread evenly (NMF MFMAs, NDR fragment reads, NGL
// global loads, NDW LDS stores per step), so the memory instructions issue between the MFMAs
// instead of in bursts that leave the matrix pipe idle.
template <int NMF, int NDR, int NGL, int NDW, int G, int I = 0>
__device__ __forceinline__ void sched_kstep() {
  if constexpr (I < G) {
    constexpr int m0 = I * NMF / G, m1 = (I + 1) * NMF / G, mh = (m0 + m1) / 2;
    constexpr int r = (I + 1) * NDR / G - I * NDR / G;
    constexpr int l = (I + 1) * NGL / G - I * NGL / G;
    constexpr int w = (I + 1) * NDW / G - I * NDW / G;
    if constexpr (mh > m0) __builtin_amdgcn_sched_group_barrier(0x008, mh - m0, 0);  // MFMA
    if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);          // LDS read
    if constexpr (l > 0) __builtin_amdgcn_sched_group_barrier(0x020, l, 0);          // global load
    if constexpr (m1 > mh) __builtin_amdgcn_sched_group_barrier(0x008, m1 - mh, 0);  // MFMA
    if constexpr (w > 0) __builtin_amdgcn_sched_group_barrier(0x200, w, 0);          // LDS write
    sched_kstep<NMF, NDR, NGL, NDW, G, I + 1>();
  }
}


// Epilogues whose fp32 output is a gradient: the tile also reports the sum of squares of
// the values it stores (GemmArgs::sq), for the global gradient norm.
template <int EPI>
constexpr bool epi_sq() { return EPI == EPI_F32 || EPI == EPI_F32_ACC; }

// Block sum of each thread's s (fixed order: waves, then wave 0..NW-1) into *out.
template <int NW>
__device__ __forceinline__ void block_sumsq_store(float s, double *out) {
  __shared__ float red[NW];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < NW; w++) t += red[w];
    *out = t;
  }
}

// Final store of one output element v (alpha already applied) for every non-CE epilogue.  NT:
// fp32 outputs go out (and, accumulating, come in) as non-temporal accesses: the weight and
// embedding gradients of a short step (2.4 GB per 256-token Qwen3-0.6B step, read back only by
// the next update) then stream past the caches the activation-gradient chain beside them works
// from (that step 7.58-7.64 -> 7.45-7.55 ms).  Not on the 256x256 tile, which reads back what it
// stored for the sums of squares;
// returns the fp32 value stored (EPI_F32, EPI_F32_ACC; else 0).
template <typename HT, int EPI, bool NT = false>
__device__ __forceinline__ float store_out(const GemmArgs &g, int row, int col, float v, bool &bad) {
  if constexpr (EPI == EPI_H16) {
    const h16_t o = HT::h(v);
    bad |= HT::bad(o);
    ((h16_t *)g.C)[(long)row * g.ldc + col] = o;
  } else if constexpr (EPI == EPI_F32) {
    float *c = (float *)g.C + (long)row * g.ldc + col;
    if constexpr (NT) __builtin_nontemporal_store(v, c);
    else *c = v;
    return v;
  } else if constexpr (EPI == EPI_F32_ACC) {
    float *c = (float *)g.C + (long)row * g.ldc + col;
    const float o = (NT ? __builtin_nontemporal_load(c) : *c) + v;
    if constexpr (NT) __builtin_nontemporal_store(o, c);
    else *c = o;
    return o;
  } else if constexpr (EPI == EPI_RESID) {
    ((float *)g.C)[(long)row * g.ldc + col] = ((const float *)g.R)[(long)row * g.ldr + col] + v;
  } else if constexpr (EPI == EPI_SWIGLU_BWD) {
    const h16_t *h = (const h16_t *)g.R + (long)row * g.ldr;
    const float h1 = HT::f(h[col]), h3 = HT::f(h[g.N + col]);
    const float sg = fast_sigmoid(h1);
    h16_t *d = (h16_t *)g.C + (long)row * g.ldc;
    const h16_t o1 = HT::h(v * h3 * sg * (1.f + h1 * (1.f - sg)));
    const h16_t o3 = HT::h(v * h1 * sg);
    bad |= HT::bad(o1) | HT::bad(o3);
    d[col] = o1;
    d[g.N + col] = o3;
  }
  return 0.f;
}

// How a split's K steps are run: the software pipeline takes two steps per iteration.
//  KM_TAIL: an odd last step is computed after the loop (the default);
//  KM_EVEN: every split has an even step count (no tail code at all);
//  KM_PAD:  an odd count runs one extra step whose A stage is zero.
// The cross-entropy epilogues hold more registers than the others: with the tail, the
// allocator copied the accumulators around the conditional compute (392 bytes of scratch per
// lane for EPI_CE_FWD); they take KM_EVEN or KM_PAD.
enum { KM_TAIL = 0, KM_EVEN = 1, KM_PAD = 2 };

// One output tile (mt, nt) of split kz: the body of the plain and the grouped kernel.
template <typename HT, int BM, int BN, int BK, int WM, int WN, bool AKC, bool BKC, int EPI, int KMODE>
__device__ __forceinline__ void gemm_body(const GemmArgs &g, const int mt, const int nt, const int kz) {
  constexpr int NTHREADS = WM * WN * 64;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  static_assert(FM >= 1 && FN >= 1, "wave tile >= 32x32");
  // 256x256 tiles: 144 KB of the 160 KB LDS of a gfx950 CU (one work-group per CU).  Two
  // named buffers (not one array), so the compiler sees that the stores into one and the
  // fragment reads from the other do not alias and can interleave them.
  typedef Stage<NTHREADS, BM, BK, AKC> SA;
  typedef Stage<NTHREADS, BN, BK, BKC> SB;
  __shared__ __attribute__((aligned(16))) h16_t lds0[SA::ELEMS + SB::ELEMS];
  __shared__ __attribute__((aligned(16))) h16_t lds1[SA::ELEMS + SB::ELEMS];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int n0 = nt * BN, m0 = mt * BM;
  const h16_t *A = (const h16_t *)g.A;
  const h16_t *B = (const h16_t *)g.B;
  // K steps of this split: [kt0, kt1)
  const int nkt = g.K / BK;
  const int kt0 = (int)((long)nkt * kz / g.split);
  const int kt1 = (int)((long)nkt * (kz + 1) / g.split);

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  // Software pipeline: while a K step's MFMAs run from one LDS buffer, the next stage (held in
  // registers since the previous step) is written into the other, and the stage after that is
  // loaded from global memory into the second register set: global loads are issued two steps
  // ahead of their use, and the LDS-only barrier lets them cross the step boundary.
  SA sa0, sa1;
  SB sb0, sb1;
  constexpr int NMF = FM * FN * (BK / 16), NDR = (FM * SA::FRAG_READS + FN * SB::FRAG_READS) * (BK / 16);
  constexpr int NGL = SA::PER + SB::PER, NDW = SA::PER + SB::PER;
  auto compute = [&](const h16_t *L) {
    const h16_t *As = L, *Bs = L + SA::ELEMS;
#pragma unroll
    for (int kk = 0; kk < BK / 16; kk++) {
      typename HT::v8 a[FM], b[FN];
#pragma unroll
      for (int i = 0; i < FM; i++) a[i] = HT::op(SA::frag(As, wm * TM + i * 32, kk, lane));
#pragma unroll
      for (int j = 0; j < FN; j++) b[j] = HT::op(SB::frag(Bs, wn * TN + j * 32, kk, lane));
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = HT::mfma32(a[i], b[j], acc[i][j]);
    }
  };
  const int n = kt1 - kt0;  // K steps of this split (>= 1)
  const int nr = KMODE == KM_PAD ? n + (n & 1) : n;  // steps run
  // Stage j of the split is loaded from K step kt0 + min(j, n - 1): the loads past the end
  // repeat the last step (valid memory, never computed), so the loop body has no branch and
  // one register allocation covers every split length.
  // SwiGLU forward: the tile's first BN/2 B rows are W1 rows n0/2.., the rest the W3 rows of
  // the same columns (B rows N/2 + n0/2..), so h1 and h3 of a column meet in one work-group
  const h16_t *Blo = B + (long)(n0 / 2) * g.ldb, *Bhi = B + ((long)g.N / 2 + n0 / 2 - BN / 2) * g.ldb;
  auto load = [&](SA &a, SB &b, int j) {
    const int kt = kt0 + min(j, n - 1);
    a.load(A, g.lda, m0, kt * BK, tid);
    if constexpr (EPI == EPI_SWIGLU_FWD) b.load_split(Blo, Bhi, g.ldb, BN / 2, kt * BK, tid);
    else b.load(B, g.ldb, n0, kt * BK, tid);
    if constexpr (KMODE == KM_PAD)
      if (j >= n) a.zero();  // the padding step adds nothing
  };
  auto store = [&](h16_t *L, SA &a, SB &b) {
    a.store(L, tid);
    b.store(L + SA::ELEMS, tid);
  };
  auto sched = [&]() { sched_kstep<NMF, NDR, NGL, NDW, NGL>(); };

  load(sa0, sb0, 0);
  store(lds0, sa0, sb0);
  load(sa0, sb0, 1);
  lds_barrier();
  for (int i = 0; i + 1 < nr; i += 2) {  // steps i (lds0) and i + 1 (lds1)
    load(sa1, sb1, i + 2);
    compute(lds0);
    store(lds1, sa0, sb0);
    sched();
    lds_barrier();
    load(sa0, sb0, i + 3);
    compute(lds1);
    store(lds0, sa1, sb1);
    sched();
    lds_barrier();
  }
  if constexpr (KMODE == KM_TAIL)
    if (n & 1) compute(lds0);  // the last step of an odd count is in lds0

  // ---- epilogue: lane owns column (lane & 31) and rows 8*(e/4) + 4*(lane/32) + e%4 ----
  const float alpha = g.alpha;
  if constexpr (EPI == EPI_CE_FWD) {
    // Per row of this N-tile: the max over the tile's columns and the sum of exp relative to
    // it, plus the target logit when the target column falls in the tile.  With C, each
    // logit v is also stored as the 16-bit e = exp(v - tile max) in [0, 1], from which the
    // gradient pass (launch_ce_grad) forms softmax - onehot once the row's log-sum-exp is
    // known, instead of a second logits GEMM.  Padding columns (>= n_valid) take no part
    // (e = 0).
    __shared__ float red_m[WN][BM], red_s[WN][BM];
#pragma unroll
    for (int i = 0; i < FM; i++) {
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int rl = wm * TM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int row = m0 + rl;
        const int tgt = g.targets[row];
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < FN; j++) {
          const int col = g.col0 + n0 + wn * TN + j * 32 + (lane & 31);  // of the full vocabulary
          const float v = col < g.n_valid ? acc[i][j][e] * alpha : -INFINITY;
          mx = fmaxf(mx, v);
          if (col == tgt) g.tgt_logit[row] = v;
        }
        mx = half_wave_max(mx);  // over the 32 lanes sharing this row (equal lane>>5)
        if ((lane & 31) == 0) red_m[wn][rl] = mx;
      }
    }
    __syncthreads();
    h16_t *ce = (h16_t *)g.C;
#pragma unroll
    for (int i = 0; i < FM; i++) {
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int rl = wm * TM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        float mx = red_m[0][rl];
#pragma unroll
        for (int w = 1; w < WN; w++) mx = fmaxf(mx, red_m[w][rl]);
        // a row with no valid column in this tile has mx = -inf and sum 0
        const float mxs = mx > -INFINITY ? mx : 0.f;
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < FN; j++) {
          const int cl = n0 + wn * TN + j * 32 + (lane & 31);  // of this launch
          const float ev = g.col0 + cl < g.n_valid ? __expf(acc[i][j][e] * alpha - mxs) : 0.f;
          s += ev;
          if (ce) ce[(long)(m0 + rl) * g.ldc + cl] = HT::h(ev);
        }
        s = half_wave_sum(s);
        if ((lane & 31) == 0) red_s[wn][rl] = s;
      }
    }
    __syncthreads();
    for (int r = tid; r < BM; r += NTHREADS) {
      float mx = red_m[0][r], s = red_s[0][r];
#pragma unroll
      for (int w = 1; w < WN; w++) {
        mx = fmaxf(mx, red_m[w][r]);
        s += red_s[w][r];
      }
      float *p = g.part + ((long)(m0 + r) * g.n_tiles + g.tile0 + nt) * 2;
      p[0] = mx;
      p[1] = s;
    }
    return;
  }

  if constexpr (EPI == EPI_SWIGLU_FWD) {
    // Wave column wn = 0 holds h1, wn = 1 h3 of the same output columns n0/2 + (local column)
    // in the same lanes and registers (a wave's N extent is BN/2).  Each rounds its values to
    // 16 bits and writes them to h13; the h3 waves pass theirs through LDS, and the h1 waves
    // write the gate from the two 16-bit values, as a separate SwiGLU pass over h13 would.
    static_assert(WN == 2 && TN * 2 == BN, "SwiGLU forward: two wave columns of BN/2");
    static_assert(WM * FM * FN * 16 * 64 <= SA::ELEMS + SB::ELEMS, "SwiGLU forward: exchange fits an LDS buffer");
    h16_t *xch = lds0;
    h16_t *h13 = (h16_t *)g.C, *gate = (h16_t *)g.C2;
    const int H = g.N / 2;
    bool bad = false, badg = false;
    lds_barrier();  // the last K step's fragment reads of lds0 are done
    if (wn == 1) {
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) {
          const int col = H + n0 / 2 + j * 32 + (lane & 31);
#pragma unroll
          for (int e = 0; e < 16; e++) {
            const int row = m0 + wm * TM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
            const h16_t o = HT::h(acc[i][j][e] * alpha);
            bad |= HT::bad(o);
            h13[(long)row * g.ldc + col] = o;
            xch[(((wm * FM + i) * FN + j) * 16 + e) * 64 + lane] = o;
          }
        }
    }
    lds_barrier();
    if (wn == 0) {
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) {
          const int col = n0 / 2 + j * 32 + (lane & 31);
#pragma unroll
          for (int e = 0; e < 16; e++) {
            const int row = m0 + wm * TM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
            const h16_t o1 = HT::h(acc[i][j][e] * alpha), o3 = xch[(((wm * FM + i) * FN + j) * 16 + e) * 64 + lane];
            bad |= HT::bad(o1);
            h13[(long)row * g.ldc + col] = o1;
            const h16_t og = swiglu_gate<HT>(o1, o3);
            badg |= HT::bad(og);
            gate[(long)row * g.ldc2 + col] = og;
          }
        }
    }
    flag_overflow(g.ovf, bad);
    flag_overflow(g.ovf2, badg);
    return;
  }

  if (g.split > 1) {  // fp32 partial tile -> workspace slice kz
    float *ws = g.ws + (long)kz * g.M * g.N;
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++) {
        const int col = n0 + wn * TN + j * 32 + (lane & 31);
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int row = m0 + wm * TM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
          ws[(long)row * g.N + col] = acc[i][j][e];
        }
      }
    return;
  }

  if constexpr (EPI == EPI_SWIGLU_BWD || EPI == EPI_CE_BWD) {
    // Through LDS, so that the 16-bit outputs (and the SwiGLU gate reads) are 16-byte row pieces
    // (in the MFMA layout each lane would touch one 2-byte element per row): pass i stages row
    // block i of every wave row (WM * 32 rows x BN fp32, the first half of the rows in lds0, the
    // second in lds1), then each thread takes 8 consecutive columns of a row.
    constexpr int SR = WM * 32, HR = SR / 2, SP = BN + 8;  // rows per pass, per buffer; pitch
    constexpr int CPR8 = BN / 8, NCHK = SR * CPR8 / NTHREADS;
    static_assert(HR * SP * 4 <= (SA::ELEMS + SB::ELEMS) * 2, "staged epilogue: a pass must fit an LDS buffer");
    static_assert(SR * CPR8 % NTHREADS == 0, "staged epilogue: whole chunks per thread");
    float *st0 = (float *)lds0, *st1 = (float *)lds1;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < FM; i++) {
      lds_barrier();  // the buffers' previous readers (last K step, previous pass) are done
      float *stw = wm < WM / 2 ? st0 : st1;
#pragma unroll
      for (int j = 0; j < FN; j++) {
        const int col = wn * TN + j * 32 + (lane & 31);
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int rr = (wm % (WM / 2)) * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
          stw[rr * SP + col] = acc[i][j][e] * alpha;
        }
      }
      lds_barrier();
#pragma unroll
      for (int c = 0; c < NCHK; c++) {
        const int chunk = tid + c * NTHREADS, row = chunk / CPR8, c8 = chunk % CPR8;
        const float *str = (row < HR ? st0 : st1) + (row % HR) * SP + c8 * 8;
        const float4 v0 = *(const float4 *)str, v1 = *(const float4 *)(str + 4);
        const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        const long grow = m0 + (row / 32) * TM + i * 32 + row % 32;
        const int gcol = n0 + c8 * 8;
        if constexpr (EPI == EPI_SWIGLU_BWD) {
          const h16_t *hb = (const h16_t *)g.R;
          h16_t *db = (h16_t *)g.C;
          const u16x8 h1v = *(const u16x8 *)(hb + grow * g.ldr + gcol);
          const u16x8 h3v = *(const u16x8 *)(hb + grow * g.ldr + g.N + gcol);
          u16x8 o1, o3;
#pragma unroll
          for (int e = 0; e < 8; e++) {
            const float h1 = HT::f(h1v[e]), h3 = HT::f(h3v[e]);
            const float sg = fast_sigmoid(h1);
            o1[e] = HT::h(v[e] * h3 * sg * (1.f + h1 * (1.f - sg)));
            o3[e] = HT::h(v[e] * h1 * sg);
            bad |= HT::bad(o1[e]) | HT::bad(o3[e]);
          }
          *(u16x8 *)(db + grow * g.ldc + gcol) = o1;
          *(u16x8 *)(db + grow * g.ldc + g.N + gcol) = o3;
        } else {
          // dlogits = (exp(logit - lse) - onehot(target)) * scale; padding columns (of the
          // full vocabulary's numbering, >= n_valid) get no gradient
          const float l = g.lse[grow];
          const int tc = g.targets[grow] - g.col0 - gcol;  // target's offset in this chunk
          const int nv = g.n_valid - g.col0 - gcol;        // valid columns in this chunk
          u16x8 o;
#pragma unroll
          for (int e = 0; e < 8; e++) {
            float p = e < nv ? __expf(v[e] - l) : 0.f;
            if (e == tc) p -= 1.f;
            o[e] = HT::h(p * g.scale);
            bad |= HT::bad(o[e]);
          }
          *(u16x8 *)((h16_t *)g.C + grow * g.ldc + gcol) = o;
        }
      }
    }
    flag_overflow(g.ovf, bad);
    return;
  }

  // The sum of squares of the stored values (epi_sq): summed as they are stored, except on
  // the 256x256 tile (128 accumulators per lane), where keeping each stored value live for it
  // pushed the registers past 256 (scratch spills); there each thread reads back the values it
  // has just stored (L2 hits), after a compiler barrier that keeps the reads from being folded
  // into the stores.  That tile runs long reductions (K >= 8192), where the read-back is
  // negligible; at 256 tokens it cost the 128x128 weight-gradient tiles ~25 us per layer.
  constexpr bool SQ_INLINE = FM * FN * 16 <= 64;
  bool bad = false;
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < FM; i++) {
#pragma unroll
    for (int j = 0; j < FN; j++) {
      const int col = n0 + wn * TN + j * 32 + (lane & 31);
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int row = m0 + wm * TM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const float o = store_out<HT, EPI, SQ_INLINE>(g, row, col, acc[i][j][e] * alpha, bad);
        if constexpr (epi_sq<EPI>() && SQ_INLINE) sq += o * o;
      }
    }
  }
  flag_overflow(g.ovf, bad);
  if constexpr (epi_sq<EPI>())
    if (g.sq) {
      if constexpr (!SQ_INLINE) {
        asm volatile("" ::: "memory");
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int j = 0; j < FN; j++) {
            const int col = n0 + wn * TN + j * 32 + (lane & 31);
#pragma unroll
            for (int e = 0; e < 16; e++) {
              const int row = m0 + wm * TM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
              const float o = ((const float *)g.C)[(long)row * g.ldc + col];
              sq += o * o;
            }
          }
      }
      block_sumsq_store<WM * WN>(sq, g.sq + (long)mt * (g.N / BN) + nt);
    }
}

// Tile order.  Work-groups go to the 8 XCDs round-robin (work-group w to XCD w % 8), and
// each XCD has its own L2.  The tiles are laid out in grouped order (groups of GM M tiles,
// the M tiles of a group in turn for each N tile, so consecutive tiles share a B tile and a
// group's A tiles recur), and XCD x takes one contiguous stretch of that sequence: the M
// tiles that share a B tile run on the same XCD and find it in its L2, as do the recurring A
// tiles.  (Handing consecutive tiles to different XCDs made every XCD fetch each B tile: 4x
// the weight bytes for a 256-token forward GEMM.)  GM = 4: a group's A tiles (4 x 512 KB at
// K = 1024) stay in the 4 MB L2 beside the streaming B tiles; 8 did not fit, and the
// 16k-token step ran 1.2% slower with it.
//
// xcd_stretch: the position in the launch's tile sequence of work-group pid of T (a
// bijection of [0, T)); grouped_tile: tile u of an num_m x num_n output in grouped order.
__device__ __forceinline__ int xcd_stretch(int pid, int T) {
  constexpr int NX = 8;
  const int x = pid % NX, q = T / NX, rem = T % NX;
  return x * q + min(x, rem) + pid / NX;
}

__device__ __forceinline__ void grouped_tile(int u, int num_m, int num_n, int &mt, int &nt) {
  constexpr int GM = 4;
  const int grp = u / (GM * num_n), first_m = grp * GM;
  const int gsz = min(num_m - first_m, GM);
  const int r = u - grp * GM * num_n;
  mt = first_m + r % gsz;
  nt = r / gsz;
}

template <typename HT, int BM, int BN, int BK, int WM, int WN, bool AKC, bool BKC, int EPI, int KMODE>
__global__ __launch_bounds__(WM * WN * 64) void gemm_kernel(GemmArgs g) {
  // The K splits (grid.z) take part in the stretches: an XCD runs all the tiles of a split
  // (tile fastest in the sequence), so a split's slice of the shared operand is fetched into one
  // L2.  With the stretches over the tile plane alone, a launch of few tiles and many splits
  // (the LM-head dX of a 256-token step: 8 tiles x 32 splits) put each split's 8 tiles on the 8
  // XCDs, and every XCD fetched every slice of dlogits (933 MB read per launch for 389 MB).
  const int num_m = gridDim.y, num_n = gridDim.x, plane = num_m * num_n;
  const int u = xcd_stretch(blockIdx.x + num_n * (blockIdx.y + num_m * blockIdx.z), plane * gridDim.z);
  int mt, nt;
  grouped_tile(u % plane, num_m, num_n, mt, nt);
  gemm_body<HT, BM, BN, BK, WM, WN, AKC, BKC, EPI, KMODE>(g, mt, nt, u / plane);
}

// Several GEMMs of one shape class in one launch (the weight gradients of a layer): problem
// p owns the work-groups [first[p], first[p + 1]) of the tile sequence, which the XCDs take
// in contiguous stretches as above.  No split-K: each tile runs its whole K range.
template <typename HT, int BM, int BN, int BK, int WM, int WN, bool AKC, bool BKC, int EPI>
__global__ __launch_bounds__(WM * WN * 64) void gemm_group_kernel(GemmGroup gg) {
  const int u = xcd_stretch(blockIdx.x, gg.first[gg.n]);
  int p = 0;
  while (p + 1 < gg.n && u >= gg.first[p + 1]) p++;
  const GemmArgs &g = gg.g[p];
  int mt, nt;
  grouped_tile(u - gg.first[p], g.M / BM, g.N / BN, mt, nt);
  gemm_body<HT, BM, BN, BK, WM, WN, AKC, BKC, EPI, KM_TAIL>(g, mt, nt, 0);
}

// Ordered sum of the split-K partials (split 0 first) followed by the epilogue; four
// consecutive columns per thread.  The partials are read KS at a time (KS divides the split,
// a power of two), all KS loads issued before the first add, so a thread waits on HBM once per
// KS partials rather than once per partial.
template <typename HT, int EPI, int KS>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmArgs g) {
  const long n4 = (long)g.M * g.N / 4;
  const long slice = (long)g.M * g.N;
  bool bad = false;
  float sq = 0.f;
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n4; i += (long)gridDim.x * 256) {
    const long e = i * 4;
    float4 p[KS];
#pragma unroll
    for (int z = 0; z < KS; z++) p[z] = *(const float4 *)(g.ws + z * slice + e);
    float4 s = p[0];
#pragma unroll
    for (int z = 1; z < KS; z++) {
      s.x += p[z].x; s.y += p[z].y; s.z += p[z].z; s.w += p[z].w;
    }
    for (int z0 = KS; z0 < g.split; z0 += KS) {
#pragma unroll
      for (int z = 0; z < KS; z++) p[z] = *(const float4 *)(g.ws + (z0 + z) * slice + e);
#pragma unroll
      for (int z = 0; z < KS; z++) {
        s.x += p[z].x; s.y += p[z].y; s.z += p[z].z; s.w += p[z].w;
      }
    }
    const int row = (int)(e / g.N), col = (int)(e % g.N);
    const float o0 = store_out<HT, EPI>(g, row, col, s.x * g.alpha, bad);
    const float o1 = store_out<HT, EPI>(g, row, col + 1, s.y * g.alpha, bad);
    const float o2 = store_out<HT, EPI>(g, row, col + 2, s.z * g.alpha, bad);
    const float o3 = store_out<HT, EPI>(g, row, col + 3, s.w * g.alpha, bad);
    if constexpr (epi_sq<EPI>()) sq += o0 * o0 + o1 * o1 + o2 * o2 + o3 * o3;
  }
  flag_overflow(g.ovf, bad);
  if constexpr (epi_sq<EPI>())
    if (g.sq) block_sumsq_store<4>(sq, g.sq + blockIdx.x);
}

}  // namespace

namespace {

// Work-groups of the ordered split-K reduction of an M x N output.
int reduce_blocks(int M, int N) { return (int)std::min<long>(((long)M * N / 4 + 255) / 256, 2048); }

template <typename HT, int BM, int BN, int BK, int WM, int WN, bool AKC, bool BKC, int EPI>
int launch_t(GemmArgs g, hipStream_t s) {
  g.n_tiles = g.part_ld > 0 ? g.part_ld : g.N / BN;
  dim3 grid(g.N / BN, g.M / BM, g.split);
  if constexpr (EPI == EPI_CE_FWD || EPI == EPI_CE_BWD) {  // never split
    if ((g.K / BK) % 2 == 0)
      hipLaunchKernelGGL((gemm_kernel<HT, BM, BN, BK, WM, WN, AKC, BKC, EPI, KM_EVEN>), grid, dim3(WM * WN * 64), 0, s, g);
    else
      hipLaunchKernelGGL((gemm_kernel<HT, BM, BN, BK, WM, WN, AKC, BKC, EPI, KM_PAD>), grid, dim3(WM * WN * 64), 0, s, g);
  } else {
    hipLaunchKernelGGL((gemm_kernel<HT, BM, BN, BK, WM, WN, AKC, BKC, EPI, KM_TAIL>), grid, dim3(WM * WN * 64), 0, s, g);
  }
  NE_HIP(hipGetLastError());
  if (g.split > 1 && !g.defer_reduce) {
    if constexpr (EPI != EPI_CE_FWD && EPI != EPI_CE_BWD && EPI != EPI_SWIGLU_FWD) {
      const int blocks = reduce_blocks(g.M, g.N);
      if (g.split == 2) hipLaunchKernelGGL((splitk_reduce_kernel<HT, EPI, 2>), dim3(blocks), dim3(256), 0, s, g);
      else if (g.split == 4) hipLaunchKernelGGL((splitk_reduce_kernel<HT, EPI, 4>), dim3(blocks), dim3(256), 0, s, g);
      else if (g.split % 8 == 0) hipLaunchKernelGGL((splitk_reduce_kernel<HT, EPI, 8>), dim3(blocks), dim3(256), 0, s, g);
      else return ne_fail(NE_ERR_ARG, "gemm: split %d is not a power of two", g.split);
      NE_HIP(hipGetLastError());
    }
  }
  return 0;
}

// Block tiles: 256x256 (8 waves of 64x128), 256x128 (8 waves of 64x64), 128x128 (4 waves of
// 64x64), 64x64 (4 waves of 32x32).  The 8-wave tiles take most of a CU's LDS (one work-group
// per CU), the 4-wave tiles fit two.
enum { TILE_256 = 0, TILE_256x128 = 1, TILE_128 = 2, TILE_64 = 3 };
constexpr int tile_bm(int t) { return t == TILE_256 || t == TILE_256x128 ? 256 : t == TILE_128 ? 128 : 64; }
constexpr int tile_bn(int t) { return t == TILE_256 ? 256 : t == TILE_64 ? 64 : 128; }

template <typename HT, bool AKC, bool BKC, int EPI>
int launch_e(GemmArgs g, int tile, hipStream_t s) {
  if (tile == TILE_256) return launch_t<HT, 256, 256, 64, 4, 2, AKC, BKC, EPI>(g, s);
  if (tile == TILE_256x128) return launch_t<HT, 256, 128, 64, 4, 2, AKC, BKC, EPI>(g, s);
  if (tile == TILE_128) return launch_t<HT, 128, 128, 64, 2, 2, AKC, BKC, EPI>(g, s);
  // The 64x64 tile serves the short-token GEMMs (a 256-token step), whose K loops are bound by
  // the latency of each step's loads: steps of 128 halve the loop's trips (the forward GEMMs of
  // a 256-token Qwen3-0.6B step: 1.41 -> 1.25 ms, the backward's 2.86 -> 2.68 ms).
  if (g.K % 128 == 0) return launch_t<HT, 64, 64, 128, 2, 2, AKC, BKC, EPI>(g, s);
  return launch_t<HT, 64, 64, 64, 2, 2, AKC, BKC, EPI>(g, s);
}

template <typename HT, bool AKC, bool BKC>
int launch_l(int epi, GemmArgs g, int tile, hipStream_t s) {
  switch (epi) {
    case EPI_H16: return launch_e<HT, AKC, BKC, EPI_H16>(g, tile, s);
    case EPI_F32: return launch_e<HT, AKC, BKC, EPI_F32>(g, tile, s);
    case EPI_F32_ACC: return launch_e<HT, AKC, BKC, EPI_F32_ACC>(g, tile, s);
    case EPI_RESID: return launch_e<HT, AKC, BKC, EPI_RESID>(g, tile, s);
    case EPI_SWIGLU_BWD: return launch_e<HT, AKC, BKC, EPI_SWIGLU_BWD>(g, tile, s);
    case EPI_CE_FWD: return launch_e<HT, AKC, BKC, EPI_CE_FWD>(g, tile, s);
    case EPI_CE_BWD: return launch_e<HT, AKC, BKC, EPI_CE_BWD>(g, tile, s);
    case EPI_SWIGLU_FWD:
      if constexpr (AKC && BKC) return launch_e<HT, AKC, BKC, EPI_SWIGLU_FWD>(g, tile, s);
      return ne_fail(NE_ERR_ARG, "gemm: the SwiGLU forward epilogue takes layout 0 (A[M,K], B[N,K])");
  }
  return ne_fail(NE_ERR_ARG, "gemm: unknown epilogue %d", epi);
}

template <typename HT>
int launch_dt(int layout, int epi, GemmArgs g, int tile, hipStream_t s) {
  switch (layout) {
    case 0: return launch_l<HT, true, true>(epi, g, tile, s);
    case 1: return launch_l<HT, false, true>(epi, g, tile, s);
    case 2: return launch_l<HT, true, false>(epi, g, tile, s);
    case 3: return launch_l<HT, false, false>(epi, g, tile, s);
  }
  return ne_fail(NE_ERR_ARG, "gemm: unknown layout %d", layout);
}

// Block tile for a shape.  256x256 when that still gives a full wave of work-groups over the
// 256 CUs; 256x128 when that does (about), or when the output is small and K very long (the
// LM-head dX of a short step: split-K fills the CUs and each weight tile is read once);
// else 128x128 when that gives at least half a wave (split-K fills the rest); else 64x64.
int gemm_tile(int M, int N, int K) {
  const long t256 = (long)(M / 256) * (N / 256), t256x128 = (long)(M / 256) * (N / 128);
  const long t128 = (long)(M / 128) * (N / 128);
  if (M % 256 == 0 && N % 256 == 0 && t256 >= 256) return TILE_256;
  if (M % 256 == 0 && N % 128 == 0 && (t256x128 >= 200 || (t128 < 128 && K >= 8192))) return TILE_256x128;
  if (M % 128 == 0 && N % 128 == 0 && t128 >= 128) return TILE_128;
  return TILE_64;
}

}  // namespace

// A large output with N (or M) not a multiple of 256 — a vocabulary of 151,936 columns — runs
// as a part of whole 256-wide tiles (which then takes the 256x256 tile) and a narrow
// remainder.  Returns the width of that main part, or 0 when the shape is not split: only
// when the main part has at least four waves of 256x256 work-groups and K >= 1024 (smaller
// shapes run faster on the narrower tile, which gives twice the work-groups).
int ragged_main(int M, int N, int K) {
  const int nm = N / 256 * 256;
  if (M % 256 || N % 256 == 0 || nm == 0 || K < 1024 || (long)(M / 256) * (nm / 256) < 1024) return 0;
  return nm;
}

int gemm_ce_tiles(int M, int N, int K) {
  const int nm = ragged_main(M, N, K);
  if (!nm) return N / tile_bn(gemm_tile(M, N, K));
  return nm / 256 + (N - nm) / tile_bn(gemm_tile(M, N - nm, K));
}

void gemm_ce_layout(int M, int N, int K, int *main_cols, int *w_main, int *w_rest) {
  const int nm = ragged_main(M, N, K);
  *main_cols = nm ? nm : N;
  *w_main = nm ? 256 : tile_bn(gemm_tile(M, N, K));
  *w_rest = nm ? tile_bn(gemm_tile(M, N - nm, K)) : *w_main;
}

bool gemm_ce_piece_ok(int M, int N, int K, int c0, int c1) {
  if (c0 == 0 && c1 == N) return true;
  if (ragged_main(M, N, K) || c0 < 0 || c1 > N || c0 >= c1) return false;
  const int tile = gemm_tile(M, N, K), bn = tile_bn(tile), w = c1 - c0;
  return c0 % bn == 0 && w % bn == 0 && gemm_tile(M, w, K) == tile && !ragged_main(M, w, K);
}

int gemm_ce_pieces(int M, int N, int K, int max_pieces, int *cut) {
  cut[0] = 0;
  cut[1] = N;
  if (max_pieces < 2 || ragged_main(M, N, K)) return 1;
  const int tile = gemm_tile(M, N, K), bn = tile_bn(tile);
  const int per = tile == TILE_256 || tile == TILE_256x128 ? 256 : 512;  // 8-wave tiles: one per CU
  const int np = std::min(max_pieces, N / bn / per);
  if (np < 2) return 1;
  for (int k = 0; k < np; k++) {
    cut[k + 1] = k + 1 < np ? (k + 1) * per * bn : N;
    if (!gemm_ce_piece_ok(M, N, K, cut[k], cut[k + 1])) {
      cut[1] = N;
      return 1;
    }
  }
  return np;
}

bool gemm_group_fits(const GemmArgs *g, int n) {
  if (n < 1 || n > GEMM_GROUP_MAX) return false;
  long tiles = 0;
  for (int i = 0; i < n; i++) {
    if (g[i].M <= 0 || g[i].N <= 0 || g[i].M % 256 || g[i].N % 256 || g[i].K < 8192 || g[i].K % 64) return false;
    tiles += (long)(g[i].M / 256) * (g[i].N / 256);
  }
  return tiles >= 192 && tiles < (1L << 30);
}

int gemm_group_launch(int dt, int epi, const GemmArgs *g, int n, hipStream_t s) {
  if (!gemm_group_fits(g, n)) return ne_fail(NE_ERR_ARG, "gemm group: shapes do not take the grouped path");
  if (epi != EPI_F32 && epi != EPI_F32_ACC) return ne_fail(NE_ERR_ARG, "gemm group: epilogue %d", epi);
  if (dt != 0 && dt != 1) return ne_fail(NE_ERR_ARG, "gemm: unknown 16-bit format %d", dt);
  GemmGroup gg = {};
  gg.n = n;
  gg.first[0] = 0;
  for (int i = 0; i < n; i++) {
    if ((g[i].lda % 8) || (g[i].ldb % 8) || (((uintptr_t)g[i].A | (uintptr_t)g[i].B) & 15))
      return ne_fail(NE_ERR_ARG, "gemm: operands need 16-byte aligned rows (ld %% 8 == 0)");
    gg.g[i] = g[i];
    gg.g[i].split = 1;
    gg.g[i].n_tiles = g[i].N / 256;
    gg.first[i + 1] = gg.first[i] + (g[i].M / 256) * (g[i].N / 256);
  }
  const dim3 grid(gg.first[n]), block(512);
  if (dt == 0) {
    if (epi == EPI_F32) hipLaunchKernelGGL((gemm_group_kernel<H16B, 256, 256, 64, 4, 2, false, false, EPI_F32>), grid, block, 0, s, gg);
    else hipLaunchKernelGGL((gemm_group_kernel<H16B, 256, 256, 64, 4, 2, false, false, EPI_F32_ACC>), grid, block, 0, s, gg);
  } else {
    if (epi == EPI_F32) hipLaunchKernelGGL((gemm_group_kernel<H16F, 256, 256, 64, 4, 2, false, false, EPI_F32>), grid, block, 0, s, gg);
    else hipLaunchKernelGGL((gemm_group_kernel<H16F, 256, 256, 64, 4, 2, false, false, EPI_F32_ACC>), grid, block, 0, s, gg);
  }
  NE_HIP(hipGetLastError());
  return 0;
}

// Block tile and K splits of a shape (ws_elems < 0: no workspace, no split).  The cross-entropy
// and SwiGLU-forward epilogues never split (they need whole sums in the tile).
static void plan(int epi, int M, int N, int K, long ws_elems, int &tile, int &split) {
  const bool nosplit_ok = epi != EPI_CE_FWD && epi != EPI_CE_BWD && epi != EPI_SWIGLU_FWD;
  tile = gemm_tile(M, N, K);
  // A long reduction into a small output (the weight gradients of a long step: K = tokens)
  // takes the 256x256 tile too when split-K can give it a full wave of work-groups: its higher
  // MFMA rate outweighs writing and summing the fp32 partials (a few % of the GEMM's time).
  if (ws_elems >= 0 && nosplit_ok && tile != TILE_256 && M % 256 == 0 && N % 256 == 0 &&
      K >= 8192) {
    const long t256 = (long)(M / 256) * (N / 256);
    int sp = 1;
    while (t256 * sp < 256 && sp < 8 && (K / 64) / (sp * 2) >= 4 && (long)M * N * sp * 2 <= ws_elems) sp *= 2;
    if (t256 * sp >= 256) tile = TILE_256;
  }
  // split K while too few work-groups would run (8-wave tiles: fewer than one per CU;
  // 4-wave tiles: fewer than 3/4 of the CUs), keeping >= 4 K steps per split.  Each split
  // adds an fp32 partial output to write and read back: at 256 tokens the partials of a
  // layer's GEMMs outweighed its weights at two work-groups per CU (target 512: 8.84 ms per
  // Qwen3-0.6B step, 256: 8.64, 192: 8.54, 128: 9.25).
  split = 1;
  if (ws_elems >= 0 && nosplit_ok) {
    const long tiles = (long)(M / tile_bm(tile)) * (N / tile_bn(tile));
    const long target = tile_bm(tile) == 256 ? 256 : 192;
    const int nkt = K / 64;
    while (tiles * split < target && nkt / (split * 2) >= 4 && split < 64 &&
           (long)M * N * split * 2 <= ws_elems)
      split *= 2;
  }
}

int gemm_splits(int epi, int M, int N, int K, long ws_elems) {
  int tile, split;
  plan(epi, M, N, K, ws_elems, tile, split);
  return split;
}

long gemm_sq_parts(int epi, int M, int N, int K, long ws_elems) {
  // the same ragged splits as gemm_launch (EPI_F32 / EPI_F32_ACC take both)
  if (const int nm = ragged_main(M, N, K))
    return gemm_sq_parts(epi, M, nm, K, ws_elems) + gemm_sq_parts(epi, M, N - nm, K, ws_elems);
  if (const int mm = ragged_main(N, M, K))
    return gemm_sq_parts(epi, mm, N, K, ws_elems) + gemm_sq_parts(epi, M - mm, N, K, ws_elems);
  int tile, split;
  plan(epi, M, N, K, ws_elems, tile, split);
  if (split > 1) return reduce_blocks(M, N);
  return (long)(M / tile_bm(tile)) * (N / tile_bn(tile));
}

int gemm_launch(int dt, int layout, int epi, GemmArgs g, hipStream_t s, int *split_out) {
  if (g.M <= 0 || g.N <= 0 || g.K <= 0 || g.M % 64 || g.N % 64 || g.K % 64)
    return ne_fail(NE_ERR_ARG, "gemm: M=%d N=%d K=%d must be positive multiples of 64", g.M, g.N, g.K);
  if ((g.lda % 8) || (g.ldb % 8) || (((uintptr_t)g.A | (uintptr_t)g.B) & 15))
    return ne_fail(NE_ERR_ARG, "gemm: operands need 16-byte aligned rows (ld %% 8 == 0)");
  if (dt != 0 && dt != 1) return ne_fail(NE_ERR_ARG, "gemm: unknown 16-bit format %d", dt);
  if (epi == EPI_SWIGLU_BWD && ((g.ldr % 8) || (g.ldc % 8) || (((uintptr_t)g.R | (uintptr_t)g.C) & 15)))
    return ne_fail(NE_ERR_ARG, "gemm: the SwiGLU backward epilogue needs 16-byte aligned h13 / dh13 rows");
  if (epi == EPI_CE_BWD && ((g.ldc % 8) || ((uintptr_t)g.C & 15)))
    return ne_fail(NE_ERR_ARG, "gemm: the cross-entropy backward needs 16-byte aligned dlogits rows");
  if (epi == EPI_SWIGLU_FWD && (!g.C || !g.C2 || g.ldc < g.N || g.ldc2 < g.N / 2 || g.N % 128))
    return ne_fail(NE_ERR_ARG, "gemm: the SwiGLU forward needs h13 [M,N] and gate [M,N/2] outputs, N %% 128 == 0");
  // ragged shapes: the main part of whole 256-wide tiles, then the rest (see ragged_main)
  if (epi != EPI_SWIGLU_BWD && epi != EPI_SWIGLU_FWD && !g.defer_reduce) {
    const size_t ce = epi == EPI_H16 || epi == EPI_CE_BWD || epi == EPI_CE_FWD ? 2 : 4;  // C element size
    if (const int nm = ragged_main(g.M, g.N, g.K)) {  // split the columns
      GemmArgs a = g, b = g;
      a.N = nm;
      b.N = g.N - nm;
      b.B = (const h16_t *)g.B + ((layout & 2) ? (long)nm : (long)nm * g.ldb);
      if (g.C) b.C = (char *)g.C + nm * ce;
      if (g.R) b.R = (const float *)g.R + nm;
      if (g.sq) b.sq = g.sq + gemm_sq_parts(epi, a.M, a.N, a.K, g.ws ? g.ws_elems : -1);
      b.col0 = g.col0 + nm;
      if (epi == EPI_CE_FWD) {
        a.part_ld = b.part_ld = g.part_ld > 0 ? g.part_ld : gemm_ce_tiles(g.M, g.N, g.K);
        b.tile0 = g.tile0 + nm / 256;
      }
      NE_CHECK(gemm_launch(dt, layout, epi, a, s, split_out));
      return gemm_launch(dt, layout, epi, b, s, nullptr);
    }
    if (epi != EPI_CE_FWD && epi != EPI_CE_BWD)
      if (const int mm = ragged_main(g.N, g.M, g.K)) {  // split the rows
        GemmArgs a = g, b = g;
        a.M = mm;
        b.M = g.M - mm;
        b.A = (const h16_t *)g.A + ((layout & 1) ? (long)mm : (long)mm * g.lda);
        if (g.C) b.C = (char *)g.C + (size_t)mm * g.ldc * ce;
        if (g.R) b.R = (const float *)g.R + (long)mm * g.ldr;
        if (g.sq) b.sq = g.sq + gemm_sq_parts(epi, a.M, a.N, a.K, g.ws ? g.ws_elems : -1);
        NE_CHECK(gemm_launch(dt, layout, epi, a, s, split_out));
        return gemm_launch(dt, layout, epi, b, s, nullptr);
      }
  }
  int tile, split;
  plan(epi, g.M, g.N, g.K, g.ws ? g.ws_elems : -1, tile, split);
  g.split = split;
  if (split_out) *split_out = g.split;
  return DISPATCH_H16(dt, launch_dt<HT>(layout, epi, g, tile, s));
}
