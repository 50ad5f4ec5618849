// Shared device helpers for the gfx950 kernels: 16-bit storage types, MFMA operand
// vectors, 64-lane wavefront reductions.
//
// Activations and the weight shadow are 16-bit, stored as raw uint16 bit patterns and
// bit-cast to the MFMA operand vectors at the instruction boundary.  The 16-bit format is
// a per-context choice: IEEE fp16 (default for training: 10-bit mantissa, 8x finer than
// bf16, same MFMA rate on gfx950; gradients carry a power-of-two scale to stay in range)
// or bf16.  Kernels are templated on a format tag (H16F / H16B).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint16_t h16_t;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

#define NE_WAVE 64

// bf16 format tag
struct H16B {
  static constexpr int id = 0;
  typedef bf16x8 v8;
  __device__ static __forceinline__ float f(h16_t h) { return __uint_as_float(((uint32_t)h) << 16); }
  // round to nearest even (finite inputs)
  __device__ static __forceinline__ h16_t h(float x) {
    uint32_t u = __float_as_uint(x);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (h16_t)(u >> 16);
  }
  __device__ static __forceinline__ bool bad(h16_t v) { return (v & 0x7F80u) == 0x7F80u; }
  __device__ static __forceinline__ v8 op(const u16x8 &v) { return __builtin_bit_cast(v8, v); }
  __device__ static __forceinline__ f32x16 mfma32(const v8 &a, const v8 &b, const f32x16 &c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ f32x4 mfma16(const v8 &a, const v8 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

// IEEE fp16 format tag
struct H16F {
  static constexpr int id = 1;
  typedef f16x8 v8;
  __device__ static __forceinline__ float f(h16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
  __device__ static __forceinline__ h16_t h(float x) { return __builtin_bit_cast(h16_t, (_Float16)x); }
  // inf or nan after conversion (|x| beyond the fp16 range)
  __device__ static __forceinline__ bool bad(h16_t v) { return (v & 0x7C00u) == 0x7C00u; }
  __device__ static __forceinline__ v8 op(const u16x8 &v) { return __builtin_bit_cast(v8, v); }
  __device__ static __forceinline__ f32x16 mfma32(const v8 &a, const v8 &b, const f32x16 &c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ f32x4 mfma16(const v8 &a, const v8 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// SwiGLU gate silu(h1) * h3 of two 16-bit values, rounded to fp32 and then to 16 bits.  The
// compiler may fuse the product and the 16-bit rounding into one mixed-precision FMA (a single
// rounding), in some kernels and not in others; the empty asm holds the fp32 product in a
// register so that every kernel computing the gate gets the same bits.
template <typename HT>
__device__ __forceinline__ h16_t swiglu_gate(h16_t a, h16_t b) {
  const float h1 = HT::f(a), h3 = HT::f(b);
  float g = h1 / (1.f + __expf(-h1)) * h3;
  asm volatile("" : "+v"(g));
  return HT::h(g);
}

// Dispatch a templated launcher on the runtime format id: DISPATCH_H16(dt, fn<HT>(args)).
#define DISPATCH_H16(dt, ...)            \
  ((dt) == 1 ? [&] { using HT = H16F; return __VA_ARGS__; }() \
             : [&] { using HT = H16B; return __VA_ARGS__; }())

// Raise a device overflow flag (non-finite 16-bit result) once per thread.
// Barrier that orders LDS only: waits for this wave's LDS operations, not for the global
// loads still in flight (they stay in flight across it).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ void flag_overflow(int *ovf, bool bad) {
  if (ovf && bad) *ovf = 1;
}


__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Reductions over the 32 lanes of a half-wave (lanes sharing lane / 32) as an xor butterfly
// of strides 1, 2, 4, 8, 16, every lane left with the same result: the first four strides as DPP
// operands of the VALU (quad permutations for 1 and 2; then, the value being uniform over each
// quad and then over each 8-lane half-row, the half-row and row mirrors pair the same groups as
// xor 4 and xor 8), the last as one swizzle (xor 16 inside 32 lanes).  Cross-lane permutes
// through LDS (ds_bpermute) for all five strides cost the cross-entropy forward epilogue
// 160 permutes per lane per pass.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float swizzle_xor16(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}
__device__ __forceinline__ float half_wave_sum(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]: xor 1
  v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]: xor 2
  v += dpp_mov<0x141>(v);  // row_half_mirror
  v += dpp_mov<0x140>(v);  // row_mirror
  return v + swizzle_xor16(v);
}
__device__ __forceinline__ float half_wave_max(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));
  v = fmaxf(v, dpp_mov<0x4E>(v));
  v = fmaxf(v, dpp_mov<0x141>(v));
  v = fmaxf(v, dpp_mov<0x140>(v));
  return fmaxf(v, swizzle_xor16(v));
}

// The same butterfly over all 64 lanes (one LDS permute for the last stride, 32).
__device__ __forceinline__ float wave_sum(float v) {
  v = half_wave_sum(v);
  return v + __shfl_xor(v, 32, 64);
}
__device__ __forceinline__ float wave_max(float v) {
  v = half_wave_max(v);
  return fmaxf(v, __shfl_xor(v, 32, 64));
}

// The same butterfly over aligned groups of W lanes (W = 8, 16, 32 or 64), the sum left in
// every lane of the group: the same partial sums added in the same order as the xor-shuffle
// butterfly of strides 1 .. W/2, so the same bits.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(W == 8 || W == 16 || W == 32 || W == 64, "group_sum: 8, 16, 32 or 64 lanes");
  if constexpr (W == 64) return wave_sum(v);
  if constexpr (W == 32) return half_wave_sum(v);
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x141>(v);
  if constexpr (W == 16) v += dpp_mov<0x140>(v);
  return v;
}

// Reductions over the 4 lane groups {l, l^16, l^32, l^48} (lanes sharing l % 16).
__device__ __forceinline__ float quad16_sum(float v) {
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}
__device__ __forceinline__ float quad16_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  v = fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}

// One element of AdamW (TD/cpu_ops.h:266-303) with bias-corrected moments, every product and
// sum written out (explicit fmaf, no contraction left to the compiler): the result does not
// depend on how a kernel that inlines it is scheduled.
struct AdamConst {
  float gs, b1, b2, ob1, ob2, ibc1, ibc2, lr, eps;
  __device__ __forceinline__ AdamConst(const float *gscale, float b1_, float b2_, float bc1, float bc2, float lr_,
                                       float eps_)
      : gs(gscale[0]), b1(b1_), b2(b2_), ob1(1.f - b1_), ob2(1.f - b2_), ibc1(1.f / bc1), ibc2(1.f / bc2),
        lr(lr_), eps(eps_) {}
};
__device__ __forceinline__ void adam_elem(const AdamConst &k, float &p, float g, float &m, float &v, float wd) {
  const float gg = g * k.gs;
  m = fmaf(k.b1, m, k.ob1 * gg);
  v = fmaf(k.b2, v, k.ob2 * (gg * gg));
  const float mh = m * k.ibc1, vh = v * k.ibc2;
  const float u = mh / (sqrtf(vh) + k.eps);
  p = fmaf(-k.lr, fmaf(wd, p, u), p);
}
