// MFMA issue ceiling (a measurement kernel, not part of the training step).
//
// Each wave runs 8 independent accumulator chains of one MFMA shape on register operands,
// with no memory traffic, so the kernel's duration against its flop count gives the rate
// the matrix cores sustain for that shape and format on this device: the denominator of
// the MFMA utilisation figures quoted for the GEMM and attention kernels.
//
// Built with the MFMA VGPR form (as the attention kernels are): with accumulators in AGPRs
// the compiler rotates the 16x16x32 chains through v_accvgpr copies every iteration, and
// the kernel then measures those copies rather than the matrix cores.
#include <type_traits>

#include "common.h"
#include "ne_internal.h"

namespace {

template <typename HT, bool BIG>
__global__ __launch_bounds__(256) void mfma_ceiling_kernel(float *out, int iters) {
  constexpr int CH = 8;
  typedef typename std::conditional<BIG, f32x16, f32x4>::type acc_t;
  constexpr int NE = BIG ? 16 : 4;
  u16x8 ra, rb;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    ra[i] = HT::h(0.001f * (float)(threadIdx.x & 63) + 0.01f * i);
    rb[i] = HT::h(0.5f - 0.01f * i);
  }
  const typename HT::v8 a = HT::op(ra), b = HT::op(rb);
  acc_t acc[CH];
#pragma unroll
  for (int c = 0; c < CH; c++)
#pragma unroll
    for (int e = 0; e < NE; e++) acc[c][e] = 0.f;
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int c = 0; c < CH; c++) {
      if constexpr (BIG) acc[c] = HT::mfma32(a, b, acc[c]);
      else acc[c] = HT::mfma16(a, b, acc[c]);
    }
  }
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < CH; c++)
#pragma unroll
    for (int e = 0; e < NE; e++) sum += acc[c][e];
  out[(long)blockIdx.x * 256 + threadIdx.x] = sum;
}

}  // namespace

int launch_mfma_ceiling(int dt, int shape, int blocks, int iters, float *out, hipStream_t s) {
  if (blocks <= 0 || iters <= 0 || (shape != 0 && shape != 1))
    return ne_fail(NE_ERR_ARG, "mfma_ceiling: blocks=%d iters=%d shape=%d", blocks, iters, shape);
  if (dt != 0 && dt != 1) return ne_fail(NE_ERR_ARG, "mfma_ceiling: unknown 16-bit format %d", dt);
  return DISPATCH_H16(dt, [&] {
    if (shape == 0) hipLaunchKernelGGL((mfma_ceiling_kernel<HT, true>), dim3(blocks), dim3(256), 0, s, out, iters);
    else hipLaunchKernelGGL((mfma_ceiling_kernel<HT, false>), dim3(blocks), dim3(256), 0, s, out, iters);
    return ne_hip_status(hipGetLastError(), "mfma_ceiling");
  }());
}
