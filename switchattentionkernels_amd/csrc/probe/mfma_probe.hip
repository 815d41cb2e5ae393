// Measurement probe for gfx950, built as its own library (libswattn_probe.so)
// and used only by bench.py: the bf16 MFMA rate this chip sustains with
// nothing but v_mfma_f32_32x32x16_bf16 in flight (operands in registers, no
// memory traffic, two waves per SIMD).  The attention kernel's fraction of
// this rate separates scheduling losses from the clock the chip holds under a
// full matrix-core load, which is below the one the published peak assumes.
// It is not part of the attention library's ABI (include/swattn.h).
//
//   int swattn_mfma_peak(int64_t iters, int32_t blocks, float* out, void* stream)
//     blocks workgroups of 256 threads, each wave iters rounds of 8 MFMAs;
//     out: blocks * 256 floats (written so the work is not optimised away).
//     Returns 0, -1 for a bad argument, or a positive hipError_t.

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace swattn {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Each wave: iters rounds of 8 MFMAs over four independent accumulators.
__global__ __launch_bounds__(256) void mfma_peak_kernel(int64_t iters, float seed, float* out) {
  const int lane = threadIdx.x & 63;
  bf16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = static_cast<__bf16>(seed * static_cast<float>(i + 1));
    b[i] = static_cast<__bf16>(seed + static_cast<float>(lane));
  }
  f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int64_t it = 0; it < iters; ++it) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c3, 0, 0, 0);
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c3, 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += c0[i] + c1[i] + c2[i] + c3[i];
  out[static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = s;
}

}  // namespace
}  // namespace swattn

using namespace swattn;

extern "C" int swattn_mfma_peak(int64_t iters, int32_t blocks, float* out, void* stream) {
  if (iters < 1 || blocks < 1 || out == nullptr) return -1;
  hipLaunchKernelGGL(mfma_peak_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), iters, 1e-3f, out);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : static_cast<int>(e);
}
