// Measurement only: the bf16 matrix-core rate this device sustains, for the benchmark's
// MFMA-utilisation figures (no counterpart in the reference).
//
// Every wave issues `iters` rounds of 16 independent v_mfma_f32_16x16x32_bf16 (the
// instruction the prefill kernels use), operands in registers, no memory traffic inside
// the loop; 16 chains cover the instruction's dependent-issue latency. Each lane writes the
// sum of its accumulators so the work is not removed. FLOPs per launch:
// blocks * 4 waves * iters * 16 * 16384.
#include "common.hpp"
#include "abi_internal.hpp"

namespace vaayu {

constexpr int kProbeChains = 16;

__global__ void __launch_bounds__(256) probe_mfma_kernel(float* __restrict__ out, int iters) {
  const uint32_t seed = opaque(threadIdx.x * 2654435761u + blockIdx.x);
  uint4 av = make_uint4(seed & 0x3F803F80u, seed | 0x3C003C00u, 0x3F003F00u, seed ^ 0x3E003E00u);
  uint4 bv = make_uint4(0x3F803F80u, seed & 0x3D003D00u, seed | 0x3B003B00u, 0x3F403F40u);
  av.x = opaque(av.x); bv.x = opaque(bv.x);
  const bf16x8 a = __builtin_bit_cast(bf16x8, av);
  const bf16x8 b = __builtin_bit_cast(bf16x8, bv);
  f32x4 acc[kProbeChains];
#pragma unroll
  for (int c = 0; c < kProbeChains; ++c) acc[c] = (f32x4){0.f, 0.f, 0.f, 0.f};
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int c = 0; c < kProbeChains; ++c)
      acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[c], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < kProbeChains; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
  out[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

}  // namespace vaayu

using namespace vaayu;

extern "C" int vaayu_probe_mfma(float* out, int32_t blocks, int32_t iters, void* stream) {
  clear_error();
  if (!out) return set_error(-1, "null pointer argument");
  if (blocks <= 0 || iters <= 0) return set_error(-1, "blocks / iters must be positive");
  hipLaunchKernelGGL(probe_mfma_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, out, iters);
  return check_launch("mfma probe");
}
