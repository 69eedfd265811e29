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

// The fp32 sums D = A B^T of the prefill kernels' MFMA sequence, for measuring their
// accumulation error against exact sums: one wave per 16x16 tile of D, lane (q, m) holding
// row m of A and of B; per K step of 128, MFMA i of quarter q takes elements
// [step + 32q + 8i, +8), the slot map of the prefill K loop, so each output accumulates
// the same products in the same 32-product groups and order as the prefill GEMMs.
__global__ void __launch_bounds__(64) probe_mfma_sum_kernel(const uint16_t* __restrict__ a,
                                                            const uint16_t* __restrict__ b,
                                                            float* __restrict__ d, int k,
                                                            int col_tiles) {
  const int rt = blockIdx.x / col_tiles, ct = blockIdx.x % col_tiles;
  const int q = threadIdx.x >> 4, m = threadIdx.x & 15;
  const uint16_t* ar = a + (int64_t)(rt * 16 + m) * k + 32 * q;
  const uint16_t* br = b + (int64_t)(ct * 16 + m) * k + 32 * q;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < k; k0 += 128) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 av = *(const uint4*)(ar + k0 + 8 * i);
      const uint4 bv = *(const uint4*)(br + k0 + 8 * i);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av),
                                                    __builtin_bit_cast(bf16x8, bv), acc, 0, 0, 0);
    }
  }
  const int cols = col_tiles * 16;
#pragma unroll
  for (int i = 0; i < 4; ++i) d[(int64_t)(rt * 16 + 4 * q + i) * cols + ct * 16 + m] = acc[i];
}

}  // namespace vaayu

using namespace vaayu;

extern "C" int vaayu_probe_mfma_sum(const void* a, const void* b, float* d, int32_t k,
                                    int32_t row_tiles, int32_t col_tiles, void* stream) {
  clear_error();
  if (!a || !b || !d) return set_error(-1, "null pointer argument");
  if (((uintptr_t)a | (uintptr_t)b) & 15) return set_error(-2, "a and b must be 16-byte aligned");
  if (k <= 0 || k % 128) return set_error(-2, "K must be a positive multiple of 128");
  if (row_tiles <= 0 || col_tiles <= 0 || (int64_t)row_tiles * col_tiles > 0x7FFFFFFF)
    return set_error(-2, "bad tile counts");
  hipLaunchKernelGGL(probe_mfma_sum_kernel, dim3((unsigned)(row_tiles * col_tiles)), dim3(64),
                     0, (hipStream_t)stream, (const uint16_t*)a, (const uint16_t*)b, d, k,
                     col_tiles);
  return check_launch("mfma sum probe");
}

extern "C" int vaayu_probe_mfma(float* out, int32_t blocks, int32_t iters, void* stream) {
  clear_error();
  if (!out) return set_error(-1, "null pointer argument");
  if (blocks <= 0 || iters <= 0) return set_error(-1, "blocks / iters must be positive");
  hipLaunchKernelGGL(probe_mfma_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, out, iters);
  return check_launch("mfma probe");
}
