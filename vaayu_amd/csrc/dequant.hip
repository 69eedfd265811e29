// Whole-blob dequant: the packed codes of one expert (all roles, one flat stream) to dense
// weights, bit-exact with `_fused_dequant_kernel` (vaayu/moe_patch.py:750-769):
//   out[i] = round_out((code_i - 2^(bits-1)) * round_out(scale[i / group]))
// The code offset is subtracted exactly in integers and the product is formed in fp32
// (exact for bf16 / fp16 outputs; the fp32 output's own rounding for fp32), then rounded
// once to the output dtype. Each thread takes one 16-byte unit (4 words): one 16-byte code
// load, one scale load per word (a group holds whole words), and its 4 * 32/bits outputs
// leave as 16-byte stores. HBM-bound: per word 4 code bytes in, 32/bits outputs out.
#include "common.hpp"
#include "abi_internal.hpp"

namespace vaayu {

__device__ __forceinline__ float load_sc(const void* p, int64_t i, int dt) {
  if (dt == DT_BF16) return load_as_float<DT_BF16>(p, i);
  if (dt == DT_FP16) return load_as_float<DT_FP16>(p, i);
  return load_as_float<DT_FP32>(p, i);
}

// Output element type of dtype code OUT.
template <int OUT> struct OutT { typedef uint16_t type; };
template <> struct OutT<DT_FP32> { typedef float type; };

template <int OUT>
__device__ __forceinline__ typename OutT<OUT>::type out_bits(float v) {
  if constexpr (OUT == DT_BF16) return __builtin_bit_cast(uint16_t, (__bf16)v);
  else if constexpr (OUT == DT_FP16) return __builtin_bit_cast(uint16_t, (_Float16)v);
  else return v;
}

template <int BITS, int OUT>
__global__ void __launch_bounds__(256)
dequant_kernel(const int32_t* __restrict__ packed, const void* __restrict__ scale, int sc_dt,
               void* __restrict__ out, int64_t n_words, int group) {
  constexpr int PER = 32 / BITS;                        // codes per word
  constexpr uint32_t mask = (1u << BITS) - 1u;
  typedef typename OutT<OUT>::type T;
  constexpr int PER_VEC = 16 / sizeof(T);               // outputs per 16-byte store
  const int64_t w0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (w0 >= n_words) return;
  const int nw = n_words - w0 >= 4 ? 4 : (int)(n_words - w0);
  uint32_t w[4] = {0u, 0u, 0u, 0u};
  float s[4];
  if (nw == 4) {
    const uint4 v = *(const uint4*)(packed + w0);       // w0 * 4 bytes: 16-byte aligned
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else {
    for (int i = 0; i < nw; ++i) w[i] = (uint32_t)packed[w0 + i];
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    s[i] = round_act<OUT>(load_sc(scale, (i < nw ? w0 + i : w0) * PER / group, sc_dt));
  T vals[4 * PER];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int c = (int)((w[i] >> (j * BITS)) & mask) - (1 << (BITS - 1));
      vals[i * PER + j] = out_bits<OUT>((float)c * s[i]);
    }
  T* dst = (T*)out + w0 * PER;
  if (nw == 4) {                                        // 4 * PER * sizeof(T) is a multiple of 16
#pragma unroll
    for (int v = 0; v < 4 * PER / PER_VEC; ++v)
    {
      uint4 chunk;
      __builtin_memcpy(&chunk, vals + v * PER_VEC, 16);
      *(uint4*)(dst + v * PER_VEC) = chunk;
    }
  } else {
    for (int e = 0; e < nw * PER; ++e) dst[e] = vals[e];
  }
}

}  // namespace vaayu

using namespace vaayu;

extern "C" int vaayu_dequant_blob(const int32_t* packed, const void* scale, int32_t scale_dtype,
                                  void* out, int32_t out_dtype, int64_t n_words, int32_t bits,
                                  int32_t group, void* stream) {
  clear_error();
  if (!packed || !scale || !out) return set_error(-1, "null pointer argument");
  if (n_words <= 0) return set_error(-1, "n_words must be positive");
  if (bits != 1 && bits != 2 && bits != 4 && bits != 8) return set_error(-2, "bit width");
  if (group <= 0 || group % (32 / bits)) return set_error(-2, "group size");
  if (scale_dtype < 0 || scale_dtype > 2 || out_dtype < 0 || out_dtype > 2)
    return set_error(-1, "dtype code");
  if (((uintptr_t)packed & 15) || ((uintptr_t)out & 15))
    return set_error(-2, "codes and output must start on 16 bytes");
  const int64_t units = (n_words + 3) / 4;
  const dim3 grid((unsigned)((units + 255) / 256)), block(256);
  hipStream_t st = (hipStream_t)stream;
#define DQ(B_, O_)                                                                         \
  hipLaunchKernelGGL((dequant_kernel<B_, O_>), grid, block, 0, st, packed, scale, scale_dtype, \
                     out, n_words, group)
#define BYOUT(B_)                          \
  if (out_dtype == DT_BF16) DQ(B_, DT_BF16); \
  else if (out_dtype == DT_FP16) DQ(B_, DT_FP16); \
  else DQ(B_, DT_FP32);
  if (bits == 4) { BYOUT(4) }
  else if (bits == 8) { BYOUT(8) }
  else if (bits == 2) { BYOUT(2) }
  else { BYOUT(1) }
#undef BYOUT
#undef DQ
  return check_launch("dequant blob");
}
