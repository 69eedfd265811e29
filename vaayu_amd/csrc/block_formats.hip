// Non-int expert formats: FP8 e4m3 with block scales, and microscaled (MX) e2m1 / e4m3
// with one e8m0 scale per 32 elements along a row. Elementwise, HBM-bound: each thread
// turns one 16-byte load of codes into the dequantized values and writes them with 16-byte
// stores.
//
// Replaces:
//   dequantize_block_scaled (vaayu/model_code/deepseek_v4/modeling_deepseek_v4.py:228-240)
//     W[i, j] = out(fp32(w[i, j]) * fp32(scale[i / bo, j / bi]))
//   upcast_from_mxfp_torch / _upcast_from_mxfp (vendor gpt_oss_triton_kernels
//   numerics_details/mxfp.py:256-299, mxfp_details/_upcast_from_mxfp.py:8-122)
//     W[r, k] = out(fp32(q[r, k]) * 2^(s[r, k / 32] - 127)), the scale being the fp32 with
//     exponent bits s (so s = 0 gives 0), and s = 0xFF giving NaN
//   (fp32 product rounded once, then one rounding to the output dtype).
#include "abi_internal.hpp"
#include "common.hpp"

namespace vaayu {

enum { FMT_E2M1 = 0, FMT_E4M3 = 1 };
enum { SC_BF16 = 0, SC_FP16 = 1, SC_FP32 = 2, SC_E8M0 = 3 };

template <int SC>
__device__ __forceinline__ float load_scale(const void* p, int64_t i) {
  if constexpr (SC == SC_E8M0) return e8m0_to_f32(((const uint8_t*)p)[i]);
  else if constexpr (SC == SC_FP32) return ((const float*)p)[i];
  else if constexpr (SC == SC_BF16) return load_as_float<DT_BF16>(p, i);
  else return load_as_float<DT_FP16>(p, i);
}

// 16 fp32 values -> the output dtype, stored at out + i (16-byte aligned when OUT != fp32 or
// i % 4 == 0).
template <int OUT>
__device__ __forceinline__ void store16(void* out, int64_t i, const float (&v)[16]) {
  if constexpr (OUT == DT_FP32) {
    float4* o = (float4*)((float*)out + i);
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
  } else {
    uint32_t w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if constexpr (OUT == DT_BF16)
        w[k] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){v[2 * k], v[2 * k + 1]}, bf16x2));
      else
        w[k] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){v[2 * k], v[2 * k + 1]}, f16x2));
    }
    uint4* o = (uint4*)((uint16_t*)out + i);
    o[0] = make_uint4(w[0], w[1], w[2], w[3]);
    o[1] = make_uint4(w[4], w[5], w[6], w[7]);
  }
}

// FP8 block dequant: one thread per 16 codes of a row. cols % 16 == 0, bi % 16 == 0.
template <int SC, int OUT>
__global__ void __launch_bounds__(256)
fp8_block_kernel(const uint4* __restrict__ w, const void* __restrict__ scale, void* __restrict__ out,
                 uint32_t rows, uint32_t u_row, uint32_t bo, uint32_t bi16, uint32_t s_cols) {
  const uint32_t row = blockIdx.y;
  const uint32_t u = blockIdx.x * 256 + threadIdx.x;   // 16-code unit within the row
  if (u >= u_row || row >= rows) return;
  const int64_t idx = (int64_t)row * u_row + u;
  const uint4 q = w[idx];
  const float s = load_scale<SC>(scale, (int64_t)(row / bo) * s_cols + u / bi16);
  const uint32_t words[4] = {q.x, q.y, q.z, q.w};
  float v[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) v[k] = e4m3_to_f32((words[k >> 2] >> (8 * (k & 3))) & 0xFFu) * s;
  store16<OUT>(out, idx * 16, v);
}

// MX upcast: one thread per group of 32 elements of a row (one e8m0 scale). When the row
// length is a multiple of 32 a group is read with 16-byte loads (e2m1: one, e4m3: two) and
// written with 16-byte stores; otherwise element by element.
template <int FMT, int OUT>
__global__ void __launch_bounds__(256)
mx_upcast_kernel(const uint8_t* __restrict__ q, const uint8_t* __restrict__ scale,
                 void* __restrict__ out, uint32_t rows, uint32_t k, uint32_t q_row,
                 uint32_t groups) {
  const uint32_t row = blockIdx.y;
  const uint32_t gi = blockIdx.x * 256 + threadIdx.x;
  if (gi >= groups || row >= rows) return;
  const float s = e8m0_to_f32(scale[(int64_t)row * groups + gi]);
  const uint8_t* qr = q + (int64_t)row * q_row;
  const int64_t o0 = (int64_t)row * k + (int64_t)gi * 32;
  const uint32_t e0 = gi * 32;
  if ((k & 31) == 0) {      // every group full, every row 16-byte aligned
    float v[32];
    if constexpr (FMT == FMT_E2M1) {
      const uint4 p = *(const uint4*)(qr + e0 / 2);
      const uint32_t words[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
      for (int b = 0; b < 16; ++b) {
        const uint32_t byte = (words[b >> 2] >> (8 * (b & 3))) & 0xFFu;
        v[2 * b] = e2m1_to_f32(byte & 0xFu) * s;
        v[2 * b + 1] = e2m1_to_f32(byte >> 4) * s;
      }
    } else {
      const uint4* p = (const uint4*)(qr + e0);
      const uint4 a = p[0], c = p[1];
      const uint32_t words[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
      for (int b = 0; b < 32; ++b) v[b] = e4m3_to_f32((words[b >> 2] >> (8 * (b & 3))) & 0xFFu) * s;
    }
    float lo[16], hi[16];
#pragma unroll
    for (int b = 0; b < 16; ++b) { lo[b] = v[b]; hi[b] = v[16 + b]; }
    store16<OUT>(out, o0, lo);
    store16<OUT>(out, o0 + 16, hi);
    return;
  }
  for (uint32_t e = e0; e < k && e < e0 + 32; ++e) {
    float c;
    if constexpr (FMT == FMT_E2M1) {
      const uint32_t byte = qr[e / 2];
      c = e2m1_to_f32((e & 1) ? (byte >> 4) : (byte & 0xFu));
    } else {
      c = e4m3_to_f32(qr[e]);
    }
    store_act<OUT>(out, (int64_t)row * k + e, c * s);
  }
}

template <int SC>
static void fp8_by_out(int od, dim3 grid, hipStream_t st, const uint4* w, const void* scale,
                       void* out, uint32_t rows, uint32_t u_row, uint32_t bo, uint32_t bi16,
                       uint32_t s_cols) {
  if (od == DT_BF16)
    hipLaunchKernelGGL((fp8_block_kernel<SC, DT_BF16>), grid, dim3(256), 0, st, w, scale, out, rows, u_row, bo, bi16, s_cols);
  else if (od == DT_FP16)
    hipLaunchKernelGGL((fp8_block_kernel<SC, DT_FP16>), grid, dim3(256), 0, st, w, scale, out, rows, u_row, bo, bi16, s_cols);
  else
    hipLaunchKernelGGL((fp8_block_kernel<SC, DT_FP32>), grid, dim3(256), 0, st, w, scale, out, rows, u_row, bo, bi16, s_cols);
}

template <int FMT>
static void mx_by_out(int od, dim3 grid, hipStream_t st, const uint8_t* q, const uint8_t* scale,
                      void* out, uint32_t rows, uint32_t k, uint32_t q_row, uint32_t groups) {
  if (od == DT_BF16)
    hipLaunchKernelGGL((mx_upcast_kernel<FMT, DT_BF16>), grid, dim3(256), 0, st, q, scale, out, rows, k, q_row, groups);
  else if (od == DT_FP16)
    hipLaunchKernelGGL((mx_upcast_kernel<FMT, DT_FP16>), grid, dim3(256), 0, st, q, scale, out, rows, k, q_row, groups);
  else
    hipLaunchKernelGGL((mx_upcast_kernel<FMT, DT_FP32>), grid, dim3(256), 0, st, q, scale, out, rows, k, q_row, groups);
}

}  // namespace vaayu

using namespace vaayu;

extern "C" int vaayu_dequant_fp8_block(const uint8_t* weight, const void* scale, int32_t scale_dtype,
                                       void* out, int32_t out_dtype, int64_t rows, int64_t cols,
                                       int64_t scale_rows, int64_t scale_cols, void* stream) {
  clear_error();
  if (!weight || !scale || !out) return set_error(-1, "null pointer argument");
  if (rows <= 0 || cols <= 0 || scale_rows <= 0 || scale_cols <= 0)
    return set_error(-1, "sizes must be positive");
  if (rows % scale_rows || cols % scale_cols)
    return set_error(-1, "the scale grid does not tile the weight");
  if (scale_dtype < 0 || scale_dtype > 3 || out_dtype < 0 || out_dtype > 2)
    return set_error(-1, "scale / output dtype");
  const int64_t bo = rows / scale_rows, bi = cols / scale_cols;
  if (cols % 16 || bi % 16) return set_error(-2, "row length and column block must be multiples of 16");
  if (((uintptr_t)weight | (uintptr_t)out) & 15) return set_error(-1, "weight and out must be 16-byte aligned");
  if (cols / 16 > (int64_t)256 * 65535 || bo > 65535) return set_error(-2, "weight too large");
  const uint32_t u_row = (uint32_t)(cols / 16);
  // more rows than one grid holds: launches of whole row blocks
  const int64_t chunk = (65535 / bo) * bo;
  hipStream_t st = (hipStream_t)stream;
  for (int64_t r0 = 0; r0 < rows; r0 += chunk) {
    const uint32_t nr = (uint32_t)(rows - r0 < chunk ? rows - r0 : chunk);
    const dim3 grid((u_row + 255) / 256, nr);
    const size_t ob = (size_t)r0 * cols * (out_dtype == DT_FP32 ? 4 : 2);
    const size_t sb = (size_t)(r0 / bo) * scale_cols *
                      (scale_dtype == SC_FP32 ? 4 : scale_dtype == SC_E8M0 ? 1 : 2);
    const uint4* w = (const uint4*)(weight + r0 * cols);
    const void* s = (const char*)scale + sb;
    void* o = (char*)out + ob;
    switch (scale_dtype) {
      case SC_BF16: fp8_by_out<SC_BF16>(out_dtype, grid, st, w, s, o, nr, u_row, (uint32_t)bo, (uint32_t)(bi / 16), (uint32_t)scale_cols); break;
      case SC_FP16: fp8_by_out<SC_FP16>(out_dtype, grid, st, w, s, o, nr, u_row, (uint32_t)bo, (uint32_t)(bi / 16), (uint32_t)scale_cols); break;
      case SC_FP32: fp8_by_out<SC_FP32>(out_dtype, grid, st, w, s, o, nr, u_row, (uint32_t)bo, (uint32_t)(bi / 16), (uint32_t)scale_cols); break;
      default: fp8_by_out<SC_E8M0>(out_dtype, grid, st, w, s, o, nr, u_row, (uint32_t)bo, (uint32_t)(bi / 16), (uint32_t)scale_cols); break;
    }
  }
  return check_launch("fp8 block dequant");
}

extern "C" int vaayu_upcast_mx(const uint8_t* q, int32_t fmt, const uint8_t* scale, void* out,
                               int32_t out_dtype, int64_t rows, int64_t k, void* stream) {
  clear_error();
  if (!q || !scale || !out) return set_error(-1, "null pointer argument");
  if (rows <= 0 || k <= 0) return set_error(-1, "sizes must be positive");
  if (fmt != FMT_E2M1 && fmt != FMT_E4M3) return set_error(-1, "format must be 0 (e2m1) or 1 (e4m3)");
  if (out_dtype < 0 || out_dtype > 2) return set_error(-1, "output dtype");
  if (fmt == FMT_E2M1 && (k & 1)) return set_error(-2, "e2m1 rows hold an even number of elements");
  if (k > (int64_t)1 << 31) return set_error(-2, "row too long");
  const uint32_t groups = (uint32_t)((k + 31) / 32);
  const uint32_t q_row = (uint32_t)(fmt == FMT_E2M1 ? k / 2 : k);
  // full groups are read and written 16 bytes at a time: needs 16-byte aligned rows
  if ((k & 31) == 0 && (((uintptr_t)q | (uintptr_t)out) & 15))
    return set_error(-1, "codes and out must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
    const uint32_t nr = (uint32_t)(rows - r0 < 65535 ? rows - r0 : 65535);
    const dim3 grid((groups + 255) / 256, nr);
    const uint8_t* qq = q + r0 * q_row;
    const uint8_t* ss = scale + r0 * groups;
    void* o = (char*)out + (size_t)r0 * k * (out_dtype == DT_FP32 ? 4 : 2);
    if (fmt == FMT_E2M1) mx_by_out<FMT_E2M1>(out_dtype, grid, st, qq, ss, o, nr, (uint32_t)k, q_row, groups);
    else mx_by_out<FMT_E4M3>(out_dtype, grid, st, qq, ss, o, nr, (uint32_t)k, q_row, groups);
  }
  return check_launch("mx upcast");
}
