// Shared device helpers for the packed-expert kernels (gfx950 / CDNA4).
//
// Numerics follow the reference's stock path rounding points
// (vaayu/packed_expert_kernels.py:75-106): a packed code c becomes the weight
//   W = round_act((c - 2^(bits-1)) * round_act(scale))
// and every value the stock path stores in the activation dtype is rounded to it
// (nearest-even, NaN kept NaN).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vaayu {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum { DT_BF16 = 0, DT_FP16 = 1, DT_FP32 = 2 };

// ── scalar loads / rounding ─────────────────────────────────────────────────────────────

template <int DT>
__device__ __forceinline__ float load_as_float(const void* p, int64_t i) {
  if constexpr (DT == DT_BF16) {
    uint32_t b = (uint32_t)((const uint16_t*)p)[i] << 16;
    return __builtin_bit_cast(float, b);
  } else if constexpr (DT == DT_FP16) {
    return (float)((const _Float16*)p)[i];
  } else {
    return ((const float*)p)[i];
  }
}

// fp32 -> the activation dtype and back: one nearest-even rounding (the hardware
// conversions, which keep a NaN a NaN).
template <int ACT>
__device__ __forceinline__ float round_act(float v) {
  if constexpr (ACT == DT_BF16) {
    return (float)(__bf16)v;
  } else if constexpr (ACT == DT_FP16) {
    return (float)(_Float16)v;
  } else {
    return v;
  }
}

template <int ACT>
__device__ __forceinline__ void store_act(void* p, int64_t i, float v) {
  if constexpr (ACT == DT_BF16) {
    ((__bf16*)p)[i] = (__bf16)v;
  } else if constexpr (ACT == DT_FP16) {
    ((_Float16*)p)[i] = (_Float16)v;
  } else {
    ((float*)p)[i] = v;
  }
}

// A constant copied into a VGPR whose value the compiler no longer knows. gfx9 VOP3 takes
// no literal operands, so with opaque masks `(a & m) | o` selects to one v_and_or_b32 and
// `(m & a) | (~m & b)` to one v_bfi_b32 (the compiler otherwise splits them around the
// literals, or turns the butterfly's selects into indexed register reads). The ops
// themselves stay ordinary compiled code: no instruction is hand-written in inline asm,
// so the compiler's hazard checks (e.g. the wait states a v_dot2c result needs before
// another VALU op reads it) cover them.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// (a & m) | o; with opaque m and o one VALU op.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
  return (a & m) | o;
}

// SiLU(g) * u with the stock rounding points: a = round(g / (1 + exp(-g))), h = round(a*u)
// (vaayu/packed_expert_kernels.py:147-150).
template <int ACT>
__device__ __forceinline__ float silu_mul(float acc_g, float acc_u) {
  float g = round_act<ACT>(acc_g);
  float u = round_act<ACT>(acc_u);
  float a = round_act<ACT>(g / (1.0f + expf(-g)));
  return round_act<ACT>(a * u);
}

// ── per-group dequant constants ─────────────────────────────────────────────────────────
//
// The codes are turned into fp16 values with an exponent "magic": a code c placed in the
// low mantissa bits under exponent 2^10 reads as 1024 + c; placed at mantissa bits 4..7
// under exponent 2^6 it reads as 64 + c. v_fma_mix then computes
//   (1024 + c) * s - (1024 + off) * s   or   (64 + c) * s - (64 + off) * s
// in fp32. Both addends are exact (s has <= 11 significant bits for bf16/fp16
// activations) and the exact result (c - off) * s has <= 19 significant bits, so the one
// fp32 rounding is exact and the later conversion to the activation dtype is the stock
// path's single rounding of the dequantized weight.
struct GroupK {
  float s;       // the scale, already rounded to the activation dtype
  float lo;      // -(1024 + off) * s
  float hi;      // -(64 + off) * s
};

template <int BITS>
__device__ __forceinline__ GroupK group_consts(float s_act) {
  constexpr float off = (float)(1 << (BITS - 1));
  GroupK k;
  k.s = s_act;
  k.lo = -(1024.0f + off) * s_act;
  k.hi = -(64.0f + off) * s_act;
  return k;
}

// ── 16-byte units: 4 words of codes -> weights in the activation dtype ─────────────────
//
// For bf16/fp16 activations the weights come out as packed pairs (element 2i in the low
// half, 2i+1 in the high half), ready for v_dot2 or an MFMA operand.

struct Masks {
  uint32_t m_lo, m_hi, magic_lo, magic_hi, m_byte;
};

__device__ __forceinline__ Masks make_masks() {
  Masks m;
  m.m_lo = opaque(0x000F000Fu);
  m.m_hi = opaque(0x00F000F0u);
  m.magic_lo = opaque(0x64006400u);   // fp16 2^10: mantissa bits 0..9
  m.magic_hi = opaque(0x54005400u);   // fp16 2^6: a code at mantissa bits 4..7 reads as 64 + c
  m.m_byte = opaque(0x00FF00FFu);
  return m;
}

// int4 word (codes 0..7) -> 4 packed weight pairs in the activation dtype (bf16 or fp16).
template <int ACT>
__device__ __forceinline__ void deq_word_i4(uint32_t w, const GroupK& k, const Masks& M,
                                            uint32_t out[4]) {
  f16x2 A = __builtin_bit_cast(f16x2, and_or(w, M.m_lo, M.magic_lo));   // c0, c4
  f16x2 B = __builtin_bit_cast(f16x2, and_or(w, M.m_hi, M.magic_hi));   // c1, c5
  uint32_t w8 = w >> 8;
  f16x2 C = __builtin_bit_cast(f16x2, and_or(w8, M.m_lo, M.magic_lo));  // c2, c6
  f16x2 D = __builtin_bit_cast(f16x2, and_or(w8, M.m_hi, M.magic_hi));  // c3, c7
  float f0 = __builtin_fmaf((float)A.x, k.s, k.lo);
  float f1 = __builtin_fmaf((float)B.x, k.s, k.hi);
  float f2 = __builtin_fmaf((float)C.x, k.s, k.lo);
  float f3 = __builtin_fmaf((float)D.x, k.s, k.hi);
  float f4 = __builtin_fmaf((float)A.y, k.s, k.lo);
  float f5 = __builtin_fmaf((float)B.y, k.s, k.hi);
  float f6 = __builtin_fmaf((float)C.y, k.s, k.lo);
  float f7 = __builtin_fmaf((float)D.y, k.s, k.hi);
  if constexpr (ACT == DT_BF16) {
    out[0] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){f0, f1}, bf16x2));
    out[1] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){f2, f3}, bf16x2));
    out[2] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){f4, f5}, bf16x2));
    out[3] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){f6, f7}, bf16x2));
  } else {
    out[0] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){f0, f1}, f16x2));
    out[1] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){f2, f3}, f16x2));
    out[2] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){f4, f5}, f16x2));
    out[3] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){f6, f7}, f16x2));
  }
}

// int8 word (codes 0..3) -> 2 packed weight pairs.
template <int ACT>
__device__ __forceinline__ void deq_word_i8(uint32_t w, const GroupK& k, const Masks& M,
                                            uint32_t out[2]) {
  f16x2 A = __builtin_bit_cast(f16x2, and_or(w, M.m_byte, M.magic_lo));       // c0, c2
  f16x2 B = __builtin_bit_cast(f16x2, and_or(w >> 8, M.m_byte, M.magic_lo));  // c1, c3
  float f0 = __builtin_fmaf((float)A.x, k.s, k.lo);
  float f1 = __builtin_fmaf((float)B.x, k.s, k.lo);
  float f2 = __builtin_fmaf((float)A.y, k.s, k.lo);
  float f3 = __builtin_fmaf((float)B.y, k.s, k.lo);
  if constexpr (ACT == DT_BF16) {
    out[0] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){f0, f1}, bf16x2));
    out[1] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){f2, f3}, bf16x2));
  } else {
    out[0] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){f0, f1}, f16x2));
    out[1] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){f2, f3}, f16x2));
  }
}

// Any bit width (1, 2, 4, 8) one code at a time, for any activation dtype: the general
// path (fp32 activations and the narrow widths).
template <int ACT, int BITS>
__device__ __forceinline__ float deq_code(uint32_t w, int j, float s_act) {
  constexpr uint32_t mask = (1u << BITS) - 1u;
  float c = (float)((w >> (j * BITS)) & mask) - (float)(1 << (BITS - 1));
  return round_act<ACT>(c * s_act);
}

// Packed-pair dot products (fp32 accumulate).
template <int ACT>
__device__ __forceinline__ float dot2(uint32_t w, uint32_t x, float acc) {
  if constexpr (ACT == DT_BF16) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w),
                                           __builtin_bit_cast(bf16x2, x), acc, false);
  } else {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), __builtin_bit_cast(f16x2, x),
                                  acc, false);
  }
}

// ── FP8 / FP4 codes and E8M0 scales ─────────────────────────────────────────────────────

// float8 e4m3fn (bias 7, no infinities, S.1111.111 is NaN) -> fp32, exact.
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  const uint32_t sign = (b & 0x80u) << 24;
  const uint32_t e = (b >> 3) & 0xFu, m = b & 7u;
  float mag;
  if (e == 0) {
    mag = (float)m * 0x1p-9f;                                   // subnormal: m/8 * 2^-6
  } else if (e == 15 && m == 7) {
    mag = __builtin_nanf("");
  } else {
    mag = __builtin_bit_cast(float, ((e + 120u) << 23) | (m << 20));
  }
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, mag) | sign);
}

// e2m1 nibble (bit 3 the sign; values 0, .5, 1, 1.5, 2, 3, 4, 6) -> fp32, exact.
__device__ __forceinline__ float e2m1_to_f32(uint32_t n) {
  const uint32_t sign = (n & 8u) << 28;
  const uint32_t e = (n >> 1) & 3u, m = n & 1u;
  const uint32_t mag = e ? (((e + 126u) << 23) | (m << 22)) : (m ? 0x3F000000u : 0u);
  return __builtin_bit_cast(float, mag | sign);
}

// E8M0 scale byte -> the fp32 with exponent bits s (s = 0 gives 0), 0xFF -> NaN.
__device__ __forceinline__ float e8m0_to_f32(uint32_t s) {
  return s == 0xFFu ? __builtin_nanf("") : __builtin_bit_cast(float, s << 23);
}

// Two fp32 values -> one packed pair of the activation dtype (bf16 or fp16), nearest-even.
template <int ACT>
__device__ __forceinline__ uint32_t pack_act(float a, float b) {
  if constexpr (ACT == DT_BF16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
}

// e4m3 word (4 codes, code k in byte k) -> 2 packed weight pairs round_act(fp32(c) * s):
// the fp32 product rounded once, then one rounding to the activation dtype. The codes are
// widened by v_cvt_pk_f32_fp8 (gfx950: OCP e4m3fn, exact for all 256 codes, NaN kept).
template <int ACT>
__device__ __forceinline__ void deq_word_e4m3(uint32_t w, float s, uint32_t out[2]) {
#if defined(__HIP_DEVICE_COMPILE__)        // gfx950 instructions: no host-pass form
  const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  out[0] = pack_act<ACT>(lo.x * s, lo.y * s);
  out[1] = pack_act<ACT>(hi.x * s, hi.y * s);
#else
  out[0] = out[1] = w;
  (void)s;
#endif
}

// e2m1 word (8 codes, code k in bits 4k..4k+3) -> 4 packed weight pairs round_act(e2m1 * s),
// s the E8M0 scale as fp32 (2^(e-127); 0 for e = 0; NaN for e = 255). The products are exact
// (e2m1 has two significant bits, s is a power of two). v_cvt_scalef32_pk_*_fp4 applies the
// scale by its exponent field, which gives 2^-127 rather than 0 for s = 0: there the codes'
// magnitude bits are cleared first (signs kept), so every product is the reference's +-0.
template <int ACT>
__device__ __forceinline__ void deq_word_e2m1(uint32_t w, float s, uint32_t out[4]) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint32_t keep = __builtin_bit_cast(uint32_t, s) == 0 ? 0x88888888u : 0xFFFFFFFFu;
  const uint32_t c = w & keep;
  if constexpr (ACT == DT_BF16) {
    out[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, s, 0));
    out[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, s, 1));
    out[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, s, 2));
    out[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, s, 3));
  } else {
    const f32x2 v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(c, s, 0);
    const f32x2 v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(c, s, 1);
    const f32x2 v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(c, s, 2);
    const f32x2 v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(c, s, 3);
    out[0] = pack_act<ACT>(v0.x, v0.y);
    out[1] = pack_act<ACT>(v1.x, v1.y);
    out[2] = pack_act<ACT>(v2.x, v2.y);
    out[3] = pack_act<ACT>(v3.x, v3.y);
  }
#else
  out[0] = out[1] = out[2] = out[3] = w;
  (void)s;
#endif
}

// ── code formats ────────────────────────────────────────────────────────────────────────
//
// Code formats F of the kernels: 1, 2, 4, 8 are packed unsigned integers of that many bits
// (offset 2^(F-1), scale rounded to the activation dtype); F_E4M3 is float8 e4m3fn with fp32
// block scales, F_MXFP4 is e2m1 with an E8M0 scale per 32 codes (both scales applied
// unrounded, as the reference's dequant does).
enum { F_MXFP4 = 104, F_E4M3 = 108 };

template <int F>
struct CodeBits {
  static constexpr int value = F % 100;
};

// A unit's scale as the weights take it: rounded to the activation dtype for integer codes,
// as is for e4m3 and e2m1.
template <int F, int ACT>
__device__ __forceinline__ float applied_scale(float s) {
  if constexpr (F < 100) return round_act<ACT>(s);
  else return s;
}

// MFMA operand i (8 weights as 4 packed pairs of the activation dtype, in code order) of one
// 16-byte unit of codes of format F (bf16 / fp16 activations): word i of 4-bit codes, words
// 2i and 2i+1 of 8-bit codes. k: the group constants of the applied scale (integer codes);
// s: the applied scale (e4m3, e2m1).
template <int F, int ACT>
__device__ __forceinline__ uint4 operand_i(const uint4& q, const GroupK& k, float s,
                                           const Masks& M, int i) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  if constexpr (F == 4 || F == F_MXFP4) {
    uint32_t p[4];
    if constexpr (F == 4) deq_word_i4<ACT>(w[i], k, M, p);
    else deq_word_e2m1<ACT>(w[i], s, p);
    return make_uint4(p[0], p[1], p[2], p[3]);
  } else {
    uint32_t p0[2], p1[2];
    if constexpr (F == 8) {
      deq_word_i8<ACT>(w[2 * i], k, M, p0);
      deq_word_i8<ACT>(w[2 * i + 1], k, M, p1);
    } else {
      deq_word_e4m3<ACT>(w[2 * i], s, p0);
      deq_word_e4m3<ACT>(w[2 * i + 1], s, p1);
    }
    return make_uint4(p0[0], p0[1], p1[0], p1[1]);
  }
}

// Group constants for a unit of format F (zero for e4m3 / e2m1, which do not use them).
template <int F>
__device__ __forceinline__ GroupK group_of(float s_applied) {
  if constexpr (F == 4 || F == 8) return group_consts<F>(s_applied);
  else return GroupK{};
}

// ── wavefront reductions ───────────────────────────────────────────────────────────────

template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = WIDTH / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

}  // namespace vaayu
