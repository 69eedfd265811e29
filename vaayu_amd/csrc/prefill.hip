// Prefill over packed experts: grouped GEMMs on MFMA (bf16/fp16 in, fp32 accumulate).
//
// Replaces the reference's three Triton launches (vaayu/packed_expert_kernels.py:179-260,
// launched by `_gate_up_g` :720-732, `_down_g` :735-749, `_reduce` :752-757) over the
// same tables `_prefill_tables` builds (:691-717):
//   tbl  [n_blocks, 2]   (packed address, scale address) of each 16-row block's expert
//   rows [n_blocks, 16]  row ids token*top_k + slot, -1 pads
//   ord  [tokens, top_k] row ids of each token's slots in ascending expert id
//
// Tile: one block of 16 rows x 64 weight rows per workgroup (4 waves x 16). Each wave
// runs v_mfma_f32_16x16x32 over K. The four 16-lane quarters of a wave each take one
// contiguous 16-byte unit of codes per K step, so a K step is 4 units; the MFMA's 32 K
// slots of quarter q map to codes [q*CPU + 8i, +8) of MFMA i. A and B use the same slot
// map, so each product is an ordinary dot over K in a fixed order. Every row's arithmetic
// is the same instruction sequence whatever its block-mates are (batch invariance), and
// nothing is split over K or accumulated atomically.
#include "common.hpp"
#include "abi_internal.hpp"

namespace vaayu {

template <int ACT>
__device__ __forceinline__ f32x4 mfma16(uint4 a, uint4 b, f32x4 c) {
  if constexpr (ACT == DT_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

__device__ __forceinline__ float load_dt(const void* p, int64_t i, int dt) {
  if (dt == DT_BF16) return load_as_float<DT_BF16>(p, i);
  if (dt == DT_FP16) return load_as_float<DT_FP16>(p, i);
  return load_as_float<DT_FP32>(p, i);
}

// B operands (8 weights each, as 4 packed pairs) of one unit of codes.
template <int BITS, int ACT>
__device__ __forceinline__ void unit_operands(uint4 q, float s_act, const Masks& M,
                                              uint4 (&b)[BITS == 4 ? 4 : 2]) {
  if constexpr (BITS == 4) {
    GroupK k = group_consts<4>(s_act);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t p[4];
      deq_word_i4<ACT>(w[i], k, M, p);
      b[i] = make_uint4(p[0], p[1], p[2], p[3]);
    }
  } else {
    GroupK k = group_consts<8>(s_act);
    uint32_t p0[2], p1[2], p2[2], p3[2];
    deq_word_i8<ACT>(q.x, k, M, p0);
    deq_word_i8<ACT>(q.y, k, M, p1);
    deq_word_i8<ACT>(q.z, k, M, p2);
    deq_word_i8<ACT>(q.w, k, M, p3);
    b[0] = make_uint4(p0[0], p0[1], p1[0], p1[1]);
    b[1] = make_uint4(p2[0], p2[1], p3[0], p3[1]);
  }
}

template <int BITS, int ACT>
__global__ void __launch_bounds__(256)
prefill_gate_up_kernel(const void* __restrict__ x, const int64_t* __restrict__ rows,
                       const int64_t* __restrict__ tbl, void* __restrict__ h, int top_k,
                       int hidden, int inter, int group, int sc_dt, int64_t gate_w,
                       int64_t gate_s, int64_t up_w, int64_t up_s) {
  constexpr int CPU = 128 / BITS;                   // codes per lane per K step
  constexpr int NM = CPU / 8;                       // MFMAs per K step
  const int b = blockIdx.x;
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int q = lane >> 4, m = lane & 15;
  const int n = blockIdx.y * 64 + wv * 16 + m;      // weight row whose B column lane m loads
  const bool n_ok = n < inter;
  const int64_t rid = rows[b * 16 + m];
  const int64_t tok = rid >= 0 ? rid / top_k : 0;   // padding rows read token 0, never stored
  const int32_t* pk = (const int32_t*)tbl[2 * b];
  const void* sc = (const void*)tbl[2 * b + 1];
  const int64_t words_row = (int64_t)hidden * BITS / 32;
  const int64_t groups_row = hidden / group;
  const int nn = n_ok ? n : 0;
  const int32_t* grow = pk + gate_w + nn * words_row;
  const int32_t* urow = pk + up_w + nn * words_row;
  const char* xrow = (const char*)x + tok * hidden * 2;
  const Masks M = make_masks();
  f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < hidden; k0 += 4 * CPU) {
    const int kc = k0 + q * CPU;
    const uint4 qg = *(const uint4*)(grow + kc * BITS / 32);
    const uint4 qu = *(const uint4*)(urow + kc * BITS / 32);
    const float sg = round_act<ACT>(load_dt(sc, gate_s + nn * groups_row + kc / group, sc_dt));
    const float su = round_act<ACT>(load_dt(sc, up_s + nn * groups_row + kc / group, sc_dt));
    uint4 bg[NM], bu[NM];
    unit_operands<BITS, ACT>(qg, sg, M, bg);
    unit_operands<BITS, ACT>(qu, su, M, bu);
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      const uint4 a = *(const uint4*)(xrow + (int64_t)(kc + 8 * i) * 2);
      ag = mfma16<ACT>(a, bg[i], ag);
      au = mfma16<ACT>(a, bu[i], au);
    }
  }
  // C layout: lane (q, m) holds rows 4q..4q+3 of the block, column m.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t r = rows[b * 16 + 4 * q + i];
    if (r >= 0 && n_ok) store_act<ACT>(h, r * inter + n, silu_mul<ACT>(ag[i], au[i]));
  }
}

template <int BITS, int ACT>
__global__ void __launch_bounds__(256)
prefill_down_kernel(const void* __restrict__ h, const int64_t* __restrict__ rows,
                    const int64_t* __restrict__ tbl, const void* __restrict__ rw, int rw_dt,
                    float* __restrict__ y, int hidden, int inter, int group, int sc_dt,
                    int64_t down_w, int64_t down_s, int w_round) {
  constexpr int CPU = 128 / BITS;
  constexpr int NM = CPU / 8;
  const int b = blockIdx.x;
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int q = lane >> 4, m = lane & 15;
  const int n = blockIdx.y * 64 + wv * 16 + m;
  const bool n_ok = n < hidden;
  const int64_t rid = rows[b * 16 + m];
  const int64_t hr = rid >= 0 ? rid : 0;
  const int32_t* pk = (const int32_t*)tbl[2 * b];
  const void* sc = (const void*)tbl[2 * b + 1];
  const int64_t words_row = (int64_t)inter * BITS / 32;
  const int64_t groups_row = inter / group;
  const int nn = n_ok ? n : 0;
  const int32_t* drow = pk + down_w + nn * words_row;
  const char* hrow = (const char*)h + hr * inter * 2;
  const Masks M = make_masks();
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < inter; k0 += 4 * CPU) {
    const int kc = k0 + q * CPU;
    const uint4 qd = *(const uint4*)(drow + kc * BITS / 32);
    const float sd = round_act<ACT>(load_dt(sc, down_s + nn * groups_row + kc / group, sc_dt));
    uint4 bd[NM];
    unit_operands<BITS, ACT>(qd, sd, M, bd);
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      const uint4 a = *(const uint4*)(hrow + (int64_t)(kc + 8 * i) * 2);
      acc = mfma16<ACT>(a, bd[i], acc);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t r = rows[b * 16 + 4 * q + i];
    if (r >= 0 && n_ok) {
      float c = round_act<ACT>(acc[i]) * load_dt(rw, r, rw_dt);
      if (w_round) c = round_act<ACT>(c);
      y[r * hidden + n] = c;
    }
  }
}

// out[t, c] = sum_k y[ord[t*top_k + k], c], sequential from 0.
__global__ void __launch_bounds__(256)
prefill_reduce_kernel(const float* __restrict__ y, const int64_t* __restrict__ ord,
                      float* __restrict__ out, int top_k, int hidden) {
  const int t = blockIdx.x;
  const int c0 = (blockIdx.y * 256 + threadIdx.x) * 4;
  if (c0 >= hidden) return;
  const int64_t* o = ord + (int64_t)t * top_k;
  if (c0 + 4 <= hidden && (hidden & 3) == 0) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k = 0; k < top_k; ++k) {
      const float4 v = *(const float4*)(y + o[k] * hidden + c0);
      acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
    *(float4*)(out + (int64_t)t * hidden + c0) = acc;
  } else {
    for (int c = c0; c < c0 + 4 && c < hidden; ++c) {
      float acc = 0.f;
      for (int k = 0; k < top_k; ++k) acc += y[o[k] * hidden + c];
      out[(int64_t)t * hidden + c] = acc;
    }
  }
}

// Why the prefill kernels cannot take this geometry, or nullptr.
const char* prefill_unsupported(const vaayu_geom* g, int act) {
  if (act != DT_BF16 && act != DT_FP16) return "activation dtype (MFMA takes bf16 / fp16)";
  if (g->bits != 4 && g->bits != 8) return "bit width (the MFMA path takes 4 and 8)";
  const int cpu = 128 / g->bits;
  if (g->group % cpu) return "group size smaller than a 16-byte unit of codes";
  if (g->hidden % (4 * cpu) || g->inter % (4 * cpu))
    return "K tile: hidden / intermediate is not a multiple of the 4-unit K step";
  return nullptr;
}

}  // namespace vaayu

using namespace vaayu;

extern "C" int vaayu_prefill_gate_up(const void* x, const int64_t* rows, const int64_t* table,
                                     void* h, int32_t n_blocks, int32_t top_k,
                                     const vaayu_geom* g, int32_t act, int32_t scale_dtype,
                                     void* stream) {
  clear_error();
  if (!x || !rows || !table || !h || !g) return set_error(-1, "null pointer argument");
  if (n_blocks <= 0 || top_k <= 0) return set_error(-1, "n_blocks / top_k must be positive");
  if (scale_dtype < 0 || scale_dtype > 2) return set_error(-1, "scale dtype");
  if (const char* why = prefill_unsupported(g, act)) return set_error(-2, why);
  const dim3 grid((unsigned)n_blocks, (unsigned)((g->inter + 63) / 64)), block(256);
  hipStream_t st = (hipStream_t)stream;
#define GU(B_, A_)                                                                        \
  hipLaunchKernelGGL((prefill_gate_up_kernel<B_, A_>), grid, block, 0, st, x, rows, table, h, \
                     top_k, g->hidden, g->inter, g->group, scale_dtype, g->gate_w, g->gate_s, \
                     g->up_w, g->up_s)
  if (g->bits == 4 && act == DT_BF16) GU(4, DT_BF16);
  else if (g->bits == 4) GU(4, DT_FP16);
  else if (act == DT_BF16) GU(8, DT_BF16);
  else GU(8, DT_FP16);
#undef GU
  return check_launch("prefill gate/up");
}

extern "C" int vaayu_prefill_down(const void* h, const int64_t* rows, const int64_t* table,
                                  const void* routing_weights, int32_t rw_dtype, float* y,
                                  int32_t n_blocks, const vaayu_geom* g, int32_t act,
                                  int32_t scale_dtype, int32_t w_round, void* stream) {
  clear_error();
  if (!h || !rows || !table || !routing_weights || !y || !g)
    return set_error(-1, "null pointer argument");
  if (n_blocks <= 0) return set_error(-1, "n_blocks must be positive");
  if (scale_dtype < 0 || scale_dtype > 2 || rw_dtype < 0 || rw_dtype > 2)
    return set_error(-1, "scale / routing-weight dtype");
  if (const char* why = prefill_unsupported(g, act)) return set_error(-2, why);
  const dim3 grid((unsigned)n_blocks, (unsigned)((g->hidden + 63) / 64)), block(256);
  hipStream_t st = (hipStream_t)stream;
#define DN(B_, A_)                                                                          \
  hipLaunchKernelGGL((prefill_down_kernel<B_, A_>), grid, block, 0, st, h, rows, table,         \
                     routing_weights, rw_dtype, y, g->hidden, g->inter, g->group, scale_dtype,  \
                     g->down_w, g->down_s, w_round)
  if (g->bits == 4 && act == DT_BF16) DN(4, DT_BF16);
  else if (g->bits == 4) DN(4, DT_FP16);
  else if (act == DT_BF16) DN(8, DT_BF16);
  else DN(8, DT_FP16);
#undef DN
  return check_launch("prefill down");
}

extern "C" int vaayu_prefill_reduce(const float* y, const int64_t* order, float* out,
                                    int32_t tokens, int32_t top_k, int32_t hidden, void* stream) {
  clear_error();
  if (!y || !order || !out) return set_error(-1, "null pointer argument");
  if (tokens <= 0 || top_k <= 0 || hidden <= 0) return set_error(-1, "sizes must be positive");
  const dim3 grid((unsigned)tokens, (unsigned)((hidden + 1023) / 1024)), block(256);
  hipLaunchKernelGGL(prefill_reduce_kernel, grid, block, 0, (hipStream_t)stream, y, order, out,
                     top_k, hidden);
  return check_launch("prefill reduce");
}
