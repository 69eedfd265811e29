// Decode kernels (shared by decode_gate_up.hip and decode_down.hip).
// One-token decode over packed experts: memory-bound GEMVs on the VALU (no MFMA).
//
// Replaces the reference's two Triton launches (vaayu/packed_expert_kernels.py:131-176,
// launched by `_gate_up` :355-371 and `_down` :374-387):
//   gate/up:  h[p, i] = round(round(SiLU(round(x.Wg[i]))) * round(x.Wu[i]))   per pair p
//   down:     out[r]  = sum over pairs p in TABLE ORDER of
//                       fl32(round(h[p].Wd[r]) * w[slot_p])  (+ round if W_ROUND)
// The pointer table is the reference's: int64 (packed address, scale address, slot) per pair.
//
// Mapping: a row of a role is a run of 16-byte units (4 words of codes). A lane group of
// LPR lanes (a power of two) covers one row; lane j owns the CH units j, j+LPR, ...,
// j+(CH-1)*LPR, so each load instruction reads LPR*16 contiguous bytes of a row and all
// CH loads of a row are issued before the first wait (CH is unrolled). The activation
// vector is staged once per block in LDS and each lane reads its CH slices from there.
// Codes are read with buffer loads (wave-uniform SGPR descriptors per role, 32-bit
// offsets, bounds-checked by the hardware), dequantized in registers (common.hpp) and
// dotted with v_dot2; each group's partial sums are reduced with a transposed butterfly.
// Nothing is atomic: the fp32 sum over pairs runs sequentially in table order out of LDS.
#pragma once
#include "common.hpp"
#include "abi_internal.hpp"

namespace vaayu {

typedef __amdgpu_buffer_rsrc_t rsrc_t;


__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(rsrc_t r, uint32_t byte_off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// The same load marked non-temporal (the cache-policy nt bit): for expert codes read once
// per call, so their lines are the first to leave L2 and the small operands the next
// kernels need (pointer tables, activations) stay cached.
__device__ __forceinline__ uint4 buf_load16_nt(rsrc_t r, uint32_t byte_off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 2);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// A scale of SW bits (8: E8M0, 16: bf16 / fp16, 32: fp32), raw (converted only where it is used,
// so the load is not waited for early).
template <int SW>
__device__ __forceinline__ uint32_t buf_load_scale(rsrc_t r, uint32_t idx) {
  if constexpr (SW == 32) return __builtin_amdgcn_raw_buffer_load_b32(r, idx * 4u, 0, 0);
  else if constexpr (SW == 16) return __builtin_amdgcn_raw_buffer_load_b16(r, idx * 2u, 0, 0);
  else return __builtin_amdgcn_raw_buffer_load_b8(r, idx, 0, 0);
}

// Raw scale bits of dtype `dt` (wave-uniform) as fp32; for 16-bit scales both readings are
// formed and one selected, which costs less than a branch.
template <int SW>
__device__ __forceinline__ float scale_value(uint32_t b, int dt) {
  if constexpr (SW == 32) {
    return __builtin_bit_cast(float, b);
  } else if constexpr (SW == 8) {
    return e8m0_to_f32(b);
  } else {
    const float as_bf16 = __builtin_bit_cast(float, b << 16);
    const float as_fp16 = (float)__builtin_bit_cast(_Float16, (uint16_t)b);
    return dt == DT_BF16 ? as_bf16 : as_fp16;
  }
}

// Dot of one 16-byte unit of codes with its activation slice `xw` (raw dwords of the
// activation dtype), accumulated into `acc`. Fast path: bf16/fp16 activations, 4- or
// 8-bit codes.
template <int BITS, int ACT>
__device__ __forceinline__ float unit_dot_fast(const uint4& q, const uint32_t* xw, float s,
                                               const Masks& M, float acc) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  if constexpr (BITS == F_E4M3) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t wp[2];
      deq_word_e4m3<ACT>(w[i], s, wp);
      acc = dot2<ACT>(wp[0], xw[2 * i], acc);
      acc = dot2<ACT>(wp[1], xw[2 * i + 1], acc);
    }
  } else if constexpr (BITS == F_MXFP4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t wp[4];
      deq_word_e2m1<ACT>(w[i], s, wp);
#pragma unroll
      for (int t = 0; t < 4; ++t) acc = dot2<ACT>(wp[t], xw[4 * i + t], acc);
    }
  } else if constexpr (BITS == 4) {
    const GroupK k = group_consts<4>(s);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t wp[4];
      deq_word_i4<ACT>(w[i], k, M, wp);
#pragma unroll
      for (int t = 0; t < 4; ++t) acc = dot2<ACT>(wp[t], xw[4 * i + t], acc);
    }
  } else {
    const GroupK k = group_consts<8>(s);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t wp[2];
      deq_word_i8<ACT>(w[i], k, M, wp);
      acc = dot2<ACT>(wp[0], xw[2 * i], acc);
      acc = dot2<ACT>(wp[1], xw[2 * i + 1], acc);
    }
  }
  return acc;
}

// General path (any activation dtype, 1/2/4/8-bit codes), one code at a time.
template <int BITS, int ACT>
__device__ __forceinline__ float unit_dot_general(const uint4& q, const uint32_t* xw,
                                                  float s_act, float acc) {
  constexpr int PER = 32 / CodeBits<BITS>::value;
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int jj = 0; jj < PER; ++jj) {
      const int e = i * PER + jj;
      float wt;
      if constexpr (BITS == F_E4M3)
        wt = round_act<ACT>(e4m3_to_f32((w[i] >> (8 * jj)) & 0xFFu) * s_act);
      else if constexpr (BITS == F_MXFP4)
        wt = round_act<ACT>(e2m1_to_f32((w[i] >> (4 * jj)) & 0xFu) * s_act);
      else
        wt = deq_code<ACT, BITS>(w[i], jj, s_act);
      float xval;
      if constexpr (ACT == DT_FP32) {
        xval = __builtin_bit_cast(float, xw[e]);
      } else if constexpr (ACT == DT_BF16) {
        const uint32_t d = xw[e >> 1];
        xval = __builtin_bit_cast(float, (e & 1) ? (d & 0xFFFF0000u) : (d << 16));
      } else {
        const f16x2 d = __builtin_bit_cast(f16x2, xw[e >> 1]);
        xval = (float)((e & 1) ? d.y : d.x);
      }
      acc = __builtin_fmaf(wt, xval, acc);
    }
  }
  return acc;
}

template <int F, int ACT>
struct Unit {
  static constexpr int CODES = 128 / CodeBits<F>::value;                    // per 16 B unit
  static constexpr int XD = (ACT == DT_FP32 ? 4 * CODES : 2 * CODES) / 4;   // x dwords
  static constexpr bool FAST = ACT != DT_FP32 && (F == 4 || F == 8 || F >= 100);
};

// mask ? a : b bitwise; with an opaque all-ones / all-zeros mask one v_bfi_b32.
__device__ __forceinline__ float bit_select(uint32_t mask, float a, float b) {
  const uint32_t ua = __builtin_bit_cast(uint32_t, a), ub = __builtin_bit_cast(uint32_t, b);
  return __builtin_bit_cast(float, (mask & ua) | (~mask & ub));
}

// Sum NV per-lane values over the `lpr` lanes of each aligned lane group (NV <= lpr, both
// powers of two). Transposed butterfly: each exchange halves the values a lane carries,
// then a plain butterfly finishes. Lane j (in-group index) ends with the group total of
// value number j / (lpr / NV).
template <int NV>
__device__ __forceinline__ float group_reduce(float (&v)[NV], int lpr, int j) {
  int m = lpr >> 1;
#pragma unroll
  for (int n = NV; n > 1; n >>= 1) {
    const uint32_t upper = opaque((j & m) ? 0xFFFFFFFFu : 0u);
#pragma unroll
    for (int i = 0; i < n / 2; ++i) {
      const float lo = v[i], hi = v[i + n / 2];
      const float send = bit_select(upper, lo, hi);
      const float keep = bit_select(upper, hi, lo);
      v[i] = keep + __shfl_xor(send, m, 64);
    }
    m >>= 1;
  }
  float r = v[0];
  for (; m >= 1; m >>= 1) r += __shfl_xor(r, m, 64);
  return r;
}

struct DecodeShape {
  int n_pairs;
  int inter, hidden;
  int units_row;         // 16 B units per row of the K dimension
  int lpr;               // lanes per row (power of two, <= 64)
  int chunks;            // units per lane per row (CH) = units_row / lpr
  int groups_row;        // scales per row
  int ushift;            // log2(units per scale group)
  int rshift;            // log2(rows per scale block): 0 but for block-scaled FP8
  int sc_dt;             // scale dtype code
  uint32_t role_bytes;   // bytes of one role's codes
  uint32_t role_scales;  // scales of one role
};

// RI rows x CH units of one role for one lane: codes and raw scale bits.
template <int RI, int CH>
struct RowTile {
  uint4 q[RI][CH];
  uint32_t s[RI][CH];
};

// Lane j's units of a row are j + c*lpr, c < CH.
template <int SW, int RI, int CH>
__device__ __forceinline__ void load_tile(RowTile<RI, CH>& t, rsrc_t codes, rsrc_t sc,
                                          const int (&rows)[RI], int j, const DecodeShape& s) {
#pragma unroll
  for (int r = 0; r < RI; ++r) {
    const uint32_t base = ((uint32_t)rows[r] * s.units_row + j) * 16u;
#pragma unroll
    for (int c = 0; c < CH; ++c) t.q[r][c] = buf_load16(codes, base + 16u * s.lpr * c);
  }
#pragma unroll
  for (int r = 0; r < RI; ++r) {
    const uint32_t sbase = ((uint32_t)rows[r] >> s.rshift) * s.groups_row;
#pragma unroll
    for (int c = 0; c < CH; ++c)
      t.s[r][c] = buf_load_scale<SW>(sc, sbase + ((j + c * s.lpr) >> s.ushift));
  }
}

template <int BITS, int ACT, int SW, int RI, int CH>
__device__ __forceinline__ void tile_dot(const RowTile<RI, CH>& t, const uint32_t* const (&xw)[CH],
                                         const Masks& M, float* acc, int stride, int sc_dt) {
  using UT = Unit<BITS, ACT>;
#pragma unroll
  for (int r = 0; r < RI; ++r) {
    float a = acc[r * stride];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const float sv = scale_value<SW>(t.s[r][c], sc_dt);
      const float s_act = BITS >= 100 ? sv : round_act<ACT>(sv);
      if constexpr (UT::FAST) {
        a = unit_dot_fast<BITS, ACT>(t.q[r][c], xw[c], s_act, M, a);
      } else {
        a = unit_dot_general<BITS, ACT>(t.q[r][c], xw[c], s_act, a);
      }
    }
    acc[r * stride] = a;
  }
}

// Block barrier that waits only for this wave's LDS traffic (not for its in-flight global
// or buffer loads, which keep streaming across the barrier).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Up to XST uint4 per thread of a vector staged into LDS by the whole block: the global
// loads are issued by stage_load (before the caller's weight loads, so the in-order
// load counter lets stage_store wait for them alone) and written by stage_store.
template <int XST>
__device__ __forceinline__ void stage_load(const uint4* __restrict__ src, int n16, uint4 (&st)[XST]) {
#pragma unroll
  for (int k = 0; k < XST; ++k) {
    // clamped, not guarded: lanes past the end re-load the last element (no branch, so
    // no wait is forced on the loads already in flight)
    st[k] = src[min((int)threadIdx.x + k * (int)blockDim.x, n16 - 1)];
  }
}

template <int XST>
__device__ __forceinline__ void stage_store(uint4* dst, int n16, const uint4 (&st)[XST]) {
#pragma unroll
  for (int k = 0; k < XST; ++k)   // lanes past the end rewrite the last element's value
    dst[min((int)threadIdx.x + k * (int)blockDim.x, n16 - 1)] = st[k];
}

// Lane j's CH activation slices (units j + c*lpr) from the LDS copy, as raw dwords.
template <int BITS, int ACT, int CH>
__device__ __forceinline__ void load_x(const uint32_t* x, int j, int lpr,
                                       uint32_t (&xw)[CH][Unit<BITS, ACT>::XD]) {
  constexpr int XD = Unit<BITS, ACT>::XD;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const uint4* src = (const uint4*)(x + (j + c * lpr) * XD);
#pragma unroll
    for (int i = 0; i < XD / 4; ++i) {
      const uint4 v = src[i];
      xw[c][4 * i] = v.x; xw[c][4 * i + 1] = v.y; xw[c][4 * i + 2] = v.z; xw[c][4 * i + 3] = v.w;
    }
  }
}

// Grid: one wave per (pair, RPW groups x RI rows); blocks of 4 waves. The block stages x
// in LDS (XST uint4 per thread) while its waves' weight loads are in flight.
template <int BITS, int ACT, int SW, int RI, int CH, int XST>
__global__ void __launch_bounds__(256)
decode_gate_up_kernel(const uint32_t* __restrict__ x, const int64_t* __restrict__ tbl,
                      void* __restrict__ h, DecodeShape s, uint32_t gate_wb, uint32_t gate_s,
                      uint32_t up_wb, uint32_t up_s) {
  using UT = Unit<BITS, ACT>;
  constexpr int NV = 2 * RI;
  extern __shared__ uint4 xl[];
  const int lane = threadIdx.x & 63;
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rpw = 64 / s.lpr;
  const int gi = lane / s.lpr, j = lane & (s.lpr - 1);
  const int rows_per_wave = rpw * RI;
  const int wpp = (s.inter + rows_per_wave - 1) / rows_per_wave;
  const int wave = blockIdx.x * 4 + wib;
  const int p = min(wave / wpp, s.n_pairs - 1);
  const bool active = wave / wpp < s.n_pairs;
  const int row0 = (wave - p * wpp) * rows_per_wave + gi * RI;
  const char* pk = (const char*)tbl[3 * p];
  const char* sc = (const char*)tbl[3 * p + 1];
  constexpr int sb = SW / 8;
  const rsrc_t G = make_rsrc(pk + gate_wb, s.role_bytes);
  const rsrc_t U = make_rsrc(pk + up_wb, s.role_bytes);
  const rsrc_t GS = make_rsrc(sc + (size_t)gate_s * sb, s.role_scales * sb);
  const rsrc_t US = make_rsrc(sc + (size_t)up_s * sb, s.role_scales * sb);
  const Masks M = make_masks();
  const int x16 = s.units_row * UT::XD / 4;          // uint4 of x

  uint4 st[XST];
  stage_load<XST>((const uint4*)x, x16, st);
  __builtin_amdgcn_sched_barrier(0);
  int rows[RI];
#pragma unroll
  for (int r = 0; r < RI; ++r) rows[r] = max(min(row0 + r, s.inter - 1), 0);   // in bounds
  RowTile<RI, CH> tg, tu;
  load_tile<SW>(tg, G, GS, rows, j, s);     // (an idle wave's loads are valid, unused)
  load_tile<SW>(tu, U, US, rows, j, s);
  __builtin_amdgcn_sched_barrier(0);
  stage_store<XST>(xl, x16, st);
  lds_barrier();
  if (!active) return;

  uint32_t xw[CH][UT::XD];
  load_x<BITS, ACT, CH>((const uint32_t*)xl, j, s.lpr, xw);
  const uint32_t* xp[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) xp[c] = xw[c];
  float acc[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) acc[i] = 0.f;
  tile_dot<BITS, ACT, SW>(tg, xp, M, acc, 2, s.sc_dt);
  tile_dot<BITS, ACT, SW>(tu, xp, M, acc + 1, 2, s.sc_dt);
  const float tot = group_reduce<NV>(acc, s.lpr, j);
  const int stride = s.lpr / NV;                     // lanes per value after the reduce
  const float partner = __shfl_xor(tot, stride, 64);  // the up total beside each gate total
  const int q = j / stride;
  if ((j % stride) == 0 && (q & 1) == 0) {
    const int row = row0 + (q >> 1);
    if (row < s.inter) store_act<ACT>(h, (int64_t)p * s.inter + row, silu_mul<ACT>(tot, partner));
  }
}

// Block: 8 waves split as pair_split x row_split. The block stages every pair's h in LDS
// (XST uint4 per thread); each wave takes pairs p = pl, pl + pair_split, ... over its
// rows; every contribution lands in LDS and the block then sums each row's contributions
// in table order.
template <int BITS, int ACT, int SW, int RI, int CH, int XST>
__global__ void __launch_bounds__(512)
decode_down_kernel(const void* __restrict__ h, const int64_t* __restrict__ tbl,
                   const void* __restrict__ rw, int rw_dt, float* __restrict__ out,
                   DecodeShape s, int pair_split, uint32_t down_wb, uint32_t down_s, int w_round) {
  using UT = Unit<BITS, ACT>;
  extern __shared__ uint4 lds[];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rpw = 64 / s.lpr;
  const int gi = lane / s.lpr, j = lane & (s.lpr - 1);
  const int row_split = 8 / pair_split;
  const int pl = wv % pair_split, rp = wv / pair_split;
  const int wg_rows = row_split * rpw * RI;
  const int row_base = blockIdx.x * wg_rows;
  const int my = (rp * rpw + gi) * RI;               // this group's first row, in-block
  const Masks M = make_masks();
  constexpr int sb = SW / 8;
  const int p16 = s.units_row * UT::XD / 4;                 // uint4 of one pair's h
  const int h16 = s.n_pairs * p16;                          // uint4 of all h
  float* cbuf = (float*)(lds + h16);
  int rows[RI];
#pragma unroll
  for (int r = 0; r < RI; ++r) rows[r] = min(row_base + my + r, s.hidden - 1);

  uint4 st[XST];
  stage_load<XST>((const uint4*)h, h16, st);
  __builtin_amdgcn_sched_barrier(0);
  // the first pair's weights go out before the staging barrier (an idle wave loads a
  // valid pair it does not use)
  RowTile<RI, CH> t;
  {
    const int p0 = min(pl, s.n_pairs - 1);
    const char* pk = (const char*)tbl[3 * p0];
    const char* sc = (const char*)tbl[3 * p0 + 1];
    load_tile<SW>(t, make_rsrc(pk + down_wb, s.role_bytes),
                  make_rsrc(sc + (size_t)down_s * sb, s.role_scales * sb), rows, j, s);
  }
  __builtin_amdgcn_sched_barrier(0);
  stage_store<XST>(lds, h16, st);
  lds_barrier();

  for (int p = pl; p < s.n_pairs; p += pair_split) {
    const char* pk = (const char*)tbl[3 * p];
    const char* sc = (const char*)tbl[3 * p + 1];
    const int64_t slot = tbl[3 * p + 2];
    if (p != pl)
      load_tile<SW>(t, make_rsrc(pk + down_wb, s.role_bytes),
                    make_rsrc(sc + (size_t)down_s * sb, s.role_scales * sb), rows, j, s);
    uint32_t xw[CH][UT::XD];
    load_x<BITS, ACT, CH>((const uint32_t*)(lds + p * p16), j, s.lpr, xw);
    const uint32_t* xp[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) xp[c] = xw[c];
    float acc[RI];
#pragma unroll
    for (int r = 0; r < RI; ++r) acc[r] = 0.f;
    tile_dot<BITS, ACT, SW>(t, xp, M, acc, 1, s.sc_dt);
    const float wgt = rw_dt == DT_FP32 ? load_as_float<DT_FP32>(rw, slot)
                    : rw_dt == DT_BF16 ? load_as_float<DT_BF16>(rw, slot)
                                       : load_as_float<DT_FP16>(rw, slot);
    const float tot = group_reduce<RI>(acc, s.lpr, j);
    const int stride = s.lpr / RI;
    if (j % stride == 0) {
      // The product is rounded to fp32 on its own (it goes to LDS before any add), as
      // stock's `y * weight` then `out +=` are two roundings.
      float c = round_act<ACT>(tot) * wgt;
      if (w_round) c = round_act<ACT>(c);
      cbuf[p * wg_rows + my + j / stride] = c;
    }
  }
  __syncthreads();
  for (int tt = threadIdx.x; tt < wg_rows; tt += blockDim.x) {
    const int row = row_base + tt;
    if (row >= s.hidden) continue;
    float o = 0.f;
    for (int q = 0; q < s.n_pairs; ++q) o += cbuf[q * wg_rows + tt];
    out[row] = o;
  }
}

// ── host-side planning ────────────────────────────────────────────────────────────────

inline int ilog2(int v) {
  int r = 0;
  while ((1 << r) < v) ++r;
  return r;
}

// Why the decode kernels cannot take this geometry, or nullptr.
inline const char* decode_unsupported(const vaayu_geom* g, int act) {
  if (g->format < 0 || g->format > 2) return "code format";
  if (g->format == VAAYU_FMT_E4M3 && g->bits != 8) return "e4m3 codes are 8 bits";
  if (g->format == VAAYU_FMT_MXFP4 && (g->bits != 4 || g->group != 32))
    return "mxfp4 codes are 4 bits with one scale per 32";
  if (g->format == VAAYU_FMT_E4M3 &&
      (g->block_rows <= 0 || (g->block_rows & (g->block_rows - 1)) ||
       g->hidden % g->block_rows || g->inter % g->block_rows))
    return "e4m3 scale blocks must be a power of two rows dividing hidden and intermediate";
  if (g->bits != 1 && g->bits != 2 && g->bits != 4 && g->bits != 8) return "bit width";
  const int cpu = 128 / g->bits;                   // codes per 16-byte unit
  if (g->group % cpu || (g->group & (g->group - 1)))
    return "group size is not a power of two holding whole 16-byte units of codes";
  if (g->hidden % cpu || g->inter % cpu) return "a row is not a whole number of 16-byte units";
  if ((g->hidden / cpu) % 2) return "hidden is not an even number of 16-byte units of codes";
  if (g->hidden % g->group || g->inter % g->group) return "a row is not whole groups";
  if ((g->gate_w | g->up_w | g->down_w) & 3) return "role offsets are not 16-byte aligned";
  if ((int64_t)g->hidden * g->inter * g->bits / 8 > INT32_MAX) return "a role is over 2 GiB";
  if (act < 0 || act > 2) return "activation dtype";
  return nullptr;
}

struct Plan {
  int lpr, ch;
};

inline constexpr int kCH[] = {1, 2, 3, 4, 7};   // the instantiated chunks per lane

// The kernels' code format F for a geometry (see Unit).
inline int code_format(const vaayu_geom* g) {
  return g->format == VAAYU_FMT_E4M3 ? F_E4M3 : g->format == VAAYU_FMT_MXFP4 ? F_MXFP4 : g->bits;
}

// Lanes per row LPR (a power of two in [min_lpr, 64]) and units per lane CH =
// units_row / LPR from the instantiated set ({1, 2, 3, 4, 7} on the fast path, {1} on the
// general one): the largest LPR that gives a wave at least `min_rows` rows, so each load
// instruction covers as many contiguous bytes of a row as possible; failing that, the
// smallest LPR that works.
inline Plan plan_row(int units_row, int min_lpr, int min_rows, bool fast) {
  Plan best{0, 0};
  for (int lpr = 64; lpr >= min_lpr; lpr >>= 1) {
    if (units_row % lpr) continue;
    const int ch = units_row / lpr;
    bool ok = ch == 1;
    if (fast)
      for (int c : kCH) ok |= c == ch;
    if (!ok) continue;
    best = Plan{lpr, ch};
    if (64 / lpr >= min_rows) break;
  }
  return best;
}

inline DecodeShape shape_for(const vaayu_geom* g, int n, int k_dim, int rows, int sc_dt,
                             const Plan& pl) {
  DecodeShape s;
  s.n_pairs = n;
  s.inter = g->inter;
  s.hidden = g->hidden;
  s.units_row = k_dim * g->bits / 128;
  s.lpr = pl.lpr;
  s.chunks = pl.ch;
  s.groups_row = k_dim / g->group;
  s.ushift = ilog2(g->group * g->bits / 128);
  s.rshift = g->format == VAAYU_FMT_E4M3 ? ilog2(g->block_rows) : 0;
  s.sc_dt = sc_dt;
  s.role_bytes = (uint32_t)((int64_t)rows * k_dim * g->bits / 8);
  s.role_scales = (uint32_t)((int64_t)(rows >> s.rshift) * k_dim / g->group);
  return s;
}


}  // namespace vaayu
