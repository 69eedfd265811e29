// One-token decode over packed experts: memory-bound GEMVs on the VALU (no MFMA).
//
// Replaces the reference's two Triton launches (vaayu/packed_expert_kernels.py:131-176,
// launched by `_gate_up` :355-371 and `_down` :374-387):
//   gate/up:  h[p, i] = round(round(SiLU(round(x.Wg[i]))) * round(x.Wu[i]))   per pair p
//   down:     out[r]  = sum over pairs p in TABLE ORDER of
//                       fl32(round(h[p].Wd[r]) * w[slot_p])  (+ round if W_ROUND)
// The pointer table is the reference's: int64 (packed address, scale address, slot) per pair.
//
// Layout on the GPU: each row of a role is a run of 16-byte units (4 words of codes). A
// "lane group" of LPR lanes covers one row: lane j takes units j, j+LPR, ... so every
// load instruction reads LPR*16 contiguous bytes of a row. The lanes keep their columns
// for every row they visit, so their slice of the activation vector is loaded once per
// unit and reused across the RI rows (and both roles) the group handles. Codes are
// dequantized in registers (common.hpp) and dotted with v_dot2; each row's partials are
// summed across its lane group with xor shuffles. Nothing is atomic: the fp32 sum over
// pairs runs sequentially in table order out of LDS.
#include "common.hpp"
#include "abi_internal.hpp"

namespace vaayu {

// Dot of one 16-byte unit of codes with the matching activation slice `xw` (raw dwords of
// the activation dtype), accumulated into `acc`.
template <int BITS, int ACT>
__device__ __forceinline__ float unit_dot(const uint32_t (&q)[4], const uint32_t* xw,
                                          float s_act, const Masks& M, float acc) {
  if constexpr (ACT != DT_FP32 && BITS == 4) {
    GroupK k = group_consts<4>(s_act);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t wp[4];
      deq_word_i4<ACT>(q[i], k, M, wp);
#pragma unroll
      for (int t = 0; t < 4; ++t) acc = dot2<ACT>(wp[t], xw[4 * i + t], acc);
    }
  } else if constexpr (ACT != DT_FP32 && BITS == 8) {
    GroupK k = group_consts<8>(s_act);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t wp[2];
      deq_word_i8<ACT>(q[i], k, M, wp);
      acc = dot2<ACT>(wp[0], xw[2 * i], acc);
      acc = dot2<ACT>(wp[1], xw[2 * i + 1], acc);
    }
  } else {
    constexpr int PER = 32 / BITS;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int e = i * PER + j;
        float w = deq_code<ACT, BITS>(q[i], j, s_act);
        float xv;
        if constexpr (ACT == DT_FP32) {
          xv = __builtin_bit_cast(float, xw[e]);
        } else if constexpr (ACT == DT_BF16) {
          uint32_t d = xw[e >> 1];
          xv = __builtin_bit_cast(float, (e & 1) ? (d & 0xFFFF0000u) : (d << 16));
        } else {
          f16x2 d = __builtin_bit_cast(f16x2, xw[e >> 1]);
          xv = (float)((e & 1) ? d.y : d.x);
        }
        acc = __builtin_fmaf(w, xv, acc);
      }
    }
  }
  return acc;
}

__device__ __forceinline__ float load_scale_rt(const void* p, int64_t i, int dt) {
  if (dt == DT_BF16) return load_as_float<DT_BF16>(p, i);
  if (dt == DT_FP16) return load_as_float<DT_FP16>(p, i);
  return load_as_float<DT_FP32>(p, i);
}

__device__ __forceinline__ float lane_group_sum(float v, int lpr) {
  for (int m = lpr >> 1; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Activation dwords per 16-byte unit of codes.
template <int BITS, int ACT>
struct UnitX {
  static constexpr int CODES = 128 / BITS;
  static constexpr int DWORDS = ACT == DT_FP32 ? CODES : CODES / 2;
};

template <int BITS, int ACT>
__device__ __forceinline__ void load_x_slice(const void* x, int64_t col, uint32_t* xw) {
  constexpr int D = UnitX<BITS, ACT>::DWORDS;
  const uint4* src = (const uint4*)((const char*)x + col * (ACT == DT_FP32 ? 4 : 2));
#pragma unroll
  for (int i = 0; i < D / 4; ++i) {
    uint4 v = src[i];
    xw[4 * i] = v.x; xw[4 * i + 1] = v.y; xw[4 * i + 2] = v.z; xw[4 * i + 3] = v.w;
  }
}

// grid: one wave per (pair, RPW*RI rows); block = 256 threads (4 waves).
template <int BITS, int ACT, int RI>
__global__ void __launch_bounds__(256)
decode_gate_up_kernel(const void* __restrict__ x, const int64_t* __restrict__ tbl,
                      void* __restrict__ h, int n_pairs, int hidden, int inter, int group,
                      int sc_dt, int lpr, int units, int64_t gate_w, int64_t gate_s,
                      int64_t up_w, int64_t up_s) {
  constexpr int CPU = UnitX<BITS, ACT>::CODES;
  constexpr int XD = UnitX<BITS, ACT>::DWORDS;
  const int lane = threadIdx.x & 63;
  const int rpw = 64 / lpr;
  const int gi = lane / lpr, j = lane % lpr;
  const int rows_per_wave = rpw * RI;
  const int waves_per_pair = (inter + rows_per_wave - 1) / rows_per_wave;
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int p = (int)(wave / waves_per_pair);
  if (p >= n_pairs) return;
  const int row0 = (int)(wave % waves_per_pair) * rows_per_wave + gi * RI;
  const int32_t* pk = (const int32_t*)tbl[3 * p];
  const void* sc = (const void*)tbl[3 * p + 1];
  const int64_t words_row = (int64_t)hidden * BITS / 32;
  const int64_t groups_row = hidden / group;
  const Masks M = make_masks();

  float ag[RI], au[RI];
#pragma unroll
  for (int r = 0; r < RI; ++r) { ag[r] = 0.f; au[r] = 0.f; }

  for (int u = 0; u < units; ++u) {
    const int unit = j + u * lpr;
    const int64_t col = (int64_t)unit * CPU;
    uint32_t qg[RI][4], qu[RI][4];
    float sg[RI], su[RI];
#pragma unroll
    for (int r = 0; r < RI; ++r) {
      const int row = row0 + r;
      if (row < inter) {
        const uint4 a = *(const uint4*)(pk + gate_w + row * words_row + unit * 4);
        const uint4 b = *(const uint4*)(pk + up_w + row * words_row + unit * 4);
        qg[r][0] = a.x; qg[r][1] = a.y; qg[r][2] = a.z; qg[r][3] = a.w;
        qu[r][0] = b.x; qu[r][1] = b.y; qu[r][2] = b.z; qu[r][3] = b.w;
        sg[r] = load_scale_rt(sc, gate_s + row * groups_row + col / group, sc_dt);
        su[r] = load_scale_rt(sc, up_s + row * groups_row + col / group, sc_dt);
      }
    }
    uint32_t xw[XD];
    load_x_slice<BITS, ACT>(x, col, xw);
#pragma unroll
    for (int r = 0; r < RI; ++r) {
      if (row0 + r < inter) {
        ag[r] = unit_dot<BITS, ACT>(qg[r], xw, round_act<ACT>(sg[r]), M, ag[r]);
        au[r] = unit_dot<BITS, ACT>(qu[r], xw, round_act<ACT>(su[r]), M, au[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RI; ++r) {
    ag[r] = lane_group_sum(ag[r], lpr);
    au[r] = lane_group_sum(au[r], lpr);
  }
#pragma unroll
  for (int r = 0; r < RI; ++r) {
    const int row = row0 + r;
    if (j == r && row < inter)
      store_act<ACT>(h, (int64_t)p * inter + row, silu_mul<ACT>(ag[r], au[r]));
  }
}

// block: `waves` waves split as pair_split x row_split; each wave takes pairs
// p = pl, pl + pair_split, ... for its RPW*RI rows; the contributions go to LDS and are
// summed in table order at the end.
template <int BITS, int ACT, int RI>
__global__ void __launch_bounds__(512)
decode_down_kernel(const void* __restrict__ h, const int64_t* __restrict__ tbl,
                   const void* __restrict__ rw, int rw_dt, float* __restrict__ out,
                   int n_pairs, int hidden, int inter, int group, int sc_dt, int lpr,
                   int units, int pair_split, int64_t down_w, int64_t down_s, int w_round) {
  constexpr int CPU = UnitX<BITS, ACT>::CODES;
  constexpr int XD = UnitX<BITS, ACT>::DWORDS;
  extern __shared__ float cbuf[];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int rpw = 64 / lpr;
  const int gi = lane / lpr, j = lane % lpr;
  const int row_split = nw / pair_split;
  const int pl = wv % pair_split, rp = wv / pair_split;
  const int wg_rows = row_split * rpw * RI;
  const int row_base = blockIdx.x * wg_rows;
  const int my0 = rp * rpw * RI + gi * RI;         // first of this group's rows, in-block
  const int64_t words_row = (int64_t)inter * BITS / 32;
  const int64_t groups_row = inter / group;
  const Masks M = make_masks();

  for (int p = pl; p < n_pairs; p += pair_split) {
    const int32_t* pk = (const int32_t*)tbl[3 * p];
    const void* sc = (const void*)tbl[3 * p + 1];
    const int64_t slot = tbl[3 * p + 2];
    const void* hp = (const char*)h + (int64_t)p * inter * (ACT == DT_FP32 ? 4 : 2);
    float acc[RI];
#pragma unroll
    for (int r = 0; r < RI; ++r) acc[r] = 0.f;
    for (int u = 0; u < units; ++u) {
      const int unit = j + u * lpr;
      const int64_t col = (int64_t)unit * CPU;
      uint32_t q[RI][4];
      float s[RI];
#pragma unroll
      for (int r = 0; r < RI; ++r) {
        const int row = row_base + my0 + r;
        if (row < hidden) {
          const uint4 a = *(const uint4*)(pk + down_w + row * words_row + unit * 4);
          q[r][0] = a.x; q[r][1] = a.y; q[r][2] = a.z; q[r][3] = a.w;
          s[r] = load_scale_rt(sc, down_s + row * groups_row + col / group, sc_dt);
        }
      }
      uint32_t xw[XD];
      load_x_slice<BITS, ACT>(hp, col, xw);
#pragma unroll
      for (int r = 0; r < RI; ++r)
        if (row_base + my0 + r < hidden)
          acc[r] = unit_dot<BITS, ACT>(q[r], xw, round_act<ACT>(s[r]), M, acc[r]);
    }
    const float wgt = load_scale_rt(rw, slot, rw_dt);
#pragma unroll
    for (int r = 0; r < RI; ++r) {
      float v = lane_group_sum(acc[r], lpr);
      // The product is rounded to fp32 on its own (stored to LDS before any add), as
      // stock's `y * weight` then `out +=` are two roundings.
      float c = round_act<ACT>(v) * wgt;
      if (w_round) c = round_act<ACT>(c);
      if (j == 0) cbuf[p * wg_rows + my0 + r] = c;
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < wg_rows; t += blockDim.x) {
    const int row = row_base + t;
    if (row >= hidden) continue;
    float o = 0.f;
    for (int p = 0; p < n_pairs; ++p) o += cbuf[p * wg_rows + t];
    out[row] = o;
  }
}

// ── host side ──────────────────────────────────────────────────────────────────────────

static int pow2_divisor(int64_t n, int cap) {
  int b = cap;
  while (b > 1 && n % b) b >>= 1;
  return b;
}

// Why the decode kernels cannot take this geometry, or nullptr.
const char* decode_unsupported(const vaayu_geom* g, int act) {
  if (g->bits != 1 && g->bits != 2 && g->bits != 4 && g->bits != 8) return "bit width";
  const int cpu = 128 / g->bits;                   // codes per 16-byte unit
  if (g->group % cpu) return "group size smaller than a 16-byte unit of codes";
  if (g->hidden % cpu || g->inter % cpu) return "a row is not a whole number of 16-byte units";
  if (g->hidden % g->group || g->inter % g->group) return "a row is not whole groups";
  if (act < 0 || act > 2) return "activation dtype";
  return nullptr;
}

template <int BITS, int ACT>
static void launch_gate_up(const void* x, const int64_t* tbl, void* h, int n, const vaayu_geom* g,
                           int sc_dt, hipStream_t st) {
  const int units_row = g->hidden * BITS / 128;
  const int lpr = pow2_divisor(units_row, 64);
  const int units = units_row / lpr;
  const int rpw = 64 / lpr;
  int ri = rpw >= 4 ? 1 : (rpw == 2 ? 2 : 4);
  const int rows_per_wave = rpw * ri;
  const int64_t waves = (int64_t)n * ((g->inter + rows_per_wave - 1) / rows_per_wave);
  const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
#define GU(RI_)                                                                             \
  hipLaunchKernelGGL((decode_gate_up_kernel<BITS, ACT, RI_>), grid, block, 0, st, x, tbl, h, n, \
                     g->hidden, g->inter, g->group, sc_dt, lpr, units, g->gate_w, g->gate_s,  \
                     g->up_w, g->up_s)
  if (ri == 1) GU(1); else if (ri == 2) GU(2); else GU(4);
#undef GU
}

template <int BITS, int ACT>
static int launch_down(const void* h, const int64_t* tbl, const void* rw, int rw_dt, float* out,
                       int n, const vaayu_geom* g, int sc_dt, int w_round, hipStream_t st) {
  const int units_row = g->inter * BITS / 128;
  const int lpr = pow2_divisor(units_row, 64);
  const int units = units_row / lpr;
  const int rpw = 64 / lpr;
  const int ri = rpw >= 8 ? 1 : (rpw >= 2 ? 2 : 4);
  const int waves = 8;
  int ps = 1;
  while (ps < waves && ps < n) ps <<= 1;           // pair split: a power of two <= 8
  const int row_split = waves / ps;
  const int wg_rows = row_split * rpw * ri;
  const size_t lds = (size_t)n * wg_rows * sizeof(float);
  if (lds > 64 * 1024) return set_error(-3, "decode down: too many pairs for one block's LDS");
  const dim3 grid((unsigned)((g->hidden + wg_rows - 1) / wg_rows)), block(64 * waves);
#define DN(RI_)                                                                               \
  hipLaunchKernelGGL((decode_down_kernel<BITS, ACT, RI_>), grid, block, lds, st, h, tbl, rw,      \
                     rw_dt, out, n, g->hidden, g->inter, g->group, sc_dt, lpr, units, ps,       \
                     g->down_w, g->down_s, w_round)
  if (ri == 1) DN(1); else if (ri == 2) DN(2); else DN(4);
#undef DN
  return 0;
}

template <template <int, int> class F, typename... A>
static int dispatch_bits_act(int bits, int act, A... args) {
#define CASE(B_, A_) if (bits == B_ && act == A_) return F<B_, A_>::run(args...);
  CASE(4, 0) CASE(4, 1) CASE(4, 2) CASE(8, 0) CASE(8, 1) CASE(8, 2)
  CASE(2, 0) CASE(2, 1) CASE(2, 2) CASE(1, 0) CASE(1, 1) CASE(1, 2)
#undef CASE
  return set_error(-2, "unsupported bit width / activation dtype");
}

template <int B, int A>
struct GateUpF {
  static int run(const void* x, const int64_t* tbl, void* h, int n, const vaayu_geom* g, int sc,
                 hipStream_t st) {
    launch_gate_up<B, A>(x, tbl, h, n, g, sc, st);
    return 0;
  }
};

template <int B, int A>
struct DownF {
  static int run(const void* h, const int64_t* tbl, const void* rw, int rw_dt, float* out, int n,
                 const vaayu_geom* g, int sc, int w_round, hipStream_t st) {
    return launch_down<B, A>(h, tbl, rw, rw_dt, out, n, g, sc, w_round, st);
  }
};

}  // namespace vaayu

using namespace vaayu;

extern "C" int vaayu_decode_gate_up(const void* x, const int64_t* table, void* h, int32_t n_pairs,
                                    const vaayu_geom* geom, int32_t act, int32_t scale_dtype,
                                    void* stream) {
  clear_error();
  if (!x || !table || !h || !geom) return set_error(-1, "null pointer argument");
  if (n_pairs <= 0) return set_error(-1, "n_pairs must be positive");
  if (scale_dtype < 0 || scale_dtype > 2) return set_error(-1, "scale dtype");
  if (const char* why = decode_unsupported(geom, act)) return set_error(-2, why);
  int rc = dispatch_bits_act<GateUpF>(geom->bits, act, x, table, h, (int)n_pairs, geom,
                                      (int)scale_dtype, (hipStream_t)stream);
  return rc ? rc : check_launch("decode gate/up");
}

extern "C" int vaayu_decode_down(const void* h, const int64_t* table, const void* routing_weights,
                                 int32_t rw_dtype, float* out, int32_t n_pairs,
                                 const vaayu_geom* geom, int32_t act, int32_t scale_dtype,
                                 int32_t w_round, void* stream) {
  clear_error();
  if (!h || !table || !routing_weights || !out || !geom)
    return set_error(-1, "null pointer argument");
  if (n_pairs <= 0) return set_error(-1, "n_pairs must be positive");
  if (scale_dtype < 0 || scale_dtype > 2 || rw_dtype < 0 || rw_dtype > 2)
    return set_error(-1, "scale / routing-weight dtype");
  if (const char* why = decode_unsupported(geom, act)) return set_error(-2, why);
  int rc = dispatch_bits_act<DownF>(geom->bits, act, h, table, routing_weights, (int)rw_dtype, out,
                                    (int)n_pairs, geom, (int)scale_dtype, (int)w_round,
                                    (hipStream_t)stream);
  return rc ? rc : check_launch("decode down");
}
