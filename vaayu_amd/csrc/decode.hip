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
// load instruction reads LPR*16 contiguous bytes of a row. Lanes keep their columns for
// every row they visit, so their slice of the activation vector sits in registers and
// is reused across the RI rows (and both roles) of the group. Codes are dequantized in
// registers (common.hpp) and dotted with v_dot2. A group's partial sums are reduced with
// a transposed butterfly (each exchange halves the values a lane carries). The pair
// index, the table entries and the expert pointers are wave-uniform scalars.
//
// Nothing is atomic: the fp32 sum over pairs runs sequentially in table order from LDS.
#include "common.hpp"
#include "abi_internal.hpp"

namespace vaayu {

template <int SC>
__device__ __forceinline__ float load_scale(const void* base, uint32_t i) {
  return load_as_float<SC>(base, (int64_t)i);
}

// Dot of one 16-byte unit of codes with the matching activation slice `xw` (raw dwords
// of the activation dtype), accumulated into `acc`. Fast path: bf16/fp16 activations,
// 4- or 8-bit codes.
template <int BITS, int ACT>
__device__ __forceinline__ float unit_dot_fast(const uint4& q, const uint32_t* xw, float s_act,
                                               const Masks& M, float acc) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  if constexpr (BITS == 4) {
    GroupK k = group_consts<4>(s_act);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t wp[4];
      deq_word_i4<ACT>(w[i], k, M, wp);
#pragma unroll
      for (int t = 0; t < 4; ++t) acc = dot2<ACT>(wp[t], xw[4 * i + t], acc);
    }
  } else {
    GroupK k = group_consts<8>(s_act);
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

// General path (any activation dtype, any of 1/2/4/8-bit codes), one code at a time.
template <int BITS, int ACT>
__device__ __forceinline__ float unit_dot_general(const uint4& q, const uint32_t* xw,
                                                  float s_act, float acc) {
  constexpr int PER = 32 / BITS;
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int jj = 0; jj < PER; ++jj) {
      const int e = i * PER + jj;
      const float wt = deq_code<ACT, BITS>(w[i], jj, s_act);
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

template <int BITS, int ACT>
struct Unit {
  static constexpr int CODES = 128 / BITS;                          // codes per 16 B unit
  static constexpr int XU = (ACT == DT_FP32 ? 4 * CODES : 2 * CODES) / 16;  // x uint4s
  static constexpr bool FAST = ACT != DT_FP32 && (BITS == 4 || BITS == 8);
};

template <int BITS, int ACT>
__device__ __forceinline__ float unit_dot(const uint4& q, const uint4 (&x)[Unit<BITS, ACT>::XU],
                                          float s_act, const Masks& M, float acc) {
  const uint32_t* xw = (const uint32_t*)&x[0];
  if constexpr (Unit<BITS, ACT>::FAST) return unit_dot_fast<BITS, ACT>(q, xw, s_act, M, acc);
  else return unit_dot_general<BITS, ACT>(q, xw, s_act, acc);
}

// Sum NV per-lane values over the `lpr` lanes of each aligned lane group (NV <= lpr, both
// powers of two). Transposed butterfly: each exchange halves the values a lane carries,
// then a plain butterfly finishes. On return lane j (in-group index) holds the group
// total of value number j / (lpr / NV).
// mask ? a : b as one v_bfi_b32 (kept opaque so the compiler does not turn the selects
// of the butterfly below into dynamically indexed register reads).
__device__ __forceinline__ float bit_select(uint32_t mask, float a, float b) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3"
      : "=v"(r)
      : "v"(mask), "v"(__builtin_bit_cast(uint32_t, a)), "v"(__builtin_bit_cast(uint32_t, b)));
  return __builtin_bit_cast(float, r);
}

template <int NV>
__device__ __forceinline__ float group_reduce(float (&v)[NV], int lpr, int j) {
  int m = lpr >> 1;
#pragma unroll
  for (int n = NV; n > 1; n >>= 1) {
    const uint32_t upper = (j & m) ? 0xFFFFFFFFu : 0u;
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
  int units_row;     // 16 B units per row of the K dimension
  int lpr;           // lanes per row (power of two, <= 64)
  int units;         // units per lane per row = units_row / lpr
  int groups_row;    // scales per row
  int ushift;        // log2(units per scale group)
};

// Grid: one wave per (pair, lpr-groups x RI rows); blocks of 4 waves.
template <int BITS, int ACT, int SC, int RI>
__global__ void __launch_bounds__(256)
decode_gate_up_kernel(const uint4* __restrict__ xv, const int64_t* __restrict__ tbl,
                      void* __restrict__ h, DecodeShape s, int gate_w4, int gate_s,
                      int up_w4, int up_s) {
  using UT = Unit<BITS, ACT>;
  constexpr int NV = 2 * RI;
  const int lane = threadIdx.x & 63;
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rpw = 64 / s.lpr;
  const int gi = lane / s.lpr, j = lane & (s.lpr - 1);
  const int rows_per_wave = rpw * RI;
  const int wpp = (s.inter + rows_per_wave - 1) / rows_per_wave;
  const int wave = blockIdx.x * 4 + wib;
  const int p = wave / wpp;
  if (p >= s.n_pairs) return;
  const int row0 = (wave - p * wpp) * rows_per_wave + gi * RI;
  const uint4* pk = (const uint4*)tbl[3 * p];
  const void* sc = (const void*)tbl[3 * p + 1];
  const uint4* G = pk + gate_w4;
  const uint4* U = pk + up_w4;
  const Masks M = make_masks();

  float acc[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) acc[i] = 0.f;
  int rows[RI];
#pragma unroll
  for (int r = 0; r < RI; ++r) rows[r] = min(row0 + r, s.inter - 1);   // loads stay in bounds

  for (int u = 0; u < s.units; ++u) {
    const int unit = j + u * s.lpr;
    uint4 qg[RI], qu[RI];
    float sg[RI], su[RI];
#pragma unroll
    for (int r = 0; r < RI; ++r) {
      const uint32_t wi = (uint32_t)rows[r] * s.units_row + unit;
      qg[r] = G[wi];
      qu[r] = U[wi];
      const uint32_t si = (uint32_t)rows[r] * s.groups_row + (unit >> s.ushift);
      sg[r] = load_scale<SC>(sc, gate_s + si);
      su[r] = load_scale<SC>(sc, up_s + si);
    }
    uint4 xs[UT::XU];
#pragma unroll
    for (int i = 0; i < UT::XU; ++i) xs[i] = xv[unit * UT::XU + i];
#pragma unroll
    for (int r = 0; r < RI; ++r) {
      acc[2 * r] = unit_dot<BITS, ACT>(qg[r], xs, round_act<ACT>(sg[r]), M, acc[2 * r]);
      acc[2 * r + 1] = unit_dot<BITS, ACT>(qu[r], xs, round_act<ACT>(su[r]), M, acc[2 * r + 1]);
    }
  }
  const float tot = group_reduce<NV>(acc, s.lpr, j);
  const int stride = s.lpr / NV;                    // lanes per value after the reduce
  const float partner = __shfl_xor(tot, stride, 64);   // the up total next to each gate total
  const int q = j / stride;
  if ((j % stride) == 0 && (q & 1) == 0) {
    const int row = row0 + (q >> 1);
    if (row < s.inter) store_act<ACT>(h, (int64_t)p * s.inter + row, silu_mul<ACT>(tot, partner));
  }
}

// Block: 8 waves split as pair_split x row_split. Each wave takes pairs
// p = pl, pl + pair_split, ... over its rows; every contribution lands in LDS and the
// block then sums each row's contributions in table order.
template <int BITS, int ACT, int SC, int RI>
__global__ void __launch_bounds__(512)
decode_down_kernel(const void* __restrict__ h, const int64_t* __restrict__ tbl,
                   const void* __restrict__ rw, int rw_dt, float* __restrict__ out,
                   DecodeShape s, int pair_split, int down_w4, int down_s, int w_round) {
  using UT = Unit<BITS, ACT>;
  extern __shared__ float cbuf[];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rpw = 64 / s.lpr;
  const int gi = lane / s.lpr, j = lane & (s.lpr - 1);
  const int row_split = 8 / pair_split;
  const int pl = wv % pair_split, rp = wv / pair_split;
  const int wg_rows = row_split * rpw * RI;
  const int row_base = blockIdx.x * wg_rows;
  const int my0 = rp * rpw * RI + gi * RI;           // first of this group's rows, in-block
  const Masks M = make_masks();
  const int x_bytes = ACT == DT_FP32 ? 4 : 2;
  int rows[RI];
#pragma unroll
  for (int r = 0; r < RI; ++r) rows[r] = min(row_base + my0 + r, s.hidden - 1);

  for (int p = pl; p < s.n_pairs; p += pair_split) {
    const uint4* D = (const uint4*)tbl[3 * p] + down_w4;
    const void* sc = (const void*)tbl[3 * p + 1];
    const int64_t slot = tbl[3 * p + 2];
    const uint4* hp = (const uint4*)((const char*)h + (int64_t)p * s.inter * x_bytes);
    float acc[RI];
#pragma unroll
    for (int r = 0; r < RI; ++r) acc[r] = 0.f;
    for (int u = 0; u < s.units; ++u) {
      const int unit = j + u * s.lpr;
      uint4 q[RI];
      float sd[RI];
#pragma unroll
      for (int r = 0; r < RI; ++r) {
        q[r] = D[(uint32_t)rows[r] * s.units_row + unit];
        sd[r] = load_scale<SC>(sc, down_s + (uint32_t)rows[r] * s.groups_row + (unit >> s.ushift));
      }
      uint4 xs[UT::XU];
#pragma unroll
      for (int i = 0; i < UT::XU; ++i) xs[i] = hp[unit * UT::XU + i];
#pragma unroll
      for (int r = 0; r < RI; ++r)
        acc[r] = unit_dot<BITS, ACT>(q[r], xs, round_act<ACT>(sd[r]), M, acc[r]);
    }
    const float wgt = rw_dt == DT_FP32 ? load_as_float<DT_FP32>(rw, slot)
                    : rw_dt == DT_BF16 ? load_as_float<DT_BF16>(rw, slot)
                                       : load_as_float<DT_FP16>(rw, slot);
    const float tot = group_reduce<RI>(acc, s.lpr, j);
    const int stride = s.lpr / RI;
    if ((j % stride) == 0) {
      // The product is rounded to fp32 on its own (it goes to LDS before any add), as
      // stock's `y * weight` then `out +=` are two roundings.
      float c = round_act<ACT>(tot) * wgt;
      if (w_round) c = round_act<ACT>(c);
      cbuf[p * wg_rows + my0 + j / stride] = c;
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < wg_rows; t += blockDim.x) {
    const int row = row_base + t;
    if (row >= s.hidden) continue;
    float o = 0.f;
    for (int p = 0; p < s.n_pairs; ++p) o += cbuf[p * wg_rows + t];
    out[row] = o;
  }
}

// ── host side ──────────────────────────────────────────────────────────────────────────

static int pow2_divisor(int64_t n, int cap) {
  int b = cap;
  while (b > 1 && n % b) b >>= 1;
  return b;
}

static int ilog2(int v) {
  int r = 0;
  while ((1 << r) < v) ++r;
  return r;
}

// Why the decode kernels cannot take this geometry, or nullptr.
const char* decode_unsupported(const vaayu_geom* g, int act) {
  if (g->bits != 1 && g->bits != 2 && g->bits != 4 && g->bits != 8) return "bit width";
  const int cpu = 128 / g->bits;                   // codes per 16-byte unit
  if (g->group % cpu || (g->group & (g->group - 1)))
    return "group size is not a power of two holding whole 16-byte units of codes";
  if (g->hidden % cpu || g->inter % cpu) return "a row is not a whole number of 16-byte units";
  if ((g->hidden / cpu) % 2) return "hidden is not an even number of 16-byte units of codes";
  if (g->hidden % g->group || g->inter % g->group) return "a row is not whole groups";
  if ((g->gate_w | g->up_w | g->down_w) & 3) return "role offsets are not 16-byte aligned";
  if (g->down_w / 4 > INT32_MAX || g->up_w / 4 > INT32_MAX) return "blob too large";
  if (act < 0 || act > 2) return "activation dtype";
  return nullptr;
}

static DecodeShape shape_for(const vaayu_geom* g, int n, int k_dim) {
  DecodeShape s;
  s.n_pairs = n;
  s.inter = g->inter;
  s.hidden = g->hidden;
  s.units_row = k_dim * g->bits / 128;
  s.lpr = pow2_divisor(s.units_row, 64);
  s.units = s.units_row / s.lpr;
  s.groups_row = k_dim / g->group;
  s.ushift = ilog2(g->group * g->bits / 128);
  return s;
}

template <int BITS, int ACT, int SC>
static int launch_gate_up(const void* x, const int64_t* tbl, void* h, int n, const vaayu_geom* g,
                          hipStream_t st) {
  DecodeShape s = shape_for(g, n, g->hidden);
  const int rpw = 64 / s.lpr;
  // rows per lane group: enough rows per wave that each wave streams several KB
  int ri = rpw >= 4 ? 1 : (rpw == 2 ? 2 : 4);
  if (2 * ri > s.lpr) ri = s.lpr / 2 > 0 ? s.lpr / 2 : 1;
  const int rows_per_wave = rpw * ri;
  const int64_t waves = (int64_t)n * ((g->inter + rows_per_wave - 1) / rows_per_wave);
  const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
  const int gw = (int)(g->gate_w / 4), uw = (int)(g->up_w / 4);
#define GU(RI_)                                                                                \
  hipLaunchKernelGGL((decode_gate_up_kernel<BITS, ACT, SC, RI_>), grid, block, 0, st,         \
                     (const uint4*)x, tbl, h, s, gw, (int)g->gate_s, uw, (int)g->up_s)
  if (ri == 1) GU(1); else if (ri == 2) GU(2); else GU(4);
#undef GU
  return 0;
}

template <int BITS, int ACT, int SC>
static int launch_down(const void* h, const int64_t* tbl, const void* rw, int rw_dt, float* out,
                       int n, const vaayu_geom* g, int w_round, hipStream_t st) {
  DecodeShape s = shape_for(g, n, g->inter);
  const int rpw = 64 / s.lpr;
  int ps = 1;
  while (ps < 8 && ps < n) ps <<= 1;               // pair split: a power of two <= 8
  const int row_split = 8 / ps;
  int ri = 1;
  while (ri < 4 && ri * 2 <= s.lpr && row_split * rpw * ri < 8) ri <<= 1;
  const int wg_rows = row_split * rpw * ri;
  const size_t lds = (size_t)n * wg_rows * sizeof(float);
  if (lds > 64 * 1024) return set_error(-3, "decode down: too many pairs for one block's LDS");
  const dim3 grid((unsigned)((g->hidden + wg_rows - 1) / wg_rows)), block(512);
  const int dw = (int)(g->down_w / 4);
#define DN(RI_)                                                                              \
  hipLaunchKernelGGL((decode_down_kernel<BITS, ACT, SC, RI_>), grid, block, lds, st, h, tbl, rw, \
                     rw_dt, out, s, ps, dw, (int)g->down_s, w_round)
  if (ri == 1) DN(1); else if (ri == 2) DN(2); else DN(4);
#undef DN
  return 0;
}

// (bits, act, scale dtype) -> template instance.
template <template <int, int, int> class F, typename... A>
static int dispatch(int bits, int act, int sc, A... args) {
#define SCS(B_, A_)                                          \
  if (bits == B_ && act == A_) {                             \
    if (sc == DT_BF16) return F<B_, A_, DT_BF16>::run(args...); \
    if (sc == DT_FP16) return F<B_, A_, DT_FP16>::run(args...); \
    return F<B_, A_, DT_FP32>::run(args...);                 \
  }
  SCS(4, 0) SCS(4, 1) SCS(4, 2) SCS(8, 0) SCS(8, 1) SCS(8, 2)
  SCS(2, 0) SCS(2, 1) SCS(2, 2) SCS(1, 0) SCS(1, 1) SCS(1, 2)
#undef SCS
  return set_error(-2, "unsupported bit width / activation dtype");
}

template <int B, int A, int S>
struct GateUpF {
  static int run(const void* x, const int64_t* tbl, void* h, int n, const vaayu_geom* g,
                 hipStream_t st) {
    return launch_gate_up<B, A, S>(x, tbl, h, n, g, st);
  }
};

template <int B, int A, int S>
struct DownF {
  static int run(const void* h, const int64_t* tbl, const void* rw, int rw_dt, float* out, int n,
                 const vaayu_geom* g, int w_round, hipStream_t st) {
    return launch_down<B, A, S>(h, tbl, rw, rw_dt, out, n, g, w_round, st);
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
  if (((uintptr_t)x) & 15) return set_error(-1, "x must be 16-byte aligned");
  if (const char* why = decode_unsupported(geom, act)) return set_error(-2, why);
  int rc = dispatch<GateUpF>(geom->bits, act, scale_dtype, x, table, h, (int)n_pairs, geom,
                             (hipStream_t)stream);
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
  if (((uintptr_t)h) & 15) return set_error(-1, "h must be 16-byte aligned");
  if (const char* why = decode_unsupported(geom, act)) return set_error(-2, why);
  int rc = dispatch<DownF>(geom->bits, act, scale_dtype, h, table, routing_weights, (int)rw_dtype,
                           out, (int)n_pairs, geom, (int)w_round, (hipStream_t)stream);
  return rc ? rc : check_launch("decode down");
}
