// Decode kernels on MFMA (bf16 / fp16 activations; int4, int8, e4m3 and e2m1 codes).
//
// Same results as the VALU kernels in decode_kernels.hpp (the stock path's rounding points,
// vaayu/packed_expert_kernels.py:131-176): only the fp32 dot products move from v_dot2 to
// v_mfma_f32_16x16x32_{bf16,f16}, which frees the VALU for the dequant (the bound of these
// kernels once their loads are in flight) and removes the cross-lane reduction.
//
// Mapping of a one-token GEMV onto a 16x16x32 MFMA: the 16 B columns are (weight row, K part)
// pairs and the A rows m < KP carry the activation vector's K part m, so D[m][c] is the dot
// of column c's K part with part m of the vector; the kernel keeps D[kp(c)][c] and sums the
// parts. Lane (q, c) (q = lane / 16, c = lane % 16) loads 16-byte unit 4*step + q of
// column c's part and dequantizes it straight into B operands; the MFMA's 32 K slots of
// quarter q map to codes [8i, 8i + 8) of that unit for operand i, and A uses the same map.
// Rows m >= KP of A are left as whatever the lanes hold: D rows other than D[kp(c)][c] are
// never read.
#pragma once
#include <algorithm>

#include "decode_kernels.hpp"

namespace vaayu {

template <int ACT>
__device__ __forceinline__ f32x4 mfma_16x16x32(uint4 a, uint4 b, f32x4 c) {
  if constexpr (ACT == DT_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// DPP moves inside each row of 16 lanes: rotate right by 4 / by 8, and lane ^ 2 in a quad.
enum { kRowRor4 = 0x124, kRowRor8 = 0x128, kQuadXor2 = 0x4E };

template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

template <int F>
struct MUnit {
  static constexpr int CPU = 128 / CodeBits<F>::value;   // codes per 16-byte unit
  static constexpr int NMF = CPU / 8;                     // MFMA operands per unit
  static constexpr bool INT = F < 100;                    // scale rounded to the act dtype
};

// The B operands of one unit of codes: NMF uint4 of 8 weights (4 packed pairs) each, in code
// order. `s` is the applied scale (rounded to the activation dtype for integer codes, raw
// fp32 / E8M0 value for e4m3 and e2m1).
template <int F, int ACT>
__device__ __forceinline__ void unit_b(const uint4& q, float s, const Masks& M,
                                       uint4 (&b)[MUnit<F>::NMF]) {
  const GroupK k = group_of<F>(s);
#pragma unroll
  for (int i = 0; i < MUnit<F>::NMF; ++i) b[i] = operand_i<F, ACT>(q, k, s, M, i);
}

// One MFMA decode launch's geometry (filled on the host by mfma_shape).
struct MShape {
  int n_pairs;
  int rows;              // output rows: inter (gate/up) or hidden (down)
  int units_row;         // 16-byte units of codes per row (the K dimension)
  int part_units;        // units per K part = units_row / KP
  int steps;             // part_units / 4: one unit per lane quarter per step
  int groups_row;        // scales per row
  int ushift;            // log2(units per scale group)
  int rshift;            // log2(rows per scale block): 0 but for block-scaled e4m3
  int sc_dt;             // scale dtype code
  int vec16;             // uint4 of the activation vector(s) staged in LDS
  uint32_t wb0, wb1;     // byte offsets of the roles' codes (gate, up; down in wb0)
  uint32_t sc0, sc1;     // element offsets of the roles' scales
  uint32_t code_bytes;   // buffer extent of the codes from the blob's packed address
  uint32_t scale_bytes;  // buffer extent of the scales from the blob's scale address
};

// fp32 dot of one lane's column part with the staged vector, one unit per step. begin()
// issues the loads (so a caller can put them in flight before it stages the vector);
// finish() runs the steps. NS > 0: exactly NS steps, every load issued up front in straight
// code (so the compiler's wait counts stay exact); NS == 0: s.steps steps in chunks of four,
// the next chunk's loads issued before the current chunk's dequant (a partial last chunk
// reads past the part, within the buffer or as zeros, and does not use it).
// cbase / sbase: byte offset of the lane's first unit and element index of its row's first
// scale; u0 its first unit's index in the row (for the scale group); `xa` the lane's A
// operands (read where a_lane). NT: the codes are requested non-temporal.
template <int F, int ACT, int SW, int NS, bool NT = true>
struct ColumnDot {
  static constexpr int NMF = MUnit<F>::NMF;
  static constexpr int NB = NS > 0 ? NS : 4;       // steps per register chunk
  rsrc_t P, S;
  uint32_t cbase, sbase, u0;
  int ushift;
  uint4 qa[NB], qb[NB];
  uint32_t sa[NB], sb[NB];

  // Requests go out as (codes, scale) of step 0, then of step 1, ...: the wait counter is
  // in order, so step i's dequant then waits only for steps 0..i, not for every code of the
  // chunk (the scheduling barriers stop the compiler from grouping all code loads first).
  __device__ __forceinline__ void load(uint4 (&qv)[NB], uint32_t (&sv)[NB], int st0) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      qv[i] = NT ? buf_load16_nt(P, cbase + (uint32_t)(st0 + i) * 64u)
                 : buf_load16(P, cbase + (uint32_t)(st0 + i) * 64u);
      sv[i] = buf_load_scale<SW>(S, sbase + ((u0 + 4u * (uint32_t)(st0 + i)) >> ushift));
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  __device__ __forceinline__ void begin(rsrc_t P_, rsrc_t S_, uint32_t cbase_, uint32_t sbase_,
                                        uint32_t u0_, const MShape& s) {
    P = P_; S = S_; cbase = cbase_; sbase = sbase_; u0 = u0_;
    ushift = s.ushift;
    load(qa, sa, 0);
  }

  __device__ __forceinline__ void step(f32x4& acc, const uint4& qv, uint32_t sv, int st,
                                       int sc_dt, const uint4* xa, bool a_lane, const Masks& M) {
    const float sc = applied_scale<F, ACT>(scale_value<SW>(sv, sc_dt));
    uint4 b[NMF];
    unit_b<F, ACT>(qv, sc, M, b);
    uint4 a[NMF];
    if (a_lane) {
#pragma unroll
      for (int i = 0; i < NMF; ++i) a[i] = xa[st * 4 * NMF + i];
    }
#pragma unroll
    for (int i = 0; i < NMF; ++i) acc = mfma_16x16x32<ACT>(a[i], b[i], acc);
  }

  __device__ __forceinline__ void chunk(f32x4& acc, const uint4 (&qv)[NB], const uint32_t (&sv)[NB],
                                        int st0, int ns, int sc_dt, const uint4* xa, bool a_lane,
                                        const Masks& M) {
#pragma unroll
    for (int i = 0; i < NB; ++i)
      if (NS > 0 || st0 + i < ns) step(acc, qv[i], sv[i], st0 + i, sc_dt, xa, a_lane, M);
  }

  __device__ __forceinline__ f32x4 finish(const MShape& s, const uint4* xa, bool a_lane,
                                          const Masks& M) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if constexpr (NS > 0) {
      chunk(acc, qa, sa, 0, NS, s.sc_dt, xa, a_lane, M);
    } else {
      const int ns = s.steps;
      for (int st0 = 0;; st0 += 2 * NB) {
        if (st0 + NB < ns) load(qb, sb, st0 + NB);
        chunk(acc, qa, sa, st0, ns, s.sc_dt, xa, a_lane, M);
        if (st0 + NB >= ns) break;
        if (st0 + 2 * NB < ns) load(qa, sa, st0 + 2 * NB);
        chunk(acc, qb, sb, st0 + NB, ns, s.sc_dt, xa, a_lane, M);
        if (st0 + 2 * NB >= ns) break;
      }
    }
    return acc;
  }
};

// ── gate/up ─────────────────────────────────────────────────────────────────────────────
//
// Grid (ceil(inter / 8), n_pairs), 4 waves. Wave w of block (bx, p) takes rows
// r0 = 8 bx + 2 w and r0 + 1 of pair p in both roles: column c = 4 kp + 2 role + (row - r0)
// over the 4 K parts kp. The block stages x in LDS (up to 4 uint4 per thread) behind an
// LDS-only barrier while the codes stream. The four parts of a column
// are summed with two row rotations, the up total is fetched beside the gate total with a
// quad exchange, and lanes 0 and 1 write h.
template <int F, int ACT, int SW, int NS, bool NT>
__global__ void __launch_bounds__(256)
mfma_gate_up_kernel(const int64_t* __restrict__ tbl, const uint32_t* __restrict__ x,
                    void* __restrict__ h, MShape s) {
  extern __shared__ uint4 xl[];
  constexpr int CPU = MUnit<F>::CPU;
  const rsrc_t X = make_rsrc(x, (uint32_t)s.vec16 * 16u);
  const int xn = (s.vec16 + 255) >> 8;                       // uint4 of x per thread, <= 4
  uint4 xs[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (k < xn) xs[k] = buf_load16(X, (threadIdx.x + k * 256u) * 16u);
  const int p = blockIdx.y;
  const char* pk = (const char*)tbl[3 * p];
  const char* sc = (const char*)tbl[3 * p + 1];
  const int lane = threadIdx.x & 63;
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, c = lane & 15;
  const int kp = c >> 2, role = (c >> 1) & 1;
  const int row0 = blockIdx.x * 8 + wib * 2;
  const int row = min(row0 + (c & 1), s.rows - 1);
  const rsrc_t P = make_rsrc(pk, s.code_bytes);
  const rsrc_t S = make_rsrc(sc, s.scale_bytes);
  const uint32_t u0 = (uint32_t)(kp * s.part_units + q);
  const uint32_t cbase = (role ? s.wb1 : s.wb0) + ((uint32_t)row * s.units_row + u0) * 16u;
  const uint32_t sbase = (role ? s.sc1 : s.sc0) + (uint32_t)(row >> s.rshift) * s.groups_row;
  ColumnDot<F, ACT, SW, NS, NT> cd;
  cd.begin(P, S, cbase, sbase, u0, s);
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (k < xn) xl[threadIdx.x + k * 256] = xs[k];
  lds_barrier();
  const Masks M = make_masks();
  // A row c < 4 is x's part c: quarter q's operands of step t start at code
  // c * part_units * CPU + (4 t + q) * CPU.
  const uint4* xa = xl + (c * s.part_units + q) * (CPU / 8);
  const f32x4 acc = cd.finish(s, xa, c < 4, M);
  float v = kp == 0 ? acc[0] : kp == 1 ? acc[1] : kp == 2 ? acc[2] : acc[3];
  v += dpp_move<kRowRor4>(v);
  v += dpp_move<kRowRor8>(v);
  const float up = dpp_move<kQuadXor2>(v);
  if (lane < 2 && row0 + lane < s.rows)
    store_act<ACT>(h, (int64_t)p * s.rows + row0 + lane, silu_mul<ACT>(v, up));
}

// ── down + the fixed-order sum ──────────────────────────────────────────────────────────
//
// Grid: ceil(hidden / BR) blocks of 8 waves, BR = NRG * RG * RW rows per block. The waves
// are RG row groups x PS pair slots (RG * PS = 8); wave (g, pl) takes, for each of its NRG
// row groups of RW = 16 / KP rows, the pairs p = pl, pl + PS, ... Column c = kp * RW + (row -
// r0) over the KP = 2^kps K parts (1, 2 or 4). The block stages every pair's h in LDS; each
// wave writes
// c_p = fl32(round(y) * w[slot]) (+ one rounding when the routing weight is in the
// activation dtype) into LDS, and after one barrier the block sums each row's contributions
// sequentially in table order. Nothing is atomic.
template <int F, int ACT, int SW, int NS, bool ONE>
__global__ void __launch_bounds__(512)
mfma_down_kernel(const int64_t* __restrict__ tbl, const void* __restrict__ h,
                 const void* __restrict__ rw, float* __restrict__ out, MShape s, int rw_dt,
                 int kps, int ps, int nrg, int w_round) {
  constexpr int CPU = MUnit<F>::CPU;
  extern __shared__ uint4 lds[];
  const rsrc_t HV = make_rsrc(h, (uint32_t)s.vec16 * 16u);
  const int hn = (s.vec16 + 511) >> 9;                       // uint4 of h per thread, <= 8
  uint4 hs[8];
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (k < hn) hs[k] = buf_load16(HV, (threadIdx.x + k * 512u) * 16u);
  const int KP = 1 << kps;                                   // K parts: 1, 2 or 4
  const int RW = 16 >> kps;                                  // rows per row group
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, c = lane & 15;
  const int kp = c >> (4 - kps);
  const int rg = 8 / ps;
  const int pl = wv % ps, g = wv / ps;
  const int br = nrg * rg * RW;                              // rows per block
  const int p16 = s.units_row * CPU / 8;                     // uint4 of one pair's h
  float* cbuf = (float*)(lds + s.vec16);
  const uint32_t u0 = (uint32_t)(kp * s.part_units + q);
  ColumnDot<F, ACT, SW, NS> cd;     // codes non-temporal: no shape measured slower with it
  // the operands of (row group 0, pair pl) go out before the staging barrier (an idle wave,
  // pl >= n_pairs, loads pair 0's and does not use them)
  auto begin = [&](int gi, int p) {
    const char* pk = (const char*)tbl[3 * p];
    const char* sc = (const char*)tbl[3 * p + 1];
    const int row = min(blockIdx.x * br + (gi * rg + g) * RW + (c & (RW - 1)), s.rows - 1);
    cd.begin(make_rsrc(pk + s.wb0, s.code_bytes),
             make_rsrc(sc + (size_t)s.sc0 * (SW / 8), s.scale_bytes),
             ((uint32_t)row * s.units_row + u0) * 16u, (uint32_t)(row >> s.rshift) * s.groups_row,
             u0, s);
  };
  begin(0, pl < s.n_pairs ? pl : 0);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int i = threadIdx.x + k * 512;
    if (k < hn && i < s.vec16) lds[i] = hs[k];
  }
  lds_barrier();
  const Masks M = make_masks();
  // One (row group, pair) of this wave: the dot, the K-part sum, the weighted contribution.
  auto one = [&](int gi, int p, bool live) {
    const int brow = (gi * rg + g) * RW;                     // first row, in-block
    const int64_t slot = tbl[3 * p + 2];
    // The routing weight is requested before the dot's steps, so its latency overlaps them,
    // as two 16-bit loads with no branch on its dtype (a branch there would wait for every
    // request of the wave): the low half, and the high half of an fp32 weight (for a 16-bit
    // weight the same half again). Both stay inside the weight's own bytes.
    const int esz = rw_dt == DT_FP32 ? 4 : 2;
    const uint16_t* wp = (const uint16_t*)((const char*)rw + slot * esz);
    const uint16_t w_lo = wp[0];
    const uint16_t w_hi = wp[esz == 4 ? 1 : 0];
    __builtin_amdgcn_sched_barrier(0);
    const uint4* xa = lds + p * p16 + (c * s.part_units + q) * (CPU / 8);
    const f32x4 acc = cd.finish(s, xa, c < KP, M);
    float v = kp == 0 ? acc[0] : kp == 1 ? acc[1] : kp == 2 ? acc[2] : acc[3];
    if (KP == 4) v += dpp_move<kRowRor4>(v);
    if (KP >= 2) v += dpp_move<kRowRor8>(v);
    const float wgt = rw_dt == DT_FP32 ? __builtin_bit_cast(float, (uint32_t)w_hi << 16 | w_lo)
                    : rw_dt == DT_BF16 ? __builtin_bit_cast(float, (uint32_t)w_lo << 16)
                                       : (float)__builtin_bit_cast(_Float16, w_lo);
    if (live && lane < RW) {
      // The product is rounded to fp32 on its own (it goes to LDS before any add), as
      // stock's `y * weight` then `out +=` are two roundings.
      float cv = round_act<ACT>(v) * wgt;
      if (w_round) cv = round_act<ACT>(cv);
      cbuf[p * br + brow + lane] = cv;
    }
  };
  if constexpr (ONE) {
    // One row group and at most one pair per wave (its requests went out before the
    // staging barrier): straight code with no branch, so each step waits only for its own
    // codes. An idle wave (pl >= n_pairs) computes pair 0 and writes nothing. Inside the
    // loops below, the compiler waits for all of a wave's requests before its first step.
    one(0, pl < s.n_pairs ? pl : 0, pl < s.n_pairs);
  } else {
    for (int gi = 0; gi < nrg; ++gi)
      for (int p = pl; p < s.n_pairs; p += ps) {
        if (gi != 0 || p != pl) begin(gi, p);
        one(gi, p, true);
      }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < br; t += blockDim.x) {
    const int row = blockIdx.x * br + t;
    if (row >= s.rows) continue;
    float o = 0.f;
    for (int pp = 0; pp < s.n_pairs; ++pp) o += cbuf[pp * br + t];
    out[row] = o;
  }
}

// ── host-side planning ──────────────────────────────────────────────────────────────────

// Whether the MFMA kernels take this launch (bf16 / fp16 activations; int4, int8, e4m3,
// e2m1 codes), else the VALU kernels run.
inline bool mfma_format(int fmt, int act) {
  return (act == DT_BF16 || act == DT_FP16) && (fmt == 4 || fmt == 8 || fmt == F_E4M3 || fmt == F_MXFP4);
}

// Geometry of one MFMA launch over rows x k_dim (codes per row) with `kp` K parts.
inline MShape mfma_shape(const vaayu_geom* g, int fmt, int n, int rows, int k_dim, int kp,
                         int sc_dt) {
  MShape s{};
  const int cpu = 128 / (fmt % 100);
  s.n_pairs = n;
  s.rows = rows;
  s.units_row = k_dim / cpu;
  s.part_units = s.units_row / kp;
  s.steps = s.part_units / 4;
  s.groups_row = k_dim / g->group;
  s.ushift = ilog2(g->group / cpu);
  s.rshift = g->format == VAAYU_FMT_E4M3 ? ilog2(g->block_rows) : 0;
  s.sc_dt = sc_dt;
  return s;
}

// Bytes of a scale of dtype code `sc` (E8M0: 1).
inline int scale_bytes_of(int sc) { return sc == DT_FP32 ? 4 : sc == VAAYU_E8M0 ? 1 : 2; }

// The MFMA kernel's shape for this launch, or false when it does not take it: hidden is a
// multiple of 16 units (4 K parts x 4 lane quarters), x fits 4 uint4 per thread, and the
// two roles lie within 4 GiB of the blob's packed address.
inline bool mfma_gate_up_plan(const vaayu_geom* g, int fmt, int act, int n, int sc, MShape& s,
                              int& xs) {
  if (!mfma_format(fmt, act)) return false;
  const int cpu = 128 / (fmt % 100);
  if (g->hidden % cpu || (g->hidden / cpu) % 16) return false;
  s = mfma_shape(g, fmt, n, g->inter, g->hidden, 4, sc);
  s.vec16 = g->hidden / 8;
  xs = (s.vec16 + 255) / 256;
  if (xs > 4) return false;
  const int64_t role_bytes = (int64_t)g->inter * g->hidden * g->bits / 8;
  const int64_t code_end = std::max(g->gate_w, g->up_w) * 4 + role_bytes;
  const int64_t role_scales = (int64_t)(g->inter >> s.rshift) * (g->hidden / g->group);
  const int64_t scale_end = (std::max(g->gate_s, g->up_s) + role_scales) * scale_bytes_of(sc);
  if (code_end > 0xFFFFFFFFll || scale_end > 0xFFFFFFFFll) return false;
  s.wb0 = (uint32_t)(g->gate_w * 4);
  s.wb1 = (uint32_t)(g->up_w * 4);
  s.sc0 = (uint32_t)g->gate_s;
  s.sc1 = (uint32_t)g->up_s;
  s.code_bytes = (uint32_t)code_end;
  s.scale_bytes = (uint32_t)scale_end;
  return true;
}

struct DownPlan {
  MShape s;
  int kp, ps, nrg;
  size_t lds;
  unsigned blocks;
};

// The MFMA kernel's plan for this launch, or false when it does not take it. K parts: the
// most of 4, 2, 1 that split the intermediate dimension into whole steps (4 units each).
// Row groups per wave (nrg) keep the grid at kMaxDownBlocks blocks at most, since every
// block stages all pairs' h. A wave starts a row group's requests only when the previous
// one is done, so each extra row group exposes a full memory latency; up to 2048 blocks
// (h re-read from L2 per block) the straight one-group kernel is the faster trade.
constexpr int64_t kMaxDownBlocks = 2048;

inline bool mfma_down_plan(const vaayu_geom* g, int fmt, int act, int n, int sc, DownPlan& d) {
  if (!mfma_format(fmt, act)) return false;
  const int cpu = 128 / (fmt % 100);
  if (g->inter % cpu) return false;
  const int units = g->inter / cpu;
  d.kp = units % 16 == 0 ? 4 : units % 8 == 0 ? 2 : units % 4 == 0 ? 1 : 0;
  if (!d.kp) return false;
  d.s = mfma_shape(g, fmt, n, g->hidden, g->inter, d.kp, sc);
  const int64_t vec16 = (int64_t)n * g->inter / 8;
  if (vec16 > 8 * 512) return false;                          // h: up to 8 uint4 per thread
  d.s.vec16 = (int)vec16;
  d.ps = 1;
  while (d.ps < 8 && d.ps < n) d.ps <<= 1;
  const int rows_g = (8 / d.ps) * (16 / d.kp);               // rows per block per row group
  const int64_t blocks1 = (g->hidden + rows_g - 1) / rows_g;
  d.nrg = (int)std::max<int64_t>(1, (blocks1 + kMaxDownBlocks - 1) / kMaxDownBlocks);
  const int br = d.nrg * rows_g;
  d.blocks = (unsigned)((g->hidden + br - 1) / br);
  d.lds = (size_t)vec16 * 16 + (size_t)n * br * sizeof(float);
  if (d.lds > 64 * 1024) return false;
  const int64_t role_bytes = (int64_t)g->hidden * g->inter * g->bits / 8;
  const int64_t role_scales = (int64_t)(g->hidden >> d.s.rshift) * (g->inter / g->group);
  if (role_bytes > 0xFFFFFFFFll || role_scales * scale_bytes_of(sc) > 0xFFFFFFFFll) return false;
  d.s.wb0 = (uint32_t)(g->down_w * 4);
  d.s.sc0 = (uint32_t)g->down_s;
  d.s.code_bytes = (uint32_t)role_bytes;
  d.s.scale_bytes = (uint32_t)(role_scales * scale_bytes_of(sc));
  return true;
}


}  // namespace vaayu
