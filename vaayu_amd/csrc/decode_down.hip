// Decode down entry: vaayu_decode_down (kernels in decode_mfma.hpp for bf16 / fp16
// activations with 4- and 8-bit codes, decode_kernels.hpp otherwise).
#include "decode_mfma.hpp"

namespace vaayu {

// Step counts with a straight-line kernel; others run the chunked loop (NS = 0).
template <int F, int ACT, int SW>
static int mfma_down_at(const void* h, const int64_t* tbl, const void* rw, int rw_dt, float* out,
                        const DownPlan& d, int w_round, hipStream_t st) {
  const int kps = d.kp == 4 ? 2 : d.kp == 2 ? 1 : 0;
  // one (row group, pair) per wave: the straight-line variant
  const bool one = d.nrg == 1 && d.ps >= d.s.n_pairs;
#define DN(NS_, ONE_) hipLaunchKernelGGL((mfma_down_kernel<F, ACT, SW, NS_, ONE_>), dim3(d.blocks), \
                                         dim3(512), d.lds, st, tbl, h, rw, out, d.s, rw_dt, kps,  \
                                         d.ps, d.nrg, w_round)
#define DN2(NS_) if (one) DN(NS_, true); else DN(NS_, false)
  switch (d.s.steps) {
    case 1: DN2(1); break;
    case 2: DN2(2); break;
    case 3: DN2(3); break;
    case 4: DN2(4); break;
    case 8: DN2(8); break;
    default: DN(0, false); break;
  }
#undef DN2
#undef DN
  return 0;
}

template <int F, int ACT>
static int mfma_down_sw(const void* h, const int64_t* tbl, const void* rw, int rw_dt, float* out,
                        const DownPlan& d, int sc, int w_round, hipStream_t st) {
  if constexpr (F == F_MXFP4) {
    if (sc == VAAYU_E8M0) return mfma_down_at<F, ACT, 8>(h, tbl, rw, rw_dt, out, d, w_round, st);
    return set_error(-2, "mxfp4 scales are E8M0");
  } else {
    if (sc == VAAYU_E8M0) return set_error(-2, "E8M0 scales go with mxfp4 codes");
    if (sc == DT_FP32) return mfma_down_at<F, ACT, 32>(h, tbl, rw, rw_dt, out, d, w_round, st);
    return mfma_down_at<F, ACT, 16>(h, tbl, rw, rw_dt, out, d, w_round, st);
  }
}

template <int BITS, int ACT, int SW, int CH>
static int down_at(const void* h, const int64_t* tbl, const void* rw, int rw_dt, float* out,
                   const DecodeShape& s, const vaayu_geom* g, int w_round, hipStream_t st) {
  constexpr int XST = 8;                               // h staged: up to 8 uint4 per thread
  int ps = 1;
  while (ps < 8 && ps < s.n_pairs) ps <<= 1;           // pair split: a power of two <= 8
  const int row_split = 8 / ps;
  const int rpw = 64 / s.lpr;
  // two rows per lane group when one would make so many blocks that staging every pair's
  // h per block costs more than it saves
  const bool ri2 = Unit<BITS, ACT>::FAST && s.lpr >= 2 &&
                   (s.hidden + row_split * rpw - 1) / (row_split * rpw) > 1024;
  const int wg_rows = row_split * rpw * (ri2 ? 2 : 1);
  const int h16 = s.n_pairs * s.units_row * Unit<BITS, ACT>::XD / 4;
  const size_t lds = (size_t)h16 * 16 + (size_t)s.n_pairs * wg_rows * sizeof(float);
  if (lds > 64 * 1024 || h16 > 512 * XST)
    return set_error(-3, "decode down: the pairs' activations do not fit one block's LDS");
  const dim3 grid((unsigned)((s.hidden + wg_rows - 1) / wg_rows)), block(512);
  if (ri2) {
    if constexpr (Unit<BITS, ACT>::FAST)
      hipLaunchKernelGGL((decode_down_kernel<BITS, ACT, SW, 2, CH, XST>), grid, block, lds, st,
                         h, tbl, rw, rw_dt, out, s, ps, (uint32_t)(g->down_w * 4),
                         (uint32_t)g->down_s, w_round);
  } else {
    hipLaunchKernelGGL((decode_down_kernel<BITS, ACT, SW, 1, CH, XST>), grid, block, lds, st, h,
                       tbl, rw, rw_dt, out, s, ps, (uint32_t)(g->down_w * 4), (uint32_t)g->down_s,
                       w_round);
  }
  return 0;
}

template <int BITS, int ACT, int SW>
static int by_ch(const void* h, const int64_t* tbl, const void* rw, int rw_dt, float* out,
                 const DecodeShape& s, const vaayu_geom* g, int w_round, hipStream_t st) {
  constexpr bool fast = Unit<BITS, ACT>::FAST;
  switch (s.chunks) {
    case 1: return down_at<BITS, ACT, SW, 1>(h, tbl, rw, rw_dt, out, s, g, w_round, st);
    case 2: if constexpr (fast) return down_at<BITS, ACT, SW, 2>(h, tbl, rw, rw_dt, out, s, g, w_round, st); break;
    case 3: if constexpr (fast) return down_at<BITS, ACT, SW, 3>(h, tbl, rw, rw_dt, out, s, g, w_round, st); break;
    case 4: if constexpr (fast) return down_at<BITS, ACT, SW, 4>(h, tbl, rw, rw_dt, out, s, g, w_round, st); break;
    case 7: if constexpr (fast) return down_at<BITS, ACT, SW, 7>(h, tbl, rw, rw_dt, out, s, g, w_round, st); break;
  }
  return set_error(-2, "decode down: no kernel for this row split");
}

template <int BITS, int ACT>
static int by_sw(const void* h, const int64_t* tbl, const void* rw, int rw_dt, float* out,
                 const DecodeShape& s, const vaayu_geom* g, int sc, int w_round, hipStream_t st) {
  if constexpr (BITS == F_MXFP4) {
    if (sc == VAAYU_E8M0) return by_ch<BITS, ACT, 8>(h, tbl, rw, rw_dt, out, s, g, w_round, st);
    return set_error(-2, "mxfp4 scales are E8M0");
  } else {
    if (sc == VAAYU_E8M0) return set_error(-2, "E8M0 scales go with mxfp4 codes");
    if (sc == DT_FP32) return by_ch<BITS, ACT, 32>(h, tbl, rw, rw_dt, out, s, g, w_round, st);
    return by_ch<BITS, ACT, 16>(h, tbl, rw, rw_dt, out, s, g, w_round, st);
  }
}

}  // namespace vaayu

using namespace vaayu;

extern "C" int vaayu_decode_down(const void* h, const int64_t* table, const void* routing_weights,
                                 int32_t rw_dtype, float* out, int32_t n_pairs,
                                 const vaayu_geom* geom, int32_t act, int32_t scale_dtype,
                                 int32_t w_round, void* stream) {
  clear_error();
  if (!h || !table || !routing_weights || !out || !geom)
    return set_error(-1, "null pointer argument");
  if (n_pairs <= 0) return set_error(-1, "n_pairs must be positive");
  if (scale_dtype < 0 || scale_dtype > 3 || rw_dtype < 0 || rw_dtype > 2)
    return set_error(-1, "scale / routing-weight dtype");
  if (((uintptr_t)h) & 15) return set_error(-1, "h must be 16-byte aligned");
  if (const char* why = decode_unsupported(geom, act)) return set_error(-2, why);
  const int fmt = code_format(geom);
  hipStream_t st = (hipStream_t)stream;
  {
    DownPlan d;
    if (mfma_down_plan(geom, fmt, act, n_pairs, scale_dtype, d)) {
      int rc;
#define BA(B_, A_) else if (fmt == B_ && act == A_) rc = mfma_down_sw<B_, A_>(h, table, routing_weights, rw_dtype, out, d, scale_dtype, w_round, st);
      if (false) rc = 0;
      BA(4, 0) BA(4, 1) BA(8, 0) BA(8, 1) BA(F_E4M3, 0) BA(F_E4M3, 1) BA(F_MXFP4, 0) BA(F_MXFP4, 1)
      else rc = set_error(-2, "unsupported code format / activation dtype");
#undef BA
      return rc ? rc : check_launch("decode down");
    }
  }
  const bool fast = (fmt == 4 || fmt == 8 || fmt >= 100) && act != DT_FP32;
  const Plan pl = plan_row(geom->inter * geom->bits / 128, 1, 1, fast);
  if (pl.lpr == 0) return set_error(-2, "decode down: no lane split of this row is built");
  const DecodeShape s = shape_for(geom, n_pairs, geom->inter, geom->hidden, scale_dtype, pl);
  int rc;
#define BA(B_, A_) else if (fmt == B_ && act == A_) rc = by_sw<B_, A_>(h, table, routing_weights, rw_dtype, out, s, geom, scale_dtype, w_round, st);
  if (false) rc = 0;
  BA(4, 0) BA(4, 1) BA(4, 2) BA(8, 0) BA(8, 1) BA(8, 2) BA(2, 0) BA(2, 1) BA(2, 2)
  BA(1, 0) BA(1, 1) BA(1, 2) BA(F_E4M3, 0) BA(F_E4M3, 1) BA(F_E4M3, 2)
  BA(F_MXFP4, 0) BA(F_MXFP4, 1) BA(F_MXFP4, 2)
  else rc = set_error(-2, "unsupported code format / activation dtype");
#undef BA
  return rc ? rc : check_launch("decode down");
}
