// Decode gate/up entry: vaayu_decode_gate_up (kernels in decode_mfma.hpp for bf16 / fp16
// activations with 4- and 8-bit codes, decode_kernels.hpp otherwise).
#include "decode_mfma.hpp"

namespace vaayu {

// Blocks the chip holds at once (256 CUs x 5 four-wave blocks). A grid within that loads
// its codes non-temporal: measured on the 8-pair Qwen3-30B-A3B-shape decode, 5.86 -> 5.23 us
// per launch, since the streamed codes no longer push the small operands of the next
// kernels out of the caches. Larger grids (Mixtral, DeepSeek-V3 experts) were slower with
// it (26.4 -> 28.1 us and 39.3 -> 43.0 us) and keep the default policy.
constexpr int64_t kResidentGateUpBlocks = 1280;

// Step counts with a straight-line kernel; others run the chunked loop (NS = 0).
template <int F, int ACT, int SW, bool NT>
static int mfma_gate_up_nt(const void* x, const int64_t* tbl, void* h, const MShape& s,
                           const dim3 grid, size_t lds, hipStream_t st) {
#define GU(NS_) hipLaunchKernelGGL((mfma_gate_up_kernel<F, ACT, SW, NS_, NT>), grid, dim3(256), \
                                   lds, st, tbl, (const uint32_t*)x, h, s)
  switch (s.steps) {
    case 1: GU(1); break;
    case 2: GU(2); break;
    case 3: GU(3); break;
    case 4: GU(4); break;
    case 8: GU(8); break;
    default: GU(0); break;
  }
#undef GU
  return 0;
}

template <int F, int ACT, int SW>
static int mfma_gate_up_at(const void* x, const int64_t* tbl, void* h, const MShape& s, int xs,
                           hipStream_t st) {
  const dim3 grid((unsigned)((s.rows + 7) / 8), (unsigned)s.n_pairs);
  const size_t lds = (size_t)xs * 256 * 16;
  if ((int64_t)grid.x * grid.y <= kResidentGateUpBlocks)
    return mfma_gate_up_nt<F, ACT, SW, true>(x, tbl, h, s, grid, lds, st);
  return mfma_gate_up_nt<F, ACT, SW, false>(x, tbl, h, s, grid, lds, st);
}

template <int F, int ACT>
static int mfma_gate_up_sw(const void* x, const int64_t* tbl, void* h, const MShape& s, int xs,
                           int sc, hipStream_t st) {
  if constexpr (F == F_MXFP4) {
    if (sc == VAAYU_E8M0) return mfma_gate_up_at<F, ACT, 8>(x, tbl, h, s, xs, st);
    return set_error(-2, "mxfp4 scales are E8M0");
  } else {
    if (sc == VAAYU_E8M0) return set_error(-2, "E8M0 scales go with mxfp4 codes");
    if (sc == DT_FP32) return mfma_gate_up_at<F, ACT, 32>(x, tbl, h, s, xs, st);
    return mfma_gate_up_at<F, ACT, 16>(x, tbl, h, s, xs, st);
  }
}

// Fast path: 4/8-bit codes with bf16/fp16 activations, any CH of the instantiated set.
// General path (fp32 activations, 1/2-bit codes): CH = 1.
template <int BITS, int ACT, int SW, int CH>
static int gate_up_at(const void* x, const int64_t* tbl, void* h, const DecodeShape& s,
                      const vaayu_geom* g, hipStream_t st) {
  constexpr int XST = 4;                               // x staged: up to 4 uint4 per thread
  const int x16 = s.units_row * Unit<BITS, ACT>::XD / 4;
  if (x16 > 256 * XST) return set_error(-2, "decode gate/up: hidden too large to stage in LDS");
  const int rows_per_wave = 64 / s.lpr;
  const int64_t waves = (int64_t)s.n_pairs * ((s.inter + rows_per_wave - 1) / rows_per_wave);
  hipLaunchKernelGGL((decode_gate_up_kernel<BITS, ACT, SW, 1, CH, XST>),
                     dim3((unsigned)((waves + 3) / 4)), dim3(256), (size_t)x16 * 16, st,
                     (const uint32_t*)x, tbl, h, s, (uint32_t)(g->gate_w * 4),
                     (uint32_t)g->gate_s, (uint32_t)(g->up_w * 4), (uint32_t)g->up_s);
  return 0;
}

template <int BITS, int ACT, int SW>
static int by_ch(const void* x, const int64_t* tbl, void* h, const DecodeShape& s,
                 const vaayu_geom* g, hipStream_t st) {
  constexpr bool fast = Unit<BITS, ACT>::FAST;
  switch (s.chunks) {
    case 1: return gate_up_at<BITS, ACT, SW, 1>(x, tbl, h, s, g, st);
    case 2: if constexpr (fast) return gate_up_at<BITS, ACT, SW, 2>(x, tbl, h, s, g, st); break;
    case 3: if constexpr (fast) return gate_up_at<BITS, ACT, SW, 3>(x, tbl, h, s, g, st); break;
    case 4: if constexpr (fast) return gate_up_at<BITS, ACT, SW, 4>(x, tbl, h, s, g, st); break;
    case 7: if constexpr (fast) return gate_up_at<BITS, ACT, SW, 7>(x, tbl, h, s, g, st); break;
  }
  return set_error(-2, "decode gate/up: no kernel for this row split");
}

template <int BITS, int ACT>
static int by_sw(const void* x, const int64_t* tbl, void* h, const DecodeShape& s,
                 const vaayu_geom* g, int sc, hipStream_t st) {
  if constexpr (BITS == F_MXFP4) {
    if (sc == VAAYU_E8M0) return by_ch<BITS, ACT, 8>(x, tbl, h, s, g, st);
    return set_error(-2, "mxfp4 scales are E8M0");
  } else {
    if (sc == VAAYU_E8M0) return set_error(-2, "E8M0 scales go with mxfp4 codes");
    if (sc == DT_FP32) return by_ch<BITS, ACT, 32>(x, tbl, h, s, g, st);
    return by_ch<BITS, ACT, 16>(x, tbl, h, s, g, st);
  }
}

}  // namespace vaayu

using namespace vaayu;

extern "C" int vaayu_decode_gate_up(const void* x, const int64_t* table, void* h, int32_t n_pairs,
                                    const vaayu_geom* geom, int32_t act, int32_t scale_dtype,
                                    void* stream) {
  clear_error();
  if (!x || !table || !h || !geom) return set_error(-1, "null pointer argument");
  if (n_pairs <= 0) return set_error(-1, "n_pairs must be positive");
  if (scale_dtype < 0 || scale_dtype > 3) return set_error(-1, "scale dtype");
  if (((uintptr_t)x) & 15) return set_error(-1, "x must be 16-byte aligned");
  if (const char* why = decode_unsupported(geom, act)) return set_error(-2, why);
  const int fmt = code_format(geom);
  hipStream_t st = (hipStream_t)stream;
  {
    MShape ms;
    int xs;
    if (mfma_gate_up_plan(geom, fmt, act, n_pairs, scale_dtype, ms, xs)) {
      int rc;
#define BA(B_, A_) else if (fmt == B_ && act == A_) rc = mfma_gate_up_sw<B_, A_>(x, table, h, ms, xs, scale_dtype, st);
      if (false) rc = 0;
      BA(4, 0) BA(4, 1) BA(8, 0) BA(8, 1) BA(F_E4M3, 0) BA(F_E4M3, 1) BA(F_MXFP4, 0) BA(F_MXFP4, 1)
      else rc = set_error(-2, "unsupported code format / activation dtype");
#undef BA
      return rc ? rc : check_launch("decode gate/up");
    }
  }
  const bool fast = (fmt == 4 || fmt == 8 || fmt >= 100) && act != DT_FP32;
  const Plan pl = plan_row(geom->hidden * geom->bits / 128, 2, 2, fast);
  if (pl.lpr == 0) return set_error(-2, "decode gate/up: no lane split of this row is built");
  const DecodeShape s = shape_for(geom, n_pairs, geom->hidden, geom->inter, scale_dtype, pl);
  int rc;
#define BA(B_, A_) else if (fmt == B_ && act == A_) rc = by_sw<B_, A_>(x, table, h, s, geom, scale_dtype, st);
  if (false) rc = 0;
  BA(4, 0) BA(4, 1) BA(4, 2) BA(8, 0) BA(8, 1) BA(8, 2) BA(2, 0) BA(2, 1) BA(2, 2)
  BA(1, 0) BA(1, 1) BA(1, 2) BA(F_E4M3, 0) BA(F_E4M3, 1) BA(F_E4M3, 2)
  BA(F_MXFP4, 0) BA(F_MXFP4, 1) BA(F_MXFP4, 2)
  else rc = set_error(-2, "unsupported code format / activation dtype");
#undef BA
  return rc ? rc : check_launch("decode gate/up");
}
