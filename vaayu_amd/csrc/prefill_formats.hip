// Prefill launches for e4m3 and e2m1 expert blobs (kernels in prefill_kernels.hpp), a compile
// unit of their own so the integer and float code families build in parallel.
#include "prefill_kernels.hpp"

namespace vaayu {

int prefill_gate_up_formats(const void* x, const int64_t* rows, const int64_t* tbl, void* h,
                            const PrefillArgs& p, const vaayu_geom* g, int act, hipStream_t st) {
  if (g->format == VAAYU_FMT_MXFP4) {
    if (act == DT_BF16) launch_prefill_gate_up<F_MXFP4, DT_BF16, 8>(x, rows, tbl, h, p, g, st);
    else launch_prefill_gate_up<F_MXFP4, DT_FP16, 8>(x, rows, tbl, h, p, g, st);
    return 0;
  }
  if (g->format != VAAYU_FMT_E4M3) return set_error(-2, "code format");
  const bool f32 = p.sc_dt == DT_FP32;
  if (act == DT_BF16) {
    if (f32) launch_prefill_gate_up<F_E4M3, DT_BF16, 32>(x, rows, tbl, h, p, g, st);
    else launch_prefill_gate_up<F_E4M3, DT_BF16, 16>(x, rows, tbl, h, p, g, st);
  } else {
    if (f32) launch_prefill_gate_up<F_E4M3, DT_FP16, 32>(x, rows, tbl, h, p, g, st);
    else launch_prefill_gate_up<F_E4M3, DT_FP16, 16>(x, rows, tbl, h, p, g, st);
  }
  return 0;
}

int prefill_down_formats(const void* h, const int64_t* rows, const int64_t* tbl, const void* rw,
                         int rw_dt, float* y, const PrefillArgs& p, const vaayu_geom* g,
                         int act, int w_round, hipStream_t st) {
  if (g->format == VAAYU_FMT_MXFP4) {
    if (act == DT_BF16)
      launch_prefill_down<F_MXFP4, DT_BF16, 8>(h, rows, tbl, rw, rw_dt, y, p, g, w_round, st);
    else
      launch_prefill_down<F_MXFP4, DT_FP16, 8>(h, rows, tbl, rw, rw_dt, y, p, g, w_round, st);
    return 0;
  }
  if (g->format != VAAYU_FMT_E4M3) return set_error(-2, "code format");
  const bool f32 = p.sc_dt == DT_FP32;
  if (act == DT_BF16) {
    if (f32) launch_prefill_down<F_E4M3, DT_BF16, 32>(h, rows, tbl, rw, rw_dt, y, p, g, w_round, st);
    else launch_prefill_down<F_E4M3, DT_BF16, 16>(h, rows, tbl, rw, rw_dt, y, p, g, w_round, st);
  } else {
    if (f32) launch_prefill_down<F_E4M3, DT_FP16, 32>(h, rows, tbl, rw, rw_dt, y, p, g, w_round, st);
    else launch_prefill_down<F_E4M3, DT_FP16, 16>(h, rows, tbl, rw, rw_dt, y, p, g, w_round, st);
  }
  return 0;
}

}  // namespace vaayu
