// Prefill entries: vaayu_prefill_gate_up / _down / _reduce (kernels in prefill_kernels.hpp).
#include "prefill_kernels.hpp"

namespace vaayu {

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

// Why the prefill kernels cannot take this geometry and scale dtype, or nullptr.
const char* prefill_unsupported(const vaayu_geom* g, int act, int sc) {
  if (g->format < 0 || g->format > 2) return "code format";
  if (act != DT_BF16 && act != DT_FP16) return "activation dtype (MFMA takes bf16 / fp16)";
  if (g->bits != 4 && g->bits != 8) return "bit width (the MFMA path takes 4 and 8)";
  if (g->format == VAAYU_FMT_E4M3 &&
      (g->bits != 8 || g->block_rows <= 0 || (g->block_rows & (g->block_rows - 1)) ||
       g->hidden % g->block_rows || g->inter % g->block_rows))
    return "e4m3 codes are 8 bits with power-of-two scale blocks tiling hidden and intermediate";
  if (g->format == VAAYU_FMT_MXFP4 && (g->bits != 4 || g->group != 32))
    return "mxfp4 codes are 4 bits with one scale per 32";
  if ((g->format == VAAYU_FMT_MXFP4) != (sc == VAAYU_E8M0)) return "E8M0 scales go with mxfp4 codes";
  const int cpu = 128 / g->bits;
  if (g->group % cpu) return "group size smaller than a 16-byte unit of codes";
  if (g->group & (g->group - 1)) return "group size is not a power of two";
  if (g->hidden % (4 * cpu) || g->inter % (4 * cpu))
    return "K tile: hidden / intermediate is not a multiple of the 4-unit K step";
  return nullptr;
}

}  // namespace vaayu

using namespace vaayu;

extern "C" int vaayu_prefill_gate_up(const void* x, const int64_t* rows, const int64_t* table,
                                     const int64_t* work, int32_t n_slots, int32_t run_blocks,
                                     void* h,
                                     int32_t n_blocks, int32_t top_k, const vaayu_geom* g,
                                     int32_t act, int32_t scale_dtype, void* stream) {
  clear_error();
  if (!x || !rows || !table || !work || !h || !g) return set_error(-1, "null pointer argument");
  if (n_blocks <= 0 || top_k <= 0) return set_error(-1, "n_blocks / top_k must be positive");
  if (n_slots < 0 || n_slots > n_blocks) return set_error(-1, "n_slots must be in [0, n_blocks]");
  if (run_blocks < 1 || run_blocks > kRunGateUp)
    return set_error(-1, "run_blocks must be in [1, vaayu_prefill_run_blocks(0)]");
  if (scale_dtype < 0 || scale_dtype > 3) return set_error(-1, "scale dtype");
  if (const char* why = prefill_unsupported(g, act, scale_dtype)) return set_error(-2, why);
  if (const char* why = rows_out_of_reach(n_blocks, top_k, 2ll * g->hidden, 0))
    return set_error(-2, why);
  const PrefillArgs p{n_blocks, (g->inter + kTileN - 1) / kTileN, top_k, g->hidden, g->inter,
                      log2_of(g->group),
                      g->format == VAAYU_FMT_E4M3 ? log2_of(g->block_rows) : 0, scale_dtype,
                      work, n_slots, run_blocks};
  hipStream_t st = (hipStream_t)stream;
  if (g->format != VAAYU_FMT_INT) {
    const int rc = prefill_gate_up_formats(x, rows, table, h, p, g, act, st);
    return rc ? rc : check_launch("prefill gate/up");
  }
#define GU(B_, A_, W_) launch_prefill_gate_up<B_, A_, W_>(x, rows, table, h, p, g, st)
#define GU2(B_, A_) if (scale_dtype == DT_FP32) GU(B_, A_, 32); else GU(B_, A_, 16)
  if (g->bits == 4 && act == DT_BF16) { GU2(4, DT_BF16); }
  else if (g->bits == 4) { GU2(4, DT_FP16); }
  else if (act == DT_BF16) { GU2(8, DT_BF16); }
  else { GU2(8, DT_FP16); }
#undef GU2
#undef GU
  return check_launch("prefill gate/up");
}

extern "C" int vaayu_prefill_down(const void* h, const int64_t* rows, const int64_t* table,
                                  const int64_t* work, int32_t n_slots, int32_t run_blocks,
                                  const void* routing_weights, int32_t rw_dtype, float* y,
                                  int32_t n_blocks, const vaayu_geom* g, int32_t act,
                                  int32_t scale_dtype, int32_t w_round, void* stream) {
  clear_error();
  if (!h || !rows || !table || !work || !routing_weights || !y || !g)
    return set_error(-1, "null pointer argument");
  if (n_blocks <= 0) return set_error(-1, "n_blocks must be positive");
  if (n_slots < 0 || n_slots > n_blocks) return set_error(-1, "n_slots must be in [0, n_blocks]");
  if (run_blocks < 1 || run_blocks > kRunDown)
    return set_error(-1, "run_blocks must be in [1, vaayu_prefill_run_blocks(1)]");
  if (scale_dtype < 0 || scale_dtype > 3 || rw_dtype < 0 || rw_dtype > 2)
    return set_error(-1, "scale / routing-weight dtype");
  if (const char* why = prefill_unsupported(g, act, scale_dtype)) return set_error(-2, why);
  if (const char* why = rows_out_of_reach(n_blocks, 1, 0, 2ll * g->inter))
    return set_error(-2, why);
  const PrefillArgs p{n_blocks, (g->hidden + kTileN - 1) / kTileN, 1, g->hidden, g->inter,
                      log2_of(g->group),
                      g->format == VAAYU_FMT_E4M3 ? log2_of(g->block_rows) : 0, scale_dtype,
                      work, n_slots, run_blocks};
  hipStream_t st = (hipStream_t)stream;
  if (g->format != VAAYU_FMT_INT) {
    const int rc = prefill_down_formats(h, rows, table, routing_weights, rw_dtype, y, p, g, act,
                                        w_round, st);
    return rc ? rc : check_launch("prefill down");
  }
#define DN(B_, A_, W_) launch_prefill_down<B_, A_, W_>(h, rows, table, routing_weights, rw_dtype, y, p, g, w_round, st)
#define DN2(B_, A_) if (scale_dtype == DT_FP32) DN(B_, A_, 32); else DN(B_, A_, 16)
  if (g->bits == 4 && act == DT_BF16) { DN2(4, DT_BF16); }
  else if (g->bits == 4) { DN2(4, DT_FP16); }
  else if (act == DT_BF16) { DN2(8, DT_BF16); }
  else { DN2(8, DT_FP16); }
#undef DN2
#undef DN
  return check_launch("prefill down");
}

// The run length (blocks) the work lists of the grouped kernels may hold: which = 0
// gate/up (prefill and fused-3D), 1 down.
extern "C" int32_t vaayu_prefill_run_blocks(int32_t which) {
  return which == 0 ? kRunGateUp : which == 1 ? kRunDown : -1;
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
