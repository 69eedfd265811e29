// Routed fused-3D MXFP4 experts (gpt-oss layout): the grouped gate/up GEMM with bias and
// the gpt-oss SwiGLU fused into its epilogue, and the grouped down GEMM with bias and the
// routing weight, over one layer's whole expert tensors.
//
// Replaces the vendored `matmul_ogs` + fused `swiglu` that the experts module runs on the
// routed rows (caller: vaayu/routed_fused3d.py:131-238; the module:
// transformers' Mxfp4GptOssExperts.forward). Arithmetic follows the vendored kernels:
// the gate/up epilogue `acc + bias` then `_swiglu_fn` (…/swiglu_details/_swiglu.py
// compute_swiglu: gate clipped above at `limit`, the linear half to [-limit, limit],
// s = gate / (1 + exp(-alpha gate)), out = fma(s, linear, s)), the down epilogue
// `(acc + bias) * gamma` (…/matmul_ogs_details/_matmul_ogs.py:310-349), both stored in
// bf16; the per-token sum over slots in ascending expert id is `vaayu_prefill_reduce`.
//
// Layout read in place, no repacking: gate_up blocks [E, 2I, H/32, 16] (row 2j = gate
// column j, row 2j+1 = up column j), scales [E, 2I, H/32] E8M0; down blocks [E, H, I/32, 16],
// scales [E, H, I/32]; biases fp32 [E, 2I] and [E, H]. The K loop runs to K rounded up to a
// whole step (128): the activations carry zeros there (the caller pads x and h), and the
// units past a row's K, which lie in the next row (at an expert's last row, the next
// expert's, whatever its bytes), take a zero scale and so zero weights: the tail adds
// exact zeros and no byte outside the routed experts' rows reaches an output. Reads past
// the tensors' ends return zeros (buffer bounds).
#include "prefill_kernels.hpp"

namespace vaayu {

// A role whose weight rows sit `code_pitch` bytes / `sc_pitch` scale bytes apart (two
// rows apart for the interleaved gate/up halves), readable up to the tensors' ends.
__device__ __forceinline__ Role make_role_pitched(const char* codes, const char* sc,
                                                  uint32_t code_pitch, uint32_t sc_pitch,
                                                  const char* codes_end, const char* sc_end,
                                                  int k, int n) {
  Role r;
  r.row_bytes = code_pitch;
  r.row_groups = sc_pitch;
  r.codes = rsrc(codes, (uint32_t)min<int64_t>(codes_end - codes, 0xFFFFFFF0ll));
  r.sc = rsrc(sc, (uint32_t)min<int64_t>(sc_end - sc, 0xFFFFFFF0ll));
  r.bf16_mask = 0u;
  r.kc_end = (uint32_t)k;
  r.n = n;
  r.gshift = 5;                 // E8M0 scale per 32 codes
  r.rshift = 0;
  return r;
}

struct Fused3DArgs {
  const int64_t* rows;
  const int64_t* tbl;           // [n_blocks, 2] (codes, scales) of each block's expert
  const int64_t* btbl;          // [n_blocks] its bias
  const int64_t* work;          // the work list (prefill_kernels.hpp: item_here)
  const char* codes_end;
  const char* sc_end;
  int n_blocks, n_tiles, top_k;
  int k, k_pad;                 // the GEMM's K and the K loop's length (whole steps)
  int n_out;                    // output columns (gate/up: I; down: H)
  int out_pitch;                // h row pitch (gate/up: I padded)
  float alpha, limit;
};

template <int S>
__device__ __forceinline__ void oss_gate_up_run(const Item& it, const Fused3DArgs& p,
                                                const void* x, void* h, char* lds0, char* lds1,
                                                int* rid_s) {
  constexpr int F = F_MXFP4, ACT = DT_BF16, SW = 8;
  constexpr int KS = 512 / CodeBits<F>::value;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int q = lane >> 4, m = lane & 15;
  const int n = it.tile * kTileN + wv * 16 + m;
  const bool n_ok = n < p.n_out;
  const int nn = n_ok ? n : 0;
  const char* pk = (const char*)p.tbl[2 * it.b];
  const char* sc = (const char*)p.tbl[2 * it.b + 1];
  const uint32_t row_b = (uint32_t)p.k / 2, row_s = (uint32_t)p.k / 32;
  const Role role[2] = {
      make_role_pitched(pk, sc, 2 * row_b, 2 * row_s, p.codes_end, p.sc_end, p.k, nn),
      make_role_pitched(pk + row_b, sc + row_s, 2 * row_b, 2 * row_s, p.codes_end, p.sc_end,
                        p.k, nn)};
  const float* bias = (const float*)p.btbl[it.b];
  const float bg = bias[2 * nn], bu = bias[2 * nn + 1];
  const int64_t* rrow = p.rows + (int64_t)it.b * 16;
  AStage<KS, S> a;
  a_plan<KS, S>(a, [&](int r) -> uint32_t {
    const int64_t rid = rrow[r];
    return rid >= 0 ? (uint32_t)(rid / p.top_k) * (uint32_t)p.k_pad * 2u : kNoRow;
  });
  if (threadIdx.x < S * 16) rid_s[threadIdx.x] = (int)rrow[threadIdx.x];
  f32x4 acc[2][S];
  run_k<F, ACT, SW, 2, S>(role, rsrc(x, kNoRow), a, lds0, lds1, p.k_pad, q, m, acc);
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rid_s[s * 16 + 4 * q + i];
      if (r >= 0 && n_ok) {
        const float g = fminf(acc[0][s][i] + bg, p.limit);
        const float u = fminf(fmaxf(acc[1][s][i] + bu, -p.limit), p.limit);
        const float sg = g / (1.f + expf(-p.alpha * g));
        store_act<ACT>(h, (int64_t)r * p.out_pitch + n, fmaf(sg, u, sg));
      }
      if (i == 3) __builtin_amdgcn_sched_barrier(0);
    }
}

template <int S>
__device__ __forceinline__ void oss_down_run(const Item& it, const Fused3DArgs& p, const void* h,
                                             const float* gammas, float* y, char* lds0,
                                             char* lds1, int* rid_s, float* w_s) {
  constexpr int F = F_MXFP4, ACT = DT_BF16, SW = 8;
  constexpr int KS = 512 / CodeBits<F>::value;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int q = lane >> 4, m = lane & 15;
  const int n = it.tile * kTileN + wv * 16 + m;
  const bool n_ok = n < p.n_out;
  const int nn = n_ok ? n : 0;
  const char* pk = (const char*)p.tbl[2 * it.b];
  const char* sc = (const char*)p.tbl[2 * it.b + 1];
  const Role role[1] = {make_role_pitched(pk, sc, (uint32_t)p.k / 2, (uint32_t)p.k / 32,
                                          p.codes_end, p.sc_end, p.k, nn)};
  const float bd = ((const float*)p.btbl[it.b])[nn];
  const int64_t* rrow = p.rows + (int64_t)it.b * 16;
  AStage<KS, S> a;
  a_plan<KS, S>(a, [&](int r) -> uint32_t {
    const int64_t rid = rrow[r];
    return rid >= 0 ? (uint32_t)rid * (uint32_t)p.k_pad * 2u : kNoRow;
  });
  float w_mine = 0.f;
  if (threadIdx.x < S * 16) {
    const int rid = (int)rrow[threadIdx.x];
    rid_s[threadIdx.x] = rid;
    w_mine = gammas[max(rid, 0)];
  }
  f32x4 acc[1][S];
  run_k<F, ACT, SW, 1, S>(role, rsrc(h, kNoRow), a, lds0, lds1, p.k_pad, q, m, acc);
  if (threadIdx.x < S * 16) w_s[threadIdx.x] = w_mine;
  __syncthreads();
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = s * 16 + 4 * q + i;
      const int r = rid_s[t];
      if (r >= 0 && n_ok)
        y[(int64_t)r * p.n_out + n] = round_act<ACT>((acc[0][s][i] + bd) * w_s[t]);
    }
}

#define VAAYU_F3D_BY_S(CALL)                                                        \
  switch (it.S) {                                                                   \
    case 1: CALL(1); break; case 2: CALL(2); break; case 3: CALL(3); break;          \
    case 4: CALL(4); break; case 5: CALL(5); break; case 6: CALL(6); break;          \
    case 7: CALL(7); break; case 8: CALL(8); break; default: break;                 \
  }
#define VAAYU_F3D_BY_S16(CALL)                                                      \
  switch (it.S) {                                                                   \
    case 1: CALL(1); break; case 2: CALL(2); break; case 3: CALL(3); break;          \
    case 4: CALL(4); break; case 5: CALL(5); break; case 6: CALL(6); break;          \
    case 7: CALL(7); break; case 8: CALL(8); break; case 9: CALL(9); break;          \
    case 10: CALL(10); break; case 11: CALL(11); break; case 12: CALL(12); break;    \
    case 13: CALL(13); break; case 14: CALL(14); break; case 15: CALL(15); break;    \
    case 16: CALL(16); break; default: break;                                       \
  }

template <int R>
__global__ void __launch_bounds__(64 * kWaves)
fused3d_gate_up_kernel(Fused3DArgs p, const void* __restrict__ x, void* __restrict__ h) {
  __shared__ __align__(1024) char lds0[tile_blocks(R) * 16 * (2 * 512 / 4)];
  __shared__ __align__(1024) char lds1[tile_blocks(R) * 16 * (2 * 512 / 4)];
  __shared__ int rid_s[R * 16];
  const Item it = item_here<R>(p.work, p.n_blocks, p.n_tiles);
#define F3_GU(S_) oss_gate_up_run<S_>(it, p, x, h, lds0, lds1, rid_s)
  if constexpr (R > kRunGateUpShort) {
    VAAYU_F3D_BY_S16(F3_GU)
  } else {
    switch (it.S) {
      case 1: F3_GU(1); break; case 2: F3_GU(2); break; case 3: F3_GU(3); break;
      case 4: F3_GU(4); break; default: break;
    }
  }
#undef F3_GU
}

template <int R>
__global__ void __launch_bounds__(64 * kWaves)
fused3d_down_kernel(Fused3DArgs p, const void* __restrict__ h, const float* __restrict__ gammas,
                    float* __restrict__ y) {
  __shared__ __align__(1024) char lds0[tile_blocks(R) * 16 * (2 * 512 / 4)];
  __shared__ __align__(1024) char lds1[tile_blocks(R) * 16 * (2 * 512 / 4)];
  __shared__ int rid_s[R * 16];
  __shared__ float w_s[R * 16];
  const Item it = item_here<R>(p.work, p.n_blocks, p.n_tiles);
#define F3_DN(S_) oss_down_run<S_>(it, p, h, gammas, y, lds0, lds1, rid_s, w_s)
  if constexpr (R > kRunDownShort) {
    VAAYU_F3D_BY_S16(F3_DN)
  } else {
    VAAYU_F3D_BY_S(F3_DN)
  }
#undef F3_DN
}

#undef VAAYU_F3D_BY_S
#undef VAAYU_F3D_BY_S16

}  // namespace vaayu

using namespace vaayu;

static int fused3d_check(int n_blocks, int top_k, int k, int k_pad, int n_out) {
  if (n_blocks < 0 || top_k <= 0) return set_error(-2, "bad block count or top_k");
  if (k <= 0 || k % 32) return set_error(-2, "K must be a positive multiple of 32");
  if (k_pad < k || k_pad % 128) return set_error(-2, "the padded K must be >= K and a multiple of 128");
  if (n_out <= 0) return set_error(-2, "no output columns");
  return 0;
}

extern "C" int vaayu_fused3d_gate_up(const void* x, const int64_t* rows, const int64_t* tbl,
                                     const int64_t* btbl, const int64_t* work, int32_t n_slots,
                                     int32_t run_blocks, void* h, int32_t n_blocks,
                                     int32_t top_k, int32_t hidden, int32_t hidden_pad,
                                     int32_t inter, int32_t inter_pad, const void* codes_end,
                                     const void* scales_end, float alpha, float limit,
                                     void* stream) {
  clear_error();
  if (!x || !rows || !tbl || !btbl || !work || !h || !codes_end || !scales_end)
    return set_error(-1, "null pointer argument");
  if (n_slots < 0 || n_slots > n_blocks) return set_error(-2, "n_slots must be in [0, n_blocks]");
  if (run_blocks < 1 || run_blocks > kRunGateUp)
    return set_error(-2, "run_blocks must be in [1, vaayu_prefill_run_blocks(0)]");
  if (int rc = fused3d_check(n_blocks, top_k, hidden, hidden_pad, inter)) return rc;
  if (inter_pad < inter) return set_error(-2, "h's row pitch is below the intermediate size");
  if (const char* why = rows_out_of_reach(n_blocks, top_k, 2ll * hidden_pad, 0))
    return set_error(-2, why);
  if (n_blocks == 0) return 0;
  Fused3DArgs p;
  p.rows = rows; p.tbl = tbl; p.btbl = btbl; p.work = work;
  p.codes_end = (const char*)codes_end; p.sc_end = (const char*)scales_end;
  p.n_blocks = n_blocks; p.n_tiles = (inter + kTileN - 1) / kTileN; p.top_k = top_k;
  p.k = hidden; p.k_pad = hidden_pad; p.n_out = inter; p.out_pitch = inter_pad;
  p.alpha = alpha; p.limit = limit;
  if (n_slots == 0) return 0;
  const dim3 grid = work_grid(n_slots, p.n_tiles), block(64 * kWaves);
  if (run_blocks <= kRunGateUpShort)
    hipLaunchKernelGGL(fused3d_gate_up_kernel<kRunGateUpShort>, grid, block, 0,
                       (hipStream_t)stream, p, x, h);
  else
    hipLaunchKernelGGL(fused3d_gate_up_kernel<kRunGateUp>, grid, block, 0, (hipStream_t)stream, p,
                       x, h);
  return check_launch("fused-3D gate/up");
}

extern "C" int vaayu_fused3d_down(const void* h, const int64_t* rows, const int64_t* tbl,
                                  const int64_t* btbl, const int64_t* work, int32_t n_slots,
                                  int32_t run_blocks, const float* gammas, float* y,
                                  int32_t n_blocks, int32_t top_k, int32_t hidden,
                                  int32_t inter, int32_t inter_pad, const void* codes_end,
                                  const void* scales_end, void* stream) {
  clear_error();
  if (!h || !rows || !tbl || !btbl || !work || !gammas || !y || !codes_end || !scales_end)
    return set_error(-1, "null pointer argument");
  if (n_slots < 0 || n_slots > n_blocks) return set_error(-2, "n_slots must be in [0, n_blocks]");
  if (run_blocks < 1 || run_blocks > kRunDown)
    return set_error(-2, "run_blocks must be in [1, vaayu_prefill_run_blocks(1)]");
  if (int rc = fused3d_check(n_blocks, top_k, inter, inter_pad, hidden)) return rc;
  if (const char* why = rows_out_of_reach(n_blocks, 1, 0, 2ll * inter_pad))
    return set_error(-2, why);
  if (n_blocks == 0) return 0;
  Fused3DArgs p;
  p.rows = rows; p.tbl = tbl; p.btbl = btbl; p.work = work;
  p.codes_end = (const char*)codes_end; p.sc_end = (const char*)scales_end;
  p.n_blocks = n_blocks; p.n_tiles = (hidden + kTileN - 1) / kTileN; p.top_k = top_k;
  p.k = inter; p.k_pad = inter_pad; p.n_out = hidden; p.out_pitch = hidden;
  p.alpha = 0.f; p.limit = 0.f;
  if (n_slots == 0) return 0;
  const dim3 grid = work_grid(n_slots, p.n_tiles), block(64 * kWaves);
  if (run_blocks <= kRunDownShort)
    hipLaunchKernelGGL(fused3d_down_kernel<kRunDownShort>, grid, block, 0, (hipStream_t)stream, p,
                       h, gammas, y);
  else
    hipLaunchKernelGGL(fused3d_down_kernel<kRunDown>, grid, block, 0, (hipStream_t)stream, p, h,
                       gammas, y);
  return check_launch("fused-3D down");
}
