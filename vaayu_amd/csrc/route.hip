// Router softmax -> top-k -> renormalise on the GPU, the decode-time expert budget on top
// of it, and the one-token decode pair table built from the result, so a decode layer
// needs no host round trip between its router and its expert kernels.
//
// Restates the reference's default routing (the `_route` branch for a router that returns
// bare logits, vaayu/moe_patch.py:2329-2334, and `route_experts`' fallback at :159-161):
//   w, idx = topk(logits.float().softmax(-1), k); w = w / w.sum(-1)
// then `truncate_top_k` (vaayu/moe_patch.py:170-215: keep the k largest, or the fewest
// slots reaching routing mass p with the dropped slots re-pointed at the top-1 expert
// with weight 0, kept weights rescaled to the row's original sum), and the decode table
// `_table_values` over the slots sorted by (expert id, slot)
// (vaayu/packed_expert_kernels.py:349-352; the caller's stable sort at
// vaayu/moe_patch.py:2386-2389), with every expert resident: its blob addresses come from
// a device table indexed by id. Ties between equal probabilities go to the lower expert id.
#include "abi_internal.hpp"
#include "common.hpp"

namespace vaayu {

constexpr int kRouteMaxExperts = 1024;
constexpr int kRouteThreads = 1024;
constexpr int kRouteMaxK = 16;

// A whole wave's max / sum: DPP inside each row of 16 lanes (lane ^ 1, lane ^ 2, rotate
// by 4, by 8), then the four rows' results read out and combined.
template <int CTRL>
__device__ __forceinline__ float route_dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float route_lane(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

template <bool MAX>
__device__ __forceinline__ float route_op(float a, float b) {
  return MAX ? fmaxf(a, b) : a + b;
}

// The block's max / sum of v over its first `nw` waves (the other waves hold the
// identity); every thread gets the result.
template <bool MAX>
__device__ __forceinline__ float block_reduce(float v, float* red, int nw) {
  v = route_op<MAX>(v, route_dpp<0xB1>(v));       // quad_perm [1,0,3,2]
  v = route_op<MAX>(v, route_dpp<0x4E>(v));       // quad_perm [2,3,0,1]
  v = route_op<MAX>(v, route_dpp<0x124>(v));      // row_ror:4
  v = route_op<MAX>(v, route_dpp<0x128>(v));      // row_ror:8
  v = route_op<MAX>(route_op<MAX>(route_lane(v, 0), route_lane(v, 16)),
                    route_op<MAX>(route_lane(v, 32), route_lane(v, 48)));
  if ((threadIdx.x & 63) == 0 && (int)(threadIdx.x >> 6) < nw) red[threadIdx.x >> 6] = v;
  __syncthreads();
  v = red[0];
#pragma unroll
  for (int w = 1; w < kRouteThreads / 64; ++w)
    if (w < nw) v = route_op<MAX>(v, red[w]);
  __syncthreads();
  return v;
}

// One token per block (a multiple of the experts rounded up to 64). Each expert's rank among the token's
// probabilities is counted directly -- split over the threads the block has to spare, a
// slice of the experts each -- so the top-k need no rounds of block-wide argmax.
// weights / ids [tokens, n_out], n_out = min(keep_k, top_k); with pair_table (tokens == 1)
// also the decode table: (packed address, scale address, slot) per slot, in (expert id,
// slot) order.
template <int DT>
__global__ void __launch_bounds__(kRouteThreads)
route_topk_kernel(const void* __restrict__ logits, int experts, int top_k, int keep_k,
                  float top_p, int renorm, float* __restrict__ weights,
                  int64_t* __restrict__ ids, const int64_t* __restrict__ expert_table,
                  int64_t* __restrict__ pair_table) {
  __shared__ int4 qk4[kRouteMaxExperts / 4];
  __shared__ int cnt_s[kRouteThreads];
  __shared__ float red[kRouteThreads / 64];
  __shared__ float sel_w[kRouteMaxK];
  __shared__ int sel_id[kRouteMaxK];
  __shared__ int64_t sel_blob[kRouteMaxK][2];
  int* qk = reinterpret_cast<int*>(qk4);
  const int64_t t = blockIdx.x;
  const int tid = threadIdx.x;
  const int epad = (experts + 63) & ~63;           // experts rounded up to whole waves
  const int parts = (int)blockDim.x / epad;        // threads counting one expert's rank
  const int part = tid / epad;
  const int e = tid - part * epad;                 // the expert this thread works on
  const bool holder = part == 0 && e < experts;    // holds the expert's logit
  const float v = holder ? load_as_float<DT>(logits, t * experts + e) : -INFINITY;
  // Each expert's blob addresses, loaded beside its logit so the table needs no second
  // trip to memory once the picks are known.
  int64_t blob0 = 0, blob1 = 0;
  if (pair_table && holder) {
    blob0 = expert_table[2 * e];
    blob1 = expert_table[2 * e + 1];
  }
  const int nw = epad >> 6;                         // the waves holding logits
  const float m = block_reduce<true>(v, red, nw);
  const float ex = holder ? expf(v - m) : 0.f;
  const float s = block_reduce<false>(ex, red, nw);
  const float pr = ex / s;
  // Keys: a probability's bits (monotone for p >= 0); a NaN probability (NaN logits make
  // the whole row NaN) ranks as -1, below every real one; the padding to a multiple of 4
  // as -2, below everything.
  const int padded = (experts + 3) & ~3;
  if (part == 0 && e < padded)
    qk[e] = e < experts ? (pr == pr ? __builtin_bit_cast(int, pr) : -1) : -2;
  __syncthreads();
  const int ke = qk[e < padded ? e : 0];
  // Expert j ranks above expert e when k_j > k_e, or k_j == k_e and j < e: k_j > ke - 1
  // for j < e, k_j > ke for j >= e. The wave's experts are [w0, w0 + 64): the groups of
  // four j wholly below or wholly above them take one threshold for every lane.
  // The wave's part and first expert, read as wave-uniform values so the branches below
  // are scalar.
  const int tlo = ke - 1, thi = ke;
  const int wpart = __builtin_amdgcn_readfirstlane(part);
  const int w0 = __builtin_amdgcn_readfirstlane((tid & ~63) - part * epad);
  int cnt = 0;                                     // the keys above expert e's
  if (wpart < parts) {                             // in this wave's slice
    const int per = (padded / 4 + parts - 1) / parts;
    const int jb = wpart * per, je = min(jb + per, padded / 4);
    const int below = min(max(w0 / 4, jb), je);        // groups wholly below w0 end here
    const int above = min(max((w0 + 64) / 4, below), je);  // wholly above start here
#pragma unroll 4
    for (int j4 = jb; j4 < below; ++j4) {
      const int4 c = qk4[j4];
      cnt += (c.x > tlo) + (c.y > tlo) + (c.z > tlo) + (c.w > tlo);
    }
    for (int j4 = below; j4 < above; ++j4) {
      const int4 c = qk4[j4];
      const int j = 4 * j4;
      cnt += (c.x > (j < e ? tlo : thi)) + (c.y > (j + 1 < e ? tlo : thi)) +
             (c.z > (j + 2 < e ? tlo : thi)) + (c.w > (j + 3 < e ? tlo : thi));
    }
#pragma unroll 4
    for (int j4 = above; j4 < je; ++j4) {
      const int4 c = qk4[j4];
      cnt += (c.x > thi) + (c.y > thi) + (c.z > thi) + (c.w > thi);
    }
  }
  cnt_s[tid] = cnt;
  __syncthreads();
  if (holder) {
    int rank = 0;
#pragma unroll
    for (int p = 0; p < kRouteThreads / 64; ++p)
      if (p < parts) rank += cnt_s[p * epad + e];
    if (rank < top_k) {
      sel_w[rank] = ke == -1 ? -0.5f : __builtin_bit_cast(float, ke);
      sel_id[rank] = e;
      sel_blob[rank][0] = blob0;
      sel_blob[rank][1] = blob1;
    }
  }
  __syncthreads();
  const int n_out = keep_k < top_k ? keep_k : top_k;
  if (tid < 64) {
    // Wave 0, lane j = slot j. The slots hold the picks by falling probability, so every
    // top-k / sort below is the slot order itself. Sums run in slot order, lane by lane
    // (the same order on every lane); slots past top_k hold 0 and add nothing.
    const int j = tid;
    const bool nan_row = sel_w[0] == -0.5f;
    const int top1 = sel_id[0];
    const int64_t top1_blob0 = sel_blob[0][0], top1_blob1 = sel_blob[0][1];
    float w = j < top_k ? sel_w[j] : 0.f;
    auto slot_sum = [](float v) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < kRouteMaxK; ++i) acc += route_lane(v, i);
      return acc;
    };
    if (renorm) w = w / slot_sum(w);
    if (n_out < top_k || top_p > 0.f) {
      float row = slot_sum(w);                           // the row's original sum
      if (fabsf(row - 1.f) < 1e-2f) row = 1.f;
      if (n_out < top_k) {
        if (j >= n_out) w = 0.f;
        w = w / slot_sum(w) * row;
      }
      if (top_p > 0.f) {
        w = w / slot_sum(w);
        float acc = 0.f, cs = 0.f;                       // inclusive prefix sum at slot j
#pragma unroll
        for (int i = 0; i < kRouteMaxK; ++i) {
          acc += route_lane(w, i);
          if (i == j) cs = acc;
        }
        if (j < n_out && !(cs - w < top_p)) {          // mass before this slot reaches p
          w = 0.f;
          sel_id[j] = top1;                              // re-pointed at the top-1 expert
          sel_blob[j][0] = top1_blob0;
          sel_blob[j][1] = top1_blob1;
        }
        w = w / slot_sum(w) * row;
      }
    }
    if (j < n_out) sel_w[j] = nan_row ? __builtin_nanf("") : w;
  }
  __syncthreads();
  if (tid < n_out) {
    const int id = sel_id[tid];
    weights[t * n_out + tid] = sel_w[tid];
    ids[t * n_out + tid] = id;
    if (pair_table) {
      int rank = 0;                  // position in the stable (expert id, slot) order
#pragma unroll
      for (int j = 0; j < kRouteMaxK; ++j)
        if (j < n_out) rank += (sel_id[j] < id) | ((sel_id[j] == id) & (j < tid));
      pair_table[3 * rank] = sel_blob[tid][0];
      pair_table[3 * rank + 1] = sel_blob[tid][1];
      pair_table[3 * rank + 2] = tid;
    }
  }
}

// The router's product for a few tokens: logits[t, e] = round_out(sum_h x[t, h] w[e, h]),
// the fp32 sum rounded once to the output dtype, as `F.linear(x, w)` stores it. One wave
// per (token, expert): 16-byte loads of x and of the expert's row, fp32 FMAs, a DPP wave
// sum. For decode-sized calls, where a library GEMM's launch and tiling dominate.
constexpr int kGemvWaves = 4;

template <int XDT, int ODT>
__global__ void __launch_bounds__(kGemvWaves * 64)
router_gemv_kernel(const void* __restrict__ x, const void* __restrict__ w, void* __restrict__ out,
                   int tokens, int hidden, int experts) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kGemvWaves + (threadIdx.x >> 6);
  if (row >= (int64_t)tokens * experts) return;          // wave-uniform
  const int t = (int)(row / experts), e = (int)(row - (int64_t)t * experts);
  const uint16_t* xr = (const uint16_t*)x + (int64_t)t * hidden;
  const uint16_t* wr = (const uint16_t*)w + (int64_t)e * hidden;
  float acc = 0.f;
  for (int k = lane * 8; k < hidden; k += 64 * 8) {       // hidden % 8 == 0
    const uint4 xv = *(const uint4*)(xr + k);
    const uint4 wv = *(const uint4*)(wr + k);
    const uint32_t xa[4] = {xv.x, xv.y, xv.z, xv.w}, wa[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float x0 = load_as_float<XDT>(&xa[j], 0), x1 = load_as_float<XDT>(&xa[j], 1);
      const float w0 = load_as_float<XDT>(&wa[j], 0), w1 = load_as_float<XDT>(&wa[j], 1);
      acc = fmaf(x0, w0, acc);
      acc = fmaf(x1, w1, acc);
    }
  }
  acc = route_op<false>(acc, route_dpp<0xB1>(acc));
  acc = route_op<false>(acc, route_dpp<0x4E>(acc));
  acc = route_op<false>(acc, route_dpp<0x124>(acc));
  acc = route_op<false>(acc, route_dpp<0x128>(acc));
  acc = (route_lane(acc, 0) + route_lane(acc, 16)) + (route_lane(acc, 32) + route_lane(acc, 48));
  if (lane == 0) store_act<ODT>(out, row, acc);
}

}  // namespace vaayu

using namespace vaayu;

extern "C" int vaayu_route_topk(const void* logits, int32_t logits_dtype, int32_t tokens,
                                int32_t experts, int32_t top_k, int32_t keep_k, float top_p,
                                int32_t renorm, float* weights, int64_t* ids,
                                const int64_t* expert_table, int64_t* pair_table,
                                void* stream) {
  clear_error();
  if (!logits || !weights || !ids) return set_error(-1, "null pointer argument");
  if (tokens <= 0) return set_error(-1, "tokens must be positive");
  if (experts <= 0 || experts > kRouteMaxExperts) return set_error(-2, "experts must be 1..1024");
  if (top_k <= 0 || top_k > kRouteMaxK || top_k > experts)
    return set_error(-2, "top_k must be 1..min(16, experts)");
  if (keep_k <= 0) return set_error(-2, "keep_k must be positive");
  if (!(top_p >= 0.f)) return set_error(-2, "top_p must be 0 (off) or positive");
  if (pair_table && (tokens != 1 || !expert_table))
    return set_error(-1, "the pair table is built for one token, from an expert table");
  // Four threads per expert (rounded up to whole waves) share the rank counting: measured
  // on MI355X at 128 experts, 512 threads beat 128, 256 and 1024.
  const int epad = (experts + 63) & ~63;
  const dim3 grid((unsigned)tokens), block((unsigned)min(kRouteThreads, 4 * epad));
  hipStream_t st = (hipStream_t)stream;
#define RT(DT_) hipLaunchKernelGGL(route_topk_kernel<DT_>, grid, block, 0, st, logits, experts, top_k, \
                                   keep_k, top_p, renorm, weights, ids, expert_table, pair_table)
  if (logits_dtype == DT_BF16) RT(DT_BF16);
  else if (logits_dtype == DT_FP16) RT(DT_FP16);
  else if (logits_dtype == DT_FP32) RT(DT_FP32);
  else return set_error(-2, "logits dtype must be 0 bf16, 1 fp16 or 2 fp32");
#undef RT
  return check_launch("route top-k");
}

extern "C" int vaayu_router_logits(const void* x, const void* w, int32_t x_dtype, void* logits,
                                   int32_t out_dtype, int32_t tokens, int32_t hidden,
                                   int32_t experts, void* stream) {
  clear_error();
  if (!x || !w || !logits) return set_error(-1, "null pointer argument");
  if (tokens <= 0 || experts <= 0 || hidden <= 0) return set_error(-2, "empty shape");
  if (hidden % 8) return set_error(-2, "hidden must be a multiple of 8");
  if (x_dtype != DT_BF16 && x_dtype != DT_FP16)
    return set_error(-2, "x and the router weight must be bf16 (0) or fp16 (1)");
  if (out_dtype != x_dtype && out_dtype != DT_FP32)
    return set_error(-2, "logits must be x's dtype or fp32 (2)");
  if ((uintptr_t)x % 16 || (uintptr_t)w % 16) return set_error(-2, "x and w must be 16-byte aligned");
  const int64_t rows = (int64_t)tokens * experts;
  if ((rows + kGemvWaves - 1) / kGemvWaves > 0x7FFFFFFF) return set_error(-2, "too many rows");
  const dim3 grid((unsigned)((rows + kGemvWaves - 1) / kGemvWaves)), block(kGemvWaves * 64);
  hipStream_t st = (hipStream_t)stream;
#define RG(X_, O_) hipLaunchKernelGGL((router_gemv_kernel<X_, O_>), grid, block, 0, st, x, w, logits, \
                                      tokens, hidden, experts)
  if (x_dtype == DT_BF16) {
    if (out_dtype == DT_FP32) RG(DT_BF16, DT_FP32); else RG(DT_BF16, DT_BF16);
  } else {
    if (out_dtype == DT_FP32) RG(DT_FP16, DT_FP32); else RG(DT_FP16, DT_FP16);
  }
#undef RG
  return check_launch("router logits");
}

