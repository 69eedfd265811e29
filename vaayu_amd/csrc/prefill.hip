// Prefill over packed experts: grouped GEMMs on MFMA (bf16/fp16 in, fp32 accumulate).
//
// Replaces the reference's three Triton launches (vaayu/packed_expert_kernels.py:179-260,
// launched by `_gate_up_g` :720-732, `_down_g` :735-749, `_reduce` :752-757) over the
// same tables `_prefill_tables` builds (:691-717):
//   tbl  [n_blocks, 2]   (packed address, scale address) of each 16-row block's expert
//   rows [n_blocks, 16]  row ids token*top_k + slot, -1 pads
//   ord  [tokens, top_k] row ids of each token's slots in ascending expert id
//
// Both GEMM kernels run v_mfma_f32_16x16x32 (bf16 or fp16 in, fp32 accumulate). The four
// 16-lane quarters of a wave each take one contiguous 16-byte unit of codes per K step, so a
// K step is 4 units; the MFMA's 32 K slots of quarter q map to codes [q*CPU + 8i, +8) of
// MFMA i. A and B use the same slot map, so each product is an ordinary dot over K in a
// fixed order. Every row's arithmetic is the same instruction sequence whatever its
// block-mates are (batch invariance), and nothing is split over K or accumulated
// atomically.
#include "common.hpp"
#include "abi_internal.hpp"

namespace vaayu {

template <int ACT>
__device__ __forceinline__ f32x4 mfma16(uint4 a, uint4 b, f32x4 c) {
  if constexpr (ACT == DT_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

__device__ __forceinline__ float load_dt(const void* p, int64_t i, int dt) {
  if (dt == DT_BF16) return load_as_float<DT_BF16>(p, i);
  if (dt == DT_FP16) return load_as_float<DT_FP16>(p, i);
  return load_as_float<DT_FP32>(p, i);
}

// B operands (8 weights each, as 4 packed pairs) of one unit of codes.
template <int BITS, int ACT>
__device__ __forceinline__ void unit_operands(uint4 q, float s_act, const Masks& M,
                                              uint4 (&b)[BITS == 4 ? 4 : 2]) {
  if constexpr (BITS == 4) {
    GroupK k = group_consts<4>(s_act);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t p[4];
      deq_word_i4<ACT>(w[i], k, M, p);
      b[i] = make_uint4(p[0], p[1], p[2], p[3]);
    }
  } else {
    GroupK k = group_consts<8>(s_act);
    uint32_t p0[2], p1[2], p2[2], p3[2];
    deq_word_i8<ACT>(q.x, k, M, p0);
    deq_word_i8<ACT>(q.y, k, M, p1);
    deq_word_i8<ACT>(q.z, k, M, p2);
    deq_word_i8<ACT>(q.w, k, M, p3);
    b[0] = make_uint4(p0[0], p0[1], p1[0], p1[1]);
    b[1] = make_uint4(p2[0], p2[1], p3[0], p3[1]);
  }
}

// ── run-tiled grouped GEMM ─────────────────────────────────────────────────────────────
//
// A work item is a RUN of up to kRun consecutive 16-row blocks of one expert (the table
// lists each expert's blocks contiguously) times 64 weight rows (N). Runs split where the
// expert changes and at block indices that are multiples of kRun, so a block can tell from
// the table alone whether it leads a run (its predecessor is another expert, or its index
// is a multiple of kRun) and how long the run is; items of non-leading blocks exit at once.
//
// Per K step (4 units of codes per weight row) the block stages the run's activation rows
// for that step in LDS (prefetched one step ahead in registers), each wave dequantizes its
// 16 weight rows' codes ONCE in VGPRs straight into MFMA B operands and runs them against
// every 16-row sub-tile of the run: the dequant cost is shared by up to kRun*16 rows. The
// A operand of sub-tile s comes from LDS with the same K-slot map as B (quarter q of the
// wave, MFMA i: codes [q*CPU + 8i, +8) of the step).
//
// XCD mapping: linear workgroup id L runs on XCD L % 8. Blocks are grouped by b / kRun
// (at most one full run per group) and group G is placed on XCD G % 8, with all of a
// group's N tiles consecutive in that XCD's order, so the items that share a run's
// activation rows share an L2.
constexpr int kRun = 8;
constexpr int kStride = 16;      // LDS row padding, bytes

struct RunInfo {
  int lead;       // 1 if this item computes
  int nblk;       // blocks in the run
};

__device__ __forceinline__ RunInfo run_of(const int64_t* __restrict__ tbl, int b, int n_blocks) {
  RunInfo r{0, 0};
  if (b >= n_blocks) return r;
  const int64_t me = tbl[2 * b];
  if (b % kRun != 0 && tbl[2 * (b - 1)] == me) return r;
  int n = 1;
  while (n < kRun && b + n < n_blocks && (b + n) % kRun != 0 && tbl[2 * (b + n)] == me) ++n;
  r.lead = 1;
  r.nblk = n;
  return r;
}

// (block b, N tile) of linear workgroup id L.
__device__ __forceinline__ void item_of(int L, int n_tiles, int& b, int& tile) {
  const int xcd = L & 7, j = L >> 3;
  const int per_group = kRun * n_tiles;                  // items of one group of blocks
  const int g = j / per_group, w = j - g * per_group;
  b = (g * 8 + xcd) * kRun + w / n_tiles;
  tile = w % n_tiles;
}

__host__ __device__ inline int items_for(int n_blocks, int n_tiles) {
  const int groups = (n_blocks + kRun - 1) / kRun;
  return ((groups + 7) / 8) * 8 * kRun * n_tiles;
}

typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ uint4 bload16(rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// A row offset that the buffer bounds check turns into zeros (padding rows), for any
// K offset added to it.
constexpr uint32_t kNoRow = 0xFFFF0000u;

// One K step of the run's activation rows: S*16 rows x KS codes (KS*2 bytes a row), in
// 16-byte pieces; piece t of thread i is row (t*256 + i) / PPR, piece (t*256 + i) % PPR.
// off[t] is that piece's byte offset in the activation buffer at K = 0 (kNoRow: padding).
template <int KS>
struct AStage {
  static constexpr int PPR = KS * 2 / 16;               // 16-byte pieces per row
  static constexpr int PER = kRun * 16 * PPR / 256;     // pieces per thread (full run)
  static constexpr int ROWS_PER_T = 256 / PPR;          // rows one piece index t covers
  uint32_t off[PER];
  uint4 v[PER];
};

// Piece offsets of this thread; `row_off(r)` = byte offset of run row r (kNoRow: padding).
template <int KS, typename RowOff>
__device__ __forceinline__ void a_plan(AStage<KS>& a, int S, RowOff row_off) {
  constexpr int PPR = AStage<KS>::PPR;
#pragma unroll
  for (int t = 0; t < AStage<KS>::PER; ++t) {
    const int idx = t * 256 + (int)threadIdx.x;
    const int r = idx / PPR, c = idx % PPR;
    const uint32_t ro = r < S * 16 ? row_off(r) : kNoRow;
    a.off[t] = ro == kNoRow ? kNoRow : ro + c * 16;
  }
}

template <int KS>
__device__ __forceinline__ bool a_live(int t, int S) {   // block-uniform
  return t * AStage<KS>::ROWS_PER_T < S * 16;
}

template <int KS>
__device__ __forceinline__ void a_load(AStage<KS>& a, rsrc_t src, int S, int k0) {
#pragma unroll
  for (int t = 0; t < AStage<KS>::PER; ++t)
    if (a_live<KS>(t, S)) a.v[t] = bload16(src, a.off[t] + (uint32_t)k0 * 2u);
}

template <int KS>
__device__ __forceinline__ void a_store(const AStage<KS>& a, char* lds, int S) {
  constexpr int PPR = AStage<KS>::PPR;
  constexpr int LROW = KS * 2 + kStride;
#pragma unroll
  for (int t = 0; t < AStage<KS>::PER; ++t) {
    if (a_live<KS>(t, S)) {
      const int idx = t * 256 + (int)threadIdx.x;
      *(uint4*)(lds + (idx / PPR) * LROW + (idx % PPR) * 16) = a.v[t];
    }
  }
}

// B codes and raw scale bits of one K step for one weight row (lane q's unit).
struct BStep {
  uint4 q;
  uint32_t s;
};

// Scale bits of dtype dt (wave-uniform) as fp32.
__device__ __forceinline__ float scale_of(uint32_t b, int dt) {
  if (dt == DT_FP32) return __builtin_bit_cast(float, b);
  const float bf = __builtin_bit_cast(float, b << 16);
  const float hf = (float)__builtin_bit_cast(_Float16, (uint16_t)b);
  return dt == DT_BF16 ? bf : hf;
}

// codes: the role's rows (code bytes); sc: the role's scales. Row n, K offset kc.
template <int BITS>
__device__ __forceinline__ BStep b_load(rsrc_t codes, rsrc_t sc, uint32_t row_bytes,
                                        uint32_t row_groups, int sb, int n, int kc, int gshift) {
  BStep r;
  r.q = bload16(codes, (uint32_t)n * row_bytes + (uint32_t)kc * BITS / 8);
  const uint32_t si = (uint32_t)n * row_groups + ((uint32_t)kc >> gshift);
  r.s = sb == 4 ? __builtin_amdgcn_raw_buffer_load_b32(sc, si * 4u, 0, 0)
                : (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(sc, si * 2u, 0, 0);
  return r;
}

template <int BITS, int ACT>
__global__ void __launch_bounds__(256)
prefill_gate_up_kernel(const void* __restrict__ x, uint32_t x_bytes, const int64_t* __restrict__ rows,
                       const int64_t* __restrict__ tbl, void* __restrict__ h, int n_blocks,
                       int n_tiles, int top_k, int hidden, int inter, int gshift, int sc_dt,
                       int64_t gate_w, int64_t gate_s, int64_t up_w, int64_t up_s) {
  constexpr int CPU = 128 / BITS;                   // codes per lane per K step
  constexpr int NM = CPU / 8;                       // MFMAs per K step per sub-tile
  constexpr int KS = 4 * CPU;                       // codes per K step
  constexpr int LROW = KS * 2 + kStride;            // LDS bytes per staged row
  __shared__ __align__(16) char lds[kRun * 16 * LROW];
  int b, tile;
  item_of(blockIdx.x, n_tiles, b, tile);
  const RunInfo run = run_of(tbl, b, n_blocks);
  if (!run.lead) return;
  const int S = run.nblk;
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int q = lane >> 4, m = lane & 15;
  const int n = tile * 64 + wv * 16 + m;            // weight row (output column) of lane m
  const bool n_ok = n < inter;
  const int nn = n_ok ? n : 0;
  const char* pk = (const char*)tbl[2 * b];
  const char* sc = (const char*)tbl[2 * b + 1];
  const int sb = sc_dt == DT_FP32 ? 4 : 2;
  const uint32_t row_bytes = (uint32_t)hidden * BITS / 8;
  const uint32_t row_groups = (uint32_t)hidden >> gshift;
  const uint32_t role_bytes = row_bytes * (uint32_t)inter;
  const uint32_t role_sc = row_groups * (uint32_t)inter * sb;
  const rsrc_t G = rsrc(pk + gate_w * 4, role_bytes), U = rsrc(pk + up_w * 4, role_bytes);
  const rsrc_t GS = rsrc(sc + gate_s * sb, role_sc), US = rsrc(sc + up_s * sb, role_sc);
  const rsrc_t X = rsrc(x, x_bytes);
  const int64_t* rrow = rows + (int64_t)b * 16;
  AStage<KS> a;
  a_plan<KS>(a, S, [&](int r) -> uint32_t {
    const int64_t rid = rrow[r];
    return rid >= 0 ? (uint32_t)(rid / top_k) * (uint32_t)hidden * 2u : kNoRow;
  });
  const Masks M = make_masks();
  f32x4 ag[kRun], au[kRun];
#pragma unroll
  for (int s = 0; s < kRun; ++s) {
    ag[s] = (f32x4){0.f, 0.f, 0.f, 0.f};
    au[s] = (f32x4){0.f, 0.f, 0.f, 0.f};
  }
  a_load<KS>(a, X, S, 0);
  BStep bg = b_load<BITS>(G, GS, row_bytes, row_groups, sb, nn, q * CPU, gshift);
  BStep bu = b_load<BITS>(U, US, row_bytes, row_groups, sb, nn, q * CPU, gshift);
  for (int k0 = 0; k0 < hidden; k0 += KS) {
    __syncthreads();                                 // previous step's LDS reads are done
    a_store<KS>(a, lds, S);
    const int kn = k0 + KS;
    if (kn < hidden) a_load<KS>(a, X, S, kn);
    uint4 og[NM], ou[NM];
    unit_operands<BITS, ACT>(bg.q, round_act<ACT>(scale_of(bg.s, sc_dt)), M, og);
    unit_operands<BITS, ACT>(bu.q, round_act<ACT>(scale_of(bu.s, sc_dt)), M, ou);
    if (kn < hidden) {
      bg = b_load<BITS>(G, GS, row_bytes, row_groups, sb, nn, kn + q * CPU, gshift);
      bu = b_load<BITS>(U, US, row_bytes, row_groups, sb, nn, kn + q * CPU, gshift);
    }
    __syncthreads();                                 // this step's rows are in LDS
#pragma unroll
    for (int s = 0; s < kRun; ++s) {
      if (s < S) {
#pragma unroll
        for (int i = 0; i < NM; ++i) {
          const uint4 av = *(const uint4*)(lds + (s * 16 + m) * LROW + (q * CPU + 8 * i) * 2);
          ag[s] = mfma16<ACT>(av, og[i], ag[s]);
          au[s] = mfma16<ACT>(av, ou[i], au[s]);
        }
      }
    }
  }
  // C layout: lane (q, m) holds rows 4q..4q+3 of sub-tile s, column m.
#pragma unroll
  for (int s = 0; s < kRun; ++s) {
    if (s < S) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t r = rrow[s * 16 + 4 * q + i];
        if (r >= 0 && n_ok) store_act<ACT>(h, r * inter + n, silu_mul<ACT>(ag[s][i], au[s][i]));
      }
    }
  }
}

template <int BITS, int ACT>
__global__ void __launch_bounds__(256)
prefill_down_kernel(const void* __restrict__ h, uint32_t h_bytes, const int64_t* __restrict__ rows,
                    const int64_t* __restrict__ tbl, const void* __restrict__ rw, int rw_dt,
                    float* __restrict__ y, int n_blocks, int n_tiles, int hidden, int inter,
                    int gshift, int sc_dt, int64_t down_w, int64_t down_s, int w_round) {
  constexpr int CPU = 128 / BITS;
  constexpr int NM = CPU / 8;
  constexpr int KS = 4 * CPU;
  constexpr int LROW = KS * 2 + kStride;
  __shared__ __align__(16) char lds[kRun * 16 * LROW];
  int b, tile;
  item_of(blockIdx.x, n_tiles, b, tile);
  const RunInfo run = run_of(tbl, b, n_blocks);
  if (!run.lead) return;
  const int S = run.nblk;
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int q = lane >> 4, m = lane & 15;
  const int n = tile * 64 + wv * 16 + m;
  const bool n_ok = n < hidden;
  const int nn = n_ok ? n : 0;
  const char* pk = (const char*)tbl[2 * b];
  const char* sc = (const char*)tbl[2 * b + 1];
  const int sb = sc_dt == DT_FP32 ? 4 : 2;
  const uint32_t row_bytes = (uint32_t)inter * BITS / 8;
  const uint32_t row_groups = (uint32_t)inter >> gshift;
  const rsrc_t D = rsrc(pk + down_w * 4, row_bytes * (uint32_t)hidden);
  const rsrc_t DS = rsrc(sc + down_s * sb, row_groups * (uint32_t)hidden * sb);
  const rsrc_t HB = rsrc(h, h_bytes);
  const int64_t* rrow = rows + (int64_t)b * 16;
  AStage<KS> a;
  a_plan<KS>(a, S, [&](int r) -> uint32_t {
    const int64_t rid = rrow[r];
    return rid >= 0 ? (uint32_t)rid * (uint32_t)inter * 2u : kNoRow;
  });
  const Masks M = make_masks();
  f32x4 acc[kRun];
#pragma unroll
  for (int s = 0; s < kRun; ++s) acc[s] = (f32x4){0.f, 0.f, 0.f, 0.f};
  a_load<KS>(a, HB, S, 0);
  BStep bd = b_load<BITS>(D, DS, row_bytes, row_groups, sb, nn, q * CPU, gshift);
  for (int k0 = 0; k0 < inter; k0 += KS) {
    __syncthreads();
    a_store<KS>(a, lds, S);
    const int kn = k0 + KS;
    if (kn < inter) a_load<KS>(a, HB, S, kn);
    uint4 od[NM];
    unit_operands<BITS, ACT>(bd.q, round_act<ACT>(scale_of(bd.s, sc_dt)), M, od);
    if (kn < inter) bd = b_load<BITS>(D, DS, row_bytes, row_groups, sb, nn, kn + q * CPU, gshift);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < kRun; ++s) {
      if (s < S) {
#pragma unroll
        for (int i = 0; i < NM; ++i) {
          const uint4 av = *(const uint4*)(lds + (s * 16 + m) * LROW + (q * CPU + 8 * i) * 2);
          acc[s] = mfma16<ACT>(av, od[i], acc[s]);
        }
      }
    }
  }
#pragma unroll
  for (int s = 0; s < kRun; ++s) {
    if (s < S) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t r = rrow[s * 16 + 4 * q + i];
        if (r >= 0 && n_ok) {
          float c = round_act<ACT>(acc[s][i]) * load_dt(rw, r, rw_dt);
          if (w_round) c = round_act<ACT>(c);
          y[r * hidden + n] = c;
        }
      }
    }
  }
}

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

// Why the prefill kernels cannot take this geometry, or nullptr.
const char* prefill_unsupported(const vaayu_geom* g, int act) {
  if (act != DT_BF16 && act != DT_FP16) return "activation dtype (MFMA takes bf16 / fp16)";
  if (g->bits != 4 && g->bits != 8) return "bit width (the MFMA path takes 4 and 8)";
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
                                     void* h, int32_t n_blocks, int32_t top_k,
                                     const vaayu_geom* g, int32_t act, int32_t scale_dtype,
                                     void* stream) {
  clear_error();
  if (!x || !rows || !table || !h || !g) return set_error(-1, "null pointer argument");
  if (n_blocks <= 0 || top_k <= 0) return set_error(-1, "n_blocks / top_k must be positive");
  if (scale_dtype < 0 || scale_dtype > 2) return set_error(-1, "scale dtype");
  if (const char* why = prefill_unsupported(g, act)) return set_error(-2, why);
  const int n_tiles = (g->inter + 63) / 64;
  int gshift = 0;
  while ((1 << gshift) < g->group) ++gshift;
  const dim3 grid((unsigned)items_for(n_blocks, n_tiles)), block(256);
  hipStream_t st = (hipStream_t)stream;
#define GU(B_, A_)                                                                        \
  hipLaunchKernelGGL((prefill_gate_up_kernel<B_, A_>), grid, block, 0, st, x, kNoRow, rows,     \
                     table, h, n_blocks, n_tiles, top_k, g->hidden, g->inter, gshift,         \
                     scale_dtype, g->gate_w, g->gate_s, g->up_w, g->up_s)
  if (g->bits == 4 && act == DT_BF16) GU(4, DT_BF16);
  else if (g->bits == 4) GU(4, DT_FP16);
  else if (act == DT_BF16) GU(8, DT_BF16);
  else GU(8, DT_FP16);
#undef GU
  return check_launch("prefill gate/up");
}

extern "C" int vaayu_prefill_down(const void* h, const int64_t* rows, const int64_t* table,
                                  const void* routing_weights, int32_t rw_dtype, float* y,
                                  int32_t n_blocks, const vaayu_geom* g, int32_t act,
                                  int32_t scale_dtype, int32_t w_round, void* stream) {
  clear_error();
  if (!h || !rows || !table || !routing_weights || !y || !g)
    return set_error(-1, "null pointer argument");
  if (n_blocks <= 0) return set_error(-1, "n_blocks must be positive");
  if (scale_dtype < 0 || scale_dtype > 2 || rw_dtype < 0 || rw_dtype > 2)
    return set_error(-1, "scale / routing-weight dtype");
  if (const char* why = prefill_unsupported(g, act)) return set_error(-2, why);
  const int n_tiles = (g->hidden + 63) / 64;
  int gshift = 0;
  while ((1 << gshift) < g->group) ++gshift;
  const dim3 grid((unsigned)items_for(n_blocks, n_tiles)), block(256);
  hipStream_t st = (hipStream_t)stream;
#define DN(B_, A_)                                                                          \
  hipLaunchKernelGGL((prefill_down_kernel<B_, A_>), grid, block, 0, st, h, kNoRow, rows, table, \
                     routing_weights, rw_dtype, y, n_blocks, n_tiles, g->hidden, g->inter,      \
                     gshift, scale_dtype, g->down_w, g->down_s, w_round)
  if (g->bits == 4 && act == DT_BF16) DN(4, DT_BF16);
  else if (g->bits == 4) DN(4, DT_FP16);
  else if (act == DT_BF16) DN(8, DT_BF16);
  else DN(8, DT_FP16);
#undef DN
  return check_launch("prefill down");
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
