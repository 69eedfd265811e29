// Prefill over packed experts: grouped GEMMs on MFMA (bf16/fp16 in, fp32 accumulate).
// Kernels shared by prefill.hip (integer codes) and prefill_formats.hip (e4m3, e2m1).
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
#pragma once
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

// ── run-tiled grouped GEMM ─────────────────────────────────────────────────────────────
//
// A work item is a RUN of up to R consecutive 16-row blocks of one expert (the table lists
// each expert's blocks contiguously) times kTileN weight rows (N); R is kRunGateUp for
// gate/up and kRunDown for down. The host lists the runs (an expert's blocks in runs of R
// from its first block on) in a work list, so only workgroups with work are launched: a
// workgroup launched only to find that it has nothing to do holds a whole CU (one gate/up
// workgroup fills one) for a few memory round trips. The kernels branch once on the run's
// length S to a K loop compiled for that S.
//
// Per K step (4 units of codes per weight row) the block stages the run's activation rows
// in LDS, each wave dequantizes its 16 weight rows' codes ONCE in VGPRs straight into MFMA B
// operands and runs them against every 16-row sub-tile of the run: the dequant cost is
// shared by up to R*16 rows. The A operand of sub-tile s comes from LDS with the same K-slot
// map as B (quarter q of the wave, MFMA i: codes [q*CPU + 8i, +8) of the step).
//
// XCD mapping: linear workgroup id L runs on XCD L % 8; the work list gives each XCD its
// runs, with all N tiles of a run consecutive in that XCD's order, so the items that share
// a run's activation rows share an L2.
//
// Runs of more than kPairS blocks take each K step as the MFMAs of the step, then the
// dequant of the next step's operands, so the two steps' operands are never live together
// and the 16-block path's 128 accumulators fit two waves per SIMD.

constexpr int kRunGateUp = 16;   // blocks per run, gate/up: the longest, and
constexpr int kRunGateUpShort = 4;  // the kernel of calls whose runs are at most this long
                                    // (128 VGPRs, so two blocks share a CU)
constexpr int kRunDown = 16;     // blocks per run, down: the longest, and
constexpr int kRunDownShort = 8; // the kernel of calls whose runs are at most this long
                                 // (118 VGPRs, so two blocks share a CU)
constexpr int kWaves = 8;        // waves per workgroup, 16 weight rows (N) each
constexpr int kTileN = 16 * kWaves;

// Work list: one int64 entry per (slot k, XCD x) at work[k * 8 + x], b * 32 + S for the
// run of S blocks that starts at table block b (S <= the kernel's run length), -1 for none.
// Workgroup L runs on XCD x = L % 8 and takes N tile j % n_tiles of the run in slot
// j / n_tiles of its XCD (j = L / 8), so all N tiles of a run share one XCD's L2 and only
// workgroups with work are launched. The host chooses which runs go to which XCD.
constexpr int kXcds = 8;
constexpr int64_t kRunShift = 5;

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

// Activation rows (x, one per token) and intermediate rows (h, one per table row) are
// addressed with 32-bit byte offsets. A launch's tables hold at most n_blocks * 16 row ids
// (token * top_k + slot), so a launch whose rows could start past kOffsetLimit bytes is
// refused: callers split such a call into token chunks. The limit leaves room below kNoRow
// for any K offset inside a row.
constexpr int64_t kOffsetLimit = 0xF0000000ll;

// Why a launch over n_blocks table blocks could address past the limit, or nullptr:
// x_row_bytes for rows read per token (gate/up), h_row_bytes per table row (down).
inline const char* rows_out_of_reach(int n_blocks, int top_k, int64_t x_row_bytes,
                                     int64_t h_row_bytes) {
  const int64_t rows = (int64_t)n_blocks * 16;
  if ((rows + top_k - 1) / top_k * x_row_bytes > kOffsetLimit)
    return "activation rows past the 32-bit offset range: launch fewer tokens per call";
  if (rows * h_row_bytes > kOffsetLimit)
    return "intermediate rows past the 32-bit offset range: launch fewer tokens per call";
  return nullptr;
}

// One K step of a run's activation rows (S*16 rows x KS codes, RB = KS*2 bytes a row) lives
// in LDS as S*16 rows of RB bytes, row r's 16-byte piece c at position c ^ swz(r) (below):
// the A reads of one MFMA (16 rows at one piece) then fall on distinct banks. Rows reach LDS by
// direct buffer->LDS loads: one wave instruction writes 1 KB (64 lanes x 16 B) contiguously,
// i.e. 1024/RB rows, so lane l of instruction g loads row g*(1024/RB) + l/PPR, the piece
// that belongs at position l % PPR. off[j] is lane's byte offset (at K = 0) in the
// activation buffer for its j-th instruction g = kWaves*j + wave (kNoRow: a padding row, read as
// zeros by the bounds check).
// Row r's 16-byte piece c sits at position c ^ swz(r) of the row. For 16 pieces a row
// (4-bit codes) the 4x4 transpose of r's low bits keeps the 16 rows an A read touches on
// distinct banks (SQ_LDS_BANK_CONFLICT: none; with r % 16 two-way conflicts, and down, whose
// A reads feed one MFMA each, ran up to 12 % slower); 8-bit codes keep r % 8.
template <int PPR>
__device__ __forceinline__ int swz(int r) {
  if constexpr (PPR == 16) return ((r >> 2) & 3) | ((r & 3) << 2);
  else return r % PPR;
}

template <int KS, int S>
struct AStage {
  static constexpr int RB = KS * 2;                     // bytes per staged row
  static constexpr int PPR = RB / 16;                   // 16-byte pieces per row
  static constexpr int RPI = 1024 / RB;                 // rows per wave instruction
  static constexpr int INSTR = S * 16 / RPI;            // instructions per step (block)
  static constexpr int PER = (INSTR + kWaves - 1) / kWaves;   // per wave
  static constexpr int BYTES = S * 16 * RB;             // one step's rows
  uint32_t off[PER];
};

template <int KS, int S, typename RowOff>
__device__ __forceinline__ void a_plan(AStage<KS, S>& a, RowOff row_off) {
  using A = AStage<KS, S>;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < A::PER; ++j) {
    const int g = kWaves * j + w;
    const int r = g * A::RPI + l / A::PPR;
    const int c = (l % A::PPR) ^ swz<A::PPR>(r);
    const uint32_t ro = g < A::INSTR ? row_off(r) : kNoRow;
    a.off[j] = ro == kNoRow ? kNoRow : ro + c * 16;
  }
}

// Issue one step's rows into `buf` (wave-uniform LDS address of the step's tile).
template <int KS, int S>
__device__ __forceinline__ void a_issue(const AStage<KS, S>& a, rsrc_t src, char* buf, int k0) {
  using A = AStage<KS, S>;
  const int w = threadIdx.x >> 6;
#pragma unroll
  for (int j = 0; j < A::PER; ++j) {
    const int g = kWaves * j + w;
    if (A::INSTR % kWaves == 0 || g < A::INSTR) {
#if defined(__HIP_DEVICE_COMPILE__)        // a gfx950 instruction: no host-pass form
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          src, (__attribute__((address_space(3))) void*)(buf + g * 1024), 16,
          a.off[j] + (uint32_t)k0 * 2u, 0, 0, 0);
#endif
    }
  }
}

// The A operand of MFMA (s, i) for lane (q, m): row 16s + m, piece q*CPU/8 + i.
template <int KS, int S, int CPU>
__device__ __forceinline__ uint4 a_read(const char* buf, int s, int i, int q, int m) {
  using A = AStage<KS, S>;
  const int r = s * 16 + m;
  const int piece = q * (CPU / 8) + i;
  return *(const uint4*)(buf + r * A::RB + ((piece ^ swz<A::PPR>(r)) * 16));
}

// B codes and raw scale bits of one K step for one weight row (lane q's unit).
struct BStep {
  uint4 q;
  uint32_t s;
};

// Raw scale bits as fp32. SW = 32: fp32 bits. SW = 8: an E8M0 exponent byte. SW = 16: bf16 or fp16 bits, chosen by
// `bf16_mask` (all ones: bf16), an opaque per-lane value so the choice is a select and not
// a branch (a branch would split the K loop's basic block).
template <int SW>
__device__ __forceinline__ float scale_of(uint32_t b, uint32_t bf16_mask) {
  if constexpr (SW == 32) {
    return __builtin_bit_cast(float, b);
  } else if constexpr (SW == 8) {
    return e8m0_to_f32(b & 0xFFu);
  } else {
    const uint32_t bf = b << 16;
    const uint32_t hf = __builtin_bit_cast(uint32_t, (float)__builtin_bit_cast(_Float16, (uint16_t)b));
    return __builtin_bit_cast(float, (bf16_mask & bf) | (~bf16_mask & hf));
  }
}

// One role of one expert as a lane reads it: codes and scales (buffer descriptors), the
// lane's weight row n (clamped into range).
struct Role {
  rsrc_t codes, sc;
  uint32_t row_bytes, row_groups;
  uint32_t bf16_mask;
  uint32_t kc_end;             // the row's K: E8M0 scales of units at or past it read as 0
  int n, gshift, rshift;       // rshift: log2(rows per scale block), 0 but for e4m3
};

template <int SW>
__device__ __forceinline__ Role make_role(const char* pk, int64_t w_off, const char* sc,
                                          int64_t s_off, int rows, int k, int bits, int gshift,
                                          int rshift, int sc_dt, int n) {
  Role r;
  constexpr int sb = SW / 8;
  r.row_bytes = (uint32_t)k * bits / 8;
  r.row_groups = (uint32_t)k >> gshift;
  r.codes = rsrc(pk + w_off * 4, r.row_bytes * (uint32_t)rows);
  r.sc = rsrc(sc + s_off * sb, r.row_groups * (uint32_t)(rows >> rshift) * sb);
  r.bf16_mask = opaque(sc_dt == DT_BF16 ? 0xFFFFFFFFu : 0u);
  r.kc_end = (uint32_t)k;
  r.n = n;
  r.gshift = gshift;
  r.rshift = rshift;
  return r;
}

template <int BITS, int SW>
__device__ __forceinline__ BStep b_load(const Role& r, int kc) {
  BStep o;
  o.q = bload16(r.codes, (uint32_t)r.n * r.row_bytes + (uint32_t)kc * BITS / 8);
  const uint32_t si = (uint32_t)(r.n >> r.rshift) * r.row_groups + ((uint32_t)kc >> r.gshift);
  if constexpr (SW == 32) {
    o.s = __builtin_amdgcn_raw_buffer_load_b32(r.sc, si * 4u, 0, 0);
  } else if constexpr (SW == 8) {
    // A unit past the row's K (a K loop padded to whole steps) would take the next row's
    // codes and scale, which may be another expert's and any byte; its scale reads as 0,
    // which makes every weight of the unit +-0 (the e2m1 dequant clears the codes'
    // magnitudes for a zero scale), so the padding adds exact zeros whatever lies there.
    const uint32_t sb = (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r.sc, si, 0, 0);
    o.s = (uint32_t)kc < r.kc_end ? sb : 0u;
  } else {
    o.s = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r.sc, si * 2u, 0, 0);
  }
  return o;
}

// One K step of a run longer than kPairS blocks (rows in `cur`, B operands `o`): this
// step's MFMAs, each A operand read from LDS two MFMA slots ahead, then the dequant of the
// next step's operands (from `raw`, into `on`), so the operands of the two steps are never
// live together. (Measured against the dequant spread between the MFMAs with both operand
// sets live: the same or faster on every workload, in 60-110 fewer VGPRs.)
template <int F, int ACT, int SW, int NR, int S>
__device__ __forceinline__ void k_step_split(const char* cur,
                                             const uint4 (&o)[NR][128 / CodeBits<F>::value / 8],
                                             const BStep (&raw)[NR], const Role (&role)[NR],
                                             uint4 (&on)[NR][128 / CodeBits<F>::value / 8],
                                             const Masks& M, int q, int m, f32x4 (&acc)[NR][S]) {
  constexpr int CPU = 128 / CodeBits<F>::value;
  constexpr int NM = CPU / 8;
  constexpr int KS = 4 * CPU;
  constexpr int SLOTS = S * NM, JOBS = NR * NM;
  // A reads ahead of their MFMAs: down's feed one MFMA each, so they run further ahead
  // (measured: Mixtral down 156 -> 149 us at four slots, DeepSeek-V3 976 -> 967)
  constexpr int AH = NR == 1 ? 4 : 2;
  uint4 ar[AH + 1];
#pragma unroll
  for (int g = 0; g < AH; ++g) ar[g] = a_read<KS, S, CPU>(cur, g / NM, g % NM, q, m);
#pragma unroll
  for (int g = 0; g < SLOTS; ++g) {
    const int s = g / NM, i = g % NM;
    if (g + AH < SLOTS)
      ar[(g + AH) % (AH + 1)] = a_read<KS, S, CPU>(cur, (g + AH) / NM, (g + AH) % NM, q, m);
    const uint4 av = ar[g % (AH + 1)];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r][s] = mfma16<ACT>(av, o[r][i], acc[r][s]);
  }
  __builtin_amdgcn_sched_group_barrier(0x100, AH + 1, 0);
#pragma unroll
  for (int g = 0; g < SLOTS; ++g) {
    __builtin_amdgcn_sched_group_barrier(0x008, NR, 0);
    if (g + AH + 1 < SLOTS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  float sn[NR];
  GroupK kn[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    sn[r] = applied_scale<F, ACT>(scale_of<SW>(raw[r].s, role[r].bf16_mask));
    kn[r] = group_of<F>(sn[r]);
  }
#pragma unroll
  for (int j = 0; j < JOBS; ++j)
    on[j / NM][j % NM] = operand_i<F, ACT>(raw[j / NM].q, kn[j / NM], sn[j / NM], M, j % NM);
  __builtin_amdgcn_sched_barrier(0);
}

// The K loop of one run: NR roles sharing the activation rows (gate/up: 2, down: 1), S
// sub-tiles of 16 rows; acc[r][s] is the 16x16 fp32 tile of role r, sub-tile s.
//
// Pipeline (two LDS tiles, lds0 and lds1, one step each; the loop runs two steps per
// iteration so every access names its tile at compile time): step t's rows are in one
// tile and its B operands are dequantized; the other tile receives step t+1's rows by
// direct loads issued before step t's MFMAs; the codes of step t+2 are requested after
// them. At the end of the step one barrier (its wait also covers the direct loads) makes
// step t+1's rows visible and frees step t's tile. Requests past the last step re-read the
// last step (no branches in the loop body; their results are not used).
// ── short runs: two K steps per barrier ──────────────────────────────────────────────────
//
// Runs of up to kPairS blocks take the K loop two steps at a time: a tile (sized for one
// step of a full run) holds two steps' activation rows, and each pair of steps starts by sending
// the next pair's rows (to the other tile) and requesting the next pair's codes, then
// computes its two steps (each step's B operands built right before its MFMAs) and ends at
// one barrier. That barrier waits for the rows just sent; the codes, requested after them,
// stay in flight until the next pair's barrier, so they have two steps to arrive, and half
// as many barriers stand in a short run's K loop. Every output takes the same MFMAs in the
// same order as in run_k, so the bits are the same whatever the run's length.
// A pair tile holds two steps of S*16 rows (S <= kPairS), inside a kernel's LDS tile
// (tile_blocks: one step of a full run, or two steps of the longest run that takes pairs).
constexpr int kPairS = 4;

constexpr int tile_blocks(int R) { return R <= kPairS ? 2 * R : R; }
static_assert(2 * kPairS <= tile_blocks(kRunGateUpShort) && 2 * kPairS <= kRunDownShort &&
                  2 * kPairS <= kRunGateUp,
              "a pair of steps must fit one LDS tile");

template <int F, int ACT, int SW, int NR, int S>
__device__ __forceinline__ void one_step(const char* buf, const BStep (&raw)[NR],
                                         const Role (&role)[NR], const Masks& M, int q, int m,
                                         f32x4 (&acc)[NR][S]) {
  constexpr int CPU = 128 / CodeBits<F>::value;
  constexpr int NM = CPU / 8;
  constexpr int KS = 4 * CPU;
  float sn[NR];
  GroupK kn[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    sn[r] = applied_scale<F, ACT>(scale_of<SW>(raw[r].s, role[r].bf16_mask));
    kn[r] = group_of<F>(sn[r]);
  }
#pragma unroll
  for (int i = 0; i < NM; ++i) {
    uint4 b[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) b[r] = operand_i<F, ACT>(raw[r].q, kn[r], sn[r], M, i);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const uint4 av = a_read<KS, S, CPU>(buf, s, i, q, m);
#pragma unroll
      for (int r = 0; r < NR; ++r) acc[r][s] = mfma16<ACT>(av, b[r], acc[r][s]);
    }
  }
}

template <int F, int ACT, int SW, int NR, int S>
__device__ __forceinline__ void pair_step(const char* cur, char* nxt, rsrc_t src,
                                          const AStage<512 / CodeBits<F>::value, S>& a, int t,
                                          int T, int last, const BStep (&c0)[NR],
                                          const BStep (&c1)[NR], BStep (&n0)[NR],
                                          BStep (&n1)[NR], const Role (&role)[NR],
                                          const Masks& M, int q, int m, f32x4 (&acc)[NR][S]) {
  constexpr int BITS = CodeBits<F>::value;
  constexpr int CPU = 128 / BITS;
  constexpr int KS = 4 * CPU;
  using A = AStage<KS, S>;
  const int k2 = min((t + 2) * KS, last), k3 = min((t + 3) * KS, last);
  a_issue<KS, S>(a, src, nxt, k2);
  a_issue<KS, S>(a, src, nxt + A::BYTES, k3);
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    n0[r] = b_load<BITS, SW>(role[r], k2 + q * CPU);
    n1[r] = b_load<BITS, SW>(role[r], k3 + q * CPU);
  }
  __builtin_amdgcn_sched_barrier(0);
  one_step<F, ACT, SW, NR, S>(cur, c0, role, M, q, m, acc);
  if (t + 1 < T) one_step<F, ACT, SW, NR, S>(cur + A::BYTES, c1, role, M, q, m, acc);
  __syncthreads();
}

template <int F, int ACT, int SW, int NR, int S>
__device__ __forceinline__ void run_k_pairs(const Role (&role)[NR], rsrc_t src,
                                            const AStage<512 / CodeBits<F>::value, S>& a,
                                            char* lds0, char* lds1, int K, int q, int m,
                                            f32x4 (&acc)[NR][S]) {
  constexpr int BITS = CodeBits<F>::value;
  constexpr int CPU = 128 / BITS;
  constexpr int KS = 4 * CPU;
  using A = AStage<KS, S>;
  static_assert(2 * S <= kRunGateUp && 2 * S <= kRunDownShort, "a pair of steps must fit one tile");
  const Masks M = make_masks();
  const int T = K / KS, last = K - KS;
  BStep c0[NR], c1[NR], n0[NR], n1[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
#pragma unroll
    for (int s = 0; s < S; ++s) acc[r][s] = (f32x4){0.f, 0.f, 0.f, 0.f};
  }
  a_issue<KS, S>(a, src, lds0, 0);
  a_issue<KS, S>(a, src, lds0 + A::BYTES, min(KS, last));
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    c0[r] = b_load<BITS, SW>(role[r], q * CPU);
    c1[r] = b_load<BITS, SW>(role[r], min(KS, last) + q * CPU);
  }
  __syncthreads();
  for (int t = 0; t < T; t += 4) {
    pair_step<F, ACT, SW, NR, S>(lds0, lds1, src, a, t, T, last, c0, c1, n0, n1, role, M, q, m, acc);
    if (t + 2 >= T) break;
    pair_step<F, ACT, SW, NR, S>(lds1, lds0, src, a, t + 2, T, last, n0, n1, c0, c1, role, M, q, m,
                                 acc);
  }
}

template <int F, int ACT, int SW, int NR, int S>
__device__ __forceinline__ void run_k(const Role (&role)[NR], rsrc_t src,
                                      const AStage<512 / CodeBits<F>::value, S>& a, char* lds0,
                                      char* lds1, int K, int q, int m, f32x4 (&acc)[NR][S]) {
  if constexpr (S <= kPairS) {
    run_k_pairs<F, ACT, SW, NR, S>(role, src, a, lds0, lds1, K, q, m, acc);
    return;
  }
  constexpr int BITS = CodeBits<F>::value;
  constexpr int CPU = 128 / BITS;
  constexpr int NM = CPU / 8;
  constexpr int KS = 4 * CPU;
  const Masks M = make_masks();
  const int last = K - KS;
  uint4 oa[NR][NM], ob[NR][NM];
  BStep raw[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int s = 0; s < S; ++s) acc[r][s] = (f32x4){0.f, 0.f, 0.f, 0.f};
  a_issue<KS, S>(a, src, lds0, 0);
#pragma unroll
  for (int r = 0; r < NR; ++r) raw[r] = b_load<BITS, SW>(role[r], q * CPU);
  __syncthreads();
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const float s0 = applied_scale<F, ACT>(scale_of<SW>(raw[r].s, role[r].bf16_mask));
    const GroupK k0 = group_of<F>(s0);
#pragma unroll
    for (int i = 0; i < NM; ++i) oa[r][i] = operand_i<F, ACT>(raw[r].q, k0, s0, M, i);
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) raw[r] = b_load<BITS, SW>(role[r], min(KS, last) + q * CPU);
  int k0 = 0;
  for (; k0 + KS < K; k0 += 2 * KS) {
    // step k0 (tile lds0, operands oa) -> step k0 + KS (tile lds1, operands ob); the
    // scheduling barriers keep the next step's loads ahead of this step's MFMAs
    a_issue<KS, S>(a, src, lds1, k0 + KS);
    __builtin_amdgcn_sched_barrier(0);
    k_step_split<F, ACT, SW, NR, S>(lds0, oa, raw, role, ob, M, q, m, acc);
#pragma unroll
    for (int r = 0; r < NR; ++r) raw[r] = b_load<BITS, SW>(role[r], min(k0 + 2 * KS, last) + q * CPU);
    __syncthreads();
    // step k0 + KS (tile lds1, operands ob) -> step k0 + 2 KS (tile lds0, operands oa)
    a_issue<KS, S>(a, src, lds0, min(k0 + 2 * KS, last));
    __builtin_amdgcn_sched_barrier(0);
    k_step_split<F, ACT, SW, NR, S>(lds1, ob, raw, role, oa, M, q, m, acc);
#pragma unroll
    for (int r = 0; r < NR; ++r) raw[r] = b_load<BITS, SW>(role[r], min(k0 + 3 * KS, last) + q * CPU);
    __syncthreads();
  }
  if (k0 < K)                                      // an odd number of steps: the last one
    k_step_split<F, ACT, SW, NR, S>(lds0, oa, raw, role, ob, M, q, m, acc);
}

struct Item {
  int b, tile, S;
};

// This workgroup's run and N tile, or S = 0 when its slot holds none (or an entry that
// does not fit the table: such an entry computes nothing).
template <int R>
__device__ __forceinline__ Item item_here(const int64_t* __restrict__ work, int n_blocks,
                                          int n_tiles) {
  const int L = blockIdx.x, x = L % kXcds, j = L / kXcds;
  const int k = j / n_tiles;
  Item it;
  it.tile = j - k * n_tiles;
  const int64_t e = work[(int64_t)k * kXcds + x];
  const int64_t b = e >> kRunShift, S = e & ((1 << kRunShift) - 1);
  const bool ok = e >= 0 && S >= 1 && S <= R && b + S <= n_blocks;
  it.b = ok ? (int)b : 0;
  it.S = ok ? (int)S : 0;
  return it;
}

template <int F, int ACT, int SW, int S>
__device__ __forceinline__ void gate_up_run(const Item& it, const void* x,
                                            const int64_t* rows, const int64_t* tbl, void* h,
                                            int top_k, int hidden, int inter, int gshift,
                                            int rshift, int sc_dt, int64_t gate_w,
                                            int64_t gate_s, int64_t up_w, int64_t up_s,
                                            char* lds0, char* lds1, int* rid_s) {
  constexpr int BITS = CodeBits<F>::value;
  constexpr int KS = 512 / BITS;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int q = lane >> 4, m = lane & 15;
  const int n = it.tile * kTileN + wv * 16 + m;         // weight row (output column) of lane m
  const bool n_ok = n < inter;
  const int nn = n_ok ? n : 0;
  const char* pk = (const char*)tbl[2 * it.b];
  const char* sc = (const char*)tbl[2 * it.b + 1];
  const Role role[2] = {
      make_role<SW>(pk, gate_w, sc, gate_s, inter, hidden, BITS, gshift, rshift, sc_dt, nn),
      make_role<SW>(pk, up_w, sc, up_s, inter, hidden, BITS, gshift, rshift, sc_dt, nn)};
  const int64_t* rrow = rows + (int64_t)it.b * 16;
  AStage<KS, S> a;
  a_plan<KS, S>(a, [&](int r) -> uint32_t {
    const int64_t rid = rrow[r];
    return rid >= 0 ? (uint32_t)(rid / top_k) * (uint32_t)hidden * 2u : kNoRow;
  });
  // the run's row ids in LDS (the K loop's first barrier publishes them) for the epilogue
  if (threadIdx.x < S * 16) rid_s[threadIdx.x] = (int)rrow[threadIdx.x];
  f32x4 acc[2][S];
  run_k<F, ACT, SW, 2, S>(role, rsrc(x, kNoRow), a, lds0, lds1, hidden, q, m, acc);
  // C layout: lane (q, m) holds rows 4q..4q+3 of sub-tile s, column m. The stores go out
  // back to back (the row ids come from LDS, so no load waits between them).
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rid_s[s * 16 + 4 * q + i];
      if (r >= 0 && n_ok)
        store_act<ACT>(h, (int64_t)r * inter + n, silu_mul<ACT>(acc[0][s][i], acc[1][s][i]));
      if (i == 3) __builtin_amdgcn_sched_barrier(0);    // one sub-tile's ids live at a time
    }
}

template <int F, int ACT, int SW, int S>
__device__ __forceinline__ void down_run(const Item& it, const void* h, const int64_t* rows,
                                         const int64_t* tbl, const void* rw, int rw_dt, float* y,
                                         int hidden, int inter, int gshift, int rshift, int sc_dt,
                                         int64_t down_w, int64_t down_s, int w_round,
                                         char* lds0, char* lds1, int* rid_s, float* w_s) {
  constexpr int BITS = CodeBits<F>::value;
  constexpr int KS = 512 / BITS;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int q = lane >> 4, m = lane & 15;
  const int n = it.tile * kTileN + wv * 16 + m;
  const bool n_ok = n < hidden;
  const int nn = n_ok ? n : 0;
  const char* pk = (const char*)tbl[2 * it.b];
  const char* sc = (const char*)tbl[2 * it.b + 1];
  const Role role[1] = {
      make_role<SW>(pk, down_w, sc, down_s, hidden, inter, BITS, gshift, rshift, sc_dt, nn)};
  const int64_t* rrow = rows + (int64_t)it.b * 16;
  AStage<KS, S> a;
  a_plan<KS, S>(a, [&](int r) -> uint32_t {
    const int64_t rid = rrow[r];
    return rid >= 0 ? (uint32_t)rid * (uint32_t)inter * 2u : kNoRow;
  });
  // The run's row ids go to LDS now (the K loop's first barrier publishes them); the
  // thread of each row also requests that row's routing weight now (two 16-bit loads, no
  // branch on the dtype: the low half, and the high half of an fp32 weight) and puts it in
  // LDS after the K loop. The epilogue then reads both from LDS: no load waits between its
  // stores.
  float w_mine = 0.f;
  if (threadIdx.x < S * 16) {
    const int rid = (int)rrow[threadIdx.x];
    rid_s[threadIdx.x] = rid;
    const int esz = rw_dt == DT_FP32 ? 4 : 2;
    const uint16_t* wp = (const uint16_t*)((const char*)rw + (int64_t)max(rid, 0) * esz);
    const uint16_t w_lo = wp[0];
    const uint16_t w_hi = wp[esz == 4 ? 1 : 0];
    w_mine = rw_dt == DT_FP32 ? __builtin_bit_cast(float, (uint32_t)w_hi << 16 | w_lo)
           : rw_dt == DT_BF16 ? __builtin_bit_cast(float, (uint32_t)w_lo << 16)
                              : (float)__builtin_bit_cast(_Float16, w_lo);
  }
  f32x4 acc[1][S];
  run_k<F, ACT, SW, 1, S>(role, rsrc(h, kNoRow), a, lds0, lds1, inter, q, m, acc);
  if (threadIdx.x < S * 16) w_s[threadIdx.x] = w_mine;
  __syncthreads();
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = s * 16 + 4 * q + i;
      const int r = rid_s[t];
      if (r >= 0 && n_ok) {
        float c = round_act<ACT>(acc[0][s][i]) * w_s[t];
        if (w_round) c = round_act<ACT>(c);
        y[(int64_t)r * hidden + n] = c;
      }
    }
}

#define VAAYU_BY_S4(CALL)                                                          \
  switch (it.S) {                                                                   \
    case 1: CALL(1); break; case 2: CALL(2); break; case 3: CALL(3); break;          \
    case 4: CALL(4); break; default: break;                                         \
  }
#define VAAYU_BY_S8(CALL)                                                          \
  switch (it.S) {                                                                   \
    case 1: CALL(1); break; case 2: CALL(2); break; case 3: CALL(3); break;          \
    case 4: CALL(4); break; case 5: CALL(5); break; case 6: CALL(6); break;          \
    case 7: CALL(7); break; case 8: CALL(8); break; default: break;                 \
  }
#define VAAYU_BY_S16(CALL)                                                         \
  switch (it.S) {                                                                   \
    case 1: CALL(1); break; case 2: CALL(2); break; case 3: CALL(3); break;          \
    case 4: CALL(4); break; case 5: CALL(5); break; case 6: CALL(6); break;          \
    case 7: CALL(7); break; case 8: CALL(8); break; case 9: CALL(9); break;          \
    case 10: CALL(10); break; case 11: CALL(11); break; case 12: CALL(12); break;    \
    case 13: CALL(13); break; case 14: CALL(14); break; case 15: CALL(15); break;    \
    case 16: CALL(16); break; default: break;                                       \
  }

template <int F, int ACT, int SW, int R>
__global__ void __launch_bounds__(64 * kWaves)
prefill_gate_up_kernel(const void* __restrict__ x, const int64_t* __restrict__ rows,
                       const int64_t* __restrict__ tbl, const int64_t* __restrict__ work,
                       void* __restrict__ h, int n_blocks,
                       int n_tiles, int top_k, int hidden, int inter, int gshift, int rshift,
                       int sc_dt, int64_t gate_w, int64_t gate_s, int64_t up_w, int64_t up_s) {
  constexpr int BITS = CodeBits<F>::value;
  __shared__ __align__(1024) char lds0[tile_blocks(R) * 16 * (2 * 512 / BITS)];
  __shared__ __align__(1024) char lds1[tile_blocks(R) * 16 * (2 * 512 / BITS)];
  const Item it = item_here<R>(work, n_blocks, n_tiles);
  __shared__ int rid_s[R * 16];
#define GU_CALL(S_) gate_up_run<F, ACT, SW, S_>(it, x, rows, tbl, h, top_k, hidden, inter, gshift, \
                                            rshift, sc_dt, gate_w, gate_s, up_w, up_s, lds0, lds1, \
                                            rid_s)
  if constexpr (R > kRunGateUpShort) {
    VAAYU_BY_S16(GU_CALL)
  } else {
    VAAYU_BY_S4(GU_CALL)
  }
#undef GU_CALL
}

template <int F, int ACT, int SW, int R>
__global__ void __launch_bounds__(64 * kWaves)
prefill_down_kernel(const void* __restrict__ h, const int64_t* __restrict__ rows,
                    const int64_t* __restrict__ tbl, const int64_t* __restrict__ work,
                    const void* __restrict__ rw, int rw_dt,
                    float* __restrict__ y, int n_blocks, int n_tiles, int hidden, int inter,
                    int gshift, int rshift, int sc_dt, int64_t down_w, int64_t down_s,
                    int w_round) {
  constexpr int BITS = CodeBits<F>::value;
  __shared__ __align__(1024) char lds0[tile_blocks(R) * 16 * (2 * 512 / BITS)];
  __shared__ __align__(1024) char lds1[tile_blocks(R) * 16 * (2 * 512 / BITS)];
  const Item it = item_here<R>(work, n_blocks, n_tiles);
  __shared__ int rid_s[R * 16];
  __shared__ float w_s[R * 16];
#define DN_CALL(S_) down_run<F, ACT, SW, S_>(it, h, rows, tbl, rw, rw_dt, y, hidden, inter, gshift, \
                                         rshift, sc_dt, down_w, down_s, w_round, lds0, lds1, \
                                         rid_s, w_s)
  if constexpr (R > kRunDownShort) {
    VAAYU_BY_S16(DN_CALL)
  } else {
    VAAYU_BY_S8(DN_CALL)
  }
#undef DN_CALL
}

#undef VAAYU_BY_S4
#undef VAAYU_BY_S8
#undef VAAYU_BY_S16

// ── launches (one compile unit per code family instantiates them) ───────────────────

// log2 of a power of two.
inline int log2_of(int v) {
  int r = 0;
  while ((1 << r) < v) ++r;
  return r;
}

struct PrefillArgs {
  int n_blocks, n_tiles, top_k, hidden, inter, gshift, rshift, sc_dt;
  const int64_t* work;    // the work list (see item_here), its slots per XCD and its
  int n_slots;            // longest run (blocks)
  int run;
};

// Workgroups of a launch over n_slots slots of n_tiles N tiles each.
inline dim3 work_grid(int n_slots, int n_tiles) {
  return dim3((unsigned)((int64_t)n_slots * kXcds * n_tiles));
}

template <int F, int ACT, int SW>
void launch_prefill_gate_up(const void* x, const int64_t* rows, const int64_t* tbl, void* h,
                            const PrefillArgs& p, const vaayu_geom* g, hipStream_t st) {
  const dim3 grid = work_grid(p.n_slots, p.n_tiles), block(64 * kWaves);
  if (p.n_slots == 0) return;
  if (p.run <= kRunGateUpShort)
    hipLaunchKernelGGL((prefill_gate_up_kernel<F, ACT, SW, kRunGateUpShort>), grid, block, 0, st,
                       x, rows, tbl, p.work, h, p.n_blocks, p.n_tiles, p.top_k, p.hidden, p.inter,
                       p.gshift, p.rshift, p.sc_dt, g->gate_w, g->gate_s, g->up_w, g->up_s);
  else
    hipLaunchKernelGGL((prefill_gate_up_kernel<F, ACT, SW, kRunGateUp>), grid, block, 0, st, x,
                       rows, tbl, p.work, h, p.n_blocks, p.n_tiles, p.top_k, p.hidden, p.inter,
                       p.gshift, p.rshift, p.sc_dt, g->gate_w, g->gate_s, g->up_w, g->up_s);
}

template <int F, int ACT, int SW>
void launch_prefill_down(const void* h, const int64_t* rows, const int64_t* tbl, const void* rw,
                         int rw_dt, float* y, const PrefillArgs& p, const vaayu_geom* g,
                         int w_round, hipStream_t st) {
  const dim3 grid = work_grid(p.n_slots, p.n_tiles), block(64 * kWaves);
  if (p.n_slots == 0) return;
  if (p.run <= kRunDownShort)
    hipLaunchKernelGGL((prefill_down_kernel<F, ACT, SW, kRunDownShort>), grid, block, 0, st, h,
                       rows, tbl, p.work, rw, rw_dt, y, p.n_blocks, p.n_tiles, p.hidden, p.inter,
                       p.gshift, p.rshift, p.sc_dt, g->down_w, g->down_s, w_round);
  else
    hipLaunchKernelGGL((prefill_down_kernel<F, ACT, SW, kRunDown>), grid, block, 0, st, h, rows,
                       tbl, p.work, rw, rw_dt, y, p.n_blocks, p.n_tiles, p.hidden, p.inter,
                       p.gshift, p.rshift, p.sc_dt, g->down_w, g->down_s, w_round);
}

// e4m3 / e2m1 launches (prefill_formats.hip): 0, or a negative code with the error set.
int prefill_gate_up_formats(const void* x, const int64_t* rows, const int64_t* tbl, void* h,
                            const PrefillArgs& p, const vaayu_geom* g, int act, hipStream_t st);
int prefill_down_formats(const void* h, const int64_t* rows, const int64_t* tbl, const void* rw,
                         int rw_dt, float* y, const PrefillArgs& p, const vaayu_geom* g,
                         int act, int w_round, hipStream_t st);

}  // namespace vaayu
