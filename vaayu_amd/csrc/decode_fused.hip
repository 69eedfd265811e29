// One-launch decode layer: the gate/up and down stages of vaayu_decode_gate_up /
// vaayu_decode_down in ONE kernel, so the down stage's code loads stream while gate/up runs
// and the layer pays one launch instead of two.
//
// Workgroups [0, G) are gate/up producers: block b takes 16 rows (2 per wave, 8 waves) of
// pair b / row_blocks, exactly the arithmetic of mfma_gate_up_kernel. Workgroups [G, G + D)
// are the down blocks of mfma_down_kernel: each requests its codes first, then waits until
// every producer of this call has published, then stages h and finishes as before.
//
// Publication without atomics or cache flushes. h is written with device-coherent stores
// (cache policy sc1: written through to the point all XCDs see) and read back with
// device-coherent loads, so no L2 write-back or invalidate is needed. Each producer b, once
// its stores have completed (s_waitcnt plus the block barrier), stores its counter
// flag[b] + 1; each down block d keeps its own count seen[d] of calls it has finished, and
// waits until every flag[b] >= seen[d] + 1. Only block b writes flag[b] and only block d
// writes seen[d], so both are plain coherent stores. After the n-th call on a sync buffer,
// every counter holds n: a sync buffer belongs to ONE launch configuration (geometry,
// n_pairs, dtypes) and starts zeroed.
//
// The wait is bounded: after kMaxPolls polls a block stores a nonzero word at sync[G + D]
// and goes on (its output is then undefined, but the kernel ends). Producers are the lowest
// workgroup ids and never wait, so they are all dispatched before any down block.
#include "decode_mfma.hpp"

namespace vaayu {

constexpr int kMaxPolls = 1 << 22;

__device__ __forceinline__ uint4 buf_load16_coherent(rsrc_t r, uint32_t byte_off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 16);   // sc1
  return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ int load_coherent(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void store_coherent(int32_t* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int ACT>
__device__ __forceinline__ uint32_t act_bits(float v) {
  if constexpr (ACT == DT_BF16) return __builtin_bit_cast(uint16_t, (__bf16)v);
  else return __builtin_bit_cast(uint16_t, (_Float16)v);
}

struct FusedShape {
  MShape gu, dn;
  int row_blocks;        // producer blocks per pair: ceil(inter / 16)
  int producers;         // G
  int consumers;         // D
  int rw_dt, kps, ps, nrg, w_round;
  int max_polls;         // bound of a down block's wait (then the error word is set)
};

// ── producer: 16 rows of one pair, both roles ────────────────────────────────────────────
template <int F, int ACT, int SW, int NS>
__device__ __forceinline__ void produce(const FusedShape& f, const int64_t* __restrict__ tbl,
                                        const uint32_t* __restrict__ x, uint16_t* __restrict__ h,
                                        int32_t* __restrict__ sync, int b, uint4* xl) {
  constexpr int CPU = MUnit<F>::CPU;
  const MShape& s = f.gu;
  int my_flag = 0;
  if (threadIdx.x == 0) my_flag = load_coherent(sync + b);          // in flight meanwhile
  const rsrc_t X = make_rsrc(x, (uint32_t)s.vec16 * 16u);
  const int xn = (s.vec16 + 511) >> 9;                                // uint4 per thread, <= 2
  uint4 xs[2];
#pragma unroll
  for (int k = 0; k < 2; ++k)
    if (k < xn) xs[k] = buf_load16(X, (threadIdx.x + k * 512u) * 16u);
  const int p = b / f.row_blocks, bx = b - p * f.row_blocks;
  const char* pk = (const char*)tbl[3 * p];
  const char* sc = (const char*)tbl[3 * p + 1];
  const int lane = threadIdx.x & 63;
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, c = lane & 15;
  const int kp = c >> 2, role = (c >> 1) & 1;
  const int row0 = bx * 16 + wib * 2;
  const int row = min(row0 + (c & 1), s.rows - 1);
  const uint32_t u0 = (uint32_t)(kp * s.part_units + q);
  ColumnDot<F, ACT, SW, NS, true> cd;
  cd.begin(make_rsrc(pk, s.code_bytes), make_rsrc(sc, s.scale_bytes),
           (role ? s.wb1 : s.wb0) + ((uint32_t)row * s.units_row + u0) * 16u,
           (role ? s.sc1 : s.sc0) + (uint32_t)(row >> s.rshift) * s.groups_row, u0, s);
#pragma unroll
  for (int k = 0; k < 2; ++k)
    if (k < xn && threadIdx.x + k * 512 < s.vec16) xl[threadIdx.x + k * 512] = xs[k];
  lds_barrier();
  const Masks M = make_masks();
  const uint4* xa = xl + (c * s.part_units + q) * (CPU / 8);
  const f32x4 acc = cd.finish(s, xa, c < 4, M);
  float v = kp == 0 ? acc[0] : kp == 1 ? acc[1] : kp == 2 ? acc[2] : acc[3];
  v += dpp_move<kRowRor4>(v);
  v += dpp_move<kRowRor8>(v);
  const float up = dpp_move<kQuadXor2>(v);
  const float hv = silu_mul<ACT>(v, up);
  // lanes 0 and 1 hold rows row0, row0 + 1: lane 0 writes both as one coherent word
  const float hv1 = __shfl_down(hv, 1, 64);
  if (lane == 0 && row0 < s.rows) {          // rows is even (the host checks), so is row0
    const uint32_t lo = act_bits<ACT>(hv), hi = act_bits<ACT>(hv1);
    store_coherent((int32_t*)(h + (int64_t)p * s.rows + row0), (int)(lo | hi << 16));
  }
  __builtin_amdgcn_s_waitcnt(0);          // this wave's stores have completed
  __syncthreads();
  if (threadIdx.x == 0) store_coherent(sync + b, my_flag + 1);
}

// ── down block: codes first, then wait for every producer, then the stage as before ──────
template <int F, int ACT, int SW, int NS, bool ONE>
__device__ __forceinline__ void consume(const FusedShape& f, const int64_t* __restrict__ tbl,
                                        const uint16_t* __restrict__ h,
                                        const void* __restrict__ rw, float* __restrict__ out,
                                        int32_t* __restrict__ sync, int d, uint4* lds) {
  constexpr int CPU = MUnit<F>::CPU;
  const MShape& s = f.dn;
  __shared__ int target_s;
  int32_t* seen = sync + f.producers;
  if (threadIdx.x == 0) target_s = load_coherent(seen + d) + 1;
  const int kps = f.kps, ps = f.ps, nrg = f.nrg;
  const int KP = 1 << kps;
  const int RW = 16 >> kps;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, c = lane & 15;
  const int kp = c >> (4 - kps);
  const int rg = 8 / ps;
  const int pl = wv % ps, g = wv / ps;
  const int br = nrg * rg * RW;
  const int p16 = s.units_row * CPU / 8;
  float* cbuf = (float*)(lds + s.vec16);
  const uint32_t u0 = (uint32_t)(kp * s.part_units + q);
  ColumnDot<F, ACT, SW, NS> cd;
  auto begin = [&](int gi, int p) {
    const char* pk = (const char*)tbl[3 * p];
    const char* sc = (const char*)tbl[3 * p + 1];
    const int row = min(d * br + (gi * rg + g) * RW + (c & (RW - 1)), s.rows - 1);
    cd.begin(make_rsrc(pk + s.wb0, s.code_bytes),
             make_rsrc(sc + (size_t)s.sc0 * (SW / 8), s.scale_bytes),
             ((uint32_t)row * s.units_row + u0) * 16u, (uint32_t)(row >> s.rshift) * s.groups_row,
             u0, s);
  };
  begin(0, pl < s.n_pairs ? pl : 0);
  __syncthreads();                                   // target_s
  const int target = target_s;
  // every producer of this call has published: wave 0 polls, the others wait at the barrier
  if (wv == 0) {
    for (int polls = 0;; ++polls) {
      bool ok = true;
      for (int j = lane; j < f.producers; j += 64) ok &= load_coherent(sync + j) >= target;
      if (__all(ok)) break;
      if (polls >= f.max_polls) {
        if (lane == 0) store_coherent(sync + f.producers + f.consumers, 1);
        break;
      }
    }
  }
  __syncthreads();
  const rsrc_t HV = make_rsrc(h, (uint32_t)s.vec16 * 16u);
  const int hn = (s.vec16 + 511) >> 9;                       // uint4 of h per thread, <= 8
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int i = threadIdx.x + k * 512;
    if (k < hn && i < s.vec16) lds[i] = buf_load16_coherent(HV, (uint32_t)i * 16u);
  }
  __syncthreads();
  const Masks M = make_masks();
  auto one = [&](int gi, int p, bool live) {
    const int brow = (gi * rg + g) * RW;
    const int64_t slot = tbl[3 * p + 2];
    const int esz = f.rw_dt == DT_FP32 ? 4 : 2;
    const uint16_t* wp = (const uint16_t*)((const char*)rw + slot * esz);
    const uint16_t w_lo = wp[0];
    const uint16_t w_hi = wp[esz == 4 ? 1 : 0];
    __builtin_amdgcn_sched_barrier(0);
    const uint4* xa = lds + p * p16 + (c * s.part_units + q) * (CPU / 8);
    const f32x4 acc = cd.finish(s, xa, c < KP, M);
    float v = kp == 0 ? acc[0] : kp == 1 ? acc[1] : kp == 2 ? acc[2] : acc[3];
    if (KP == 4) v += dpp_move<kRowRor4>(v);
    if (KP >= 2) v += dpp_move<kRowRor8>(v);
    const float wgt = f.rw_dt == DT_FP32 ? __builtin_bit_cast(float, (uint32_t)w_hi << 16 | w_lo)
                    : f.rw_dt == DT_BF16 ? __builtin_bit_cast(float, (uint32_t)w_lo << 16)
                                         : (float)__builtin_bit_cast(_Float16, w_lo);
    if (live && lane < RW) {
      float cv = round_act<ACT>(v) * wgt;
      if (f.w_round) cv = round_act<ACT>(cv);
      cbuf[p * br + brow + lane] = cv;
    }
  };
  if constexpr (ONE) {
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
    const int row = d * br + t;
    if (row >= s.rows) continue;
    float o = 0.f;
    for (int pp = 0; pp < s.n_pairs; ++pp) o += cbuf[pp * br + t];
    out[row] = o;
  }
  if (threadIdx.x == 0) store_coherent(seen + d, target);
}

template <int F, int ACT, int SW, int NSG, int NSD, bool ONE>
__global__ void __launch_bounds__(512)
fused_decode_kernel(const int64_t* __restrict__ tbl, const uint32_t* __restrict__ x,
                    uint16_t* __restrict__ h, const void* __restrict__ rw,
                    float* __restrict__ out, int32_t* __restrict__ sync, FusedShape f) {
  extern __shared__ uint4 lds[];
  const int b = blockIdx.x;
  if (b < f.producers)
    produce<F, ACT, SW, NSG>(f, tbl, x, h, sync, b, lds);
  else
    consume<F, ACT, SW, NSD, ONE>(f, tbl, h, rw, out, sync, b - f.producers, lds);
}

}  // namespace vaayu

using namespace vaayu;

namespace {

struct FusedPlan {
  FusedShape f;
  size_t lds;
  bool one;
};

// The fused launch's plan, or a reason it cannot run (nullptr when it can).
const char* fused_plan(const vaayu_geom* g, int act, int n, int sc, int rw_dt, int w_round,
                       int max_polls, FusedPlan& fp) {
  if (const char* why = decode_unsupported(g, act)) return why;
  const int fmt = code_format(g);
  if (!mfma_format(fmt, act)) return "the one-launch layer takes bf16 / fp16 activations and "
                                    "4- or 8-bit codes";
  MShape gu;
  int xs;
  DownPlan dn;
  if (!mfma_gate_up_plan(g, fmt, act, n, sc, gu, xs) || !mfma_down_plan(g, fmt, act, n, sc, dn))
    return "no MFMA plan for this geometry";
  if (gu.vec16 > 2 * 512) return "hidden too large to stage in one 512-thread block";
  if (g->inter % 2) return "odd intermediate size";
  FusedShape& f = fp.f;
  f.gu = gu;
  f.dn = dn.s;
  f.row_blocks = (g->inter + 15) / 16;
  f.producers = f.row_blocks * n;
  f.consumers = (int)dn.blocks;
  f.rw_dt = rw_dt;
  f.kps = dn.kp == 4 ? 2 : dn.kp == 2 ? 1 : 0;
  f.ps = dn.ps;
  f.nrg = dn.nrg;
  f.w_round = w_round;
  f.max_polls = max_polls > 0 ? max_polls : kMaxPolls;
  fp.lds = std::max<size_t>((size_t)gu.vec16 * 16, dn.lds);
  fp.one = dn.nrg == 1 && dn.ps >= n;
  return nullptr;
}

template <int F, int ACT, int SW>
int launch_fused(const FusedPlan& fp, const int64_t* tbl, const void* x, void* h, const void* rw,
                 float* out, int32_t* sync, hipStream_t st) {
  const dim3 grid((unsigned)(fp.f.producers + fp.f.consumers)), block(512);
  const int nsg = fp.f.gu.steps, nsd = fp.f.dn.steps;
#define FD(NSG_, NSD_, ONE_)                                                                  \
  hipLaunchKernelGGL((fused_decode_kernel<F, ACT, SW, NSG_, NSD_, ONE_>), grid, block, fp.lds, st, \
                     tbl, (const uint32_t*)x, (uint16_t*)h, rw, out, sync, fp.f)
  // straight-line step counts of the measured shapes; others run the chunked loops
  if (nsg == 4 && nsd == 3 && fp.one) FD(4, 3, true);
  else if (nsg == 4 && nsd == 3) FD(4, 3, false);
  else if (fp.one) FD(0, 0, true);
  else FD(0, 0, false);
#undef FD
  return 0;
}

template <int F, int ACT>
int fused_sw(const FusedPlan& fp, int sc, const int64_t* tbl, const void* x, void* h,
             const void* rw, float* out, int32_t* sync, hipStream_t st) {
  if constexpr (F == F_MXFP4) {
    if (sc == VAAYU_E8M0) return launch_fused<F, ACT, 8>(fp, tbl, x, h, rw, out, sync, st);
    return set_error(-2, "mxfp4 scales are E8M0");
  } else {
    if (sc == VAAYU_E8M0) return set_error(-2, "E8M0 scales go with mxfp4 codes");
    if (sc == DT_FP32) return launch_fused<F, ACT, 32>(fp, tbl, x, h, rw, out, sync, st);
    return launch_fused<F, ACT, 16>(fp, tbl, x, h, rw, out, sync, st);
  }
}

}  // namespace

extern "C" int32_t vaayu_decode_fused_sync_words(int32_t n_pairs, const vaayu_geom* geom,
                                                 int32_t act, int32_t scale_dtype) {
  clear_error();
  if (!geom || n_pairs <= 0) return set_error(-1, "bad arguments");
  FusedPlan fp;
  if (const char* why = fused_plan(geom, act, n_pairs, scale_dtype, DT_FP32, 0, 0, fp))
    return set_error(-2, why);
  return fp.f.producers + fp.f.consumers + 1;
}

extern "C" int vaayu_decode_fused(const void* x, const int64_t* table, const void* routing_weights,
                                  int32_t rw_dtype, float* out, void* h, int32_t* sync,
                                  int32_t n_pairs, const vaayu_geom* geom, int32_t act,
                                  int32_t scale_dtype, int32_t w_round, int32_t max_polls,
                                  void* stream) {
  clear_error();
  if (!x || !table || !routing_weights || !out || !h || !sync || !geom)
    return set_error(-1, "null pointer argument");
  if (n_pairs <= 0) return set_error(-1, "n_pairs must be positive");
  if (scale_dtype < 0 || scale_dtype > 3 || rw_dtype < 0 || rw_dtype > 2)
    return set_error(-1, "scale / routing-weight dtype");
  if ((((uintptr_t)x) & 15) || (((uintptr_t)h) & 15) || (((uintptr_t)sync) & 3))
    return set_error(-1, "x and h must be 16-byte aligned, sync 4-byte aligned");
  FusedPlan fp;
  if (const char* why = fused_plan(geom, act, n_pairs, scale_dtype, rw_dtype, w_round, max_polls,
                                  fp))
    return set_error(-2, why);
  const int fmt = code_format(geom);
  hipStream_t st = (hipStream_t)stream;
  int rc;
#define BA(B_, A_) else if (fmt == B_ && act == A_) rc = fused_sw<B_, A_>(fp, scale_dtype, table, x, h, routing_weights, out, sync, st);
  if (false) rc = 0;
  BA(4, 0) BA(4, 1) BA(8, 0) BA(8, 1) BA(F_E4M3, 0) BA(F_E4M3, 1) BA(F_MXFP4, 0) BA(F_MXFP4, 1)
  else rc = set_error(-2, "unsupported code format / activation dtype");
#undef BA
  return rc ? rc : check_launch("fused decode");
}
