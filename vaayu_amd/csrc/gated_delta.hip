// Decode kernels for gated-delta-net mixers: the recurrent gated delta rule, the
// one-token causal depthwise conv update, and the gated RMSNorm.
//
// Restates the reference's fused seams (vaayu/gated_delta_kernels.py:66-230): `_rule_kernel`
// (:66-110), `_conv_kernel` (:148-175) and `_norm_kernel` (:205-222), which replace
// transformers' torch fallbacks `torch_recurrent_gated_delta_rule`, `causal_conv1d_update`
// and `*RMSNormGated.forward`. Arithmetic in fp32 at the reference kernels' rounding points.
#include "abi_internal.hpp"
#include "common.hpp"

namespace vaayu {

// ── dtype-generic scalar access (the small operands: per-step scalars, conv taps) ──────

__device__ __forceinline__ float ld_any(const void* p, int64_t i, int dt) {
  if (dt == DT_BF16) return load_as_float<DT_BF16>(p, i);
  if (dt == DT_FP16) return load_as_float<DT_FP16>(p, i);
  return load_as_float<DT_FP32>(p, i);
}

__device__ __forceinline__ float round_any(float v, int dt) {
  if (dt == DT_BF16) return round_act<DT_BF16>(v);
  if (dt == DT_FP16) return round_act<DT_FP16>(v);
  return v;
}

__device__ __forceinline__ void st_any(void* p, int64_t i, float v, int dt) {
  if (dt == DT_BF16) store_act<DT_BF16>(p, i, v);
  else if (dt == DT_FP16) store_act<DT_FP16>(p, i, v);
  else store_act<DT_FP32>(p, i, v);
}

__device__ __forceinline__ float sigmoidf(float x) { return 1.f / (1.f + expf(-x)); }

template <int CTRL>
__device__ __forceinline__ float gdn_dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the wave: DPP inside rows of 16 lanes, then the four rows' results.
__device__ __forceinline__ float wave_sum(float v) {
  v += gdn_dpp<0xB1>(v);      // quad_perm [1,0,3,2]
  v += gdn_dpp<0x4E>(v);      // quad_perm [2,3,0,1]
  v += gdn_dpp<0x124>(v);     // row_ror:4
  v += gdn_dpp<0x128>(v);     // row_ror:8
  const auto lane = [&](int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
  };
  return (lane(0) + lane(16)) + (lane(32) + lane(48));
}

// ── the recurrent gated delta rule ─────────────────────────────────────────────────────
//
// Per step of one (batch, value head):
//   h *= exp(g);  delta = (v - sum_k h[k] * k[k]) * beta;  h += k[k] * delta;
//   o = sum_k h[k] * q[k]
// with q, k l2-normalised in fp32 (eps 1e-6) when asked and q scaled by `scale`.

constexpr int kGdnWaves = 4;

struct GdnRuleArgs {
  const void *q, *k, *v, *g, *beta, *h0;
  void* o;
  float* ht;
  int64_t sq[3], sk[3], sv[3], sg[3], sb[3], sh[4];
  int B, T, HV, K, V;
  float scale;
  int g_dt, beta_dt, l2, store_ht, has_h0;
};

// One workgroup per (batch, value head, 16 value columns): a (batch, head) spreads over
// V/16 workgroups, since the kernel's time is load and store latency, not arithmetic (a
// 64-column tile took 9.3 us against 6.7 for Qwen3-Next's decode shape). The fp32 state
// slice stays in registers for every step: lane l of wave w holds column l & 15 and the
// KW2 rows of k-group (w << 2) | (l >> 4). The sums over K add the lane's rows, then the
// wave's four k-groups (lane ^ 16, lane ^ 32), then the four waves in wave order. GB: g
// and beta read as fp32 and the activation dtype (the mixers' own) with no dtype branch.
// Every load of a step is issued before its first wait, the first step's before the state.
constexpr int kGdnVT = 16;

template <int ACT, int HDT, int KW2, bool GB>
__global__ void __launch_bounds__(kGdnWaves * 64) gdn_rule_kernel(GdnRuleArgs a) {
  constexpr int KMAX = 16 * KW2;
  __shared__ float qs[KMAX], ks[KMAX];
  __shared__ float red[kGdnWaves][kGdnVT];
  __shared__ float nrm[2][kGdnWaves];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int col = lane & 15, kg = (w << 2) | (lane >> 4);
  const int vi = blockIdx.x * kGdnVT + col;
  const int bh = blockIdx.y, b = bh / a.HV, hh = bh - b * a.HV;
  const bool vok = vi < a.V;
  float qv = 0.f, kv = 0.f, vv = 0.f, graw = 0.f, beta = 0.f;
  auto load_step = [&](int t) {
    if (tid < a.K) {
      qv = load_as_float<ACT>(a.q, b * a.sq[0] + t * a.sq[1] + hh * a.sq[2] + tid);
      kv = load_as_float<ACT>(a.k, b * a.sk[0] + t * a.sk[1] + hh * a.sk[2] + tid);
    } else {
      qv = kv = 0.f;
    }
    vv = vok ? load_as_float<ACT>(a.v, b * a.sv[0] + t * a.sv[1] + hh * a.sv[2] + vi) : 0.f;
    const int64_t gi = b * a.sg[0] + t * a.sg[1] + hh * a.sg[2];
    const int64_t bi = b * a.sb[0] + t * a.sb[1] + hh * a.sb[2];
    if constexpr (GB) {
      graw = load_as_float<DT_FP32>(a.g, gi);
      beta = load_as_float<ACT>(a.beta, bi);
    } else {
      graw = ld_any(a.g, gi, a.g_dt);
      beta = ld_any(a.beta, bi, a.beta_dt);
    }
  };
  if (a.T > 0) load_step(0);
  float h[KW2];
#pragma unroll
  for (int i = 0; i < KW2; ++i) {
    const int kk = kg * KW2 + i;
    h[i] = (a.has_h0 && vok && kk < a.K)
               ? load_as_float<HDT>(a.h0, b * a.sh[0] + hh * a.sh[1] + kk * a.sh[2] + vi * a.sh[3])
               : 0.f;
  }
  auto sum_k = [&](float part) {                 // over the 16 k-groups, fixed order
    part += __shfl_xor(part, 16);
    part += __shfl_xor(part, 32);
    if (lane < 16) red[w][lane] = part;
    __syncthreads();
    const float r = (red[0][col] + red[1][col]) + (red[2][col] + red[3][col]);
    __syncthreads();
    return r;
  };
  for (int t = 0; t < a.T; ++t) {
    if (t > 0) load_step(t);
    if (a.l2) {
      const float sqq = wave_sum(qv * qv), skk = wave_sum(kv * kv);
      if (lane == 0) { nrm[0][w] = sqq; nrm[1][w] = skk; }
      __syncthreads();
      const float tq = (nrm[0][0] + nrm[0][1]) + (nrm[0][2] + nrm[0][3]);
      const float tk = (nrm[1][0] + nrm[1][1]) + (nrm[1][2] + nrm[1][3]);
      qv = qv * rsqrtf(tq + 1e-6f);
      kv = kv * rsqrtf(tk + 1e-6f);
    }
    qv = qv * a.scale;
    if (tid < KMAX) { qs[tid] = qv; ks[tid] = kv; }     // rows past K hold 0
    const float decay = expf(graw);
    __syncthreads();
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < KW2; ++i) {
      h[i] = h[i] * decay;
      part += h[i] * ks[kg * KW2 + i];
    }
    const float kvm = sum_k(part);
    const float delta = (vv - kvm) * beta;
    float po = 0.f;
#pragma unroll
    for (int i = 0; i < KW2; ++i) {
      h[i] = h[i] + ks[kg * KW2 + i] * delta;
      po += h[i] * qs[kg * KW2 + i];
    }
    const float ov = sum_k(po);
    if (tid < kGdnVT && vok)
      store_act<ACT>(a.o, (((int64_t)b * a.T + t) * a.HV + hh) * a.V + vi, ov);
  }
  if (a.store_ht && vok) {
#pragma unroll
    for (int i = 0; i < KW2; ++i) {
      const int kk = kg * KW2 + i;
      if (kk < a.K) a.ht[((int64_t)bh * a.K + kk) * a.V + vi] = h[i];
    }
  }
}

// ── the one-token causal conv update ───────────────────────────────────────────────────
//
// One thread per (batch, channel): shift the state left one slot, append x, the depthwise
// dot, + bias, silu -- every value passing through the weight dtype as the torch fallback's
// `cat([state, x]).to(weight.dtype)` makes it, the state written back in its own dtype.

struct GdnConvArgs {
  const void* x;
  void* state;
  const void* w;
  const void* bias;
  void* o;
  int64_t sx_b, sx_d, ss_b, ss_d, ss_w, sw_d, sw_w;
  int B, D, W;
  int x_dt, s_dt, w_dt, b_dt, has_bias;
};

// Every tap, weight and the bias are read before the first state write (the writes alias
// the reads), so they arrive together: up to kConvTaps taps in registers, wider kernels
// through the loop.
constexpr int kConvTaps = 8;

__global__ void __launch_bounds__(256) gdn_conv_kernel(GdnConvArgs a) {
  const int d = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (d >= a.D) return;
  const float bx = ld_any(a.x, b * a.sx_b + d * a.sx_d, a.x_dt);
  const int64_t sp = b * a.ss_b + d * a.ss_d;
  const int64_t wp = d * a.sw_d;
  const float bias = a.has_bias ? ld_any(a.bias, d, a.b_dt) : 0.f;
  float acc = 0.f;
  if (a.W <= kConvTaps) {
    float sv[kConvTaps], wv[kConvTaps];
#pragma unroll
    for (int j = 0; j < kConvTaps; ++j) {
      sv[j] = j + 1 < a.W ? ld_any(a.state, sp + (j + 1) * a.ss_w, a.s_dt) : 0.f;
      wv[j] = j < a.W ? ld_any(a.w, wp + j * a.sw_w, a.w_dt) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < kConvTaps; ++j) {
      if (j + 1 < a.W) {
        const float sj = round_any(sv[j], a.w_dt);
        st_any(a.state, sp + j * a.ss_w, sj, a.s_dt);
        acc += sj * wv[j];
      } else if (j + 1 == a.W) {
        const float xw = round_any(bx, a.w_dt);
        st_any(a.state, sp + j * a.ss_w, xw, a.s_dt);
        acc += xw * wv[j];
      }
    }
  } else {
    for (int j = 0; j < a.W - 1; ++j) {
      const float sj = round_any(ld_any(a.state, sp + (j + 1) * a.ss_w, a.s_dt), a.w_dt);
      st_any(a.state, sp + j * a.ss_w, sj, a.s_dt);
      acc += sj * ld_any(a.w, wp + j * a.sw_w, a.w_dt);
    }
    const float xw = round_any(bx, a.w_dt);
    st_any(a.state, sp + (a.W - 1) * a.ss_w, xw, a.s_dt);
    acc += xw * ld_any(a.w, wp + (a.W - 1) * a.sw_w, a.w_dt);
  }
  acc += bias;
  acc = round_any(acc, a.w_dt);
  const float y = round_any(acc * sigmoidf(acc), a.w_dt);
  st_any(a.o, (int64_t)b * a.D + d, y, a.x_dt);
}

// ── the gated RMSNorm ──────────────────────────────────────────────────────────────────
//
// One wave per row: rmsnorm in fp32 -> round to the input dtype -> x weight -> (round,
// when the product stays in the input dtype) -> x silu(gate) in fp32 -> round.

struct GdnNormArgs {
  const void *x, *z, *w;
  void* o;
  int64_t sx_r, sx_n, sz_r, sz_n, sw;
  int64_t rows;
  int N;
  float eps;
  int x_dt, z_dt, w_dt, round_mid;
};

// Rows of up to 64 * kNormPer elements are read once, x, z and w together, before the
// reduction; longer rows take a second pass.
constexpr int kNormPer = 4;

__global__ void __launch_bounds__(256) gdn_norm_kernel(GdnNormArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= a.rows) return;                             // wave-uniform
  float xs[kNormPer], zs[kNormPer], ws[kNormPer];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kNormPer; ++i) {
    const int n = lane + 64 * i;
    const bool ok = n < a.N;
    xs[i] = ok ? ld_any(a.x, r * a.sx_r + n * a.sx_n, a.x_dt) : 0.f;
    zs[i] = ok ? ld_any(a.z, r * a.sz_r + n * a.sz_n, a.z_dt) : 0.f;
    ws[i] = ok ? ld_any(a.w, n * a.sw, a.w_dt) : 0.f;
  }
#pragma unroll
  for (int i = 0; i < kNormPer; ++i) ss += xs[i] * xs[i];
  for (int n = lane + 64 * kNormPer; n < a.N; n += 64) {
    const float xv = ld_any(a.x, r * a.sx_r + n * a.sx_n, a.x_dt);
    ss += xv * xv;
  }
  const float inv = rsqrtf(wave_sum(ss) / (float)a.N + a.eps);
  auto out = [&](int n, float xv, float zv, float wv) {
    float y = round_any(xv * inv, a.x_dt);
    y = wv * y;
    if (a.round_mid) y = round_any(y, a.x_dt);
    st_any(a.o, r * a.N + n, y * (zv * sigmoidf(zv)), a.x_dt);
  };
#pragma unroll
  for (int i = 0; i < kNormPer; ++i)
    if (lane + 64 * i < a.N) out(lane + 64 * i, xs[i], zs[i], ws[i]);
  for (int n = lane + 64 * kNormPer; n < a.N; n += 64)
    out(n, ld_any(a.x, r * a.sx_r + n * a.sx_n, a.x_dt), ld_any(a.z, r * a.sz_r + n * a.sz_n, a.z_dt),
        ld_any(a.w, n * a.sw, a.w_dt));
}

}  // namespace vaayu

using namespace vaayu;

static bool gdn_dt_ok(int dt) { return dt == DT_BF16 || dt == DT_FP16 || dt == DT_FP32; }

extern "C" int vaayu_gdn_rule(const void* q, const void* k, const void* v, const void* g,
                              const void* beta, const void* h0, void* o, float* ht,
                              const int64_t* strides, int32_t B, int32_t T, int32_t HV,
                              int32_t K, int32_t V, float scale, int32_t act_dtype,
                              int32_t g_dtype, int32_t beta_dtype, int32_t h0_dtype,
                              int32_t l2norm, void* stream) {
  clear_error();
  if (!q || !k || !v || !g || !beta || !o || !strides) return set_error(-1, "null pointer argument");
  if (B <= 0 || T < 0 || HV <= 0 || K <= 0 || V <= 0) return set_error(-2, "empty or negative shape");
  if (K > kGdnWaves * 64) return set_error(-2, "K must be at most 256");
  if (B * HV > 65535) return set_error(-2, "batch x heads must be at most 65535");
  if (!gdn_dt_ok(act_dtype) || !gdn_dt_ok(g_dtype) || !gdn_dt_ok(beta_dtype) ||
      (h0 && !gdn_dt_ok(h0_dtype)))
    return set_error(-2, "dtype codes must be 0 bf16, 1 fp16 or 2 fp32");
  GdnRuleArgs a;
  a.q = q; a.k = k; a.v = v; a.g = g; a.beta = beta; a.h0 = h0; a.o = o; a.ht = ht;
  for (int i = 0; i < 3; ++i) {
    a.sq[i] = strides[i]; a.sk[i] = strides[3 + i]; a.sv[i] = strides[6 + i];
    a.sg[i] = strides[9 + i]; a.sb[i] = strides[12 + i];
  }
  for (int i = 0; i < 4; ++i) a.sh[i] = strides[15 + i];
  a.B = B; a.T = T; a.HV = HV; a.K = K; a.V = V; a.scale = scale;
  a.g_dt = g_dtype; a.beta_dt = beta_dtype; a.l2 = l2norm != 0;
  a.store_ht = ht != nullptr; a.has_h0 = h0 != nullptr;
  const int hdt = h0 ? h0_dtype : DT_FP32;
  hipStream_t st = (hipStream_t)stream;
  const bool gb = g_dtype == DT_FP32 && beta_dtype == act_dtype;
  const dim3 grid((unsigned)((V + kGdnVT - 1) / kGdnVT), (unsigned)(B * HV)),
      block(kGdnWaves * 64);
#define GR(A_, H_, KW_)                                                                    \
  if (gb) hipLaunchKernelGGL((gdn_rule_kernel<A_, H_, KW_, true>), grid, block, 0, st, a); \
  else hipLaunchKernelGGL((gdn_rule_kernel<A_, H_, KW_, false>), grid, block, 0, st, a)
#define GR_KW(A_, H_) \
  if (K <= 16 * 4) GR(A_, H_, 4); else if (K <= 16 * 8) GR(A_, H_, 8); else GR(A_, H_, 16)
#define GR_H(A_) \
  if (hdt == DT_BF16) { GR_KW(A_, DT_BF16); } else if (hdt == DT_FP16) { GR_KW(A_, DT_FP16); } \
  else { GR_KW(A_, DT_FP32); }
  if (act_dtype == DT_BF16) { GR_H(DT_BF16); }
  else if (act_dtype == DT_FP16) { GR_H(DT_FP16); }
  else { GR_H(DT_FP32); }
#undef GR_H
#undef GR_KW
#undef GR
  return check_launch("gated delta rule");
}

extern "C" int vaayu_gdn_conv_update(const void* x, void* state, const void* w, const void* bias,
                                     void* o, const int64_t* strides, int32_t B, int32_t D,
                                     int32_t W, int32_t x_dtype, int32_t state_dtype,
                                     int32_t w_dtype, int32_t bias_dtype, void* stream) {
  clear_error();
  if (!x || !state || !w || !o || !strides) return set_error(-1, "null pointer argument");
  if (B <= 0 || D <= 0 || W <= 0) return set_error(-2, "empty or negative shape");
  if (B > 65535) return set_error(-2, "batch must be at most 65535");
  if (!gdn_dt_ok(x_dtype) || !gdn_dt_ok(state_dtype) || !gdn_dt_ok(w_dtype) ||
      (bias && !gdn_dt_ok(bias_dtype)))
    return set_error(-2, "dtype codes must be 0 bf16, 1 fp16 or 2 fp32");
  GdnConvArgs a;
  a.x = x; a.state = state; a.w = w; a.bias = bias; a.o = o;
  a.sx_b = strides[0]; a.sx_d = strides[1]; a.ss_b = strides[2]; a.ss_d = strides[3];
  a.ss_w = strides[4]; a.sw_d = strides[5]; a.sw_w = strides[6];
  a.B = B; a.D = D; a.W = W;
  a.x_dt = x_dtype; a.s_dt = state_dtype; a.w_dt = w_dtype; a.b_dt = bias_dtype;
  a.has_bias = bias != nullptr;
  const dim3 grid((unsigned)((D + 255) / 256), (unsigned)B), block(256);
  hipLaunchKernelGGL(gdn_conv_kernel, grid, block, 0, (hipStream_t)stream, a);
  return check_launch("gated delta conv update");
}

extern "C" int vaayu_gdn_gated_norm(const void* x, const void* z, const void* w, void* o,
                                    const int64_t* strides, int64_t rows, int32_t N, float eps,
                                    int32_t x_dtype, int32_t z_dtype, int32_t w_dtype,
                                    int32_t round_mid, void* stream) {
  clear_error();
  if (!x || !z || !w || !o || !strides) return set_error(-1, "null pointer argument");
  if (rows < 0 || N <= 0) return set_error(-2, "empty or negative shape");
  if (rows == 0) return 0;
  if ((rows + 3) / 4 > 0x7FFFFFFF) return set_error(-2, "too many rows");
  if (!gdn_dt_ok(x_dtype) || !gdn_dt_ok(z_dtype) || !gdn_dt_ok(w_dtype))
    return set_error(-2, "dtype codes must be 0 bf16, 1 fp16 or 2 fp32");
  GdnNormArgs a;
  a.x = x; a.z = z; a.w = w; a.o = o;
  a.sx_r = strides[0]; a.sx_n = strides[1]; a.sz_r = strides[2]; a.sz_n = strides[3];
  a.sw = strides[4];
  a.rows = rows; a.N = N; a.eps = eps;
  a.x_dt = x_dtype; a.z_dt = z_dtype; a.w_dt = w_dtype; a.round_mid = round_mid != 0;
  const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  hipLaunchKernelGGL(gdn_norm_kernel, grid, block, 0, (hipStream_t)stream, a);
  return check_launch("gated rmsnorm");
}
