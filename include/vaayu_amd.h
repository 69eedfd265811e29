/* vaayu_amd: packed-expert routed-MoE kernels for MI355X (gfx950), C ABI.
 *
 * Every entry point takes raw device pointers (the caller owns all memory, e.g. torch
 * tensors' data_ptr()), plain sizes, dtype codes and a hipStream_t passed as void*. No
 * entry point allocates device memory, synchronises, or calls back into the host: each
 * enqueues kernels on `stream` and returns, so a caller may record them into a HIP graph.
 *
 * Return value: 0 on success; a negative value for a rejected call (bad argument, or a
 * geometry the kernels do not take), with the reason in vaayu_last_error(); a positive
 * value is the hipError_t of a failed launch.
 *
 * dtype codes are the reference's `_DTYPE_CODE` (vaayu/packed_expert_kernels.py:70):
 * 0 = bfloat16, 1 = float16, 2 = float32.
 */
#ifndef VAAYU_AMD_H
#define VAAYU_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VAAYU_ABI_VERSION 12

enum { VAAYU_BF16 = 0, VAAYU_FP16 = 1, VAAYU_FP32 = 2 };

/* Scale dtype code for E8M0 exponent bytes (MXFP4 scales). */
enum { VAAYU_E8M0 = 3 };

/* Code formats of an expert blob. VAAYU_FMT_INT: the reference's packed unsigned integer
 * codes (`bits` wide, offset 2^(bits-1)), `group` codes per scale along a row. VAAYU_FMT_E4M3:
 * float8 e4m3fn codes (bits = 8), one fp32 scale per block_rows x group tile, the weight
 * fp32(code) * scale rounded to the activation dtype, as `dequantize_block_scaled`
 * (vaayu/model_code/deepseek_v4/modeling_deepseek_v4.py:228-240). VAAYU_FMT_MXFP4: e2m1
 * codes (bits = 4, even element in the low nibble), one E8M0 scale per 32 codes along a
 * row, as `upcast_from_mxfp_torch` (vendor gpt_oss_triton_kernels
 * numerics_details/mxfp.py:256-299). Codes are packed along the last dim in 32-bit words,
 * roles gate, down, up in that order, like the reference's int blobs. */
enum { VAAYU_FMT_INT = 0, VAAYU_FMT_E4M3 = 1, VAAYU_FMT_MXFP4 = 2 };

/* One packed expert blob's geometry: `geom = (bits, group, roles)` and the per-role
 * (word offset, scale offset) that `_layout` derives from it
 * (vaayu/packed_expert_kernels.py:301-309). gate/up are [inter, hidden], down is
 * [hidden, inter], codes packed along the last dim. */
typedef struct vaayu_geom {
    int32_t bits;      /* code width: 1, 2, 4 or 8 */
    int32_t group;     /* codes per scale along a row */
    int32_t hidden;    /* H */
    int32_t inter;     /* I */
    int64_t gate_w, gate_s;
    int64_t up_w, up_s;
    int64_t down_w, down_s;
    int32_t format;      /* VAAYU_FMT_* */
    int32_t block_rows;  /* rows per scale (VAAYU_FMT_E4M3), else 1 */
} vaayu_geom;

int vaayu_abi_version(void);
const char *vaayu_last_error(void);

/* The decode and prefill entries take every code format above (prefill: 4- and 8-bit
 * codes, bf16 / fp16 activations), scale_dtype 0 bf16, 1 fp16, 2 fp32 or 3 E8M0 (E8M0 with
 * VAAYU_FMT_MXFP4 only). */

/* Decode, gate/up stage. Replaces `_gate_up` / `_gate_up_kernel`
 * (vaayu/packed_expert_kernels.py:355-371, 131-150).
 * x      [hidden] activations (dtype `act`)
 * table  int64 [n_pairs * 3]: (packed address, scale address, slot) per pair -- the
 *        reference's `_table_values` (:349-352), on the device
 * h      [n_pairs, inter] (dtype `act`) <- round(SiLU(round(x.Wg))) * round(x.Wu), rounded */
int vaayu_decode_gate_up(const void *x, const int64_t *table, void *h, int32_t n_pairs,
                         const vaayu_geom *geom, int32_t act, int32_t scale_dtype, void *stream);

/* Decode, down stage and the fixed-order sum. Replaces `_down` / `_down_kernel`
 * (vaayu/packed_expert_kernels.py:374-387, 153-176).
 * out [hidden] fp32, OVERWRITTEN with the sum over pairs in table order of
 * fl32(round(h[p].Wd) * routing_weights[slot_p]), rounded again when w_round != 0
 * (routing weights already in the activation dtype). */
int vaayu_decode_down(const void *h, const int64_t *table, const void *routing_weights,
                      int32_t rw_dtype, float *out, int32_t n_pairs, const vaayu_geom *geom,
                      int32_t act, int32_t scale_dtype, int32_t w_round, void *stream);

/* Prefill, gate/up stage over 16-row blocks of one expert each. Replaces `_gate_up_g` /
 * `_gate_up_grouped` (vaayu/packed_expert_kernels.py:720-732, 179-215).
 * x     [tokens, hidden] contiguous (dtype `act`: bf16 or fp16)
 * rows  int64 [n_blocks * 16]: row ids token*top_k + slot, -1 pads a block
 * table int64 [n_blocks * 2]: (packed address, scale address) of each block's expert
 * work  int64 [n_slots * 8]: the launch's work items (no counterpart in the reference,
 *       whose launch covers every block): work[k * 8 + x] = b * 32 + S for a run of S
 *       blocks of one expert starting at table block b (1 <= S <= the run length
 *       vaayu_prefill_run_blocks(0) gives), or -1; each run is computed for every N tile on
 *       XCD x. Every block of the table must lie in exactly one run; an entry that does
 *       not fit the table computes nothing. n_slots in [0, n_blocks].
 * run_blocks  the longest run in `work` (calls whose runs are at most 4 blocks long take a
 *       kernel that fits two workgroups per CU); an entry longer than run_blocks computes
 *       nothing.
 * h     [tokens * top_k, inter] (dtype `act`); padding rows are never written
 * x and h rows are addressed with 32-bit byte offsets: a launch whose tables could hold
 * rows past 0xF0000000 bytes (n_blocks * 16 / top_k tokens of x) is refused with -2; split
 * such a call into token chunks (every row's arithmetic is independent of its launch-mates). */
int vaayu_prefill_gate_up(const void *x, const int64_t *rows, const int64_t *table,
                          const int64_t *work, int32_t n_slots, int32_t run_blocks, void *h,
                          int32_t n_blocks,
                          int32_t top_k, const vaayu_geom *geom, int32_t act,
                          int32_t scale_dtype, void *stream);

/* Prefill, down stage. Replaces `_down_g` / `_down_grouped`
 * (vaayu/packed_expert_kernels.py:735-749, 218-247).
 * y [tokens * top_k, hidden] fp32 <- fl32(round(h[row].Wd) * routing_weights[row]),
 * rounded again when w_round != 0; routing_weights contiguous [tokens * top_k].
 * work / n_slots as for vaayu_prefill_gate_up, with runs of at most
 * vaayu_prefill_run_blocks(1) blocks; run_blocks: the longest run in `work` (calls whose
 * runs are at most 8 blocks long take a kernel that fits two workgroups per CU). An entry
 * longer than run_blocks computes nothing.
 * Refused with -2 when n_blocks * 16 rows of h would reach past 0xF0000000 bytes. */
int vaayu_prefill_down(const void *h, const int64_t *rows, const int64_t *table,
                       const int64_t *work, int32_t n_slots, int32_t run_blocks,
                       const void *routing_weights,
                       int32_t rw_dtype, float *y, int32_t n_blocks, const vaayu_geom *geom,
                       int32_t act, int32_t scale_dtype, int32_t w_round, void *stream);

/* The longest run (16-row blocks) a work item of the grouped kernels takes: which = 0
 * gate/up (vaayu_prefill_gate_up, vaayu_fused3d_gate_up), 1 down (vaayu_prefill_down,
 * vaayu_fused3d_down); -1 otherwise. No counterpart in the reference (its BLOCK_M plan
 * has no runs). */
int32_t vaayu_prefill_run_blocks(int32_t which);

/* Prefill reduce. Replaces `_reduce` / `_reduce_kernel` (vaayu/packed_expert_kernels.py:752-757,
 * 250-260): out[t] = sum over k, in `order`'s order, of y[order[t*top_k + k]], fp32 from 0.
 * out [tokens, hidden] contiguous fp32, overwritten. */
int vaayu_prefill_reduce(const float *y, const int64_t *order, float *out, int32_t tokens,
                         int32_t top_k, int32_t hidden, void *stream);

/* Whole-blob dequant. Replaces `_fused_dequant_kernel` (vaayu/moe_patch.py:750-769), the
 * function `dequantize_expert_blob` (:849-868) runs: out[i] = round_out((code_i -
 * 2^(bits-1)) * round_out(scale[i / group])) over n_words * 32/bits codes, bit-exact.
 * packed and out must start on 16 bytes (-2 otherwise). */
int vaayu_dequant_blob(const int32_t *packed, const void *scale, int32_t scale_dtype, void *out,
                       int32_t out_dtype, int64_t n_words, int32_t bits, int32_t group,
                       void *stream);

/* FP8 e4m3 block-scaled dequant. Replaces `dequantize_block_scaled`
 * (vaayu/model_code/deepseek_v4/modeling_deepseek_v4.py:228-240):
 * out[i, j] = round_out(fp32(weight[i, j]) * fp32(scale[i / bo, j / bi])), the fp32 product
 * rounded once, with bo = rows / scale_rows and bi = cols / scale_cols derived from the shapes.
 * weight uint8 [rows, cols] (float8_e4m3fn bits), row-major; scale [scale_rows, scale_cols] of
 * scale_dtype 0 bf16, 1 fp16, 2 fp32, 3 e8m0 (uint8 exponent, 0xFF = NaN); out [rows, cols]
 * of out_dtype 0 bf16, 1 fp16, 2 fp32. cols and bi multiples of 16. Bit-exact. */
int vaayu_dequant_fp8_block(const uint8_t *weight, const void *scale, int32_t scale_dtype,
                            void *out, int32_t out_dtype, int64_t rows, int64_t cols,
                            int64_t scale_rows, int64_t scale_cols, void *stream);

/* Microscaled upcast along the last axis. Replaces `upcast_from_mxfp_torch` and its Triton
 * twin `_upcast_from_mxfp` (vendor gpt_oss_triton_kernels numerics_details/mxfp.py:256-299,
 * mxfp_details/_upcast_from_mxfp.py:8-122): out[r, e] = round_out(fp32(q[r, e]) * 2^(s - 127))
 * with s = scale[r, e / 32] taken as the fp32 of exponent bits s (s = 0 gives 0) and
 * s = 0xFF giving NaN. fmt 0: e2m1, two per byte, even element in the low nibble
 * (q [rows, k / 2]); fmt 1: e4m3 (q [rows, k]). scale uint8 [rows, ceil(k / 32)]; out
 * [rows, k] of out_dtype 0 bf16, 1 fp16, 2 fp32. Bit-exact. */
int vaayu_upcast_mx(const uint8_t *q, int32_t fmt, const uint8_t *scale, void *out,
                    int32_t out_dtype, int64_t rows, int64_t k, void *stream);

/* Router top-k on the GPU, the decode-time expert budget, and the one-token decode table
 * built from them. Replaces the reference's default routing,
 * `torch.topk(logits.float().softmax(-1), k)` then `w / w.sum(-1)` (the `_route` branch for a
 * router returning bare logits, vaayu/moe_patch.py:2329-2334, and `route_experts`' fallback,
 * :159-161), `truncate_top_k(w, idx, keep_k, top_p)` on it (vaayu/moe_patch.py:170-215),
 * and the host round trip that sorts the slots by expert id and builds `_table_values`
 * (vaayu/moe_patch.py:2386-2389, vaayu/packed_expert_kernels.py:349-352) -- for experts
 * that are all resident.
 * logits       [tokens, experts] of logits_dtype (0 bf16, 1 fp16, 2 fp32), contiguous
 * top_k        the router's k; keep_k: the slots kept (n_out = min(keep_k, top_k), the k
 *              largest, rescaled to the row's original sum); top_p: 0 = off, else keep the
 *              fewest slots whose normalised weight reaches top_p and re-point each dropped
 *              slot at the top-1 expert with weight 0
 * weights      fp32 [tokens, n_out] <- the softmax probabilities of the picks in descending
 *              order (ties to the lower expert id), divided by their sum when renorm != 0,
 *              then the budget above
 * ids          int64 [tokens, n_out] <- their expert ids
 * expert_table int64 [experts, 2]: (packed address, scale address) of each expert's blob
 * pair_table   int64 [n_out * 3] or NULL; with tokens == 1 <- (packed address, scale
 *              address, slot) per slot in the stable (expert id, slot) order: the decode
 *              entries' table
 * experts 1..1024, top_k 1..min(16, experts), keep_k >= 1, top_p >= 0. NaN logits give NaN
 * weights. */
int vaayu_route_topk(const void *logits, int32_t logits_dtype, int32_t tokens, int32_t experts,
                     int32_t top_k, int32_t keep_k, float top_p, int32_t renorm, float *weights,
                     int64_t *ids, const int64_t *expert_table, int64_t *pair_table,
                     void *stream);

/* The router's product for decode-sized calls (ABI 6): logits [tokens, experts] <-
 * round_out(x [tokens, hidden] . w [experts, hidden]^T), the fp32 sum rounded once, as the
 * model's gate `F.linear(x, w)` stores it (the `router(flat_hidden)` call of `_route`,
 * vaayu/moe_patch.py:2327). x and w bf16 (0) or fp16 (1), contiguous, 16-byte aligned,
 * hidden a multiple of 8; out_dtype x's dtype or fp32 (2). */
int vaayu_router_logits(const void *x, const void *w, int32_t x_dtype, void *logits,
                        int32_t out_dtype, int32_t tokens, int32_t hidden, int32_t experts,
                        void *stream);

/* Gated-delta-net decode kernels (ABI 4). dtype codes 0 bf16, 1 fp16, 2 fp32. */

/* The recurrent gated delta rule over T steps: replaces the reference's `_rule_kernel` /
 * `fused_recurrent_rule` (vaayu/gated_delta_kernels.py:66-133), the drop-in for
 * transformers' `torch_recurrent_gated_delta_rule`. Per (batch, value head):
 *   h *= exp(g); delta = (v - h^T k) * beta; h += k delta^T; o = h^T q
 * with q, k l2-normalised in fp32 (eps 1e-6) when l2norm != 0 and q scaled by `scale`.
 * q, k [B, T, HV, K] and v [B, T, HV, V] of act_dtype, last dim contiguous; g, beta
 * [B, T, HV] (g_dtype, beta_dtype); h0 [B, HV, K, V] of h0_dtype or NULL (zeros);
 * o [B, T, HV, V] act_dtype, contiguous; ht fp32 [B, HV, K, V] contiguous or NULL.
 * strides: 19 element strides -- q (b, t, h), k (b, t, h), v (b, t, h), g (b, t, h),
 * beta (b, t, h), h0 (b, h, k, v). K <= 256, B * HV <= 65535. */
int vaayu_gdn_rule(const void *q, const void *k, const void *v, const void *g,
                   const void *beta, const void *h0, void *o, float *ht,
                   const int64_t *strides, int32_t B, int32_t T, int32_t HV, int32_t K,
                   int32_t V, float scale, int32_t act_dtype, int32_t g_dtype,
                   int32_t beta_dtype, int32_t h0_dtype, int32_t l2norm, void *stream);

/* The one-token causal depthwise conv update: replaces `_conv_kernel` /
 * `fused_conv_update` (vaayu/gated_delta_kernels.py:136-190), the drop-in for transformers'
 * `causal_conv1d_update` at one token. Shifts `state` [B, D, W] left one slot in place and
 * appends x, every value passing through the weight dtype; o [B, D] (x_dtype, contiguous)
 * <- silu(round_w(sum_j state_j w_j + bias)), rounded to the weight dtype.
 * x [B, D, 1]; w [D, W]; bias [D] or NULL. strides: x (b, d), state (b, d, w), w (d, w).
 * B <= 65535. */
int vaayu_gdn_conv_update(const void *x, void *state, const void *w, const void *bias, void *o,
                          const int64_t *strides, int32_t B, int32_t D, int32_t W,
                          int32_t x_dtype, int32_t state_dtype, int32_t w_dtype,
                          int32_t bias_dtype, void *stream);

/* The gated RMSNorm of a gated-delta mixer: replaces `_norm_kernel` / `fused_gated_norm`
 * (vaayu/gated_delta_kernels.py:197-235), the drop-in for `*RMSNormGated.forward(x, gate)`.
 * Per row of N: y = round_x(x * rsqrt(mean(x^2) + eps)); y = w * y (rounded to x's dtype
 * when round_mid != 0); o = round_x(y * silu(z)). x, z [rows, N] with strides (row, n); w [N]
 * with stride; o [rows, N] x_dtype, contiguous. strides: x (r, n), z (r, n), w. */
int vaayu_gdn_gated_norm(const void *x, const void *z, const void *w, void *o,
                         const int64_t *strides, int64_t rows, int32_t N, float eps,
                         int32_t x_dtype, int32_t z_dtype, int32_t w_dtype, int32_t round_mid,
                         void *stream);

/* Routed fused-3D MXFP4 experts (gpt-oss layout), ABI 5. Replaces the vendored `matmul_ogs`
 * calls with the fused `swiglu` that the experts module runs on the routed rows (caller:
 * vaayu/routed_fused3d.py:131-238; vendor gpt_oss_triton_kernels matmul_ogs.py,
 * matmul_ogs_details/_matmul_ogs.py:310-349, swiglu_details/_swiglu.py compute_swiglu).
 * Weights are read in place from the layer's whole tensors: gate_up blocks
 * [E, 2I, H/32, 16] (row 2j gate column j, row 2j+1 up column j) + E8M0 scales [E, 2I, H/32];
 * down blocks [E, H, I/32, 16] + scales [E, H, I/32]. rows / n_blocks: the prefill block plan
 * (16 row ids per block, row id = token * top_k + slot, -1 padding); tbl [n_blocks, 2]: the
 * block's expert (codes address, scales address); btbl [n_blocks]: its fp32 bias address;
 * work / n_slots (/ run_blocks): the launch's work list, as for vaayu_prefill_gate_up /
 * vaayu_prefill_down.
 * codes_end / scales_end: the tensors' ends (reads past them return zeros). H, I multiples
 * of 32; hidden_pad / inter_pad: multiples of 128 at least H / I, the row pitches of x and
 * h, whose padding columns must hold zeros. */

/* h [tokens * top_k, inter_pad] bf16 <- bf16(swiglu(x_row . W_gu^T + b)) per live row:
 * gate clipped above at `limit`, up to [-limit, limit], s = gate / (1 + exp(-alpha gate)),
 * h = fma(s, up, s). x [tokens, hidden_pad] bf16. */
int vaayu_fused3d_gate_up(const void *x, const int64_t *rows, const int64_t *tbl,
                          const int64_t *btbl, const int64_t *work, int32_t n_slots,
                          int32_t run_blocks, void *h, int32_t n_blocks, int32_t top_k,
                          int32_t hidden, int32_t hidden_pad, int32_t inter, int32_t inter_pad,
                          const void *codes_end, const void *scales_end, float alpha,
                          float limit, void *stream);

/* y [tokens * top_k, hidden] fp32 <- bf16((h_row . W_down^T + b) * gammas[row]) per live row;
 * `vaayu_prefill_reduce` then sums each token's slots in ascending expert id. */
int vaayu_fused3d_down(const void *h, const int64_t *rows, const int64_t *tbl,
                       const int64_t *btbl, const int64_t *work, int32_t n_slots,
                       int32_t run_blocks, const float *gammas, float *y, int32_t n_blocks,
                       int32_t top_k, int32_t hidden, int32_t inter, int32_t inter_pad,
                       const void *codes_end, const void *scales_end, void *stream);

/* One-token decode that allocates nothing. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments and result as
 * vaayu_decode_gate_up followed by vaayu_decode_down, without `h`: the intermediate
 * [n_pairs, inter] lives in a file-scope device array of
 * vaayu_decode_noalloc_scratch_bytes() bytes (4 MiB) held by each GPU until the process
 * ends. Returns -3 when n_pairs * inter * sizeof(act) exceeds it. Calls that overlap on
 * one GPU (other streams or threads) share the array and race. The first call on a device
 * looks the array's address up (hipGetSymbolAddress); make it outside a graph capture. */
int vaayu_decode_noalloc(const void *x, const int64_t *table, const void *routing_weights,
                         int32_t rw_dtype, float *out, int32_t n_pairs, const vaayu_geom *geom,
                         int32_t act, int32_t scale_dtype, int32_t w_round, void *stream);
int64_t vaayu_decode_noalloc_scratch_bytes(void);

/* Decode, both stages in ONE launch. Replaces the `_gate_up` + `_down` pair
 * (vaayu/packed_expert_kernels.py:355-387) that `_launch` / the per-layer graph run
 * (:390-396, 578-654): same arguments and result as vaayu_decode_gate_up followed by
 * vaayu_decode_down (h [n_pairs, inter] is the caller's buffer), bf16 / fp16 activations and
 * 4- / 8-bit codes only. The down workgroups request their codes while the gate/up
 * workgroups run and wait on per-workgroup counters in `sync` (int32
 * [vaayu_decode_fused_sync_words(...)], zeroed before its first call): one sync buffer
 * per launch configuration (geometry, n_pairs, dtypes), used by one stream at a time.
 * max_polls bounds a down workgroup's wait (0: about a second); past it the last word of
 * sync is set nonzero and the output is undefined. */
int vaayu_decode_fused(const void *x, const int64_t *table, const void *routing_weights,
                       int32_t rw_dtype, float *out, void *h, int32_t *sync, int32_t n_pairs,
                       const vaayu_geom *geom, int32_t act, int32_t scale_dtype,
                       int32_t w_round, int32_t max_polls, void *stream);
/* Words of vaayu_decode_fused's sync buffer for this configuration, or a negative code. */
int32_t vaayu_decode_fused_sync_words(int32_t n_pairs, const vaayu_geom *geom, int32_t act,
                                      int32_t scale_dtype);

/* Measurement only (no counterpart in the reference): `blocks` workgroups of 4 waves each
 * issue `iters` rounds of 16 independent v_mfma_f32_16x16x32_bf16 from registers; out
 * [blocks * 256] fp32 receives one sum per lane. 2 * 16 * 16 * 32 * 16 * iters * 4 * blocks
 * FLOPs per launch: the benchmark's measured bf16 matrix-core peak. */
int vaayu_probe_mfma(float *out, int32_t blocks, int32_t iters, void *stream);

/* Measurement only (no counterpart in the reference): d [16 row_tiles, 16 col_tiles] fp32
 * = a [16 row_tiles, k] times b [16 col_tiles, k]^T (both bf16, row-major), accumulated in
 * fp32 by v_mfma_f32_16x16x32_bf16 in the prefill kernels' K order (per 128-element step,
 * quarter q of MFMA i takes elements 32q + 8i .. +8). For measuring their accumulation error
 * against exact sums; k a positive multiple of 128. */
int vaayu_probe_mfma_sum(const void *a, const void *b, float *d, int32_t k, int32_t row_tiles,
                         int32_t col_tiles, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* VAAYU_AMD_H */
