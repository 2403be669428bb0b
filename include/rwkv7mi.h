/*
 * rwkv7mi — C ABI of the MI355X (gfx950) RWKV-7 inference hot path.
 *
 * Every entry point takes raw device pointers, element counts and a
 * hipStream_t passed as `void*` (NULL = the legacy default stream), launches
 * asynchronously, and returns 0 on success or a negative RWKV7MI_E* code.
 * On failure `rwkv7mi_last_error()` returns a message for the calling thread.
 * No entry point allocates device memory unless its comment says so; callers
 * own every buffer.  Nothing here touches torch types.
 *
 * Layout conventions (match the reference adapter, rwkv-rs/hf-adapter 0.8.1):
 *   vectors  r,w,k,v,kk,a,g : [B, H, N] (decode) or [B, T, H, N] (sequence),
 *                             contiguous, N = 64 (head size).
 *   state                   : [B, H, N, N] fp32, row = value channel,
 *                             column = key channel ("native V x K").
 *   MM8 weight              : w_u8 [I, O] uint8, O contiguous (= Linear.weight.T),
 *                             mx, rx [O]; my, ry [I] (stored [I,1] by the reference).
 *   W4 group weight         : packed [O, I/2] uint8 (low nibble = even input),
 *                             scales [O, I/group] .
 *   MM4 affine weight       : packed [I, O_pad/2] uint8 (low nibble = even output),
 *                             mx, rx [O_pad]; my, ry [I].
 *
 * dtype codes: RWKV7MI_F32 = 0, RWKV7MI_F16 = 1, RWKV7MI_BF16 = 2.
 */
#ifndef RWKV7MI_H
#define RWKV7MI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  RWKV7MI_F32 = 0,
  RWKV7MI_F16 = 1,
  RWKV7MI_BF16 = 2
};

enum {
  RWKV7MI_OK = 0,
  RWKV7MI_EINVAL = -1,   /* bad shape / dtype / pointer argument          */
  RWKV7MI_ELAUNCH = -2,  /* the HIP runtime rejected a launch or call     */
  RWKV7MI_ESIZE = -3     /* workspace or scratch too small                */
};

/* GEMV/GEMM epilogues (MM8, W4 group, MM4). */
enum {
  RWKV7MI_EPI_NONE = 0,      /* y = x @ W (+ bias)                         */
  RWKV7MI_EPI_RELU2 = 1,     /* y = relu(x @ W (+ bias))^2                 */
  RWKV7MI_EPI_RESIDUAL = 2   /* y = residual + x @ W (+ bias)              */
};

/* ---------------------------------------------------------------- status */

/* Message of the last failed call on this thread ("" if none). */
const char* rwkv7mi_last_error(void);
/* Library ABI version (major * 100 + minor). */
int rwkv7mi_abi_version(void);

/* ------------------------------------------------ wkv7 single-token decode */

/* One-token DPLR update + readout.
 *   S' = S * w[None,:] - (S @ kk) (kk * a)^T + v k^T ;  y = S' r
 * Replaces fused_recurrent_update / torch_recurrent_update
 * (rwkv7_hf/fused_recurrent_update.py:1214, :757) and the torch graph-body
 * form _recurrent_update_batched (rwkv7_hf/native_jit_recurrent.py:60).
 * state_out may equal state_in (in-place update).  y has act_dtype. */
int rwkv7mi_wkv7_decode_update(const void* r, const void* w, const void* k,
                               const void* v, const void* kk, const void* a,
                               const float* state_in, float* state_out,
                               void* y, int64_t B, int64_t H, int64_t N,
                               int act_dtype, int w_dtype, void* stream);

/* Update + readout + per-head GroupNorm(eps) + bonus (sum r*k*r_k)*v + gate g.
 * Replaces fused_recurrent_output_prepare
 * (rwkv7_hf/fused_recurrent_update.py:967) / torch_recurrent_output_prepare
 * (:846).  r_k [H,N], gn_w/gn_b [H*N] have param_dtype. */
int rwkv7mi_wkv7_decode_output_prepare(
    const void* r, const void* w, const void* k, const void* v,
    const void* kk, const void* a, const float* state_in, float* state_out,
    const void* g, const void* r_k, const void* gn_w, const void* gn_b,
    void* out, int64_t B, int64_t H, int64_t N, float eps, int act_dtype,
    int w_dtype, int param_dtype, void* stream);

/* Raw-input decode fusion: kk = normalize(k_raw * k_k), k = k_raw*(1+(a-1)k_a),
 * w = exp(-0.606531*sigmoid(w_raw)), then as output_prepare.
 * Replaces fused_recurrent_output_prepare_raw
 * (rwkv7_hf/fused_recurrent_update.py:1089, kernel :155).
 * v_mode: 0 = use v as given; 1 = layer 0: copy v into v_first;
 *         2 = v = v + (v_first - v) * v_gate (v_gate already sigmoid'd),
 *             the V interpolation of rwkv7_hf/native.py:219-223.
 * v_first / v_gate may be NULL when v_mode == 0. */
int rwkv7mi_wkv7_decode_output_prepare_raw(
    const void* r, const void* w_raw, const void* k_raw, const void* v,
    const void* a, const float* state_in, float* state_out, const void* g,
    const void* k_k, const void* k_a, const void* r_k, const void* gn_w,
    const void* gn_b, void* out, void* v_first, const void* v_gate,
    int v_mode, int64_t B, int64_t H, int64_t N, float eps, int act_dtype,
    int param_dtype, void* stream);

/* rwkv7mi_wkv7_decode_output_prepare_raw with the W/A/G/V LoRA up projections
 * fused in: the second half of fused_wavg_lora (rwkv7_hf/fused_lora.py:706)
 * followed by fused_recurrent_output_prepare_raw (fused_recurrent_update.py
 * :1089).  lora_part holds the partials of rwkv7mi_lora_down_multi over the
 * same (nprob, ranks, rows = B, D); problems 0 w_raw, 1 a, 2 g, 3 v_gate with
 * w_up[p] [H*N, rank_p], b_up[p] [H*N] or NULL, activations 0 none, 1 tanh,
 * 2 sigmoid.  Each (batch, head) workgroup computes its own 64 channels of
 * every up projection, rounded to act_dtype as the reference's tensors are.
 * B <= 64; ranks multiples of 8, at most 128; nprob 3 or 4 (4 when
 * v_mode == 2).  lora_splits: the number of K ranges in lora_part (0: the
 * split rwkv7mi_lora_down_multi uses for these ranks and D; 1: the whole-K
 * sums of rwkv7mi_mm8t_lnmix_multi). */
int rwkv7mi_wkv7_decode_lora_output_prepare(
    const void* r, const void* k_raw, const void* v, const float* lora_part,
    int64_t nprob, const int64_t* ranks, const void* const* w_up,
    const void* const* b_up, const int* act_down, const int* act_up, int64_t D,
    int64_t lora_splits, const float* state_in, float* state_out, const void* k_k,
    const void* k_a,
    const void* r_k, const void* gn_w, const void* gn_b, void* out, void* v_first,
    int v_mode, int64_t B, int64_t H, int64_t N, float eps, int act_dtype,
    int param_dtype, void* stream);

/* ----------------------------------------------------- wkv7 sequence scans */

/* Sequential on-chip scan over T tokens (T x the decode update), y [B,T,H,N].
 * Replaces fused_recurrent_scan / torch_recurrent_scan
 * (rwkv7_hf/fused_recurrent_update.py:1299, :800). */
int rwkv7mi_wkv7_scan(const void* r, const void* w, const void* k,
                      const void* v, const void* kk, const void* a,
                      const float* state_in, float* state_out, void* y,
                      int64_t B, int64_t T, int64_t H, int64_t N,
                      int act_dtype, int w_dtype, void* stream);

/* Chunked DPLR prefill (chunk C = 16): same result as the sequential scan.
 * w is the per-step decay (w_is_log = 0), its natural log (w_is_log = 1) or
 * the raw pre-activation w_raw of the clamp-w scan (w_is_log = 2: decay
 * exp(-0.606531 sigmoid(w_raw)) formed in-kernel).  Any T >= 0 (a ragged tail
 * chunk is handled).  Replaces self_chunk_rwkv7 (rwkv7_hf/self_chunk_rwkv7.py:33),
 * dplr_chunk_scan (rwkv7_hf/dplr_prefill.py:505) and, with w_is_log = 2,
 * fused_recurrent_scan_clampw (rwkv7_hf/fused_recurrent_update.py:1420). */
int rwkv7mi_wkv7_chunk_prefill(const void* r, const void* w, const void* k,
                               const void* v, const void* kk, const void* a,
                               const float* state_in, float* state_out,
                               void* y, int64_t B, int64_t T, int64_t H,
                               int64_t N, int64_t chunk, int w_is_log,
                               int act_dtype, int w_dtype, void* stream);

/* Sticky status bits of the chunk kernel on the current device since the last
 * clear: 1 = a bounded wait between the kernel's waves gave up (that call's
 * output is void), 2 = a chunk's log2-decay span exceeded 252 and the gate
 * factors were clamped to 2^+-126.  Synchronises the device; clear != 0 resets
 * the word.  This build's own diagnostic (no reference counterpart: the
 * reference's Triton scans have no cross-wave waits). */
int rwkv7mi_wkv7_chunk_status(int clear, int* status);

/* ------------------------------------------- wkv7 with an fp16 state (opt-in) */

/* The optional fp16-state lane.  Every tensor is fp16 except elapsed (int32
 * [B]); state [B,H,64,64] fp16 is updated in place; N must be 64.  The state
 * math is packed fp16 FMAs in a fixed order (one rounding each) and the decay
 * enters as wd = exp(-e^-1/2 sigmoid(w)) - 1 + 2^-41 int32(0x9E3779B9 phase),
 * phase = elapsed[b] + 64 h + i (+ token index).
 *
 * Decode from raw projections [B,H,64] with GroupNorm, bonus and gate, out
 * [B,H,64]; k_k, k_a, r_k, gn_w, gn_b [H*64].  advance_elapsed != 0 adds 1 to
 * every elapsed[b] after all heads have read it (a second launch on the same
 * stream).  v_mode (this build's extension, as in
 * rwkv7mi_wkv7_decode_output_prepare_raw): 0 = v as given; 1 = copy v into
 * v_first; 2 = v + (v_first - v) * v_gate with fp16 rounding after each
 * operation (v_first / v_gate may be NULL when unused).
 * Replaces rwkv7_native_fp16_recurrent_output_raw_cuda
 * (rwkv7_hf/native_wkv_fp16.py:463-514, kernel :200-336) behind
 * native_fp16_recurrent_output_prepare_raw (:678). */
int rwkv7mi_wkv7_fp16_decode_output_prepare_raw(
    const void* r, const void* w_raw, const void* k_raw, const void* v,
    const void* a, void* state, const void* g, const void* k_k,
    const void* k_a, const void* r_k, const void* gn_w, const void* gn_b,
    int32_t* elapsed, int advance_elapsed, void* out, void* v_first,
    const void* v_gate, int v_mode, int64_t B, int64_t H, int64_t N, float eps,
    void* stream);

/* The same decode with the W/A/G[/V] LoRA up projections inside the kernel,
 * as rwkv7mi_wkv7_decode_lora_output_prepare does for an fp32 state: the
 * down projections' fp32 partials lora_part ([problem][split][B][rank], from
 * rwkv7mi_lora_down_multi with lora_splits = 0, or whole sums / K-chunk sums
 * with lora_splits >= 1) are summed and activated per problem, rounded to
 * fp16, and each (batch, head) workgroup computes its 64 channels of w_raw,
 * a, g and v_gate, each rounded to fp16, before the fp16-state update above.
 * B <= 64; ranks multiples of 8 up to 128; v_mode 2 needs nprob 4.
 * Replaces fused_wavg_lora's up half (rwkv7_hf/fused_lora.py:706) followed by
 * native_fp16_recurrent_output_prepare_raw (rwkv7_hf/native_wkv_fp16.py:678)
 * in the reference's fp16 decode (rwkv7_hf/native_jit_decode.py:762-784). */
int rwkv7mi_wkv7_fp16_decode_lora_output_prepare(
    const void* r, const void* k_raw, const void* v, const float* lora_part,
    int64_t nprob, const int64_t* ranks, const void* const* w_up,
    const void* const* b_up, const int* act_down, const int* act_up, int64_t D,
    int64_t lora_splits, void* state, const void* k_k, const void* k_a,
    const void* r_k, const void* gn_w, const void* gn_b, int32_t* elapsed,
    int advance_elapsed, void* out, void* v_first, int v_mode, int64_t B,
    int64_t H, int64_t N, float eps, void* stream);

/* T >= 1 tokens of prepared vectors [B,T,H,64]: w raw (plus w0 [H*64] in
 * fp32 when w0 != NULL), neg_kk = -kk, kka = kk*a; out [B,T,H,64] is the raw
 * readout y.  elapsed is read, not advanced.  Inputs and state 16-byte
 * aligned.  Replaces rwkv7_native_fp16_sequence_cuda
 * (rwkv7_hf/native_wkv_fp16.py:516-583, kernel :338-436) behind
 * native_fp16_sequence (:756). */
int rwkv7mi_wkv7_fp16_sequence(const void* r, const void* w, const void* w0,
                               const void* k, const void* v, const void* neg_kk,
                               const void* kka, void* state,
                               const int32_t* elapsed, void* out, int64_t B,
                               int64_t T, int64_t H, int64_t N, void* stream);

/* ------------------------------------------------------------------- MM8 */

/* Device packer of the uint8 affine format.  weight [I,O] (= Linear.weight.T)
 * in w_dtype; outputs w_u8 [I,O]; mx, rx [O]; my, ry [I] in w_dtype, with
 * rx/16 and ry/16 stored exactly as rwkv7_hf/native_quant_mm8.py:62-97.
 * Needs a float workspace of (2*I + 2*O) floats. */
int rwkv7mi_mm8_pack(const void* weight, int64_t I, int64_t O, int w_dtype,
                     uint8_t* w_u8, void* mx, void* rx, void* my, void* ry,
                     float* workspace, void* stream);

/* Bytes of workspace rwkv7mi_mm8_matmul needs for `rows` activation rows. */
size_t rwkv7mi_mm8_workspace_bytes(int64_t rows, int64_t I, int64_t O);

/* y[rows,O] = epilogue(x[rows,I] @ dequant(W)), dequant as
 * (w+0.5)*ry[i]*rx[o] + my[i] + mx[o] with fp32 accumulation.
 * Replaces mm8_matmul_triton / mm8_gemv_triton / MM8Linear.forward
 * (rwkv7_hf/native_quant_mm8.py:468, :383, :594).  `workspace` holds
 * split-K partials and per-tile counters; its counter region must be zero on
 * the first call and is left zero by every call (see rwkv7mi_mm8_workspace_bytes).
 * bias [O] / residual [rows,O] may be NULL. */
int rwkv7mi_mm8_matmul(const void* x, const uint8_t* w_u8, const void* mx,
                       const void* rx, const void* my, const void* ry,
                       const void* bias, const void* residual, void* y,
                       int64_t rows, int64_t I, int64_t O, int epilogue,
                       int act_dtype, int meta_dtype, void* workspace,
                       size_t workspace_bytes, void* stream);

/* Materialise the dequantized weight out [I,O] = (w+0.5)*ry*rx + my + mx
 * (fp32 math, one rounding to out_dtype), the reference's dequantize_mm8
 * (rwkv7_hf/native_quant_mm8.py:100-108); used before a library GEMM when a
 * prefill has many rows.  O % 4 == 0, I <= 65535. */
int rwkv7mi_mm8_dequant(const uint8_t* w_u8, const void* mx, const void* rx,
                        const void* my, const void* ry, void* out, int64_t I,
                        int64_t O, int meta_dtype, int out_dtype, void* stream);

/* Blocked MM8 (the decode path).  Same values as the [I,O] format; the bytes
 * are stored per output-column group g (16 outputs) and K block b (128
 * inputs) as one 2048-byte tile at byte (g*KB + b)*2048, KB = ceil(I/128),
 * holding at byte 1024*h + 16*(16*q + c) + e the weight of output 16*g + c
 * and input 128*b + 64*h + 16*q + e (h<2, q<4, c<16, e<16), zero padded:
 * rwkv7mi_mm8t_blocked_bytes(I, O) bytes.  A wave's 128-input step of 16
 * outputs is one contiguous 2 KB run.  The reference's w_u8 buffer
 * (rwkv7_hf/native_quant_mm8.py:583, uint8 [in, out]) converts with
 * rwkv7mi_mm8t_block / _unblock; the reference picks its own per-device
 * buffer layout the same way (q_row [out, in] at :578-580). */

size_t rwkv7mi_mm8t_blocked_bytes(int64_t I, int64_t O);

/* src element (output o, input i) at src[o*stride_o + i*stride_i] (e.g. the
 * reference w_u8 [I,O]: stride_o 1, stride_i O) -> w_blk; w_blk 16-byte
 * aligned. */
int rwkv7mi_mm8t_block(const uint8_t* src, int64_t stride_o, int64_t stride_i,
                       int64_t I, int64_t O, uint8_t* w_blk, void* stream);
/* w_blk -> dst[o*stride_o + i*stride_i]. */
int rwkv7mi_mm8t_unblock(const uint8_t* w_blk, int64_t I, int64_t O, uint8_t* dst,
                         int64_t stride_o, int64_t stride_i, void* stream);

/* Packer from Linear.weight [O,I] itself: same outputs as rwkv7mi_mm8_pack on
 * weight.T, with w_t [O,I].  Workspace as for rwkv7mi_mm8_pack. */
int rwkv7mi_mm8_pack_t(const void* weight, int64_t I, int64_t O, int w_dtype,
                       uint8_t* w_t, void* mx, void* rx, void* my, void* ry,
                       float* workspace, void* stream);

/* y[rows,O] = epilogue(x[rows,I] @ dequant(W)) over blocked w_blk; no
 * workspace, deterministic.  Replaces mm8_gemv_triton / mm8_matmul_triton /
 * MM8Linear.forward (rwkv7_hf/native_quant_mm8.py:383, :468, :594).
 * I % 16 == 0; x, w_blk, my, ry 16-byte aligned; y may alias residual. */
int rwkv7mi_mm8t_matmul(const void* x, const uint8_t* w_blk, const void* mx,
                        const void* rx, const void* my, const void* ry,
                        const void* bias, const void* residual, void* y,
                        int64_t rows, int64_t I, int64_t O, int epilogue,
                        int act_dtype, int meta_dtype, void* stream);

/* Up to 4 rwkv7mi_mm8t_matmul problems of one shape in one launch (the
 * r/k/v projections of rwkv7_hf/native.py:193-195).  Arrays have nprob
 * entries; bias and residual arrays may be NULL. */
int rwkv7mi_mm8t_matmul_multi(int nprob, const void* const* x,
                              const uint8_t* const* w_blk, const void* const* mx,
                              const void* const* rx, const void* const* my,
                              const void* const* ry, const void* const* bias,
                              const void* const* residual, void* const* y,
                              const int* epilogue, int64_t rows, int64_t I,
                              int64_t O, int act_dtype, int meta_dtype,
                              void* stream);

/* rwkv7mi_mm8t_matmul_multi with a workspace for split K: when the rows' x'
 * (rows x in_features x 4 bytes) exceeds one LDS chunk, the inputs split into
 * ranges of one chunk each, every workgroup stages its range once for all its
 * column groups, and a second launch adds the ranges' fp32 partials in order
 * (deterministic) and applies bias and epilogue.  `workspace` (16-byte
 * aligned) must hold rwkv7mi_mm8t_matmul_workspace_bytes (0 when the call
 * does not split; the workspace may then be NULL). */
size_t rwkv7mi_mm8t_matmul_workspace_bytes(int nprob, int64_t rows, int64_t I,
                                           int64_t O);
int rwkv7mi_mm8t_matmul_multi_ws(int nprob, const void* const* x,
                                 const uint8_t* const* w_blk,
                                 const void* const* mx, const void* const* rx,
                                 const void* const* my, const void* const* ry,
                                 const void* const* bias,
                                 const void* const* residual, void* const* y,
                                 const int* epilogue, int64_t rows, int64_t I,
                                 int64_t O, int act_dtype, int meta_dtype,
                                 void* workspace, size_t workspace_bytes,
                                 void* stream);

/* rwkv7mi_mm8t_matmul_multi (no split K, at most 16 rows) with the decode
 * LoRA down projections in the same launch: workgroups past the products
 * compute lora_part[p][z][row][n] = sum_{k in range z} lora_x[p][row,k]
 * lora_w_down[p][n,k] over lora_splits K ranges of I inputs (the layout
 * rwkv7mi_wkv7_decode_lora_output_prepare reads with lora_splits = that count),
 * for up to four problems of lora_ranks[p] (multiples of 8, at most 256),
 * lora_x in act_dtype [rows, I].  The products are those of the plain call.
 * Replaces the grouped R/K/V dispatch plus fused_wavg_lora's down launch of
 * the decode step (rwkv7_hf/native_jit_graph_dispatch.py:449-801,
 * rwkv7_hf/fused_lora.py:706). */
int rwkv7mi_mm8t_matmul_multi_lora(int nprob, const void* const* x,
                                   const uint8_t* const* w_blk,
                                   const void* const* mx, const void* const* rx,
                                   const void* const* my, const void* const* ry,
                                   const void* const* bias,
                                   const void* const* residual, void* const* y,
                                   const int* epilogue, int64_t rows, int64_t I,
                                   int64_t O, int act_dtype, int meta_dtype,
                                   int64_t lora_nprob, const void* const* lora_x,
                                   const void* const* lora_w_down,
                                   const int64_t* lora_ranks, int64_t lora_splits,
                                   float* lora_part, size_t lora_part_bytes,
                                   void* stream);

/* The split-K products of rwkv7mi_mm8t_matmul_multi_ws for one problem
 * without the second launch: the ranges' fp32 partials stay in `workspace`
 * as part[(s * rows + row) * O + o] (s < *splits), each already carrying its
 * range's share of the row-sum terms, so y = sum_s part[s] (+ bias) in range
 * order.  The consumer adds them, e.g. rwkv7mi_attn_norm_mix6_parts for the
 * FFN value's residual.  Refuses shapes that do not split.  Replaces the
 * value projection of the decode FFN (rwkv7_hf/native_jit_graph_dispatch.py:
 * 594-598) at 3..16 rows, where x' exceeds one LDS chunk. */
int rwkv7mi_mm8t_matmul_partials(const void* x, const uint8_t* w_blk,
                                 const void* mx, const void* rx, const void* my,
                                 const void* ry, int64_t rows, int64_t I,
                                 int64_t O, int act_dtype, int meta_dtype,
                                 void* workspace, size_t workspace_bytes,
                                 int* splits, void* stream);

/* Many-row form of rwkv7mi_mm8t_matmul_multi for 17..256 rows (bsz-64
 * decode, short prefills): 64-row x 128-column MFMA tiles over split K, with
 * x' = x * ry rounded once to fp16 and the weights centred (w - 128) so that
 * the rounding touches only the centred term (relative error ~1e-4 of the
 * result's scale).  With more than one split, fp32 partials go to
 * `workspace` (>= rwkv7mi_mm8t_gemm_workspace_bytes, 256-byte aligned) and a
 * second launch adds them in split order: deterministic, no atomics.
 * splits = 0 picks the count.  Replaces mm8_matmul_triton's materialising
 * route for rows > fused_max_rows (rwkv7_hf/native_quant_mm8.py:468-507,
 * :100-126) and MM8Linear.forward (:594) at those row counts. */
size_t rwkv7mi_mm8t_gemm_workspace_bytes(int nprob, int64_t rows, int64_t I,
                                         int64_t O, int splits);
int rwkv7mi_mm8t_gemm_multi(int nprob, const void* const* x,
                            const uint8_t* const* w_blk, const void* const* mx,
                            const void* const* rx, const void* const* my,
                            const void* const* ry, const void* const* bias,
                            const void* const* residual, void* const* y,
                            const int* epilogue, int64_t rows, int64_t I,
                            int64_t O, int act_dtype, int meta_dtype,
                            int splits, void* workspace,
                            size_t workspace_bytes, void* stream);

/* rwkv7mi_mm8t_gemm_multi (17..64 rows) with the decode LoRA down
 * projections as tail workgroups of the tile launch, the same partial layout
 * as rwkv7mi_mm8t_matmul_multi_lora.  The products are those of the plain
 * call.  Replaces the grouped R/K/V dispatch plus fused_wavg_lora's down
 * launch of the decode step (rwkv7_hf/native_jit_graph_dispatch.py:449-801,
 * rwkv7_hf/fused_lora.py:706). */
int rwkv7mi_mm8t_gemm_multi_lora(int nprob, const void* const* x,
                                 const uint8_t* const* w_blk,
                                 const void* const* mx, const void* const* rx,
                                 const void* const* my, const void* const* ry,
                                 const void* const* bias,
                                 const void* const* residual, void* const* y,
                                 const int* epilogue, int64_t rows, int64_t I,
                                 int64_t O, int act_dtype, int meta_dtype,
                                 int splits, void* workspace,
                                 size_t workspace_bytes, int64_t lora_nprob,
                                 const void* const* lora_x,
                                 const void* const* lora_w_down,
                                 const int64_t* lora_ranks, int64_t lora_splits,
                                 float* lora_part, size_t lora_part_bytes,
                                 void* stream);

/* Prefill GEMM over the blocked layout for many rows (long prompts): up to
 * four problems of one shape, y = epilogue(x @ W_hat (+ bias)), on 256 x 256
 * MFMA tiles that dequantise the MM8 bytes in registers -- the weight is
 * never materialised -- with the per-row sums taken by the same MFMAs.  fp16
 * activations and fp16 metadata; rows * I * 2 < 2^31 (callers split longer
 * inputs); no workspace.  Replaces the materialising route of
 * mm8_matmul_triton for rows > fused_max_rows
 * (rwkv7_hf/native_quant_mm8.py:468-507, :100-126) used by the prefill
 * projections (rwkv7_hf/native_jit_prefill.py:542-631, 955-1013). */
int rwkv7mi_mm8t_gemm_prefill(int nprob, const void* const* x,
                              const uint8_t* const* w_blk, const void* const* mx,
                              const void* const* rx, const void* const* my,
                              const void* const* ry, const void* const* bias,
                              const void* const* residual, void* const* y,
                              const int* epilogue, int64_t rows, int64_t I,
                              int64_t O, int act_dtype, int meta_dtype,
                              void* stream);

/* Workspace bytes rwkv7mi_mm8t_gemm_prefill_ws needs for nprob problems of
 * in_features I, out_features O: nprob * ceil(O / 16) * ceil(I / 64) * 2048
 * (each problem's fp16 dequantised weight); 0 for a bad shape. */
int64_t rwkv7mi_mm8t_gemm_prefill_ws_bytes(int nprob, int64_t I, int64_t O);

/* The prefill GEMM as the reference computes it, the faster form on gfx950:
 * the dequantised weight W_hat = (w + 0.5) ry rx + my + mx, rounded once to
 * the activation type (the bytes rwkv7mi_mm8_dequant writes), is
 * materialised into the workspace in MFMA operand order, then
 * y = epilogue(x @ W_hat (+ bias)) runs on 256 x 256 MFMA tiles.  fp16 or
 * bf16 activations with metadata of the same type.  Same arguments as rwkv7mi_mm8t_gemm_prefill plus the
 * workspace (16-byte aligned, at least rwkv7mi_mm8t_gemm_prefill_ws_bytes;
 * its contents are overwritten).  Replaces mm8_matmul_triton's route for
 * rows > fused_max_rows, dequantize_mm8 then x @ W_hat
 * (rwkv7_hf/native_quant_mm8.py:468-507, :100-119), used by the prefill
 * projections (rwkv7_hf/native_jit_prefill.py:542-631, 955-1013). */
int rwkv7mi_mm8t_gemm_prefill_ws(int nprob, const void* const* x,
                                 const uint8_t* const* w_blk,
                                 const void* const* mx, const void* const* rx,
                                 const void* const* my, const void* const* ry,
                                 const void* const* bias,
                                 const void* const* residual, void* const* y,
                                 const int* epilogue, int64_t rows, int64_t I,
                                 int64_t O, int act_dtype, int meta_dtype,
                                 void* ws, int64_t ws_bytes, void* stream);

/* The same prefill GEMM for unquantised fp16 or bf16 nn.Linear weights W [O, I]
 * (y = epilogue(x @ W^T (+ bias))): W is copied into the workspace in MFMA
 * operand order, then the 256 x 256 MFMA GEMM runs with the epilogue
 * fused.  Activations and weights of one type (fp16 or bf16), I % 16 == 0,
 * the workspace as for
 * rwkv7mi_mm8t_gemm_prefill_ws (rwkv7mi_mm8t_gemm_prefill_ws_bytes).
 * Replaces the unquantised projections' torch GEMM of the prefill
 * (rwkv7_hf/native_jit_prefill.py:542-631, 955-1013). */
int rwkv7mi_dense_gemm_prefill_ws(int nprob, const void* const* x,
                                  const void* const* W, const void* const* bias,
                                  const void* const* residual, void* const* y,
                                  const int* epilogue, int64_t rows, int64_t I,
                                  int64_t O, int act_dtype, void* ws,
                                  int64_t ws_bytes, void* stream);

/* Allocation-free form of rwkv7mi_mm8t_gemm_multi (same arguments and results,
 * no workspace argument).  No counterpart in the reference: it is for callers
 * that cannot allocate (code under hipGraph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Its scratch is a fixed per-GPU device
 * array of RWKV7MI_MM8T_GEMM_SCRATCH_BYTES (80 MiB: every 7.2B projection
 * at 64 rows, the 4096 x 65536 head included) held until the process ends;
 * calls needing more (see rwkv7mi_mm8t_gemm_workspace_bytes) return
 * RWKV7MI_ESIZE.  Every call on one GPU shares that array, so calls that
 * overlap on one GPU (different streams or threads) race; the kernels write
 * every scratch byte they read, so nothing needs clearing between calls. */
#define RWKV7MI_MM8T_GEMM_SCRATCH_BYTES (80u << 20)
int rwkv7mi_mm8t_gemm_multi_noalloc(int nprob, const void* const* x,
                                    const uint8_t* const* w_blk,
                                    const void* const* mx, const void* const* rx,
                                    const void* const* my, const void* const* ry,
                                    const void* const* bias,
                                    const void* const* residual, void* const* y,
                                    const int* epilogue, int64_t rows, int64_t I,
                                    int64_t O, int act_dtype, int meta_dtype,
                                    int splits, void* stream);

/* Decode LN + token-shift mix fused into the out-major MM8 GEMV: for up to
 * four problems of one shape, h = LayerNorm(x) (x [rows, I] the residual
 * rows, ln_w / ln_b [I]), x_p = round(h + (prev - h) * mix_p) and
 * y_p = x_p @ W_p with epilogue_p (none or relu^2).  Writes h to h_out
 * [rows, I] (may be NULL) and aux_out[a] = h + (prev - h) * aux_mix[a] for
 * a < naux (<= 4).  prev is only read.  Replaces fused_attn_norm_mix6_decode /
 * fused_ffn_add_norm_mix_decode (rwkv7_hf/fused_decode_norm_mix.py:161, 296)
 * feeding MM8Linear (native_quant_mm8.py:564-628).  All activation-side
 * tensors and the MM8 metadata in act_dtype (fp16 or bf16); rows <= 2 at
 * I = 4096 (the rows must fit one x' staging batch).  Outputs must not alias
 * x or prev.  With lora_w (NULL for none; rows <= 2), also the first half of
 * fused_wavg_lora (rwkv7_hf/fused_lora.py:706) on the extra mixes:
 * lora_out[off_a + row*rank_a + j] = aux_out[a][row] . lora_w[a][j] in fp32
 * (lora_w[a] [rank_a, I] in act_dtype, off_a = rows * sum of the earlier
 * ranks) — the one-split layout rwkv7mi_wkv7_decode_lora_output_prepare
 * reads with lora_splits = 1. */
int rwkv7mi_mm8t_lnmix_multi(int nprob, const void* x, const void* prev,
                             const void* ln_w, const void* ln_b, float eps,
                             const void* const* mix, const uint8_t* const* w_blk,
                             const void* const* mx, const void* const* rx,
                             const void* const* my, const void* const* ry,
                             void* const* y, const int* epilogue, void* h_out,
                             int naux, const void* const* aux_mix, void* const* aux_out,
                             const void* const* lora_w, const int64_t* lora_ranks,
                             float* lora_out, int64_t rows, int64_t I, int64_t O,
                             int act_dtype, void* stream);

/* dequantize_mm8 (rwkv7_hf/native_quant_mm8.py:100-108) from w_blk into out
 * [O,I] (Linear.weight layout) for a library GEMM on long prefills.
 * I % 4 == 0. */
int rwkv7mi_mm8t_dequant(const uint8_t* w_blk, const void* mx, const void* rx,
                         const void* my, const void* ry, void* out, int64_t I,
                         int64_t O, int meta_dtype, int out_dtype, void* stream);

/* ------------------------------------------------------------ MM4 affine */

/* Device packer of the 4-bit affine format, quantize_mm4
 * (rwkv7_hf/native_quant_mm4.py:77-105): weight [I,O] (= Linear.weight.T) in
 * w_dtype; O is padded to even Mp with a zero column as the reference does;
 * outputs packed [I, Mp/2] (byte = u4[i,2b] | u4[i,2b+1] << 4), mx, rx_s [Mp],
 * my, ry_s [I] in w_dtype (rx/4, ry/4).  Workspace 2*I + 2*Mp floats. */
int rwkv7mi_mm4_pack(const void* weight, int64_t I, int64_t O, int w_dtype,
                     uint8_t* packed, void* mx, void* rx_s, void* my,
                     void* ry_s, float* workspace, void* stream);

/* Same values from Linear.weight [O,I], packed along the inputs for the fused
 * GEMV: packed_t [Mp, I/2], byte (o, a) = u4[2a,o] | u4[2a+1,o] << 4 (I even;
 * row O of an odd O holds the pad column's nibbles).
 * The reference keeps its own per-device buffer layouts (MM4Linear,
 * rwkv7_hf/native_quant_mm4.py:587-619). */
int rwkv7mi_mm4_pack_t(const void* weight, int64_t I, int64_t O, int w_dtype,
                       uint8_t* packed_t, void* mx, void* rx_s, void* my,
                       void* ry_s, float* workspace, void* stream);

/* y[rows,O] = epilogue(x @ dequant(W)), (u4+0.5)*ry_s*rx_s + my + mx with fp32
 * accumulation, over packed_t.  Replaces mm4_gemv_triton / mm4_matmul_triton /
 * MM4Linear.forward (rwkv7_hf/native_quant_mm4.py:545-578, :621-660).
 * I % 32 == 0; x, packed_t, my, ry_s 16-byte aligned; y may alias residual. */
int rwkv7mi_mm4t_matmul(const void* x, const uint8_t* packed_t, const void* mx,
                        const void* rx_s, const void* my, const void* ry_s,
                        const void* bias, const void* residual, void* y,
                        int64_t rows, int64_t I, int64_t O, int epilogue,
                        int act_dtype, int meta_dtype, void* stream);

/* dequantize_mm4 (rwkv7_hf/native_quant_mm4.py:108-122) from the reference
 * layout packed [I, ceil(O/2)] into out [I, O] (fp32 math, one rounding). */
int rwkv7mi_mm4_dequant(const uint8_t* packed, const void* mx, const void* rx_s,
                        const void* my, const void* ry_s, void* out, int64_t I,
                        int64_t O, int meta_dtype, int out_dtype, void* stream);

/* y[rows,O] = epilogue(x @ dequant(W)) straight from the reference layout
 * packed [I, Mp/2] (nibble pairs along the outputs; Mp even, O <= Mp):
 * rx_s * sum x*ry_s*(u4+0.5) on MFMA with fp32 accumulation (x*ry_s split
 * into fp16 hi + lo), plus sum x*my + mx * sum x in fp32.  Replaces the fused
 * mm4_gemv_triton / mm4_batched_gemv_triton / mm4_batched_dot_triton /
 * mm4_matmul_triton kernels (rwkv7_hf/native_quant_mm4.py:158-288,
 * :458-578).  rows are taken 16 at a time; workspace of
 * rwkv7mi_mm4_matmul_workspace_bytes(I, Mp), 16-byte aligned, holds the
 * K-range partials (reduced in a fixed order, no atomics); y may alias
 * residual. */
size_t rwkv7mi_mm4_matmul_workspace_bytes(int64_t I, int64_t Mp);
int rwkv7mi_mm4_matmul(const void* x, const uint8_t* packed, const void* mx,
                       const void* rx_s, const void* my, const void* ry_s,
                       const void* bias, const void* residual, void* y,
                       int64_t rows, int64_t I, int64_t O, int64_t Mp,
                       int epilogue, int act_dtype, int meta_dtype,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Decode attention-side entry for 1..8 rows, fp16 / bf16: layer 0's
 * pre-norm (pre_w / pre_b; the normalised row goes to x_out), h = LayerNorm
 * (h_out), the r / k / v mixed rows of mixes {r, w, k, v, a, g} (outs[3]),
 * and the LoRA down projections of up to four problems as K-chunk partial
 * sums part[q][c][row][j] = sum over chunk c of mix_{lora_mix[q]}(h) . W_q[j]
 * (W_q [rank_q, D] in the activation dtype; problem q starts at float
 * offset sum_{q'<q} chunks*rows*rank_q'), which the fused wkv decode kernel
 * takes with lora_splits = chunks -- fused_attn_norm_mix6_decode
 * (rwkv7_hf/fused_decode_norm_mix.py:161-293) plus the down half of
 * fused_wavg_lora (rwkv7_hf/fused_lora.py:706).  D a multiple of 128, at
 * most 4096; outputs must not alias x or prev. */
int rwkv7mi_attn_mix_lora(const void* x, void* x_out, const void* prev,
                          void* h_out, const void* ln_w, const void* ln_b,
                          const void* pre_w, const void* pre_b,
                          const void* const* mixes, void* const* outs,
                          int64_t nlora, const void* const* lora_w,
                          const int64_t* ranks, const int* lora_mix,
                          float* part, int64_t rows, int64_t D, float eps,
                          int act_dtype, int param_dtype, void* stream);

/* K-chunks rwkv7mi_attn_mix_lora splits width D into (0: D unsupported). */
int rwkv7mi_attn_mix_lora_chunks(int64_t D);

/* ------------------------------------------------------------ state slots */

/* Row copies between layer-major state pools and dense batches (the serving
 * state-slot pool of docs/integrations/RWKV7_STATE_CACHE_ABI.md:52-133:
 * gather / scatter / clone / reset of scheduled slots, NativeRWKV7Cache's
 * select_batch / reorder semantics, rwkv7_hf/model_cache.py:335-343).  Row r
 * of layer l is copied from src + l*src_layer_stride + src_rows[r]*
 * src_row_stride to dst + l*dst_layer_stride + dst_rows[r]*dst_row_stride
 * (byte strides; a NULL index array is the identity; src_rows / dst_rows /
 * active are device arrays), rows with active[r] == 0 are left untouched, and
 * src == NULL writes zeros.  row_bytes, pointers and strides 16-byte
 * aligned; nrows, nlayers <= 65535. */
int rwkv7mi_slot_copy(const void* src, int64_t src_layer_stride,
                      int64_t src_row_stride, const int64_t* src_rows, void* dst,
                      int64_t dst_layer_stride, int64_t dst_row_stride,
                      const int64_t* dst_rows, const uint8_t* active,
                      int64_t nrows, int64_t row_bytes, int64_t nlayers,
                      void* stream);

/* ------------------------------------------------------- greedy selection */

/* out[r] = argmax of row r of x [rows, n] (row stride ld elements, act dtype),
 * as the reference's greedy decode loop takes it with torch
 * (`out.logits[:, -1:].argmax(dim=-1)`, bench/bench_native_quant_e2e_decode.py:
 * 424-437): ties go to the smaller index and NaN beats every number.  out2,
 * when not NULL, receives the same indices (the decode graph writes its next
 * input tokens and the caller's copy in one launch).  x 16-byte aligned,
 * ld * element size a multiple of 16. */
int rwkv7mi_argmax_rows(const void* x, int64_t rows, int64_t n, int64_t ld,
                        int dtype, int64_t* out, int64_t* out2, void* stream);

/* rwkv7mi_argmax_rows in two launches over many workgroups per row (slices
 * of 4096 fp16 / 2048 fp32 entries, then one wave per row over the slices'
 * bests), with the same result and rules; `workspace` (8-byte aligned) holds
 * rwkv7mi_argmax_workspace_bytes(rows, n, dtype).  rows <= 65535. */
size_t rwkv7mi_argmax_workspace_bytes(int64_t rows, int64_t n, int dtype);
int rwkv7mi_argmax_rows_ws(const void* x, int64_t rows, int64_t n, int64_t ld,
                           int dtype, int64_t* out, int64_t* out2,
                           void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ LoRA */

/* Bytes of workspace rwkv7mi_lora_multi needs (fp32 split-K partials). */
size_t rwkv7mi_lora_workspace_bytes(int64_t nprob, const int64_t* ranks,
                                    int64_t rows, int64_t D);

/* Up to four LoRA projections sharing x's shape, as in fused_wavg_lora /
 * fused_wag_lora (rwkv7_hf/fused_lora.py:706, :559; torch form :795-803):
 *   y_i = act_up_i(act_down_i(x_i @ w_down_i^T) @ w_up_i^T + b_up_i)
 * x_i [rows,D], w_down_i [rank_i,D], w_up_i [A,rank_i], b_up_i [A] or NULL
 * (b_up may be NULL), y_i [rows,A]; activations 0 none, 1 tanh, 2 sigmoid.
 * The intermediate is rounded to act_dtype as the reference's tensor is.
 * rank_i a multiple of 8, at most 256; D a multiple of 8. */
int rwkv7mi_lora_multi(int64_t nprob, const void* const* xs,
                       const void* const* w_down, const void* const* w_up,
                       const void* const* b_up, void* const* ys,
                       const int64_t* ranks, const int* act_down,
                       const int* act_up, int64_t rows, int64_t D, int64_t A,
                       int act_dtype, void* workspace, size_t workspace_bytes,
                       void* stream);

/* The down projections of rwkv7mi_lora_multi alone (the first half of
 * fused_wavg_lora, rwkv7_hf/fused_lora.py:706): fp32 partial sums
 * [problem][ks][rows][rank] in the workspace, for
 * rwkv7mi_wkv7_decode_lora_output_prepare.  rows <= 64. */
int rwkv7mi_lora_down_multi(int64_t nprob, const void* const* xs,
                            const void* const* w_down, const int64_t* ranks,
                            const int* act_down, int64_t rows, int64_t D,
                            int act_dtype, void* workspace, size_t workspace_bytes,
                            void* stream);

/* ---------------------------------------------------------- W4 group-128 */

/* Device packer of the symmetric group W4 format of
 * rwkv7_hf/sm70_quant.py:502-519: weight [O,I] -> packed [O,I/2],
 * scales [O,I/group] (w_dtype).  group in {128, 256}. */
int rwkv7mi_w4g_pack(const void* weight, int64_t O, int64_t I, int64_t group,
                     int w_dtype, uint8_t* packed, void* scales, void* stream);

/* y[rows,O] = epilogue(x @ W^T), W[o,i] = (nib - 8) * scales[o, i/group].
 * Replaces w4_groupwise_linear (rwkv7_hf/sm70_quant.py:579). */
int rwkv7mi_w4g_matmul(const void* x, const uint8_t* packed,
                       const void* scales, const void* bias,
                       const void* residual, void* y, int64_t rows, int64_t O,
                       int64_t I, int64_t group, int epilogue, int act_dtype,
                       int scale_dtype, void* stream);

/* Asymmetric group-wise W4 (min/max affine, group 128 / 256): per (row o,
 * group g) s = max((max - min) / 15, 1e-8), b = min, q = clamp(rint((w - b)
 * / s), 0, 15) in fp32; packed [O, I/2] as rwkv7mi_w4g_pack (low nibble =
 * even input), scales and biases [O, I/group] in the weight dtype;
 * W[o,i] = q s + b.  The reference's only asymmetric group format is MLX's
 * affine mode (rwkv7_hf/mlx_quant.py:258-290, Apple only), which this format
 * follows in form; its parity with MLX is unpinned (no MLX here). */
int rwkv7mi_w4a_pack(const void* weight, int64_t O, int64_t I, int64_t group,
                     int w_dtype, uint8_t* packed, void* scales, void* biases,
                     void* stream);
/* y = epilogue(x W^T + bias) with the affine W above; rows any, fp32
 * accumulation, the same epilogues as rwkv7mi_w4g_matmul. */
int rwkv7mi_w4a_matmul(const void* x, const uint8_t* packed,
                       const void* scales, const void* biases,
                       const void* bias, const void* residual, void* y,
                       int64_t rows, int64_t O, int64_t I, int64_t group,
                       int epilogue, int act_dtype, int scale_dtype,
                       void* stream);

/* ------------------------------------------------ LayerNorm + token shift */

/* Decode LN + six token-shift mixes per row (D <= 8192):
 *   [x = LN_pre(x) written back when pre_w != NULL]  h = LN(x; ln_w, ln_b, eps);
 *   outs[i] = h + (prev - h) * mixes[i] (i < nmix);  prev <- h.
 * Replaces fused_attn_norm_mix6_decode (rwkv7_hf/fused_decode_norm_mix.py:161).
 * x and prev must not alias.  mixes / outs are arrays of nmix pointers. */
int rwkv7mi_attn_norm_mix6(void* x, void* prev, const void* ln_w,
                           const void* ln_b, const void* pre_w,
                           const void* pre_b, const void* const* mixes,
                           void* const* outs, int64_t nmix, int64_t rows,
                           int64_t D, float eps, int act_dtype,
                           int param_dtype, void* stream);

/* rwkv7mi_attn_norm_mix6 (no pre-norm) that first finishes the residual add
 * of the previous layer's split FFN value: x = round(sum_s part[s *
 * part_stride + row * D + i] + x), the splits (1..4) added in order as the
 * split reduce would, written back to x, then the norm and mixes as above
 * (rwkv7_hf/native_jit_graph_dispatch.py:594-598 then
 * fused_decode_norm_mix.py:161). part 16-byte aligned fp32. */
int rwkv7mi_attn_norm_mix6_parts(void* x, void* prev, const void* ln_w,
                                 const void* ln_b, const void* const* mixes,
                                 void* const* outs, int64_t nmix,
                                 const float* part, int64_t splits,
                                 int64_t part_stride, int64_t rows, int64_t D,
                                 float eps, int act_dtype, int param_dtype,
                                 void* stream);

/* x = residual (+ attn_out -> residual_out); h = LN(x);
 * mixed = h + (prev - h) * mix; prev <- h.
 * Replaces fused_ffn_add_norm_mix_decode (rwkv7_hf/fused_decode_norm_mix.py:296). */
int rwkv7mi_ffn_add_norm_mix(const void* residual, const void* attn_out,
                             void* prev, const void* ln_w, const void* ln_b,
                             const void* mix, void* residual_out, void* mixed,
                             int64_t rows, int64_t D, float eps, int act_dtype,
                             int param_dtype, void* stream);

/* Sequence form over x [B,T,D]: h_t = LN(x_t), prev_t = h_{t-1} (prev_in for
 * t = 0), outs[i] = h + (prev - h) * mixes[i]; prev_out <- h_{T-1}.
 * ln_w = ln_b = NULL: h = x (x already normalised, the reference's convention).
 * Replaces fused_attn_sequence_shift_mix / fused_ffn_sequence_shift_mix
 * (rwkv7_hf/fused_time_mix.py:413, :470).  prev_in != prev_out. */
int rwkv7mi_seq_norm_mix(const void* x, const void* prev_in, void* prev_out,
                         const void* ln_w, const void* ln_b,
                         const void* const* mixes, void* const* outs,
                         int64_t nmix, int64_t B, int64_t T, int64_t D,
                         float eps, int act_dtype, int param_dtype,
                         void* stream);

/* y = LN(x) over rows of D (F.layer_norm; used for the pre-norm and the final
 * norm before the LM head, rwkv7_hf/native_jit_prefill.py:1024-1036). */
int rwkv7mi_layer_norm(const void* x, void* y, const void* w, const void* b,
                       int64_t rows, int64_t D, float eps, int act_dtype,
                       int param_dtype, void* stream);

/* ------------------------------------------------ dense LoRA projections */

/* Up to 4 independent y_i = act_i(x_i @ W_i^T + bias_i) in one launch,
 * W_i [N_i, K_i] (nn.Linear layout), K_i % 8 == 0, act in
 * {0 none, 1 tanh, 2 sigmoid, 3 relu^2}.  Replaces the W/A/G/V LoRA down and
 * up projections of fused_wavg_lora (rwkv7_hf/fused_lora.py:706). */
int rwkv7mi_dense_multi(const void* const* xs, const void* const* Ws,
                        const void* const* biases, void* const* ys,
                        const int64_t* Ns, const int64_t* Ks, const int* acts,
                        int64_t nprob, int64_t rows, int act_dtype,
                        void* stream);

/* ------------------------------------------- scan input / output prep */

/* state_prep flags */
#define RWKV7MI_PREP_A_RAW 1     /* a is pre-sigmoid: a = sigmoid(a) first */
#define RWKV7MI_PREP_VGATE_RAW 2 /* v_gate is pre-sigmoid */
#define RWKV7MI_PREP_W_DECAY 4   /* w_out = exp(log decay), else the log decay */

/* Per (row, head): kk = normalize(k_raw * k_k), k_out = k_raw*(1+(a-1)*k_a),
 * w_out = -0.606531*sigmoid(w_raw) (natural-log decay) or its exp (flag
 * RWKV7MI_PREP_W_DECAY), in fp32 (w_dtype F32) or the activation dtype, and
 * v_out = v_raw after the V interpolation (v_mode 0: as is; 1: v_first = v;
 * 2: v += (v_first - v) * v_gate).  v_out may be v_raw.
 * Replaces fused_prefill_state_prep (rwkv7_hf/fused_prefill.py:184). */
int rwkv7mi_state_prep(const void* k_raw, const void* a, const void* w_raw,
                       const void* v_raw, void* v_out, void* v_first,
                       const void* v_gate, const void* k_k, const void* k_a,
                       void* kk_out, void* k_out, void* w_out, int64_t rows,
                       int64_t H, int64_t N, int v_mode, int flags,
                       int act_dtype, int param_dtype, int w_dtype,
                       void* stream);

/* out = (GroupNorm_H(y) + (sum_head r*k*r_k) * v) * g per (row, head).
 * Replaces fused_attn_output_prepare (rwkv7_hf/fused_output.py:190). */
int rwkv7mi_output_prepare(const void* y, const void* r, const void* k,
                           const void* v, const void* g, const void* r_k,
                           const void* gn_w, const void* gn_b, void* out,
                           int64_t rows, int64_t H, int64_t N, float eps,
                           int act_dtype, int param_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RWKV7MI_H */
