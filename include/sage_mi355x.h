/*
 * sage_mi355x.h -- C ABI of the MI355X (gfx950) SageAttention forward and backward.
 *
 * Drop-in boundary for the attention op that sqcu/futudiffu registers as
 *   futudiffu_ii::sage_attn_masked(q, k, v, block_mask, sm_scale) -> (out, lse)
 *   futudiffu_ii::sage_attn(q, k, v, sm_scale)                   -> (out, lse)
 * (src_ii/attention_srcii.py:54-64 and :109-119).  Those ops call
 * sage_attn_forward_masked_with_lse / sage_attn_forward_with_lse
 * (src/futudiffu/sage_attention.py:461-531, :271-341), which smooth K, then
 * launch one Triton kernel that quantizes Q and K inside the attention loop.
 * Here the same work is split in two entry points with plain pointers:
 * sage_quantize_qkv (smoothing + all quantization, memory-bound) and
 * sage_attn_fwd (8-bit MFMA QK^T, fp32 online softmax, fp8/bf16 PV).
 *
 * Every pointer is device memory owned by the caller; the library never
 * allocates or frees.  Every entry point is stateless, takes the HIP stream to
 * launch on, never synchronizes, and returns 0 on success or a SAGE_ERR_*
 * code, with a message available from sage_last_error() (thread-local).
 *
 * Tensor layouts (BH = B*H, Np = N rounded up to a multiple of 128):
 *   q, k, v      bf16 [BH, N, D] contiguous, D in {64, 128}.
 *   q_codes,
 *   k_codes      int8 or fp8-e4m3fn codes, BH*Np*D bytes, "row fragment"
 *                order: for each 32-token block rb, each 32-channel chunk c,
 *                each lane L = 32*h + r (h in {0,1}, r in [0,32)):
 *                16 bytes = X[32*rb + r][32*c + 16*h + 0..15].
 *                Byte offset = ((rb*(D/32) + c)*64 + L)*16.
 *   q_scale,
 *   k_scale      fp32; per token [BH, Np] (granularity 0) or per 64-token
 *                block [BH, Np/64] (granularity 1).  q_scale includes
 *                sm_scale*log2(e) (sage_kernels.py:1422).
 *   v_codes      pv_kind 1 (fp8): BH*Np*D bytes; for each 64-token tile t,
 *                32-channel block j, key half b in {0,1}, lane L = 32*h + r:
 *                16 bytes, byte 4*jj + i = Vc[64t + 32b + 8jj + 4h + i][32j + r].
 *                Byte offset = (((t*(D/32) + j)*2 + b)*64 + L)*16.
 *                pv_kind 0 (bf16): BH*Np*D*2 bytes; for each t, j, b, and
 *                half tt in {0,1}, lane L: 8 bf16, element 4*jj + i =
 *                V[64t + 32b + 16tt + 8jj + 4h + i][32j + r].
 *                Byte offset = ((((t*(D/32) + j)*2 + b)*2 + tt)*64 + L)*16.
 *   v_scale      fp8 PV only: fp32 [BH, Np/64, D], one scale per (64-token
 *                block, channel) (sage_kernels.py:1143-1148).
 *   k_mean       bf16 [BH, D] smoothing mean (written when smooth_k != 0).
 *   out          bf16 [B, H, N, D] contiguous (out_layout 0), or
 *                bf16 [B, N, H, D] contiguous (out_layout 1): the
 *                [B, N, H*D] input of the out-projection, written without the
 *                caller's transpose copy (transformer.py:471).
 *   lse        fp32 [BH, N], log2 domain: m + log2(l) in sm_scale*log2(e)
 *                units (sage_kernels.py:1468-1471).  Rows that see no key
 *                get out = 0 and lse = -inf.
 */
#ifndef SAGE_MI355X_H
#define SAGE_MI355X_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SAGE_ABI_VERSION 6

enum sage_status {
  SAGE_OK = 0,
  SAGE_ERR_ARG = 1,         /* bad shape, kind or null pointer            */
  SAGE_ERR_ALIGN = 2,       /* pointer not 16-byte aligned                 */
  SAGE_ERR_WORKSPACE = 3,   /* workspace missing or too small              */
  SAGE_ERR_LAUNCH = 4       /* hipLaunchKernel / hipGetLastError failed    */
};

enum sage_qk_kind { SAGE_QK_INT8 = 0, SAGE_QK_FP8 = 1 };
enum sage_pv_kind { SAGE_PV_BF16 = 0, SAGE_PV_FP8 = 1 };
enum sage_granularity { SAGE_GRAN_TOKEN = 0, SAGE_GRAN_BLOCK64 = 1 };
enum sage_out_layout { SAGE_OUT_BHND = 0, SAGE_OUT_BNHD = 1 };

/* Version of this ABI (SAGE_ABI_VERSION).  No reference counterpart. */
int sage_abi_version(void);

/* Message for the last non-zero status returned on this thread.
 * Replaces the reference's Python AssertionError/ValueError text
 * (sage_attention.py:487-488, :518-519). */
const char* sage_last_error(void);

/* Np for a sequence length: N rounded up to a multiple of 128. */
int64_t sage_padded_len(int64_t n);

/* Bytes of device workspace sage_quantize_qkv and sage_quantize_from_qkv
 * need when smoothing: fp64 column sums of K per head and 256-token chunk,
 * [bh][ceil(n/256)][d], an 8-byte flag per chunk, and per head an 8-byte
 * flag and the fp32 mean of K (written, then read, by the call; no prior
 * contents needed).  16-byte aligned.  Concurrent calls need separate
 * workspaces. */
size_t sage_quant_workspace_bytes(int64_t bh, int64_t n, int64_t d);

/* K smoothing + Q/K (and, for fp8 PV, V) quantization.
 * Replaces _smooth_k (sage_attention.py:63-71, applied at :490-491) and the
 * in-kernel Q/K quantization of _sage_attn_fwd_int8qk_bf16pv_masked_lse
 * (sage_kernels.py:1415-1422, :1443-1449), its fp8 counterparts (:250-258,
 * :272-280) and the V quantization of _sage_attn_fwd_fp8qk_fp8pv_lse
 * (:1143-1148).  Codes are bit-exact with those formulas given k_mean.
 * For pv_kind 0, v_out receives V (bf16, unmodified values) in the bf16
 * fragment order above and v_scale may be NULL.  sm_scale_log2e is folded
 * into q_scale (sage_attention.py:493-495).  smooth_k = 0 skips smoothing
 * (configure_sage(smooth_k=False), sage_attention.py:37-60). */
int sage_quantize_qkv(const void* q, const void* k, const void* v,
                      int64_t bh, int64_t n, int64_t d,
                      int qk_kind, int pv_kind, int granularity, int smooth_k,
                      float sm_scale_log2e,
                      void* q_codes, float* q_scale,
                      void* k_codes, float* k_scale,
                      void* v_out, float* v_scale,
                      void* k_mean,
                      void* workspace, size_t workspace_bytes,
                      hipStream_t stream);

/* The q/k/v producer: QKV split + per-head RMSNorm + Flux RoPE + transpose.
 * Replaces fused_qkv_postprocess (src/futudiffu/fused_kernels.py:271-390,
 * op :613-643).
 *   qkv        bf16 [B, N, 3*H*D] (the QKV projection output).
 *   q_norm_w,
 *   k_norm_w   fp32 [D] RMSNorm weights.
 *   freqs      fp32 [B*N, D/2, 2, 2] rotary matrices [[cos, -sin], [sin, cos]].
 *   q_out,
 *   k_out,
 *   v_out      bf16 [B, H, N, D].
 * q' = rope(x * rrms * w) with rrms = 1 / sqrt(mean(x^2) + norm_eps) per
 * token and head; the sum of squares is exact (fp64) and every other step a
 * separately rounded fp32 operation, so results are reproducible bit for bit.
 * V is copied unchanged.  All pointers 16-byte aligned. */
int sage_qkv_postprocess(const void* qkv, const float* q_norm_w, const float* k_norm_w,
                         const float* freqs, int64_t b, int64_t h, int64_t n, int64_t d,
                         float norm_eps, void* q_out, void* k_out, void* v_out,
                         hipStream_t stream);

/* Gradient of the producer with respect to the projection output.
 * Replaces the autograd formula of fused_qkv_postprocess
 * (src/futudiffu/fused_kernels.py:711-783): per token and head, the incoming
 * q / k gradient through the rotation's transpose, then the RMSNorm backward
 * rrms * (g*w - x * rrms^2 * sum(g*w * x) / D); v's gradient passes through.
 * The norm weights and rotations get no gradient, as in the reference.
 *   qkv, q_norm_w, k_norm_w, freqs, b, h, n, d, norm_eps  as in
 *                sage_qkv_postprocess (the forward's inputs).
 *   grad_q,
 *   grad_k,
 *   grad_v     bf16 [B, H, N, D] gradients of the producer's outputs.
 *   dqkv       bf16 [B, N, 3*H*D].
 * fp32 arithmetic with fp64 row sums.  All pointers 16-byte aligned. */
int sage_qkv_postprocess_bwd(const void* qkv, const float* q_norm_w, const float* k_norm_w,
                             const float* freqs, const void* grad_q, const void* grad_k,
                             const void* grad_v, int64_t b, int64_t h, int64_t n, int64_t d,
                             float norm_eps, void* dqkv, hipStream_t stream);

/* sage_quantize_qkv applied to the outputs of sage_qkv_postprocess, without
 * writing them: the producer runs inside the quantization kernels, which read
 * the projection output directly (half the HBM traffic of producer +
 * quantization).  Outputs are bit-identical to that two-call sequence.  No
 * reference counterpart (the reference writes bf16 q, k, v, fused_kernels.py
 * :372-385, and its attention quantizes them again).  Same outputs, workspace
 * and kinds as sage_quantize_qkv with bh = b*h. */
int sage_quantize_from_qkv(const void* qkv, const float* q_norm_w, const float* k_norm_w,
                           const float* freqs, int64_t b, int64_t h, int64_t n, int64_t d,
                           float norm_eps, int qk_kind, int pv_kind, int granularity,
                           int smooth_k, float sm_scale_log2e,
                           void* q_codes, float* q_scale, void* k_codes, float* k_scale,
                           void* v_out, float* v_scale, void* k_mean,
                           void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Bytes of device workspace sage_attn_fwd needs for B x H heads of N tokens
 * of dimension D: per-batch (min doc, max doc, #valid, #padding) summaries of
 * every 64-key tile and 32- and 128-row query block and the scheduled
 * key-tile range of every 128-row query block (written and used when doc_ids
 * is given), then the fp32 partial results of the key-tile pieces of
 * the 128-row items that an unmasked launch splits (the items past the last
 * whole round of 512 resident workgroups) and an 8-byte arrival counter per
 * split item (the last piece to finish merges the item's partials; the
 * counters need no clearing, each call tags them with a value no earlier
 * call used).  Enough for every launch of that shape.  No reference
 * counterpart (the Triton launch needs no workspace). */
size_t sage_attn_workspace_bytes(int64_t b, int64_t h, int64_t n, int64_t d);

/* Bytes of device workspace a sage_attn_fwd launch with a tile_mask or
 * doc_ids needs: the summaries only, since masked launches split no item
 * (a few KB; 7 KB for the packed 1x30x6912 batch).  No reference
 * counterpart. */
size_t sage_attn_masked_workspace_bytes(int64_t b, int64_t h, int64_t n, int64_t d);

/* Fused attention forward over pre-quantized operands.
 * Replaces the launch of _sage_attn_fwd_int8qk_bf16pv_masked_lse
 * (sage_kernels.py:1378-1477, launched at sage_attention.py:521-529) and the
 * unmasked dispatch of sage_attn_forward_with_lse (sage_attention.py:316-339).
 *   tile_mask     optional uint8 reference block mask, entries [z][i][j] for
 *                 query tile i (128 rows) x key tile j (64 keys); z stride
 *                 mask_stride_z (0 broadcasts a 2D mask, sage_attention.py:512-519);
 *                 mask_nq x mask_nkv must equal ceil(N/128) x ceil(N/64).
 *                 0 skips the tile pair (sage_kernels.py:1428-1436).
 *                 Each byte is read as part of its aligned 4-byte word, so
 *                 the allocation must stay readable up to the next multiple
 *                 of 4 bytes past the last entry (hipMalloc and the torch
 *                 caching allocator hand out 256-byte granules).
 *   doc_ids       optional int32 [B, N] per-token document ids for exact
 *                 masking: key n is visible to query m iff doc[n] >= 0 and
 *                 (doc[m] == doc[n] or doc[m] < 0).  Fully masked tiles issue
 *                 no MFMA.
 *   n             at most 2^22 (one head's operands are addressed with
 *                 32-bit byte offsets).
 *   h             heads per batch (row z of q belongs to batch z / h).
 *   workspace     device memory of sage_attn_workspace_bytes(b, h, n, d)
 *                 bytes (sage_attn_masked_workspace_bytes when tile_mask or
 *                 doc_ids is given), 16-byte aligned.  Concurrent calls need
 *                 separate workspaces.
 *   out_layout    SAGE_OUT_BHND (the reference op's output) or SAGE_OUT_BNHD
 *                 (fuses JointAttention's out.transpose(1, 2).reshape(b, -1,
 *                 H*D), transformer.py:471).  Values are bit-identical
 *                 between the two layouts. */
int sage_attn_fwd(const void* q_codes, const float* q_scale,
                  const void* k_codes, const float* k_scale,
                  const void* v_in, const float* v_scale,
                  int64_t b, int64_t h, int64_t n, int64_t d,
                  int qk_kind, int pv_kind, int granularity,
                  const uint8_t* tile_mask, int64_t mask_stride_z,
                  int64_t mask_nq, int64_t mask_nkv,
                  const int32_t* doc_ids,
                  void* workspace, size_t workspace_bytes,
                  void* out, int out_layout, float* lse,
                  hipStream_t stream);

/* Bytes of device scratch behind sage_attn_fwd_noalloc (per GPU). */
#define SAGE_NOALLOC_SCRATCH_BYTES (16u << 20)

/* sage_attn_fwd without the workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * workspace lives in a fixed device array of SAGE_NOALLOC_SCRATCH_BYTES per
 * GPU, held until the process ends; launches whose workspace (as
 * sage_attn_fwd: sage_attn_workspace_bytes unmasked,
 * sage_attn_masked_workspace_bytes with a tile mask or document ids) exceeds
 * it are rejected with SAGE_ERR_WORKSPACE before any launch (the unmasked
 * 1x30x4416x128 headline needs 6.9 MB, the masked packed 1x30x6912 batch
 * 7 KB).  The call allocates and frees
 * nothing and needs no memory cleared beforehand: every byte of scratch it
 * reads was written earlier in the same call, except the split items'
 * arrival counters, whose per-call tag makes another call's value count as
 * zero.  Every call on one GPU shares
 * that GPU's scratch, so calls that overlap on one GPU (other streams, other
 * threads) race; calls ordered on one stream do not.  The stream must belong
 * to the current device.  The first call on a device looks the array's
 * address up (hipGetSymbolAddress).  Other arguments, results and errors as
 * sage_attn_fwd, bit-identical to it. */
int sage_attn_fwd_noalloc(const void* q_codes, const float* q_scale,
                          const void* k_codes, const float* k_scale,
                          const void* v_in, const float* v_scale,
                          int64_t b, int64_t h, int64_t n, int64_t d,
                          int qk_kind, int pv_kind, int granularity,
                          const uint8_t* tile_mask, int64_t mask_stride_z,
                          int64_t mask_nq, int64_t mask_nkv,
                          const int32_t* doc_ids,
                          void* out, int out_layout, float* lse,
                          hipStream_t stream);

/* Reference tile mask from device per-token document ids.
 * Replaces the host construction of build_block_mask /
 * build_block_mask_from_packing_info (src_ii/block_mask.py:35-129): Q tile i
 * (128 tokens) and KV tile j (64 tokens) take the id of their first token
 * (tile starts clamped to n-1, :84-93), and mask[z][i][j] = 1 iff the ids
 * are equal (:96-97).  Ids below zero (padding, as _pad_plan_to_fixed_len
 * writes them, forward_packed.py:56-62) count as pad_fill; 0 reproduces the
 * reference, where tokens past the last segment belong to document 0
 * (block_mask.py:75-79).
 *   doc_ids   int32 [b, n] device memory.
 *   mask      uint8 [b, ceil(n/128), ceil(n/64)] (b = 1: the 2D reference mask). */
int sage_build_tile_mask(const int32_t* doc_ids, int64_t b, int64_t n,
                         int32_t pad_fill, uint8_t* mask, hipStream_t stream);

/* Exact per-token document ids from varlen segment offsets, for the doc_ids
 * argument of sage_attn_fwd.  No reference counterpart: it replaces the host
 * list that build_packed_sequence fills per segment
 * (src_ii/transformer.py:137-153) with the cu_seqlens form.
 *   cu_seqlens  int32 [b, n_segments + 1] device memory, nondecreasing per
 *               batch row; segment s covers tokens [cu[s], cu[s+1]).
 *   doc_ids     int32 [b, n]: the segment index, or -1 for tokens outside
 *               every segment (padding).
 * Offsets that are not nondecreasing give unspecified ids, never an
 * out-of-bounds access. */
int sage_doc_ids_from_cu_seqlens(const int32_t* cu_seqlens, int64_t b,
                                 int64_t n_segments, int64_t n,
                                 int32_t* doc_ids, hipStream_t stream);

/* Bytes of the workspace sage_attn_bwd needs for b*h heads of n tokens of
 * dimension D: the per-token Q / smoothed-K codes, scales and K mean, the
 * K column-sum partials, bf16 operand images of dO, Q and the smoothed K
 * (the bf16 v_codes layout above), D = rowsum(dO * O) (fp32 [BH, Np]), the
 * document-id summaries, and the fp32 partial dQ of the last dQ items, which
 * run as two key-tile halves (8 MB at D = 128).  No reference counterpart
 * (the Triton launcher allocates these with torch). */
size_t sage_attn_bwd_workspace_bytes(int64_t b, int64_t h, int64_t n, int64_t d);

/* Attention backward: dQ, dK, dV from the forward's inputs, output and LSE.
 * Replaces sage_attn_backward_masked (sage_attention.py:534-648) and
 * sage_attn_backward (:344-458): the D pre-pass (sage_kernels.py:321-349),
 * the dK/dV kernel (:805-916, tile-masked :1491-1615) and the dQ kernel
 * (:918-1030, tile-masked :1617-1722), int8 or fp8 QK (:356-590).  P is
 * recomputed from per-token codes of Q and of K (smoothed again when
 * smooth_k != 0, which must match the forward), p = 2^(s - lse):
 *   dV = bf16(P)^T dO, dK = bf16(dS * sm_scale)^T Q, dQ = (bf16(dS) K~) * sm_scale,
 *   dS = P (dO V^T - D), each output rounded once to bf16.
 *   q, k, v, out,
 *   dout, dq, dk, dv  bf16 [BH, N, D] contiguous (the [B, H, N, D] tensors).
 *   lse               fp32 [BH, N] from sage_attn_fwd (rows at -inf get no
 *                     gradient).
 *   qk_kind           SAGE_QK_INT8 (the reference's production backward) or
 *                     SAGE_QK_FP8 (its fp8 kernels, :356-590).
 *   sm_scale,
 *   sm_scale_log2e    the softmax scale and its product with log2(e), the
 *                     latter formed in double and rounded once (as passed to
 *                     sage_quantize_qkv).
 *   tile_mask, doc_ids  as in sage_attn_fwd; use the forward's.
 *   workspace         sage_attn_bwd_workspace_bytes(b, h, n, d) bytes,
 *                     16-byte aligned; concurrent calls need separate ones. */
int sage_attn_bwd(const void* q, const void* k, const void* v,
                  const void* out, const float* lse, const void* dout,
                  int64_t b, int64_t h, int64_t n, int64_t d,
                  int qk_kind, int smooth_k, float sm_scale, float sm_scale_log2e,
                  const uint8_t* tile_mask, int64_t mask_stride_z,
                  int64_t mask_nq, int64_t mask_nkv,
                  const int32_t* doc_ids,
                  void* workspace, size_t workspace_bytes,
                  void* dq, void* dk, void* dv,
                  hipStream_t stream);

/* Parity: sage_attn_fwd with per-token scales, no mask and the [B, H, N, D]
 * output, which also stores the QK^T accumulators its own loop consumes, tile
 * by tile, as that loop forms them (the split tail pieces included): s_out
 * [B*H, Np, Np] 32-bit words, row = query, column = key; int32 sums for
 * SAGE_QK_INT8, the bit patterns of the fp32 sums for SAGE_QK_FP8.  Entries
 * of rows below 32*ceil(n/32) and keys below 64*ceil(n/64) are written,
 * others are left as they were.  Exposes the result of tl.dot(q, k) before
 * dequantization (int8 sage_kernels.py:1451, fp8 :282).  Other arguments as
 * sage_attn_fwd; slower (the accumulators are stored from inside the
 * loop). */
int sage_attn_qk_accumulators(const void* q_codes, const float* q_scale,
                              const void* k_codes, const float* k_scale,
                              const void* v_in, const float* v_scale,
                              int64_t b, int64_t h, int64_t n, int64_t d,
                              int qk_kind, int pv_kind, void* workspace, size_t workspace_bytes,
                              void* out, float* lse, int32_t* s_out,
                              hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SAGE_MI355X_H */
