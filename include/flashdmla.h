/*
 * flashdmla.h -- C ABI of the MI355X-native Flash-DMLA attention backend (gfx950).
 *
 * Every entry point:
 *   - takes caller-owned device pointers and explicit element strides (the last dimension of
 *     every bf16 tensor must be contiguous and 16-byte aligned);
 *   - is asynchronous and stream-ordered on `stream` (a hipStream_t; NULL = default stream);
 *   - allocates nothing: scratch memory is a caller-provided `workspace` whose size comes from
 *     the matching *_workspace_bytes() query;
 *   - returns DMLA_OK (0) or a negative status; dmla_last_error() then describes the failure.
 *
 * The reference's launchers (e.g. `fa2_forward`, csrc/attention/fa2_fwd.cu:139-156) take
 * `(const float* Q, const float* K, const float* V, float* O, int Nq, int Nk, int d, int dv,
 *  float scale, int warps_per_block, cudaStream_t)` and return void, silently doing nothing on
 * bad arguments (fa2_fwd.cu:149).  The entry points below keep that calling pattern --
 * raw pointers, sizes, scale, stream -- and add batch/head strides, bf16 storage, the saved
 * softmax statistics of README.md:12 and an error status.
 *
 * Element types: `bf16` tensors are passed as `const void*` holding IEEE bfloat16 values;
 * statistics are fp32; page tables and sequence lengths are int32.
 */
#ifndef FLASHDMLA_H
#define FLASHDMLA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DMLA_OK 0
#define DMLA_ERR_INVALID_ARG (-1)  /* null pointer, bad shape, stride or alignment */
#define DMLA_ERR_UNSUPPORTED (-2)  /* a shape outside the compiled kernel family */
#define DMLA_ERR_WORKSPACE (-3)    /* workspace missing or too small */
#define DMLA_ERR_HIP (-4)          /* the HIP runtime reported an error at launch */

typedef void* dmla_stream_t; /* hipStream_t */

/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int dmla_version(void);

/* Message for the most recent failing call on this host thread ("" if none). */
const char* dmla_last_error(void);

/*
 * Cache-latent DMLA forward (prefill).
 * Replaces: fa2_forward (csrc/attention/fa2_fwd.cu:139-156) specialised to the cache-latent
 * mode of README.md:15 -- the role of the absent csrc/attention/fa2_dmla_fwd.cu
 * (README.md:45).
 *
 *   q     [B, H, Sq, d_qk] bf16    strides (q_sb, q_sh, q_ss)
 *   k_lat [B, Sk, d_qk]    bf16    strides (k_sb, k_ss); shared by all H heads;
 *                                  V_lat is k_lat[..., :d_v]
 *   o     [B, H, Sq, d_v]  bf16    strides (o_sb, o_sh, o_ss)
 *   m, l  [B, H, Sq]       fp32    contiguous; may both be NULL (statistics not written)
 *
 *   m[b,h,i] = max_j s_ij and l[b,h,i] = sum_j exp(s_ij - m[b,h,i]) over unmasked keys j, with
 *   s_ij = softmax_scale * q_i . k_j (natural-log units, the recurrence of fa_fwd.cu:81-123).
 *   causal != 0 masks key j > i + (Sk - Sq).  A row with no unmasked key gets o = 0,
 *   m = -inf, l = 0 (the 1/l guard of fa_fwd.cu:117-118).
 *
 * Supported: d_qk = 576, d_v = 512 (DeepSeek-V3 absorbed latent shape).
 */
int dmla_fwd_cache_latent(const void* q, const void* k_lat, void* o, float* m, float* l,
                          int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t d_qk,
                          int64_t d_v, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t k_sb,
                          int64_t k_ss, int64_t o_sb, int64_t o_sh, int64_t o_ss,
                          float softmax_scale, int causal, dmla_stream_t stream);

/*
 * On-the-fly DMLA forward (prefill): per-head latent projections inside the kernel.
 * Replaces: fa2_forward (csrc/attention/fa2_fwd.cu:139-156) in the on-the-fly mode of
 * README.md:14 -- the role of the absent csrc/attention/fa2_dmla_fwd.cu (README.md:45).
 *
 *   q      [B, H, Sq, d_lat]   bf16  strides (q_sb, q_sh, q_ss)
 *   k, v   [B, Sk, H, d_in]    bf16  strides (k_sb, k_ss, k_sh), (v_sb, v_ss, v_sh)
 *   wk, wv [H, d_in, d_lat]    bf16  strides (w_sh, w_si, 1), shared by both
 *   o      [B, H, Sq, d_lat]   bf16  strides (o_sb, o_sh, o_ss)
 *   m, l   [B, H, Sq]          fp32  contiguous; may both be NULL
 *
 *   K_lat[b,h] = k[b,:,h,:] wk[h] and V_lat[b,h] = v[b,:,h,:] wv[h] inside the kernel, then
 *   o = softmax(softmax_scale q K_lat^T (+ causal mask)) V_lat with the statistics of
 *   dmla_fwd_cache_latent (natural-log units; m = -inf, l = 0, o = 0 for a row without an
 *   unmasked key).  causal != 0 masks key j > i + (Sk - Sq).
 *   Precision: the scores take q as given (bf16) against K_lat * softmax_scale * log2(e) kept
 *   as a bf16 pair hi + lo (~2^-17 relative); V_lat and the probabilities P enter the PV
 *   product as fp16 (V_lat saturates beyond |65504|).  Inputs must be finite: the kernel is
 *   built without NaN handling in its max reductions, so a NaN input gives unspecified (not
 *   necessarily NaN) outputs in the rows it reaches.
 * Supported: d_in = 128, d_lat = 64, row strides of k and v below 2^24 elements.
 */
int dmla_fwd_onthefly(const void* q, const void* k, const void* v, const void* wk, const void* wv,
                      void* o, float* m, float* l, int64_t B, int64_t H, int64_t Sq, int64_t Sk,
                      int64_t d_in, int64_t d_lat, int64_t q_sb, int64_t q_sh, int64_t q_ss,
                      int64_t k_sb, int64_t k_ss, int64_t k_sh, int64_t v_sb, int64_t v_ss,
                      int64_t v_sh, int64_t w_sh, int64_t w_si, int64_t o_sb, int64_t o_sh,
                      int64_t o_ss, float softmax_scale, int causal, dmla_stream_t stream);

/*
 * Paged-KV DMLA decode (one query token per sequence).
 * No reference counterpart exists (the reference has no paged decode); it is the decode form
 * of fa2_forward (fa2_fwd.cu:139-156) over the latent cache.
 *
 *   q             [B, H, d_qk]                 bf16  strides (q_sb, q_sh)
 *   kv_pool       [num_pages, page_size, d_qk] bf16  strides (kv_sp, kv_ss); V = [..., :d_v]
 *   block_table   [B, max_pages_per_seq]       int32 row stride bt_sb; entries in [0, num_pages)
 *   cache_seqlens [B]                          int32 context length of each sequence
 *   o             [B, H, d_v]                  bf16  strides (o_sb, o_sh)
 *   lse           [B, H]                       fp32  contiguous, natural log; may be NULL
 *
 * Sequence b attends its first cache_seqlens[b] tokens; token t lives in page
 * block_table[b, t / page_size] at row t % page_size.  Lengths above
 * max_pages_per_seq * page_size are clamped to it.  A page index outside [0, num_pages) is
 * never dereferenced: the sequence's output and lse are set to NaN instead.
 * Supported: d_qk = 576, d_v = 512, page_size = 64.
 *
 * dmla_decode_paged leaves the decode plan (the layout of dmla_decode_plan) at the head of the
 * workspace and keeps the split partials in the rest: for B <= 512 (and at most 512 ranges)
 * the decode kernel builds the plan itself and stores it there, otherwise dmla_decode_plan
 * runs first and dmla_decode_paged_planned follows.  The workspace is always required.
 */
int64_t dmla_decode_workspace_bytes(int64_t B, int64_t H, int64_t d_v, int64_t max_pages_per_seq);
int dmla_decode_paged(const void* q, const void* kv_pool, const int32_t* block_table,
                      const int32_t* cache_seqlens, void* o, float* lse, int64_t B, int64_t H,
                      int64_t d_qk, int64_t d_v, int64_t page_size, int64_t num_pages,
                      int64_t max_pages_per_seq, int64_t q_sb, int64_t q_sh, int64_t kv_sp,
                      int64_t kv_ss, int64_t bt_sb, int64_t o_sb, int64_t o_sh,
                      float softmax_scale, void* workspace, int64_t workspace_bytes,
                      dmla_stream_t stream);

/*
 * dmla_decode_paged without a workspace, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  Same arguments and results as dmla_decode_paged; the plan
 * and split partials live in a static device array of DMLA_NOALLOC_SCRATCH_BYTES per GPU
 * (held until the process ends), and a batch whose dmla_decode_workspace_bytes exceeds it is
 * rejected with DMLA_ERR_WORKSPACE.  Nothing is allocated and no memory is cleared (every byte
 * a call reads it has written first).  All calls on one GPU share that GPU's array, so calls
 * that overlap on one GPU (on different streams, or from several threads) race.
 */
#define DMLA_NOALLOC_SCRATCH_BYTES (64ll << 20)
int dmla_decode_paged_noalloc(const void* q, const void* kv_pool, const int32_t* block_table,
                              const int32_t* cache_seqlens, void* o, float* lse, int64_t B, int64_t H,
                              int64_t d_qk, int64_t d_v, int64_t page_size, int64_t num_pages,
                              int64_t max_pages_per_seq, int64_t q_sb, int64_t q_sh, int64_t kv_sp,
                              int64_t kv_ss, int64_t bt_sb, int64_t o_sb, int64_t o_sh,
                              float softmax_scale, dmla_stream_t stream);

/*
 * Decode tile-scheduler plan, computed on the device from cache_seqlens (no reference
 * counterpart; the step between the block table and the decode kernel).  The 32-token key
 * tiles of all sequences, in order, are cut into R ranges (R = CUs / head groups of 64 heads,
 * more if a range's pages could exceed 128), each processed by one workgroup per head group.
 * Every piece of a sequence inside a range is one split of it (a segment of the workgroup's
 * work); sequences with several splits are merged by the LSE combine.  A segment has a fixed
 * cost (loading Q and its first tile, writing its output) of about 16 tiles, so the ranges are
 * equal in a weighted space where each nonempty sequence is preceded by 16 virtual tiles:
 * every workgroup gets about the same work whatever the lengths.  plan (int32,
 * dmla_decode_plan_bytes bytes):
 *   [0..7]   B, R, W (weighted tiles per range), total tiles, total splits, segment cost, 0, 0
 *   then     tile_prefix[B + 1], split_base[B + 1], num_splits[B], first_range[B],
 *            range_start[R + 1], range_first_b[R]
 * A plan depends on cache_seqlens only, so one plan serves every layer of a decode step.
 */
int64_t dmla_decode_plan_bytes(int64_t B, int64_t H, int64_t max_pages_per_seq);
int dmla_decode_plan(const int32_t* cache_seqlens, int64_t B, int64_t H, int64_t max_pages_per_seq,
                     int32_t* plan, int64_t plan_bytes, dmla_stream_t stream);

/*
 * dmla_decode_paged with a precomputed plan for the same B, H, max_pages_per_seq and
 * cache_seqlens on this device.  workspace holds the split partials:
 * dmla_decode_workspace_bytes - dmla_decode_plan_bytes bytes.
 */
int dmla_decode_paged_planned(const void* q, const void* kv_pool, const int32_t* block_table,
                              const int32_t* cache_seqlens, void* o, float* lse, int64_t B, int64_t H,
                              int64_t d_qk, int64_t d_v, int64_t page_size, int64_t num_pages,
                              int64_t max_pages_per_seq, int64_t q_sb, int64_t q_sh, int64_t kv_sp,
                              int64_t kv_ss, int64_t bt_sb, int64_t o_sb, int64_t o_sh,
                              float softmax_scale, const int32_t* plan, void* workspace,
                              int64_t workspace_bytes, dmla_stream_t stream);

/*
 * Paged latent-cache append: writes new rows into the pages the decode reads.
 * No reference counterpart (the reference has no paged cache); it is the producer side of
 * dmla_decode_paged's block-table gather.
 *
 *   kv_pool      [num_pages, page_size, d] bf16  strides (kv_sp, kv_ss); written in place
 *   block_table  [B, max_pages_per_seq]    int32 row stride bt_sb
 *   cache_seqlens[B]                       int32 tokens already cached (not updated here)
 *   new_lens     [B]                       int32 rows to append per sequence (<= n_new); may be NULL
 *   new_kv       [B, n_new, d]             bf16  strides (nk_sb, nk_ss)
 *   bad_index_flag                         int32 device word; may be NULL
 *
 * Row t < new_lens[b] of sequence b goes to position p = cache_seqlens[b] + t: page
 * block_table[b, p / page_size], row p % page_size.  A row whose page slot is past
 * max_pages_per_seq or whose page index is outside [0, num_pages) is not written, and
 * *bad_index_flag is set to 1 (the caller clears it beforehand).  d must be a multiple of 8.
 */
int dmla_kv_append(void* kv_pool, const int32_t* block_table, const int32_t* cache_seqlens,
                   const int32_t* new_lens, const void* new_kv, int32_t* bad_index_flag, int64_t B,
                   int64_t n_new, int64_t d, int64_t page_size, int64_t num_pages,
                   int64_t max_pages_per_seq, int64_t kv_sp, int64_t kv_ss, int64_t bt_sb,
                   int64_t nk_sb, int64_t nk_ss, dmla_stream_t stream);

/*
 * Split-KV log-sum-exp combine, the last step of split decoding, as a standalone op.
 * No reference counterpart; dmla_decode_paged runs the same kernel on its own partials.
 *
 *   part_o   [B, S, H, d] fp32, element strides (po_sb, po_ss, po_sh), last dim contiguous;
 *            each split's output normalised over that split's keys
 *   part_lse [B, S, H]    fp32, strides (lse_sb, lse_ss, lse_sh), natural log (-inf: empty)
 *   num_splits [B]        int32 splits used per sequence (<= S); NULL = all S
 *   o        [B, H, d]    bf16, strides (o_sb, o_sh)
 *   lse      [B, H]       fp32 contiguous; may be NULL
 *
 *   o = sum_s w_s o_s / sum_s w_s with w_s = exp(lse_s - max_s lse_s), lse = max + log(sum w);
 *   a sequence whose splits all have lse = -inf gets o = 0 and lse = -inf; a NaN lse in any
 *   split makes o and lse NaN.  d % 4 == 0 and B * H < 2^31.
 */
int dmla_lse_combine(const float* part_o, const float* part_lse, const int32_t* num_splits, void* o,
                     float* lse, int64_t B, int64_t H, int64_t max_splits, int64_t d, int64_t po_sb,
                     int64_t po_ss, int64_t po_sh, int64_t lse_sb, int64_t lse_ss, int64_t lse_sh,
                     int64_t o_sb, int64_t o_sh, dmla_stream_t stream);

/*
 * Cache-latent DMLA backward from the forward's saved statistics.
 * Replaces: fa2_backward (csrc/attention/fa2_bwd.cu:319-356, math of :198-310) specialised
 * to the cache-latent mode of README.md:12,15 -- the role of the absent
 * csrc/attention/fa2_dmla_bwd.cu (README.md:46).
 *
 *   q, k_lat, o    as for dmla_fwd_cache_latent (o is the forward's output)
 *   dout   [B, H, Sq, d_v]  bf16  strides (do_sb, do_sh, do_ss)
 *   m, l   [B, H, Sq]       fp32  contiguous, exactly as dmla_fwd_cache_latent wrote them
 *   dq     [B, H, Sq, d_qk] bf16, or fp32 when dq_fp32 != 0; strides (dq_sb, dq_sh, dq_ss)
 *   dk_lat [B, Sk, d_qk]    bf16, or fp32 when dk_fp32 != 0; strides (dk_sb, dk_ss)
 *
 *   P = exp(s - m) / l, D_i = sum_d dout_i * o_i, dP = dout V^T, dS = P * (dP - D),
 *   dq = scale dS K_lat, dk_lat = scale sum_h dS^T q + [sum_h P^T dout, 0]  (the V_lat
 *   gradient folded into the first d_v columns).  Rows with l = 0 contribute nothing.
 *   S = q K^T and dP = dout V^T use the bf16 inputs as they are; dS^T q, P^T dout and dS K
 *   take fp16 operands (P and dS rounded to fp16; q, dout, K converted to fp16, exact for
 *   magnitudes in fp16's normal range, saturating above 65504).  dout and dS enter them
 *   scaled by 2^e, the power of two (e >= 0, chosen on the device) that brings the call's
 *   largest |dout| into [4, 8), and dq, dk_lat leave scaled back: small gradients keep fp16's
 *   full precision, and dout 2^-s gives exactly 2^-s times the gradients of dout.  All
 *   products accumulate in fp32.
 *   The result is deterministic (no atomics).  workspace: device memory of at least
 *   dmla_bwd_workspace_bytes(...) bytes for the same sizes on the current device, 16-byte
 *   aligned; its contents on entry do not matter.  The workspace grows linearly in Sq and Sk:
 *   dS is kept only for the (row, key) blocks that the causal mask leaves, and when that would
 *   pass DMLA_BWD_DS_CAP_BYTES (or the environment variable DMLA_BWD_DS_CAP_BYTES, read at
 *   each call) the rows are processed in chunks whose dS fits it, dk_lat accumulating in fp32
 *   across the chunks (in the workspace when dk_lat is bf16).
 *   The default cap, 2 GiB, holds a causal S = 8192 of 16 heads in one chunk (each chunk
 *   repeats the dQ kernel's K_lat^T staging and the reduction: 4.48 against 3.40 ms there
 *   under a 512 MiB cap).
 * Supported: d_qk = 576, d_v = 512.
 */
#define DMLA_BWD_DS_CAP_BYTES (2048ll << 20)
int64_t dmla_bwd_workspace_bytes(int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t d_qk,
                                 int64_t d_v, int causal);
int dmla_bwd_cache_latent(const void* q, const void* k_lat, const void* o, const void* dout,
                          const float* m, const float* l, void* dq, void* dk_lat, int64_t B,
                          int64_t H, int64_t Sq, int64_t Sk, int64_t d_qk, int64_t d_v,
                          int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t k_sb, int64_t k_ss,
                          int64_t o_sb, int64_t o_sh, int64_t o_ss, int64_t do_sb, int64_t do_sh,
                          int64_t do_ss, int64_t dq_sb, int64_t dq_sh, int64_t dq_ss,
                          int64_t dk_sb, int64_t dk_ss, int dq_fp32, int dk_fp32,
                          float softmax_scale, int causal, void* workspace,
                          int64_t workspace_bytes, dmla_stream_t stream);

/*
 * On-the-fly DMLA backward from the forward's saved statistics.
 * Replaces: fa2_backward (csrc/attention/fa2_bwd.cu:319-356, math of :198-310) in the
 * on-the-fly mode of README.md:14, whose WK / WV are learnable -- the role of the absent
 * csrc/attention/fa2_dmla_bwd.cu (README.md:46) for that mode.  The reference has no code for
 * it; the gradients are those of dmla_fwd_onthefly's math.
 *
 *   q, k, v, wk, wv, o  as for dmla_fwd_onthefly (o is the forward's output)
 *   dout   [B, H, Sq, d_lat]  bf16  strides (do_sb, do_sh, do_ss)
 *   m, l   [B, H, Sq]         fp32  contiguous, exactly as dmla_fwd_onthefly wrote them
 *   dq     [B, H, Sq, d_lat]  bf16, or fp32 when dq_fp32 != 0; strides (dq_sb, dq_sh, dq_ss)
 *   dk, dv [B, Sk, H, d_in]   bf16, or fp32 when dkv_fp32 != 0; strides (dk_sb, dk_ss, dk_sh),
 *                             shared by both
 *   dwk, dwv [H, d_in, d_lat] bf16, or fp32 when dw_fp32 != 0; strides (dw_sh, dw_si, 1),
 *                             shared by both
 *
 *   With K_lat, V_lat recomputed as in the forward, P = exp(s - m) / l, D_i = sum dout_i o_i,
 *   dS = P * (dP - D) with dP = dout V_lat^T:
 *     dq = scale dS K_lat,  dK_lat = scale dS^T q,  dV_lat = P^T dout,
 *     dk[b,:,h,:] = dK_lat[b,h] wk[h]^T,  dwk[h] = sum_b k[b,:,h,:]^T dK_lat[b,h]  (same for v).
 *   Rows with l = 0 contribute nothing.  Products accumulate in fp32.  The dK_lat / dV_lat side
 *   (and through it dk, dv, dwk, dwv) takes bf16 operands, every rounded one (K_lat, V_lat, P,
 *   dS, dK_lat, dV_lat) as a bf16 pair hi + lo (within 2^-16 relative); dq takes fp16 operands
 *   (q, dout converted exactly for magnitudes in fp16's normal range; K_lat, V_lat, dS rounded
 *   to fp16), with dout and dS scaled by the same power of two as in dmla_bwd_cache_latent
 *   and dq scaled back.  Deterministic (no atomics).  workspace: device memory of at least
 *   dmla_bwd_onthefly_workspace_bytes(...) bytes, 16-byte aligned; its contents on entry do not
 *   matter.
 * Supported: d_in = 128, d_lat = 64, 0 < Sq, Sk <= 2^24, row strides of q, dout, k, v below 2^24.
 */
int64_t dmla_bwd_onthefly_workspace_bytes(int64_t B, int64_t H, int64_t Sq, int64_t Sk,
                                          int64_t d_in, int64_t d_lat);
int dmla_bwd_onthefly(const void* q, const void* k, const void* v, const void* wk,
                      const void* wv, const void* o, const void* dout, const float* m,
                      const float* l, void* dq, void* dk, void* dv, void* dwk, void* dwv,
                      int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t d_in, int64_t d_lat,
                      int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t k_sb, int64_t k_ss,
                      int64_t k_sh, int64_t v_sb, int64_t v_ss, int64_t v_sh, int64_t w_sh,
                      int64_t w_si, int64_t o_sb, int64_t o_sh, int64_t o_ss, int64_t do_sb,
                      int64_t do_sh, int64_t do_ss, int64_t dq_sb, int64_t dq_sh, int64_t dq_ss,
                      int64_t dk_sb, int64_t dk_ss, int64_t dk_sh, int64_t dw_sh, int64_t dw_si,
                      int dq_fp32, int dkv_fp32, int dw_fp32, float softmax_scale, int causal,
                      void* workspace, int64_t workspace_bytes, dmla_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHDMLA_H */
