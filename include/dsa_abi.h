/*
 * dsa_abi.h -- C ABI of libdsa_amd.so, the MI355X (gfx950) DSA sparse-attention hot path.
 *
 * The reference (maomaocun/mcore-bridge) reaches this arithmetic through Python calls into
 * Megatron-Core's DSA module; each entry point below replaces one of those calls:
 *
 *   dsa_indexer_scores + dsa_topk
 *       replace fused_qk_topk_naive(q, k, weights, index_topk, mask), called from
 *       DSAIndexer.forward_with_scores, reference src/mcore_bridge/patcher.py:349-358
 *       (returns index_scores [B,S,S] and topk_indices [B,S,min(K,S)], patcher.py:357).
 *   dsa_sparse_mla_fwd
 *       replaces the un-fused sparse attention of DSAttention, invoked through
 *       self.core_attention(...) at src/mcore_bridge/model/modules/multi_latent_attention.py:262-270.
 *   dsa_sparse_mla_bwd
 *       replaces torch autograd through that un-fused attention (the reference defines no
 *       custom backward; multi_latent_attention.py:262-270 is the forward call site).
 *   dsa_indexer_prologue (+ _bwd)
 *       replaces the tail of DSAIndexer.forward_before_topk after its projections,
 *       patcher.py:268-300 (and torch autograd through it).
 *   dsa_indexer_kl_target (+ _from_bwd), dsa_indexer_kl_loss, dsa_indexer_selected_scores (+ _bwd)
 *       replace megatron-core's compute_dsa_indexer_loss with the sparse loss (enabled by
 *       dsa_indexer_loss_coeff / dsa_indexer_use_sparse_loss, src/mcore_bridge/config/
 *       model_config.py:204-205) and torch autograd through the index scores of
 *       fused_qk_topk_naive (patcher.py:338-376) at the selected slots.
 *
 * Conventions
 *   - All pointers are device pointers on the current HIP device, except where noted.
 *   - Tensors are dense, row-major, and 16-byte aligned: q [T, H, 576] bf16, kv [N, 576] bf16,
 *     out [T, H, 512] bf16, lse [T, H] fp32 (natural log), idx [T, K] int32.
 *   - Indices are global row ids into kv (packed THD tokens, or cache rows); -1 = no key.
 *     The valid indices of one row must be distinct (a top-k never repeats a key); ids outside
 *     [0, n_kv) are treated like -1.
 *   - Documents: cu_seqlens [n_seq + 1] int32 on the device, cu[0] = 0, cu[n_seq] = T.
 *   - The caller owns every buffer, including workspaces; the library allocates no memory at
 *     run time (its one static device array, the 64 MiB scratch of
 *     dsa_sparse_mla_decode_noalloc, is reserved on each GPU when the library's code object
 *     is loaded there), keeps no pointer past the call, and launches everything on `stream`
 *     (hipStream_t, NULL = default stream) without synchronising the host.
 *   - Return 0 on success, a negative dsa_status otherwise; dsa_strerror() explains it.
 *     No C++ exception crosses the ABI.  Argument checks run before any device work, so an
 *     error return means nothing was launched.
 *   - Every entry point that launches work then checks the current device once per device:
 *     one that is not gfx950 (or no current device) gives DSA_ERR_DEVICE.  Launch shapes
 *     follow the device's compute units (the decode key splits fill them; a partitioned MI355X
 *     exposes fewer) and its XCDs (32 CUs each; the XCD-aware work order of the prefill kernels).
 */
#ifndef DSA_ABI_H_
#define DSA_ABI_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  DSA_OK = 0,
  DSA_ERR_INVALID_ARG = -1,   /* null pointer, bad shape, misaligned buffer, bad stride */
  DSA_ERR_UNSUPPORTED = -2,   /* valid request this build does not implement (e.g. d_qk != 576) */
  DSA_ERR_WORKSPACE = -3,     /* workspace missing or smaller than *_workspace_size() */
  DSA_ERR_LAUNCH = -4,        /* a kernel launch failed (HIP error) */
  DSA_ERR_DEVICE = -5,        /* no usable gfx950 device */
  DSA_ERR_SCRATCH = -6        /* request exceeds the static scratch of an allocation-free entry point */
} dsa_status;

typedef enum { DSA_BF16 = 0, DSA_FP8_E4M3 = 1 } dsa_dtype;

/* ABI version (major * 100 + minor). */
int dsa_abi_version(void);
/* Static description of a status code. */
const char* dsa_strerror(int status);

/* Per-query visible-key rows of packed prefill tokens: row_base[t] = start of t's document,
 * row_len[t] = t - start + 1 (causal) or the document length.  Feeds the indexer and top-k.
 * Replaces the dense [B,S,S] causal float mask built by DSAttention before the indexer call
 * (mask argument of fused_qk_topk_naive, patcher.py:358). */
int dsa_build_rows(const int32_t* cu_seqlens, int n_seq, int total_q, int causal,
                   int32_t* row_base, int32_t* row_len, void* stream);

/* Lightning-indexer prologue: the tail of DSAIndexer.forward_before_topk after its three
 * projections (reference src/mcore_bridge/patcher.py:268-300, RoPE helper _apply_rope
 * patcher.py:304-324 over the patched _apply_rotary_pos_emb_bshd,
 * src/mcore_bridge/model/modules/transformer_layer.py:240-278), fused into one pass:
 *   k = LayerNorm(k_lin; ln_weight, ln_bias, eps)                      (patcher.py:281-282)
 *   RoPE on dims [0, 64) of every q and k row: optional de-interleave (rope_deinterleave =
 *   dsa_indexer_rotary_interleaved), half-split or interleaved rotate_half (rotary_interleaved =
 *   config.rotary_interleaved), cos/sin of freqs scaled by mscale; bf16 rounding as the
 *   reference's bf16 ops (patcher.py:275,287)
 *   q, k = normalised 128-point Walsh-Hadamard transform (rotate_activation, patcher.py:292-293)
 *   w_out = w_lin * w_scale_heads * w_scale_softmax, rounded to bf16 after each product
 *   (patcher.py:299-300: Hi^-0.5 and softmax_scale = Di^-0.5)
 * q_lin [total_q, n_heads, 128] (token stride q_stride_t), k_lin [total_q, 128], w_lin [total_q,
 * n_heads], bf16; ln_weight, ln_bias [128] fp32; freqs [total_q, 64] fp32 rotary angles.
 * out_dtype DSA_BF16: q_out [total_q, n_heads, 128], k_out [total_q, 128] bf16.  DSA_FP8_E4M3:
 * OCP e4m3fn with one absmax scale per row, q_scale [total_q, n_heads], k_scale [total_q]
 * (x = x8 * scale, scale = absmax / 448), the fp8 input layout of dsa_indexer_scores.
 * w_out [total_q, n_heads] fp32.  n_heads <= 64, head_dim = 128, rope_dim = 64 (the reference's
 * x_pe split is its RoPE width only when head_dim = 2 * rope_dim). */
int dsa_indexer_prologue(const void* q_lin, int64_t q_stride_t, const void* k_lin, int64_t k_stride_t,
                         const void* w_lin, int64_t w_stride_t, const float* ln_weight, const float* ln_bias,
                         const float* freqs, int64_t freqs_stride_t, int total_q, int n_heads, int head_dim,
                         int rope_dim, float eps, float mscale, float w_scale_heads, float w_scale_softmax,
                         int rope_deinterleave, int rotary_interleaved, int out_dtype, void* q_out,
                         float* q_scale, void* k_out, float* k_scale, float* w_out, void* stream);

/* Workspace bytes for dsa_indexer_prologue_bwd. */
size_t dsa_indexer_prologue_bwd_workspace_size(int total_q);

/* Backward of dsa_indexer_prologue with bf16 outputs (replaces torch autograd through the tail
 * of DSAIndexer.forward_before_topk, patcher.py:268-300, and _apply_rope, patcher.py:304-324):
 * given dq [total_q, n_heads, 128], dk [total_q, 128], dw [total_q, n_heads] fp32 (gradients of
 * the prologue outputs, contiguous), writes the gradients of the projections' outputs dq_lin,
 * dk_lin, dw_lin (bf16, token strides as given) and of k_norm's weight and bias (dln_weight,
 * dln_bias [128] fp32, summed over tokens).  The forward's bf16 roundings pass the gradient
 * through unchanged (the chain rule of the exact operations); the other arguments are those of
 * the forward call. */
int dsa_indexer_prologue_bwd(const float* dq, const float* dk, const float* dw, const void* k_lin,
                             int64_t k_stride_t, const float* ln_weight, const float* freqs, int64_t freqs_stride_t,
                             int total_q, int n_heads, int head_dim, int rope_dim, float eps, float mscale,
                             float w_scale_heads, float w_scale_softmax, int rope_deinterleave,
                             int rotary_interleaved, void* dq_lin, int64_t dq_lin_stride_t, void* dk_lin,
                             int64_t dk_lin_stride_t, void* dw_lin, int64_t dw_lin_stride_t, float* dln_weight,
                             float* dln_bias, void* workspace, size_t workspace_bytes, void* stream);

/* Lightning-indexer scores (scoring half of fused_qk_topk_naive, patcher.py:358):
 *   scores[t, j] = sum_h w[t,h] * relu(q[t,h,:] . k[row_base[t] + j, :]),  j < row_len[t].
 * q [total_q, n_heads, head_dim], k [n_k, head_dim] in bf16 or OCP e4m3fn (then q_scale
 * [total_q, n_heads] and k_scale [n_k] fp32 dequantise: x = x8 * scale); w [total_q, n_heads]
 * fp32.  n_heads <= 64, head_dim in {64, 128}.  scores [total_q, pitch] fp32, pitch >=
 * max_row_len; with fill_masked the columns [row_len, pitch) are set to -inf (the reference's
 * masked layout). */
int dsa_indexer_scores(const void* q, int q_dtype, const float* q_scale, const void* k, int k_dtype,
                       const float* k_scale, const float* w, const int32_t* row_base,
                       const int32_t* row_len, int total_q, int n_k, int n_heads, int head_dim,
                       int max_row_len, float* scores, int64_t pitch, int fill_masked, void* stream);

/* Top-k selection half of fused_qk_topk_naive (patcher.py:358): for each row the min(topk,
 * row_len) largest scores (ties -> lower key), emitted as key ids row_base + j in ascending
 * order, padded with -1.  out_idx [rows, topk] int32; out_count [rows] (nullable); every
 * row_len <= pitch.  workspace (nullable, 16-byte aligned, at least dsa_topk_workspace_size
 * bytes) lets fewer than 256 rows longer than 16384 keys (decode) split each row over several
 * workgroups -- the same indices bit for bit; null keeps one workgroup per row. */
size_t dsa_topk_workspace_size(int rows, int64_t pitch, int topk);
int dsa_topk(const float* scores, int64_t pitch, const int32_t* row_base, const int32_t* row_len,
             int rows, int topk, int32_t* out_idx, int32_t* out_count, void* workspace,
             size_t workspace_bytes, void* stream);

/* Sparse MLA forward (DSAttention's un-fused sparse attention, multi_latent_attention.py:262-270),
 * absorbed MQA-latent form: out[t,h] = softmax_j(sm_scale * q[t,h] . kv[idx[t,j]]) kv[idx[t,j], :512],
 * lse[t,h] = ln sum_j exp(sm_scale * q[t,h] . kv[idx[t,j]]).  d_qk must be 576, d_v 512.
 * causal != 0 additionally ignores indices > t (the reference's triu mask).  A row without
 * a valid index yields out = 0, lse = -inf.  sm_scale must be finite and > 0 (the reference's
 * softmax scale 1/sqrt(d) * mscale^2 always is). */
int dsa_sparse_mla_fwd(const void* q, const void* kv, const int32_t* idx, int total_q, int n_kv,
                       int n_heads, int d_qk, int d_v, int topk, float sm_scale, int causal,
                       void* out, float* lse, void* stream);

/* dsa_sparse_mla_fwd with a per-head attention sink: sinks [n_heads] fp32 natural-log logits of
 * a column with no value row, out[t,h] = sum_j p_j kv[idx[t,j], :512] with p_j = exp(a_j) /
 * (sum_k exp(a_k) + exp(sinks[h])), a_j = sm_scale * q[t,h] . kv[idx[t,j]], and lse[t,h] =
 * ln(sum_k exp(a_k) + exp(sinks[h])) (a row without a valid index: out = 0, lse = sinks[h]).
 * Replaces the core attention of the reference's DeepSeek-V4 layers with its
 * core_attention.attn_sink (src/mcore_bridge/model/gpts/deepseek_v4.py:443; the layer
 * :61-328, whose core attention is megatron-core's).  sinks == NULL is dsa_sparse_mla_fwd.
 * d_qk 576, or 512 for V4's 512-wide heads: q [total_q, n_heads, 512] without a rope part, kv
 * rows still 576 wide with columns 512..575 zero (not read: the scores contract over the 512
 * latent dims). */
int dsa_sparse_mla_fwd_sink(const void* q, const void* kv, const int32_t* idx, int total_q, int n_kv,
                            int n_heads, int d_qk, int d_v, int topk, float sm_scale, int causal,
                            const float* sinks, void* out, float* lse, void* stream);

/* Decode rows for the indexer and top-k: sequence b's new token (position L_b - 1) sees its
 * whole cache, rows [cu_cache[b], cu_cache[b+1]) of the packed cache: row_base[b] = cu_cache[b],
 * row_len[b] = L_b.  cu_cache [batch + 1] int32 on the device.  No reference counterpart: the
 * reference's DSA has no KV cache (patcher.py:256 asserts no packing, deepseek_v4.py:94-95 no
 * inference); this is the decode restriction of the causal rows of dsa_build_rows. */
int dsa_build_decode_rows(const int32_t* cu_cache, int batch, int32_t* row_base, int32_t* row_len,
                          void* stream);
/* Workspace bytes for dsa_sparse_mla_decode on the current device (0 when the batch alone fills
 * the device): the key splits are sized by the device's compute units (256 on a whole MI355X;
 * without a current device, 256 is assumed). */
size_t dsa_sparse_mla_decode_workspace_size(int batch, int n_heads, int topk);
/* The same for a device of n_cu compute units (sizing ahead of time, e.g. for a partitioned
 * MI355X); 0 for n_cu < 1.  No reference counterpart (as dsa_sparse_mla_decode). */
size_t dsa_sparse_mla_decode_workspace_size_for(int batch, int n_heads, int topk, int n_cu);
/* Sparse MLA decode: one new query per sequence, q [batch, H, 576] bf16, over its selected rows
 * of the latent cache kv_cache [n_kv, 576] (idx [batch, topk] global cache row ids, -1 pad).
 * out [batch, H, 512] bf16, lse [batch, H] fp32.  Same arithmetic as dsa_sparse_mla_fwd with
 * causal = 0 (the new token sees every cached row); the selected rows are split across
 * workgroups and merged by their LSE, so a small batch still fills the device.  No reference
 * counterpart (decode is not implemented by the reference, see dsa_build_decode_rows); the
 * attention it computes is that of multi_latent_attention.py:262-270 for the last row. */
int dsa_sparse_mla_decode(const void* q, const void* kv_cache, const int32_t* idx, int batch, int n_kv,
                          int n_heads, int d_qk, int d_v, int topk, float sm_scale, void* out, float* lse,
                          void* workspace, size_t workspace_bytes, void* stream);
/* Allocation-free form of dsa_sparse_mla_decode.  No counterpart in the reference: it exists for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments minus the workspace, same kernels, split and
 * results; the split partials live in a static device array of the library,
 * dsa_sparse_mla_decode_scratch_bytes() = 64 MiB per GPU the library runs on, held until the
 * process ends.  Requests whose partials exceed it (dsa_sparse_mla_decode_workspace_size() > 64 MiB)
 * return DSA_ERR_SCRATCH; under this build's split rule the partials never exceed 65,280 rows
 * (67,107,840 bytes), so every request fits.  Calls neither allocate
 * nor free memory.  All calls on one GPU share its scratch: calls that overlap in time on one GPU
 * (different streams, or host threads without ordering) race on it. */
size_t dsa_sparse_mla_decode_scratch_bytes(void);
int dsa_sparse_mla_decode_noalloc(const void* q, const void* kv_cache, const int32_t* idx, int batch, int n_kv,
                                  int n_heads, int d_qk, int d_v, int topk, float sm_scale, void* out, float* lse,
                                  void* stream);

/* Workspace bytes for dsa_sparse_mla_bwd in one pass over all total_q query rows (the staged P
 * and dS tiles, ~4.5 KB per selected (query, key) pair of G rows and pair rows, key counters). */
size_t dsa_sparse_mla_bwd_workspace_size(int total_q, int n_kv, int n_heads, int topk);

/* Workspace bytes for dsa_sparse_mla_bwd run in passes of chunk_q query rows (rounded up to a
 * multiple of 256): a bounded workspace for long sequences.  No reference counterpart (torch
 * autograd has no workspace); for callers that must cap the backward's scratch memory. */
size_t dsa_sparse_mla_bwd_workspace_size_chunked(int total_q, int n_kv, int n_heads, int topk, int chunk_q);

/* Sparse MLA backward (autograd of dsa_sparse_mla_fwd; replaces torch autograd through the
 * un-fused attention called at multi_latent_attention.py:262-270).  Writes dq [T, H, 576] bf16
 * and dkv [n_kv, 576] fp32 (every row written; rows no query selected are zero).
 * n_heads <= 128 and a multiple of 16.  With a workspace of at least
 * dsa_sparse_mla_bwd_workspace_size() it runs in one pass; with a smaller one (at least the
 * chunked size of 256 rows) it runs in passes of the most multiples of 256 query rows that fit,
 * in query order, adding each pass's dkv into the previous ones.  dkv is the same bit for bit
 * from run to run for a given workspace size (the per-key sums run in ascending query order);
 * different pass sizes may differ in the last fp32 bits.  total_q == 0 writes dkv = 0 and
 * touches nothing else (the per-query pointers and the workspace may then be NULL). */
int dsa_sparse_mla_bwd(const void* q, const void* kv, const int32_t* idx, const void* out,
                       const void* dout, const float* lse, int total_q, int n_kv, int n_heads,
                       int d_qk, int d_v, int topk, float sm_scale, int causal, void* dq, float* dkv,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Backward of dsa_sparse_mla_fwd_sink (autograd of the same reference V4 core attention,
 * deepseek_v4.py:443): dq and dkv as dsa_sparse_mla_bwd_ex (flags: 0 or DSA_BWD_G_INT8, below)
 * given the sink forward's out and lse (its P and Delta are then the sink softmax's), plus
 * dsinks [n_heads] fp32 = -sum_t exp(sinks[h] - lse[t,h]) * rowsum(dout[t,h] * out[t,h]), a
 * fixed-order sum (the same bit for bit from run to run).  The workspace holds the rowsums
 * [total_q, n_heads] fp32 at its end and the backward's own workspace before them: at least
 * dsa_sparse_mla_bwd_sink_workspace_size() bytes for one pass (a smaller one runs the passes of
 * dsa_sparse_mla_bwd).  Unknown flags: DSA_ERR_INVALID_ARG (0 bytes from the size query).
 * d_qk 576, or 512 as for dsa_sparse_mla_fwd_sink: q and dq [total_q, n_heads, 512], kv and dkv
 * rows 576 wide (dkv columns 512..575 then come out zero). */
size_t dsa_sparse_mla_bwd_sink_workspace_size(int total_q, int n_kv, int n_heads, int topk, int flags);
int dsa_sparse_mla_bwd_sink(const void* q, const void* kv, const int32_t* idx, const void* out,
                            const void* dout, const float* lse, const float* sinks, int total_q, int n_kv,
                            int n_heads, int d_qk, int d_v, int topk, float sm_scale, int causal, void* dq,
                            float* dkv, float* dsinks, int flags, void* workspace, size_t workspace_bytes,
                            void* stream);

/* DeepSeek-V4 compressor (the compressed layers' `core_attention.compressor` and the CSA
 * indexer's compressor, parameters ape / linear_wkv / linear_wgate / norm mapped at
 * src/mcore_bridge/model/gpts/deepseek_v4.py:447-464; the module itself lives in megatron-core,
 * outside the reference): every complete window of `rate` tokens of each document becomes one
 * entry, out[e] = RMSNorm(sum_s softmax_s(gate[t_s] + ape[s]) * kv[t_s]) * norm_w, the softmax
 * per channel over the window's slots; with overlap (CSA) kv and gate are 2 * dim wide and
 * entry e pools the previous window's first halves and its own second halves (a document's
 * first window: its own only).  Pooled sums are rounded to bf16 before the norm, the normalised
 * row to bf16 before the weight (the module's dtype steps).
 *   kv, gate: [total_tokens, channels] bf16, row strides kv_stride / gate_stride (elements, even
 *     multiples of 8); channels = 2 * dim (overlap) or dim; dim in {64, 128, 256, 512};
 *   ape [rate, channels] bf16, norm_w [dim] bf16, out [n_entries, dim] bf16 (document order);
 *   doc_table: device int32 [3, n_docs + 1] -- cu_seqlens, entry offsets (prefix sums of
 *     len / rate, the last one n_entries) and item offsets (prefix sums of ceil(len / rate), the
 *     last one n_items); cu_seqlens[n_docs] = total_tokens.  A window whose rows fall outside
 *     [0, total_tokens) (a table that breaks these rules) yields a zero entry and no gradient.
 * No reference counterpart in this repository (its compressor runs in megatron-core); the
 * computation follows transformers' DeepseekV4 compressor, which the CPU oracle restates. */
int dsa_v4_compress_fwd(const void* kv, const void* gate, int64_t kv_stride, int64_t gate_stride, const void* ape,
                        const void* norm_w, const int32_t* doc_table, int n_docs, int total_tokens, int n_entries,
                        int channels, int dim, int rate, int overlap, float eps, void* out, void* stream);

/* Workspace bytes for dsa_v4_compress_bwd. */
size_t dsa_v4_compress_bwd_workspace_size(int n_entries, int n_items, int channels, int dim, int rate);

/* Backward of dsa_v4_compress_fwd given dout [n_entries, dim] bf16: dkv and dgate [total_tokens,
 * channels] bf16 (row strides dkv_stride / dgate_stride; every element of every row written,
 * zero where a token feeds no entry), dape [rate, channels] and dnorm_w [dim] fp32.  The pooling
 * is recomputed from kv and gate; deterministic (fixed-order sums, no atomics). */
int dsa_v4_compress_bwd(const void* kv, const void* gate, int64_t kv_stride, int64_t gate_stride, const void* ape,
                        const void* norm_w, const int32_t* doc_table, int n_docs, int total_tokens, int n_entries,
                        int n_items, int channels, int dim, int rate, int overlap, float eps, const void* dout,
                        void* dkv, void* dgate, int64_t dkv_stride, int64_t dgate_stride, float* dape,
                        float* dnorm_w, void* workspace, size_t workspace_bytes, void* stream);

/* DeepSeek-V4 per-head row transforms around the core attention (deepseek_v4.py:114-142, the q
 * path's weightless per-head RMS norm and RoPE; :287-318, the output's inverse RoPE and the
 * grouped output projection's [G, T, H * dim / G] view; the torch ops of those lines, one pass
 * each here).  RoPE is interleaved on the last rope_dim dims of each row: pairs (2i, 2i + 1)
 * rotate by (cos, sin)[t, i] of the row's token t (tables [tokens, angle_stride] fp32, the
 * attention mscale already applied; inverse = 1 negates sin).  dim in {64, 128, 256, 512},
 * rope_dim a multiple of 8 up to dim.
 * dsa_v4_norm_rope: x, out [rows, dim] bf16, rows = tokens * n_heads (token t = row / n_heads);
 *   norm = 1: y = bf16(x * rsqrt(mean x^2 + eps)) before the rotation, norm = 0: rotation only.
 * dsa_v4_norm_rope_bwd: dx [rows, dim] bf16 from dout (and x when norm = 1). */
int dsa_v4_norm_rope(const void* x, int64_t rows, int n_heads, int dim, int rope_dim, const float* cos,
                     const float* sin, int64_t angle_stride, int norm, float eps, int inverse, void* out,
                     void* stream);
int dsa_v4_norm_rope_bwd(const void* x, const void* dout, int64_t rows, int n_heads, int dim, int rope_dim,
                         const float* cos, const float* sin, int64_t angle_stride, int norm, float eps, int inverse,
                         void* dx, void* stream);
/* dsa_v4_out_rope_group: o [tokens, n_heads, dim] bf16 -> og [groups, tokens, (n_heads / groups) *
 *   dim] bf16 with each row rotated (inverse = 1: the output's inverse RoPE); n_heads divisible by
 *   groups.  dsa_v4_out_rope_group_bwd: d_o [tokens, n_heads, dim] from dog in og's layout. */
int dsa_v4_out_rope_group(const void* o, int tokens, int n_heads, int dim, int rope_dim, int groups,
                          const float* cos, const float* sin, int64_t angle_stride, int inverse, void* og,
                          void* stream);
int dsa_v4_out_rope_group_bwd(const void* dog, int tokens, int n_heads, int dim, int rope_dim, int groups,
                              const float* cos, const float* sin, int64_t angle_stride, int inverse, void* d_o,
                              void* stream);

/* Flags of dsa_sparse_mla_bwd_ex.
 * DSA_BWD_G_INT8: stage the per-(query, key) dKV partial rows as int8 with a bf16 scale per 32
 *   dims (640 bytes a row instead of 1152 in bf16): ~45% less of the backward's largest memory
 *   traffic and of that part of the workspace, at a larger dkv rounding error (normalised error
 *   ~0.5% against ~0.16% with bf16 rows, from the int8 steps of max|g|/127 per 32-dim group).
 *   dq is unchanged; dkv stays the same bit for bit from run to run. */
#define DSA_BWD_G_INT8 1

/* Workspace bytes for dsa_sparse_mla_bwd_ex with `flags`: chunk_q == 0 for one pass over all
 * total_q rows, else passes of chunk_q rows (rounded up to a multiple of 256).  0 for invalid
 * arguments or unknown flags. */
size_t dsa_sparse_mla_bwd_workspace_size_ex(int total_q, int n_kv, int n_heads, int topk, int chunk_q, int flags);

/* dsa_sparse_mla_bwd with flags (DSA_BWD_G_INT8 or 0) and optional per-stage timing events (see
 * dsa_sparse_mla_bwd_timed; NULL = untimed).  No reference counterpart for the flags (torch
 * autograd has no staging); flags == 0 is dsa_sparse_mla_bwd.  Unknown flags:
 * DSA_ERR_INVALID_ARG. */
int dsa_sparse_mla_bwd_ex(const void* q, const void* kv, const int32_t* idx, const void* out,
                          const void* dout, const float* lse, int total_q, int n_kv, int n_heads,
                          int d_qk, int d_v, int topk, float sm_scale, int causal, void* dq, float* dkv,
                          int flags, void* workspace, size_t workspace_bytes, void* const* stage_events,
                          void* stream);

/* dsa_sparse_mla_bwd with per-stage timing, for profilers and benchmarks (no reference
 * counterpart; the product path is dsa_sparse_mla_bwd).  stage_events: 6 hipEvent_t the caller
 * created with timing enabled, recorded on `stream` before the pair ordering, then after it and
 * after each of the score/probability, dQ, dKV-partial and dKV-reduce stages; NULL = untimed. */
int dsa_sparse_mla_bwd_timed(const void* q, const void* kv, const int32_t* idx, const void* out,
                             const void* dout, const float* lse, int total_q, int n_kv, int n_heads,
                             int d_qk, int d_v, int topk, float sm_scale, int causal, void* dq,
                             float* dkv, void* workspace, size_t workspace_bytes,
                             void* const* stage_events, void* stream);

/* ---- Indexer KL loss (dsa_indexer_loss_coeff > 0 with dsa_indexer_use_sparse_loss,
 * src/mcore_bridge/config/model_config.py:204-205; the loss itself is megatron-core's
 * compute_dsa_indexer_loss, which the reference runs through torch autograd). ---- */

/* Target of the sparse indexer loss: target[t, j] = (1/H) sum_h exp(sm_scale * q[t,h] .
 * kv[idx[t,j]] - lse[t,h]) -- the head-summed attention probability of each selected key,
 * L1-normalised -- recomputed from the sparse forward's lse.  target [total_q, topk] fp32, 0 at
 * invalid slots.  q, kv, idx, lse as for dsa_sparse_mla_fwd; n_heads <= 128; topk <= 8192. */
int dsa_indexer_kl_target(const void* q, const void* kv, const int32_t* idx, const float* lse, int total_q,
                          int n_kv, int n_heads, int d_qk, int topk, float sm_scale, int causal, float* target,
                          void* stream);

/* The same target from the workspace of a dsa_sparse_mla_bwd call that just ran on the same q,
 * kv, idx, lse (same total_q, n_kv, n_heads, topk, causal; no other call on that workspace in
 * between): its first stage recomputes P for every head and stages it in bf16, so the target is
 * the head mean of those tiles and no S product is recomputed.  Stream-ordered after that call.
 * Needs that call's one-pass workspace (dsa_sparse_mla_bwd_workspace_size() bytes): a chunked
 * backward keeps only its last pass's tiles (DSA_ERR_WORKSPACE). */
int dsa_indexer_kl_target_from_bwd(const void* bwd_workspace, size_t bwd_workspace_bytes, const int32_t* idx,
                                   int total_q, int n_kv, int n_heads, int topk, int causal, float* target,
                                   void* stream);

/* ---- Dense indexer loss statistics (dsa_indexer_loss_coeff > 0 with
 * dsa_indexer_use_sparse_loss = False, the reference default, src/mcore_bridge/config/
 * model_config.py:204-205: megatron-core's compute_dsa_indexer_loss targets the head-summed dense
 * attention of each query over every key of its document).  Query t's keys are the kv rows
 * row_base[t] .. row_base[t] + row_len[t] - 1 (dsa_build_rows; a row with row_base outside kv is
 * empty, lengths are clipped to kv).  q [total_q, n_heads, 576] bf16, kv [n_kv, 576] bf16;
 * n_heads <= 128; any row length (no index row). ---- */

/* lse[t, h] = ln sum_j exp(sm_scale * q[t,h] . kv[row_base[t] + j]) over the query's keys (-inf
 * for an empty row), [total_q, n_heads] fp32. */
int dsa_dense_attention_lse(const void* q, const void* kv, const int32_t* row_base, const int32_t* row_len,
                            int total_q, int n_kv, int n_heads, int d_qk, float sm_scale, float* lse, void* stream);

/* target[t, j] = (1/H) sum_h exp(sm_scale * q[t,h] . kv[row_base[t] + j] - lse[t,h]) for j <
 * min(row_len[t], pitch), 0 for the other j < pitch; [total_q, pitch] fp32, lse from
 * dsa_dense_attention_lse. */
int dsa_dense_attention_target(const void* q, const void* kv, const float* lse, const int32_t* row_base,
                               const int32_t* row_len, int total_q, int n_kv, int n_heads, int d_qk, int pitch,
                               float sm_scale, float* target, void* stream);

/* Backward of the dense index scores (the [B, S, S] scores of fused_qk_topk_naive, patcher.py:338-376,
 * over every visible key, through which the dense indexer loss trains the indexer; the reference
 * runs torch autograd through them): with I[t, j] = sum_h w[t,h] relu(q[t,h] . k[row_base[t] + j])
 * and d_scores [total_q, pitch] = dL/dI (columns j >= min(row_len[t], pitch) are ignored),
 *   dq[t,h] = w[t,h] sum_j dI 1[z>0] k,   dw[t,h] = sum_j dI relu(z),
 *   dk[s]   = sum over (t, h) seeing s of dI w[t,h] 1[z>0] q[t,h]                     (all fp32).
 * Rows as for dsa_dense_attention_lse (k [n_k, 128]), and monotone: row_base[t] and row_base[t] +
 * row_len[t] nondecreasing in t (what dsa_build_rows and dsa_build_decode_rows give).  q
 * [total_q, n_heads, 128] bf16, w [total_q, n_heads] fp32; n_heads <= 64.  Deterministic (no
 * atomics: per-chunk partial dk tiles in the workspace, summed in a fixed order). */
size_t dsa_dense_indexer_scores_bwd_workspace_size(int total_q, int n_k);
int dsa_dense_indexer_scores_bwd(const void* q, const void* k, const float* w, const int32_t* row_base,
                                 const int32_t* row_len, int total_q, int n_k, int n_heads, int head_dim,
                                 const float* d_scores, int pitch, float* dq, float* dw, float* dk, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* Per-query KL of the sparse indexer loss and its gradient: with pI = softmax of index_sel over
 * the valid slots of row t, kl[t] = sum_j target (ln(target + 1e-10) - ln(pI + 1e-10)) and
 * d_index[t, j] = grad_scale * d kl[t] / d index_sel[t, j] (0 at invalid slots).  The loss of the
 * reference is coeff * mean_t kl[t]: pass grad_scale = coeff * dL / total_q. */
int dsa_indexer_kl_loss(const float* index_sel, const float* target, const int32_t* idx, int total_q, int n_kv,
                        int topk, int causal, float grad_scale, float* kl, float* d_index, void* stream);

/* Indexer scores of the selected slots (the values fused_qk_topk_naive, patcher.py:338-376,
 * scores at the keys its top-k keeps): scores[t, j] = sum_h w[t,h] relu(q[t,h] . k[idx[t,j]]),
 * -inf at invalid slots.  q [total_q, n_heads, 128] bf16, k [n_k, 128] bf16, w [total_q,
 * n_heads] fp32 (the prologue's w_out), idx [total_q, topk]; n_heads <= 64, topk <= 4096. */
int dsa_indexer_selected_scores(const void* q, const void* k, const float* w, const int32_t* idx, int total_q,
                                int n_k, int n_heads, int head_dim, int topk, int causal, float* scores,
                                void* stream);

/* Workspace bytes for dsa_indexer_scores_bwd. */
size_t dsa_indexer_scores_bwd_workspace_size(int total_q, int n_k, int topk);

/* Backward of dsa_indexer_selected_scores (replaces torch autograd through the indexer scores
 * of patcher.py:338-376 for the selected slots) given d_index = dL/dscores [total_q, topk]:
 * dq [total_q, n_heads, 128] fp32, dw [total_q, n_heads] fp32, dk [n_k, 128] fp32 (every row
 * written; rows no query selected are zero).  Shapes and limits as for the forward.
 * total_q == 0 writes dk = 0 and touches nothing else (the other pointers and the workspace
 * may then be NULL). */
int dsa_indexer_scores_bwd(const void* q, const void* k, const float* w, const int32_t* idx, const float* d_index,
                           int total_q, int n_k, int n_heads, int head_dim, int topk, int causal, float* dq,
                           float* dw, float* dk, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSA_ABI_H_ */
