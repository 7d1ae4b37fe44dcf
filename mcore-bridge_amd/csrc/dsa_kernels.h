// Internal launch interface between the C-ABI layer (dsa_abi.cpp) and the HIP kernels.
// Pointers are device pointers; strides are in elements.  The C-ABI validates every field
// before a launcher is called, so the kernels may assume the documented shapes.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dsa {

typedef __bf16 bf16_t;

struct SparseFwdParams {
  const bf16_t* q;      // [total_q, n_heads, q_dim], token stride q_stride_t
  const bf16_t* kv;     // [n_kv, 576], row stride kv_stride
  const int32_t* idx;   // [total_q, topk] global kv row ids, -1 = none
  bf16_t* out;          // [total_q, n_heads, 512], token stride out_stride_t
  float* lse;           // [total_q, n_heads] natural-log LSE, token stride lse_stride_t
  int total_q, n_heads, n_kv, topk, causal;
  int n_split;          // key splits per query (1 = whole row; > 1: out/lse are [total_q*n_split]
                        // rows of normalised partials for launch_decode_combine)
  int split_keys;       // index slots per split (multiple of 32 when n_split > 1; = topk otherwise)
  int64_t q_stride_t, kv_stride, idx_stride, out_stride_t, lse_stride_t;
  float scale_log2;     // softmax scale * log2(e)
  int n_xcd;            // XCDs of the device (xcd_remap / xcd_grid)
  const float* sinks;   // [n_heads] per-head attention-sink logits (natural), or null; n_split == 1
  int q_dim;            // 576, or 512: q rows without the rope part (it counts as zero; the kv
                        // rows' rope region must then be zero too)
};

// Per-pair dKV partial rows ("G rows") of the sparse backward, written by B3 and summed per key
// by B5, in one of two formats:
//   bf16 (default): the 576 dims as bf16, 1152 bytes (for 512-wide q rows, q_dim = 512: the 512
//     latent dims, 1024 bytes; the workspace keeps the 1152-byte sizing).
//   int8 (DSA_BWD_G_INT8): 640 bytes, five 128-byte lines.  Dims are grouped by 32 (groups
//     0..15 latent, 16..17 rope), each group with its own scale s = max|g| / 127 rounded up to
//     bf16, so |g / s| <= 127; a dim is stored as u = rint(g / s) + 128 (offset binary, 1..255)
//     and read back as (u - 128) * s.  Bytes 0..511: latent dims 0..511.  Bytes 512..639: 8
//     slots of 16 bytes; slot j holds rope dims 512 + 8j .. +7 (8 bytes), then the bf16 scales
//     of groups 3j, 3j + 1, 3j + 2 (zero past group 17) and 2 zero bytes.
constexpr int kGRowBytesBf16 = 1152;
constexpr int kGRowBytesI8 = 640;

struct SparseBwdParams {
  const bf16_t* q;      // [total_q, n_heads, q_dim]; dq alike
  const bf16_t* kv;     // [n_kv, 576]
  const int32_t* idx;   // [total_q, topk]
  const bf16_t* out;    // [total_q, n_heads, 512]
  const bf16_t* dout;   // [total_q, n_heads, 512]
  const float* lse;     // [total_q, n_heads]
  bf16_t* dq;           // [total_q, n_heads, 576]
  float* dkv;           // [n_kv, 576] fp32 (fully written, no accumulation into old contents)
  // workspace (carved by the C-ABI from one caller buffer)
  bf16_t* p_stage;      // [total_q, topk_pad/32, n_heads, 32]  P (one contiguous tile per key block)
  bf16_t* ds_stage;     // [total_q, topk_pad/32, n_heads, 32]  scale * dS
  char* g_stage;        // [total_q * topk + 1] G rows (g_int8 ? kGRowBytesI8 : kGRowBytesBf16
                        // bytes each), key-major order
  int64_t g_sink_row;   // last row of g_stage: write target of pairs that select nothing
  int g_int8;           // G row format: 0 bf16, 1 int8 with per-32-dim scales
  int64_t* pair_pos;    // [total_q, topk] row of G for each pair (-1 = not selected)
  int64_t* csr_offsets; // [n_kv + 1]
  int32_t* csr_counts;  // [csr_count_entries(total_q, n_kv)] scratch of the pair ordering
  int total_q, n_heads, n_kv, topk, topk_pad, causal;
  int q_offset;         // position of row 0 (the causal test is key <= q_offset + row): a query chunk
  int dkv_accumulate;   // 1: B5 adds into dkv (the later chunks of a chunked backward)
  int64_t q_stride_t, kv_stride, idx_stride, out_stride_t, dout_stride_t, lse_stride_t, dq_stride_t, dkv_stride;
  float scale, scale_log2;
  int n_xcd;            // XCDs of the device (xcd_remap / xcd_grid)
  int q_dim;            // 576, or 512 (q and dq rows without the rope part: it counts as zero)
  float* delta_out;     // [total_q, n_heads] rowsum(dO * O) written by B1 (token stride n_heads), or null
};

struct IndexerParams {
  const void* q;        // [total_q, n_heads, head_dim] bf16 or e4m3fn
  const float* q_scale; // [total_q, n_heads] (fp8 only) or null
  const void* k;        // [n_k, head_dim] bf16 or e4m3fn
  const float* k_scale; // [n_k] (fp8 only) or null
  const float* w;       // [total_q, n_heads]
  const int32_t* row_base;  // per query: key id of score column 0
  const int32_t* row_len;   // per query: number of visible keys
  float* scores;        // [total_q, pitch]; column j <-> key row_base[t] + j
  int total_q, n_heads, head_dim, fp8, max_row_len;
  int64_t pitch;
  int fill_masked;      // also write -inf into columns [row_len, pitch)
  int chunk;            // keys per wave work item (power of two in [256, 4096]); 0 = launcher picks
};

struct TopkParams {
  const float* scores;       // [rows, pitch]
  const int32_t* row_base;   // per row: key id of column 0
  const int32_t* row_len;    // per row: number of valid columns
  int32_t* out_idx;          // [rows, topk] key ids, ascending, -1 padded
  int32_t* out_count;        // [rows] number selected, or null
  int rows, topk;
  int64_t pitch;
  // split selection of few long rows (null: one workgroup per row); set by launch_topk
  uint32_t* cand_key;        // [rows, n_slices, topk] order keys of the slices' candidates
  int32_t* cand_idx;         // [rows, n_slices, topk] their key ids
  int slice, n_slices;
  int cache_elems;           // LDS cache entries of the launch (set by launch_topk)
};

struct PrologueParams {
  const bf16_t* q_lin;  // [total_q, n_heads, 128] = wq_b(qr), token stride q_stride_t
  const bf16_t* k_lin;  // [total_q, 128] = wk(x), token stride k_stride_t
  const bf16_t* w_lin;  // [total_q, n_heads] = weights_proj(x), token stride w_stride_t
  const float* ln_w;    // [128] k_norm weight
  const float* ln_b;    // [128] k_norm bias
  const float* freqs;   // [total_q, 64] rotary angles, token stride freqs_stride_t
  void* q_out;          // [total_q, n_heads, 128] bf16 or e4m3fn
  float* q_scale;       // [total_q, n_heads] (fp8 only)
  void* k_out;          // [total_q, 128] bf16 or e4m3fn
  float* k_scale;       // [total_q] (fp8 only)
  float* w_out;         // [total_q, n_heads] fp32 (values exact in bf16)
  int total_q, n_heads, deinterleave, rotary_interleaved, out_fp8;
  float eps, mscale, w_scale_heads, w_scale_softmax;
  int64_t q_stride_t, k_stride_t, w_stride_t, freqs_stride_t;
};

struct KlTargetParams {
  const bf16_t* q;      // [total_q, n_heads, 576], token stride q_stride_t
  const bf16_t* kv;     // [n_kv, 576]
  const int32_t* idx;   // [total_q, topk]
  const float* lse;     // [total_q, n_heads] natural-log LSE of the sparse forward
  float* target;        // [total_q, topk] head-averaged probabilities (0 at invalid slots)
  int total_q, n_heads, n_kv, topk, causal;
  int64_t q_stride_t, idx_stride, lse_stride_t, target_stride;
  float scale_log2;     // softmax scale * log2(e)
  int n_xcd;            // XCDs of the device (xcd_remap / xcd_grid)
};

// Dense attention statistics of the dense indexer loss (dsa_dense_kl.hip): query t's keys are
// the kv rows row_base[t] .. row_base[t] + row_len[t] - 1.
struct DenseKlParams {
  const bf16_t* q;          // [total_q, n_heads, 576], token stride q_stride_t
  const bf16_t* kv;         // [n_kv, 576]
  const int32_t* row_base;  // [total_q]
  const int32_t* row_len;   // [total_q]
  const float* lse;         // target: [total_q, n_heads] natural-log dense LSE
  float* lse_out;           // LSE: [total_q, n_heads]
  float* target;            // target: [total_q, pitch] (row stride target_stride)
  int total_q, n_heads, n_kv, pitch;
  int64_t q_stride_t, target_stride;
  float scale_log2;         // softmax scale * log2(e)
  int n_xcd;                // XCDs of the device (xcd_remap / xcd_grid)
  // sparse target (index rows instead of key ranges): idx [total_q, pitch] kv row ids, -1 = none;
  // entries outside kv or (causal) after the query are none too
  const int32_t* idx;
  int64_t idx_stride;
  int causal;
};

struct KlFromPParams {
  const bf16_t* p_stage;  // the sparse backward's staged P tiles [total_q][topk_pad / 32][n_heads][32]
  const int32_t* idx;     // [total_q, topk]
  float* target;          // [total_q, topk]
  int total_q, n_heads, n_kv, topk, topk_pad, causal;
  int64_t idx_stride, target_stride;
};

struct KlLossParams {
  const float* index_sel;  // [total_q, topk] index scores of the selected slots
  const float* target;     // [total_q, topk]
  const int32_t* idx;      // [total_q, topk]
  float* kl;               // [total_q] per-query KL
  float* d_index;          // [total_q, topk] grad_scale * d KL_t / d index_sel (0 at invalid slots)
  int total_q, topk, n_kv, causal;
  int64_t index_stride, target_stride, idx_stride, d_stride;
  float grad_scale;
};

struct PrologueBwdParams {
  const float* dq;      // [total_q, n_heads, 128] dL/dq (prologue output)
  const float* dk;      // [total_q, 128] dL/dk
  const float* dw;      // [total_q, n_heads] dL/dw
  const bf16_t* k_lin;  // [total_q, 128], token stride k_stride_t (LayerNorm input)
  const float* ln_w;    // [128]
  const float* freqs;   // [total_q, 64], token stride freqs_stride_t
  bf16_t* dq_lin;       // [total_q, n_heads * 128], token stride dq_lin_stride_t
  bf16_t* dk_lin;       // [total_q, 128], token stride dk_lin_stride_t
  bf16_t* dw_lin;       // [total_q, n_heads], token stride dw_lin_stride_t
  float* dln_w;         // [128]
  float* dln_b;         // [128]
  float* dln_part;      // workspace: [total_q, 256] per-token rows + [64, 256] partial sums
  int total_q, n_heads, deinterleave, rotary_interleaved;
  float eps, mscale, w_scale_heads, w_scale_softmax;
  int64_t k_stride_t, freqs_stride_t, dq_lin_stride_t, dk_lin_stride_t, dw_lin_stride_t;
};

// Indexer scores of the selected slots, I[t, j] = sum_h w[t,h] relu(q[t,h] . k[idx[t,j]]), and
// their backward (bf16 q / k, head_dim 128, n_heads <= 64).
struct IdxSelParams {
  const bf16_t* q;       // [total_q, n_heads, 128], token stride q_stride_t
  const bf16_t* k;       // [n_k, 128]
  const float* w;        // [total_q, n_heads]
  const int32_t* idx;    // [total_q, topk]
  float* scores;         // forward: [total_q, topk] (-inf at invalid slots)
  const float* d_index;  // backward: [total_q, topk] dL/dI
  float* dq;             // backward: [total_q, n_heads, 128] fp32
  float* dw;             // backward: [total_q, n_heads] fp32
  float* dk;             // backward: [n_k, 128] fp32 (every row written)
  // backward workspace
  bf16_t* g_stage;       // [total_q * topk + 1, 128] per-pair dk rows in key-major order
  int64_t g_sink_row;    // last row of g_stage (pairs that select nothing)
  int64_t* pair_pos;     // [total_q, topk]
  int64_t* csr_offsets;  // [n_k + 1]
  int32_t* csr_counts;   // [csr_count_entries(total_q, n_k)]
  int total_q, n_heads, n_k, topk, causal;
  int64_t q_stride_t, idx_stride, scores_stride, d_stride;
  int n_xcd;             // XCDs of the device (xcd_remap / xcd_grid)
};

// Dense score backward (every visible key of each query, dsa_indexer_bwd.hip): query t's keys are
// the k rows row_base[t] .. row_base[t] + row_len[t] - 1, with row_base and row_base + row_len
// nondecreasing in t (document rows, decode rows, compressed-entry rows).
constexpr int kDenseDkKeys = 128;   // keys per key tile of the dk kernel
constexpr int kDenseQChunk = 256;   // queries per work item of the dk kernel
struct DenseIdxBwdParams {
  const bf16_t* q;            // [total_q, n_heads, 128]
  const bf16_t* k;            // [n_k, 128]
  const float* w;             // [total_q, n_heads]
  const int32_t* row_base;    // [total_q]
  const int32_t* row_len;     // [total_q]
  const float* d_scores;      // [total_q, pitch]: column j of row t = key row_base[t] + j
  float* dq;                  // [total_q, n_heads, 128]
  float* dw;                  // [total_q, n_heads]
  float* dk;                  // [n_k, 128]
  float* dk_part;             // [n_tiles, max_chunks, 128 keys, 128 dims] partial dk tiles
  int total_q, n_heads, n_k, pitch;
  int n_tiles, max_chunks;
  int n_xcd;
};
int launch_dense_scores_bwd(const DenseIdxBwdParams& p, hipStream_t stream);

int launch_sparse_mla_fwd(const SparseFwdParams& p, hipStream_t stream);
// ev (nullable): 6 events recorded around the stages B4 | B1 | B2 | B3 | B5.
int launch_sparse_mla_bwd(const SparseBwdParams& p, hipStream_t stream, hipEvent_t const* ev);
// B3 with int8 G rows (p.g_int8), launched by launch_sparse_mla_bwd.
void launch_bwd_g_i8(const SparseBwdParams& p, hipStream_t stream);
int launch_zero_rows(float* rows, int n_rows, int64_t stride, int width, hipStream_t stream);
int launch_indexer_scores(const IndexerParams& p, hipStream_t stream);
int launch_topk(const TopkParams& p, hipStream_t stream);
// Workspace bytes of launch_topk's split selection (cand_key + cand_idx); 0 when it is not used.
size_t topk_workspace_size(int rows, int64_t pitch, int topk);
int launch_indexer_prologue(const PrologueParams& p, hipStream_t stream);
int launch_indexer_prologue_bwd(const PrologueBwdParams& p, hipStream_t stream);
int launch_indexer_kl_target(const KlTargetParams& p, hipStream_t stream);
int launch_indexer_kl(const KlLossParams& p, hipStream_t stream);
int launch_indexer_kl_target_from_p(const KlFromPParams& p, hipStream_t stream);
int launch_dense_lse(const DenseKlParams& p, hipStream_t stream);
int launch_dense_target(const DenseKlParams& p, hipStream_t stream);
int launch_sparse_target(const DenseKlParams& p, hipStream_t stream);
int launch_indexer_selected_scores(const IdxSelParams& p, hipStream_t stream);
int launch_indexer_scores_bwd(const IdxSelParams& p, hipStream_t stream);
// Key-major order of the selected (query, slot) pairs, ascending in query inside each key
// (row t is at position t_offset + t for the causal test): csr_offsets [n_kv + 1] and the row of
// every pair, pair_pos [total_q, topk] (-1 = not
// selected); csr_counts is scratch of csr_count_entries() int32.  topk <= 4096.
// The query rows are cut into csr_groups() runs (at most 256, at most 2^24 run x key counters).
inline int csr_groups(int total_q, int n_kv) {
  const int64_t cap = (int64_t(1) << 24) / (n_kv > 0 ? n_kv : 1);
  int64_t g = total_q < 256 ? total_q : 256;
  if (g > cap) g = cap;
  return g > 0 ? (int)g : 1;
}
inline size_t csr_count_entries(int total_q, int n_kv) {
  return (size_t)(csr_groups(total_q, n_kv) + 1) * (size_t)(n_kv > 0 ? n_kv : 0);
}
void launch_pair_csr(const int32_t* idx, int64_t idx_stride, int total_q, int topk, int n_kv, int causal,
                     int t_offset, int32_t* csr_counts, int64_t* csr_offsets, int64_t* pair_pos, hipStream_t stream);
// d sinks[h] = -sum_t exp(sinks[h] - lse[t, h]) * delta[t, h] (the gradient of per-head
// attention-sink logits from the forward's sink-including LSE and B1's Delta), one fixed-order
// reduction per head.
// scratch (at least sink_grad_scratch_bytes(n_heads), or null for the one-level form) holds the
// partial sums of long batches
size_t sink_grad_scratch_bytes(int n_heads);
int launch_sink_grad(const float* sinks, const float* lse, const float* delta, int total_q, int n_heads,
                     float* dsinks, float* scratch, size_t scratch_bytes, hipStream_t stream);
int launch_decode_combine(const bf16_t* part_o, const float* part_lse, int batch, int n_heads, int n_split,
                          bf16_t* out, float* lse, hipStream_t stream);
// Static per-device scratch of the allocation-free decode entry point (64 MiB): device address of
// the current device's copy, looked up with hipGetSymbolAddress on the first call per device.
// 0 on success, -5 no usable device, -4 lookup failed.
constexpr size_t kDecodeScratchBytes = size_t(64) << 20;
int decode_scratch_address(void** out);
int launch_build_decode_rows(const int32_t* cu_cache, int batch, int32_t* row_base, int32_t* row_len,
                             hipStream_t stream);
int launch_build_rows(const int32_t* cu_seqlens, int n_seq, int total_q, int causal, int32_t* row_base,
                      int32_t* row_len, hipStream_t stream);

// DeepSeek-V4 compressor (dsa_v4_compress.hip): softmax-gated pooling of each complete window of
// `rate` tokens + RMS norm.  doc_table = device int32 [3][n_docs + 1]: token offsets, entry offsets
// (prefix sums of len / rate), backward item offsets (prefix sums of ceil(len / rate)).
struct CompressParams {
  const bf16_t* kv;         // [total_tokens, channels], row stride kv_stride
  const bf16_t* gate;       // [total_tokens, channels], row stride gate_stride
  const bf16_t* ape;        // [rate, channels]
  const bf16_t* norm_w;     // [dim]
  const int32_t* doc_table;
  int n_docs, total_tokens, n_entries, n_items, channels, dim, rate, overlap;
  float eps;
  int64_t kv_stride, gate_stride;
  bf16_t* out;              // forward: [n_entries, dim]
  const bf16_t* dout;       // backward: [n_entries, dim]
  bf16_t* dkv;              // backward: [total_tokens, channels], row stride dkv_stride
  bf16_t* dgate;            // backward: [total_tokens, channels], row stride dgate_stride
  int64_t dkv_stride, dgate_stride;
  float* dnorm_part;        // backward workspace: [bwd_wg, dim]
  float* dape_part;         // backward workspace: [ape_chunks, rate, channels]
  int32_t* entry_tok;       // backward workspace: [n_entries] first token of each entry's window
};
struct CompressBwdGrid {
  int bwd_wg, ape_chunks, entries_per_chunk;
  int64_t dnorm_floats, dape_floats;   // workspace floats of the two partial buffers
  int64_t entry_ints;                  // workspace int32 of the entry_tok row
};
CompressBwdGrid compress_bwd_grid(int n_entries, int n_items, int channels, int dim, int rate);
int launch_v4_compress_fwd(const CompressParams& p, hipStream_t stream);

// DeepSeek-V4 row transforms (dsa_v4_rope.hip): weightless RMS norm + interleaved RoPE of q rows,
// and the output's inverse RoPE written in the grouped projection's layout.
struct RopeParams {
  const bf16_t* x;      // norm_rope: rows [rows, dim] (forward input; backward: the forward's input)
                        // out_rope_group forward: o [tokens, n_heads, dim]
  const bf16_t* dout;   // norm_rope backward: [rows, dim]; out_rope_group backward: [groups, tokens, HG*dim]
  bf16_t* out;          // norm_rope forward: [rows, dim]; out_rope_group forward: [groups, tokens, HG*dim]
  bf16_t* dx;           // backward: [rows, dim]
  const float* cos;     // [tokens, angle_stride] (first rope_dim / 2 used), mscale applied
  const float* sin;
  int64_t rows, angle_stride;
  int tokens, n_heads, dim, rope_dim, groups, norm, inverse;
  float eps;
};
// which: 0 norm_rope forward, 1 norm_rope backward, 2 out_rope_group forward, 3 its backward
int launch_v4_rope(int which, const RopeParams& p, hipStream_t stream);
// dape [rate, channels] and dnorm [dim] fp32 outputs
int launch_v4_compress_bwd(const CompressParams& p, float* dape, float* dnorm, hipStream_t stream);

}  // namespace dsa
