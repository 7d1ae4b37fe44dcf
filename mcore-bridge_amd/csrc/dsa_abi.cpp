// C-ABI entry points of libdsa_amd.so: argument validation, workspace carving, launch.
// Declarations and the reference interfaces they replace: include/dsa_abi.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <mutex>

#include "../../include/dsa_abi.h"
#include "dsa_kernels.h"

namespace {

constexpr int kDqk = 576;
constexpr int kDv = 512;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
int topk_pad(int topk) { return (topk + 31) / 32 * 32; }

size_t align_up(size_t x) { return (x + 255) / 256 * 256; }

struct BwdLayout {
  size_t p_stage, ds_stage, g_stage, pair_pos, offsets, counts, total;
};

// G row bytes of a backward's flags (format: dsa_kernels.h)
size_t g_row_bytes(int flags) { return (flags & DSA_BWD_G_INT8) ? dsa::kGRowBytesI8 : dsa::kGRowBytesBf16; }

BwdLayout bwd_layout(int total_q, int n_kv, int n_heads, int topk, int flags = 0) {
  BwdLayout L{};
  const size_t stage = align_up(sizeof(uint16_t) * (size_t)total_q * n_heads * topk_pad(topk));
  size_t off = 0;
  L.p_stage = off; off += stage;
  L.ds_stage = off; off += stage;
  L.g_stage = off; off += align_up(g_row_bytes(flags) * ((size_t)total_q * topk + 1));
  L.pair_pos = off; off += align_up(sizeof(int64_t) * (size_t)total_q * topk);
  L.offsets = off; off += align_up(sizeof(int64_t) * ((size_t)n_kv + 1));
  L.counts = off; off += align_up(sizeof(int32_t) * dsa::csr_count_entries(total_q, n_kv));
  L.total = off;
  return L;
}

// Query rows per pass of the sparse backward for a workspace of `bytes`: total_q when the whole
// layout fits, else the most whole units of kBwdChunkUnit rows whose layout fits (0: none).
constexpr int kBwdChunkUnit = 256;
int bwd_chunk_rows(int total_q, int n_kv, int n_heads, int topk, size_t bytes, int flags) {
  if (bwd_layout(total_q, n_kv, n_heads, topk, flags).total <= bytes) return total_q;
  int lo = 0, hi = total_q / kBwdChunkUnit;   // units; layouts grow with the rows
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (bwd_layout(mid * kBwdChunkUnit, n_kv, n_heads, topk, flags).total <= bytes) lo = mid;
    else hi = mid - 1;
  }
  return lo * kBwdChunkUnit;
}

struct IdxBwdLayout {
  size_t g_stage, pair_pos, offsets, counts, total;
};

IdxBwdLayout idx_bwd_layout(int total_q, int n_k, int topk) {
  IdxBwdLayout L{};
  size_t off = 0;
  L.g_stage = off; off += align_up(sizeof(uint16_t) * ((size_t)total_q * topk + 1) * 128);
  L.pair_pos = off; off += align_up(sizeof(int64_t) * (size_t)total_q * topk);
  L.offsets = off; off += align_up(sizeof(int64_t) * ((size_t)n_k + 1));
  L.counts = off; off += align_up(sizeof(int32_t) * dsa::csr_count_entries(total_q, n_k));
  L.total = off;
  return L;
}

// The current device as the launches need it: a gfx950 check, its compute units (the decode
// key splits fill them) and its XCDs (the XCD-aware grids), looked up once per device.  An
// MI355X exposes 256 CUs in 8 XCDs of 32; a partitioned one (CPX / DPX modes) fewer of both.
struct DeviceInfo {
  int status;   // DSA_OK, or DSA_ERR_DEVICE when there is no current device or it is not gfx950
  int n_cu, n_xcd;
};
constexpr int kMaxDevices = 64;
constexpr int kCusPerXcd = 32;
constexpr int kDefaultCus = 256;   // sizing queries on a host without a device
std::mutex g_dev_mu;
DeviceInfo g_dev[kMaxDevices];
bool g_dev_known[kMaxDevices];

int xcds_of(int n_cu) {
  int x = 1;
  while (x < 8 && 2 * x * kCusPerXcd <= n_cu) x *= 2;
  return x;
}

DeviceInfo current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();   // leave no sticky error behind for the caller's next HIP call
    return DeviceInfo{DSA_ERR_DEVICE, 0, 0};
  }
  std::lock_guard<std::mutex> lock(g_dev_mu);
  if (!g_dev_known[dev]) {
    hipDeviceProp_t prop;
    DeviceInfo d{DSA_ERR_DEVICE, 0, 0};
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess && std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 &&
        prop.multiProcessorCount > 0) {
      d = DeviceInfo{DSA_OK, prop.multiProcessorCount, xcds_of(prop.multiProcessorCount)};
    } else {
      (void)hipGetLastError();
    }
    g_dev[dev] = d;
    g_dev_known[dev] = true;
  }
  return g_dev[dev];
}

// CU count that sizes the decode splits: the current device's, or kDefaultCus without one.
int sizing_cus() {
  const DeviceInfo d = current_device();
  return d.status == DSA_OK ? d.n_cu : kDefaultCus;
}

// Decode key splits: enough (sequence, split) work items to give every CU one workgroup
// (the forward kernel holds one workgroup per CU), at least 4 key blocks of 32 per split.
struct DecodeSplit {
  int n_split, split_keys;
};

DecodeSplit decode_split(int batch, int n_heads, int topk, int n_cu) {
  const int items = batch * ((n_heads + 127) / 128);
  const int blocks = (topk + 31) / 32;
  int n = (std::max(n_cu, 1) + items - 1) / items;
  n = std::max(1, std::min(n, blocks / 4));
  const int per = (blocks + n - 1) / n;                 // blocks per split
  return DecodeSplit{(blocks + per - 1) / per, per * 32};
}

size_t decode_workspace(int batch, int n_heads, int topk, int n_cu) {
  const DecodeSplit d = decode_split(batch, n_heads, topk, n_cu);
  if (d.n_split == 1) return 0;
  const size_t rows = (size_t)batch * d.n_split * n_heads;
  return align_up(rows * kDv * sizeof(uint16_t)) + align_up(rows * sizeof(float));
}

}  // namespace

// Every entry point that launches work checks the current device first (after its argument
// checks, so invalid arguments are reported the same with or without a device).
#define DSA_CHECK_DEVICE(dev)              \
  const DeviceInfo dev = current_device(); \
  if (dev.status != DSA_OK) return dev.status

extern "C" {

int dsa_abi_version(void) { return 101; }

const char* dsa_strerror(int status) {
  switch (status) {
    case DSA_OK: return "ok";
    case DSA_ERR_INVALID_ARG: return "invalid argument (null pointer, shape, alignment or stride)";
    case DSA_ERR_UNSUPPORTED: return "unsupported configuration for this build";
    case DSA_ERR_WORKSPACE: return "workspace missing or too small";
    case DSA_ERR_LAUNCH: return "kernel launch failed";
    case DSA_ERR_DEVICE: return "no usable gfx950 device";
    case DSA_ERR_SCRATCH:
      return "request needs more than the static scratch of the allocation-free entry point "
             "(dsa_sparse_mla_decode_scratch_bytes); use the workspace form";
    default: return "unknown dsa status";
  }
}

int dsa_build_rows(const int32_t* cu_seqlens, int n_seq, int total_q, int causal, int32_t* row_base,
                   int32_t* row_len, void* stream) {
  if (n_seq < 1 || total_q < 0) return DSA_ERR_INVALID_ARG;
  if (total_q == 0) return DSA_OK;
  if (!cu_seqlens || !row_base || !row_len) return DSA_ERR_INVALID_ARG;
  DSA_CHECK_DEVICE(dev);
  return dsa::launch_build_rows(cu_seqlens, n_seq, total_q, causal, row_base, row_len, as_stream(stream));
}

int dsa_indexer_prologue(const void* q_lin, int64_t q_stride_t, const void* k_lin, int64_t k_stride_t,
                         const void* w_lin, int64_t w_stride_t, const float* ln_weight, const float* ln_bias,
                         const float* freqs, int64_t freqs_stride_t, int total_q, int n_heads, int head_dim,
                         int rope_dim, float eps, float mscale, float w_scale_heads, float w_scale_softmax,
                         int rope_deinterleave, int rotary_interleaved, int out_dtype, void* q_out,
                         float* q_scale, void* k_out, float* k_scale, float* w_out, void* stream) {
  if (total_q < 0 || n_heads < 1 || !(eps >= 0.f) || !std::isfinite(mscale) || !std::isfinite(w_scale_heads) ||
      !std::isfinite(w_scale_softmax))
    return DSA_ERR_INVALID_ARG;
  if (n_heads > 64 || head_dim != 128 || rope_dim != 64) return DSA_ERR_UNSUPPORTED;
  if (out_dtype != DSA_BF16 && out_dtype != DSA_FP8_E4M3) return DSA_ERR_UNSUPPORTED;
  const bool fp8 = out_dtype == DSA_FP8_E4M3;
  if (total_q == 0) return DSA_OK;
  if (!q_lin || !k_lin || !w_lin || !ln_weight || !ln_bias || !freqs || !q_out || !k_out || !w_out)
    return DSA_ERR_INVALID_ARG;
  if (fp8 && (!q_scale || !k_scale)) return DSA_ERR_INVALID_ARG;
  // rows are read and written as 2-element words
  if (q_stride_t < (int64_t)n_heads * head_dim || k_stride_t < head_dim || w_stride_t < n_heads ||
      freqs_stride_t < rope_dim || (q_stride_t & 1) || (k_stride_t & 1))
    return DSA_ERR_INVALID_ARG;
  auto al4 = [](const void* x) { return (reinterpret_cast<uintptr_t>(x) & 3u) == 0; };
  if (!al4(q_lin) || !al4(k_lin) || !al4(q_out) || !al4(k_out)) return DSA_ERR_INVALID_ARG;
  dsa::PrologueParams p{};
  p.q_lin = static_cast<const dsa::bf16_t*>(q_lin);
  p.k_lin = static_cast<const dsa::bf16_t*>(k_lin);
  p.w_lin = static_cast<const dsa::bf16_t*>(w_lin);
  p.ln_w = ln_weight; p.ln_b = ln_bias; p.freqs = freqs;
  p.q_out = q_out; p.q_scale = q_scale; p.k_out = k_out; p.k_scale = k_scale; p.w_out = w_out;
  p.total_q = total_q; p.n_heads = n_heads;
  p.deinterleave = rope_deinterleave ? 1 : 0; p.rotary_interleaved = rotary_interleaved ? 1 : 0;
  p.out_fp8 = fp8 ? 1 : 0;
  p.eps = eps; p.mscale = mscale; p.w_scale_heads = w_scale_heads; p.w_scale_softmax = w_scale_softmax;
  p.q_stride_t = q_stride_t; p.k_stride_t = k_stride_t; p.w_stride_t = w_stride_t; p.freqs_stride_t = freqs_stride_t;
  DSA_CHECK_DEVICE(dev);
  return dsa::launch_indexer_prologue(p, as_stream(stream));
}

size_t dsa_indexer_prologue_bwd_workspace_size(int total_q) {
  if (total_q < 0) return 0;
  return sizeof(float) * ((size_t)total_q + 64) * 256;
}

int dsa_indexer_prologue_bwd(const float* dq, const float* dk, const float* dw, const void* k_lin,
                             int64_t k_stride_t, const float* ln_weight, const float* freqs, int64_t freqs_stride_t,
                             int total_q, int n_heads, int head_dim, int rope_dim, float eps, float mscale,
                             float w_scale_heads, float w_scale_softmax, int rope_deinterleave,
                             int rotary_interleaved, void* dq_lin, int64_t dq_lin_stride_t, void* dk_lin,
                             int64_t dk_lin_stride_t, void* dw_lin, int64_t dw_lin_stride_t, float* dln_weight,
                             float* dln_bias, void* workspace, size_t workspace_bytes, void* stream) {
  if (total_q < 0 || n_heads < 1 || !(eps >= 0.f) || !std::isfinite(mscale) || !std::isfinite(w_scale_heads) ||
      !std::isfinite(w_scale_softmax))
    return DSA_ERR_INVALID_ARG;
  if (n_heads > 64 || head_dim != 128 || rope_dim != 64) return DSA_ERR_UNSUPPORTED;
  if (!ln_weight || !dln_weight || !dln_bias) return DSA_ERR_INVALID_ARG;
  if (total_q > 0 && (!dq || !dk || !dw || !k_lin || !freqs || !dq_lin || !dk_lin || !dw_lin))
    return DSA_ERR_INVALID_ARG;
  if (k_stride_t < head_dim || freqs_stride_t < rope_dim || dq_lin_stride_t < (int64_t)n_heads * head_dim ||
      dk_lin_stride_t < head_dim || dw_lin_stride_t < n_heads || (k_stride_t & 1) || (dq_lin_stride_t & 1) ||
      (dk_lin_stride_t & 1))
    return DSA_ERR_INVALID_ARG;
  auto al8 = [](const void* x) { return (reinterpret_cast<uintptr_t>(x) & 7u) == 0; };
  auto al4 = [](const void* x) { return (reinterpret_cast<uintptr_t>(x) & 3u) == 0; };
  if (!al8(dq) || !al8(dk) || !al4(k_lin) || !al4(dq_lin) || !al4(dk_lin)) return DSA_ERR_INVALID_ARG;
  if (!workspace || workspace_bytes < dsa_indexer_prologue_bwd_workspace_size(total_q) || !al8(workspace))
    return DSA_ERR_WORKSPACE;
  dsa::PrologueBwdParams p{};
  p.dq = dq; p.dk = dk; p.dw = dw;
  p.k_lin = static_cast<const dsa::bf16_t*>(k_lin);
  p.ln_w = ln_weight; p.freqs = freqs;
  p.dq_lin = static_cast<dsa::bf16_t*>(dq_lin);
  p.dk_lin = static_cast<dsa::bf16_t*>(dk_lin);
  p.dw_lin = static_cast<dsa::bf16_t*>(dw_lin);
  p.dln_w = dln_weight; p.dln_b = dln_bias;
  p.dln_part = static_cast<float*>(workspace);
  p.total_q = total_q; p.n_heads = n_heads;
  p.deinterleave = rope_deinterleave ? 1 : 0; p.rotary_interleaved = rotary_interleaved ? 1 : 0;
  p.eps = eps; p.mscale = mscale; p.w_scale_heads = w_scale_heads; p.w_scale_softmax = w_scale_softmax;
  p.k_stride_t = k_stride_t; p.freqs_stride_t = freqs_stride_t; p.dq_lin_stride_t = dq_lin_stride_t;
  p.dk_lin_stride_t = dk_lin_stride_t; p.dw_lin_stride_t = dw_lin_stride_t;
  DSA_CHECK_DEVICE(dev);
  return dsa::launch_indexer_prologue_bwd(p, as_stream(stream));
}

int dsa_indexer_scores(const void* q, int q_dtype, const float* q_scale, const void* k, int k_dtype,
                       const float* k_scale, const float* w, const int32_t* row_base, const int32_t* row_len,
                       int total_q, int n_k, int n_heads, int head_dim, int max_row_len, float* scores,
                       int64_t pitch, int fill_masked, void* stream) {
  if (total_q < 0 || n_k < 0 || n_heads < 1 || max_row_len < 0 || pitch < max_row_len) return DSA_ERR_INVALID_ARG;
  if (total_q == 0) return DSA_OK;
  if (!q || !k || !w || !row_base || !row_len || !scores) return DSA_ERR_INVALID_ARG;
  if (q_dtype != k_dtype || (q_dtype != DSA_BF16 && q_dtype != DSA_FP8_E4M3)) return DSA_ERR_UNSUPPORTED;
  const bool fp8 = q_dtype == DSA_FP8_E4M3;
  if (fp8 && (!q_scale || !k_scale)) return DSA_ERR_INVALID_ARG;
  if (n_heads > 64 || (head_dim != 64 && head_dim != 128)) return DSA_ERR_UNSUPPORTED;
  if (!aligned16(q) || !aligned16(k)) return DSA_ERR_INVALID_ARG;
  dsa::IndexerParams p{};
  p.q = q; p.q_scale = q_scale; p.k = k; p.k_scale = k_scale; p.w = w;
  p.row_base = row_base; p.row_len = row_len; p.scores = scores;
  p.total_q = total_q; p.n_heads = n_heads; p.head_dim = head_dim; p.fp8 = fp8 ? 1 : 0;
  p.max_row_len = max_row_len; p.pitch = pitch; p.fill_masked = fill_masked ? 1 : 0;
  DSA_CHECK_DEVICE(dev);
  return dsa::launch_indexer_scores(p, as_stream(stream));
}

size_t dsa_topk_workspace_size(int rows, int64_t pitch, int topk) {
  return dsa::topk_workspace_size(rows, pitch, topk);
}

int dsa_topk(const float* scores, int64_t pitch, const int32_t* row_base, const int32_t* row_len, int rows,
             int topk, int32_t* out_idx, int32_t* out_count, void* workspace, size_t workspace_bytes,
             void* stream) {
  if (rows < 0 || topk < 1 || pitch < 0) return DSA_ERR_INVALID_ARG;
  if (rows == 0) return DSA_OK;
  if (!scores || !row_base || !row_len || !out_idx) return DSA_ERR_INVALID_ARG;
  dsa::TopkParams p{};
  p.scores = scores; p.row_base = row_base; p.row_len = row_len; p.out_idx = out_idx; p.out_count = out_count;
  p.rows = rows; p.topk = topk; p.pitch = pitch;
  const size_t ws = dsa::topk_workspace_size(rows, pitch, topk);
  if (workspace && ws > 0) {
    if (workspace_bytes < ws || !aligned16(workspace)) return DSA_ERR_WORKSPACE;
    const size_t n = ws / (sizeof(uint32_t) + sizeof(int32_t));
    p.cand_key = static_cast<uint32_t*>(workspace);
    p.cand_idx = reinterpret_cast<int32_t*>(p.cand_key + n);
  }
  DSA_CHECK_DEVICE(dev);
  return dsa::launch_topk(p, as_stream(stream));
}

int dsa_sparse_mla_fwd(const void* q, const void* kv, const int32_t* idx, int total_q, int n_kv, int n_heads,
                       int d_qk, int d_v, int topk, float sm_scale, int causal, void* out, float* lse,
                       void* stream) {
  if (d_qk != kDqk) return DSA_ERR_UNSUPPORTED;
  return dsa_sparse_mla_fwd_sink(q, kv, idx, total_q, n_kv, n_heads, d_qk, d_v, topk, sm_scale, causal, nullptr,
                                 out, lse, stream);
}

int dsa_sparse_mla_fwd_sink(const void* q, const void* kv, const int32_t* idx, int total_q, int n_kv, int n_heads,
                            int d_qk, int d_v, int topk, float sm_scale, int causal, const float* sinks, void* out,
                            float* lse, void* stream) {
  if (total_q < 0 || n_kv < 0 || n_heads < 1 || topk < 1 || !std::isfinite(sm_scale) || !(sm_scale > 0.f))
    return DSA_ERR_INVALID_ARG;
  if ((d_qk != kDqk && d_qk != kDv) || d_v != kDv) return DSA_ERR_UNSUPPORTED;
  if (total_q == 0) return DSA_OK;
  if (!q || !kv || !idx || !out || !lse || n_kv < 1) return DSA_ERR_INVALID_ARG;
  if (!aligned16(q) || !aligned16(kv) || !aligned16(out)) return DSA_ERR_INVALID_ARG;
  dsa::SparseFwdParams p{};
  p.q_dim = d_qk;   // 512: q rows without the rope part
  p.q = static_cast<const dsa::bf16_t*>(q);
  p.kv = static_cast<const dsa::bf16_t*>(kv);
  p.idx = idx;
  p.out = static_cast<dsa::bf16_t*>(out);
  p.lse = lse;
  p.total_q = total_q; p.n_heads = n_heads; p.n_kv = n_kv; p.topk = topk; p.causal = causal ? 1 : 0;
  p.n_split = 1; p.split_keys = topk;
  p.q_stride_t = (int64_t)n_heads * d_qk; p.kv_stride = kDqk; p.idx_stride = topk;
  p.out_stride_t = (int64_t)n_heads * kDv; p.lse_stride_t = n_heads;
  p.scale_log2 = sm_scale * 1.4426950408889634f;
  p.sinks = sinks;
  DSA_CHECK_DEVICE(dev);
  p.n_xcd = dev.n_xcd;
  return dsa::launch_sparse_mla_fwd(p, as_stream(stream));
}

int dsa_build_decode_rows(const int32_t* cu_cache, int batch, int32_t* row_base, int32_t* row_len, void* stream) {
  if (batch < 0) return DSA_ERR_INVALID_ARG;
  if (batch == 0) return DSA_OK;
  if (!cu_cache || !row_base || !row_len) return DSA_ERR_INVALID_ARG;
  DSA_CHECK_DEVICE(dev);
  return dsa::launch_build_decode_rows(cu_cache, batch, row_base, row_len, as_stream(stream));
}

size_t dsa_sparse_mla_decode_workspace_size(int batch, int n_heads, int topk) {
  if (batch < 0 || n_heads < 1 || topk < 1) return 0;
  return decode_workspace(batch, n_heads, topk, sizing_cus());
}

size_t dsa_sparse_mla_decode_workspace_size_for(int batch, int n_heads, int topk, int n_cu) {
  if (batch < 0 || n_heads < 1 || topk < 1 || n_cu < 1) return 0;
  return decode_workspace(batch, n_heads, topk, n_cu);
}

int dsa_sparse_mla_decode(const void* q, const void* kv_cache, const int32_t* idx, int batch, int n_kv,
                          int n_heads, int d_qk, int d_v, int topk, float sm_scale, void* out, float* lse,
                          void* workspace, size_t workspace_bytes, void* stream) {
  if (batch < 0 || n_kv < 0 || n_heads < 1 || topk < 1 || !std::isfinite(sm_scale) || !(sm_scale > 0.f))
    return DSA_ERR_INVALID_ARG;
  if (d_qk != kDqk || d_v != kDv) return DSA_ERR_UNSUPPORTED;
  if (batch == 0) return DSA_OK;
  if (!q || !kv_cache || !idx || !out || !lse || n_kv < 1) return DSA_ERR_INVALID_ARG;
  if (!aligned16(q) || !aligned16(kv_cache) || !aligned16(out)) return DSA_ERR_INVALID_ARG;
  const int n_cu = sizing_cus();
  const DecodeSplit d = decode_split(batch, n_heads, topk, n_cu);
  const size_t need = decode_workspace(batch, n_heads, topk, n_cu);
  if (need > 0 && (!workspace || workspace_bytes < need || !aligned16(workspace))) return DSA_ERR_WORKSPACE;
  DSA_CHECK_DEVICE(dev);
  dsa::SparseFwdParams p{};
  p.n_xcd = dev.n_xcd;
  p.q = static_cast<const dsa::bf16_t*>(q);
  p.kv = static_cast<const dsa::bf16_t*>(kv_cache);
  p.idx = idx;
  p.total_q = batch; p.n_heads = n_heads; p.n_kv = n_kv; p.topk = topk; p.causal = 0;
  p.n_split = d.n_split; p.split_keys = d.n_split == 1 ? topk : d.split_keys;
  p.q_stride_t = (int64_t)n_heads * kDqk; p.kv_stride = kDqk; p.idx_stride = topk;
  p.out_stride_t = (int64_t)n_heads * kDv; p.lse_stride_t = n_heads;
  p.scale_log2 = sm_scale * 1.4426950408889634f;
  if (d.n_split == 1) {
    p.out = static_cast<dsa::bf16_t*>(out);
    p.lse = lse;
    return dsa::launch_sparse_mla_fwd(p, as_stream(stream));
  }
  char* ws = static_cast<char*>(workspace);
  const size_t rows = (size_t)batch * d.n_split * n_heads;
  dsa::bf16_t* part_o = reinterpret_cast<dsa::bf16_t*>(ws);
  float* part_lse = reinterpret_cast<float*>(ws + align_up(rows * kDv * sizeof(uint16_t)));
  p.out = part_o;
  p.lse = part_lse;
  int rc = dsa::launch_sparse_mla_fwd(p, as_stream(stream));
  if (rc != 0) return rc;
  return dsa::launch_decode_combine(part_o, part_lse, batch, n_heads, d.n_split, static_cast<dsa::bf16_t*>(out),
                                    lse, as_stream(stream));
}

size_t dsa_sparse_mla_decode_scratch_bytes(void) { return dsa::kDecodeScratchBytes; }

int dsa_sparse_mla_decode_noalloc(const void* q, const void* kv_cache, const int32_t* idx, int batch, int n_kv,
                                  int n_heads, int d_qk, int d_v, int topk, float sm_scale, void* out, float* lse,
                                  void* stream) {
  if (batch < 0 || n_kv < 0 || n_heads < 1 || topk < 1 || !std::isfinite(sm_scale) || !(sm_scale > 0.f))
    return DSA_ERR_INVALID_ARG;
  if (d_qk != kDqk || d_v != kDv) return DSA_ERR_UNSUPPORTED;
  if (batch == 0) return DSA_OK;
  const size_t need = decode_workspace(batch, n_heads, topk, sizing_cus());
  if (need > dsa::kDecodeScratchBytes) return DSA_ERR_SCRATCH;
  void* scratch = nullptr;
  if (need > 0) {
    const int rc = dsa::decode_scratch_address(&scratch);
    if (rc != 0) return rc == -5 ? DSA_ERR_DEVICE : DSA_ERR_LAUNCH;
  }
  // the same kernels and split as dsa_sparse_mla_decode, with the partials in the static scratch
  // (every split writes all of its rows, so nothing needs clearing between calls)
  return dsa_sparse_mla_decode(q, kv_cache, idx, batch, n_kv, n_heads, d_qk, d_v, topk, sm_scale, out, lse,
                               scratch, need > 0 ? dsa::kDecodeScratchBytes : 0, stream);
}

size_t dsa_sparse_mla_bwd_workspace_size(int total_q, int n_kv, int n_heads, int topk) {
  if (total_q < 0 || n_kv < 0 || n_heads < 1 || topk < 1) return 0;
  return bwd_layout(total_q, n_kv, n_heads, topk).total;
}

size_t dsa_sparse_mla_bwd_workspace_size_chunked(int total_q, int n_kv, int n_heads, int topk, int chunk_q) {
  return dsa_sparse_mla_bwd_workspace_size_ex(total_q, n_kv, n_heads, topk, chunk_q < 1 ? -1 : chunk_q, 0);
}

size_t dsa_sparse_mla_bwd_workspace_size_ex(int total_q, int n_kv, int n_heads, int topk, int chunk_q, int flags) {
  if (total_q < 0 || n_kv < 0 || n_heads < 1 || topk < 1 || chunk_q < 0 || (flags & ~DSA_BWD_G_INT8)) return 0;
  const int rows =
      chunk_q == 0 ? total_q : std::min(total_q, (chunk_q + kBwdChunkUnit - 1) / kBwdChunkUnit * kBwdChunkUnit);
  return bwd_layout(rows, n_kv, n_heads, topk, flags).total;
}

int dsa_sparse_mla_bwd(const void* q, const void* kv, const int32_t* idx, const void* out, const void* dout,
                       const float* lse, int total_q, int n_kv, int n_heads, int d_qk, int d_v, int topk,
                       float sm_scale, int causal, void* dq, float* dkv, void* workspace,
                       size_t workspace_bytes, void* stream) {
  return dsa_sparse_mla_bwd_ex(q, kv, idx, out, dout, lse, total_q, n_kv, n_heads, d_qk, d_v, topk, sm_scale,
                               causal, dq, dkv, 0, workspace, workspace_bytes, nullptr, stream);
}

int dsa_sparse_mla_bwd_timed(const void* q, const void* kv, const int32_t* idx, const void* out,
                             const void* dout, const float* lse, int total_q, int n_kv, int n_heads, int d_qk,
                             int d_v, int topk, float sm_scale, int causal, void* dq, float* dkv,
                             void* workspace, size_t workspace_bytes, void* const* stage_events, void* stream) {
  return dsa_sparse_mla_bwd_ex(q, kv, idx, out, dout, lse, total_q, n_kv, n_heads, d_qk, d_v, topk, sm_scale,
                               causal, dq, dkv, 0, workspace, workspace_bytes, stage_events, stream);
}

}  // extern "C"

namespace {
// The sparse backward; delta_out (nullable) receives rowsum(dO * O) [total_q, n_heads].
int sparse_bwd(const void* q, const void* kv, const int32_t* idx, const void* out, const void* dout, const float* lse,
               int total_q, int n_kv, int n_heads, int d_qk, int d_v, int topk, float sm_scale, int causal, void* dq,
               float* dkv, int flags, void* workspace, size_t workspace_bytes, void* const* stage_events,
               float* delta_out, void* stream) {
  if (total_q < 0 || n_kv < 1 || n_heads < 1 || topk < 1 || !std::isfinite(sm_scale)) return DSA_ERR_INVALID_ARG;
  if (flags & ~DSA_BWD_G_INT8) return DSA_ERR_INVALID_ARG;
  if ((d_qk != kDqk && d_qk != kDv) || d_v != kDv) return DSA_ERR_UNSUPPORTED;   // 512: the sink entry only
  if (n_heads > 128 || n_heads % 16 != 0) return DSA_ERR_UNSUPPORTED;
  if (!dkv || !aligned16(dkv)) return DSA_ERR_INVALID_ARG;
  // no query rows: every key's gradient is an empty sum (the per-query buffers and the
  // workspace are not touched and may be null; the timed variant has no stages to record)
  if (total_q == 0) {
    if (stage_events) return DSA_ERR_INVALID_ARG;
    DSA_CHECK_DEVICE(dev0);
    return dsa::launch_zero_rows(dkv, n_kv, kDqk, kDqk, as_stream(stream)) == 0 ? DSA_OK : DSA_ERR_LAUNCH;
  }
  if (!q || !kv || !idx || !out || !dout || !lse || !dq) return DSA_ERR_INVALID_ARG;
  if (!aligned16(q) || !aligned16(kv) || !aligned16(out) || !aligned16(dout) || !aligned16(dq))
    return DSA_ERR_INVALID_ARG;
  // query rows per pass: all of them when the whole layout fits the workspace, else the most
  // whole units of kBwdChunkUnit rows whose layout fits (the timed variant needs one pass)
  const int chunk = bwd_chunk_rows(total_q, n_kv, n_heads, topk, workspace_bytes, flags);
  if (!workspace || chunk == 0 || !aligned16(workspace)) return DSA_ERR_WORKSPACE;
  if (stage_events && chunk < total_q) return DSA_ERR_WORKSPACE;
  DSA_CHECK_DEVICE(dev);
  const BwdLayout L = bwd_layout(chunk, n_kv, n_heads, topk, flags);
  char* ws = static_cast<char*>(workspace);
  dsa::SparseBwdParams p{};
  p.n_xcd = dev.n_xcd;
  p.kv = static_cast<const dsa::bf16_t*>(kv);
  p.dkv = dkv;
  p.p_stage = reinterpret_cast<dsa::bf16_t*>(ws + L.p_stage);
  p.ds_stage = reinterpret_cast<dsa::bf16_t*>(ws + L.ds_stage);
  p.g_stage = ws + L.g_stage;
  p.g_int8 = (flags & DSA_BWD_G_INT8) ? 1 : 0;
  p.pair_pos = reinterpret_cast<int64_t*>(ws + L.pair_pos);
  p.csr_offsets = reinterpret_cast<int64_t*>(ws + L.offsets);
  p.csr_counts = reinterpret_cast<int32_t*>(ws + L.counts);
  p.n_heads = n_heads; p.n_kv = n_kv; p.topk = topk; p.topk_pad = topk_pad(topk);
  p.causal = causal ? 1 : 0;
  p.q_dim = d_qk;   // 512: q and dq rows without the rope part
  p.q_stride_t = (int64_t)n_heads * d_qk; p.kv_stride = kDqk; p.idx_stride = topk;
  p.out_stride_t = (int64_t)n_heads * kDv; p.dout_stride_t = (int64_t)n_heads * kDv;
  p.lse_stride_t = n_heads; p.dq_stride_t = (int64_t)n_heads * d_qk; p.dkv_stride = kDqk;
  p.scale = sm_scale;
  p.scale_log2 = sm_scale * 1.4426950408889634f;
  if (stage_events)
    for (int i = 0; i < 6; ++i)
      if (!stage_events[i]) return DSA_ERR_INVALID_ARG;
  // passes in query order: the first writes dkv, the later ones add to it (a fixed order, so the
  // result is the same from run to run for a given workspace size)
  for (int c0 = 0; c0 < total_q; c0 += chunk) {
    const int rows = std::min(chunk, total_q - c0);
    p.q = static_cast<const dsa::bf16_t*>(q) + (int64_t)c0 * p.q_stride_t;
    p.idx = idx + (int64_t)c0 * topk;
    p.out = static_cast<const dsa::bf16_t*>(out) + (int64_t)c0 * p.out_stride_t;
    p.dout = static_cast<const dsa::bf16_t*>(dout) + (int64_t)c0 * p.dout_stride_t;
    p.lse = lse + (int64_t)c0 * n_heads;
    p.dq = static_cast<dsa::bf16_t*>(dq) + (int64_t)c0 * p.dq_stride_t;
    p.total_q = rows;
    p.q_offset = c0;
    p.dkv_accumulate = c0 > 0 ? 1 : 0;
    p.g_sink_row = (int64_t)rows * topk;
    p.delta_out = delta_out ? delta_out + (int64_t)c0 * n_heads : nullptr;
    const int rc = dsa::launch_sparse_mla_bwd(p, as_stream(stream), reinterpret_cast<hipEvent_t const*>(stage_events));
    if (rc != 0) return rc;
  }
  return DSA_OK;
}
}  // namespace

extern "C" {

int dsa_sparse_mla_bwd_ex(const void* q, const void* kv, const int32_t* idx, const void* out, const void* dout,
                          const float* lse, int total_q, int n_kv, int n_heads, int d_qk, int d_v, int topk,
                          float sm_scale, int causal, void* dq, float* dkv, int flags, void* workspace,
                          size_t workspace_bytes, void* const* stage_events, void* stream) {
  if (d_qk != kDqk) return DSA_ERR_UNSUPPORTED;
  return sparse_bwd(q, kv, idx, out, dout, lse, total_q, n_kv, n_heads, d_qk, d_v, topk, sm_scale, causal, dq, dkv,
                    flags, workspace, workspace_bytes, stage_events, nullptr, stream);
}

size_t dsa_sparse_mla_bwd_sink_workspace_size(int total_q, int n_kv, int n_heads, int topk, int flags) {
  if (total_q < 0 || n_kv < 0 || n_heads < 1 || topk < 1 || (flags & ~DSA_BWD_G_INT8)) return 0;
  return bwd_layout(total_q, n_kv, n_heads, topk, flags).total + align_up(sizeof(float) * (size_t)total_q * n_heads);
}

int dsa_sparse_mla_bwd_sink(const void* q, const void* kv, const int32_t* idx, const void* out, const void* dout,
                            const float* lse, const float* sinks, int total_q, int n_kv, int n_heads, int d_qk,
                            int d_v, int topk, float sm_scale, int causal, void* dq, float* dkv, float* dsinks,
                            int flags, void* workspace, size_t workspace_bytes, void* stream) {
  if (total_q < 0 || n_heads < 1 || (flags & ~DSA_BWD_G_INT8)) return DSA_ERR_INVALID_ARG;
  if (!sinks || !dsinks) return DSA_ERR_INVALID_ARG;
  // Delta [total_q, n_heads] sits at the end of the workspace; the passes take the rest
  const size_t dbytes = align_up(sizeof(float) * (size_t)total_q * n_heads);
  if (!workspace || workspace_bytes < dbytes || !aligned16(workspace)) return DSA_ERR_WORKSPACE;
  const size_t rest = (workspace_bytes - dbytes) / 256 * 256;
  float* delta = reinterpret_cast<float*>(static_cast<char*>(workspace) + rest);
  if (total_q == 0) {
    const int rc = sparse_bwd(q, kv, idx, out, dout, lse, 0, n_kv, n_heads, d_qk, d_v, topk, sm_scale, causal, dq,
                              dkv, flags, workspace, rest, nullptr, nullptr, stream);
    if (rc != DSA_OK) return rc;
    return dsa::launch_sink_grad(sinks, lse, delta, 0, n_heads, dsinks, nullptr, 0, as_stream(stream)) == 0
               ? DSA_OK
               : DSA_ERR_LAUNCH;
  }
  const int rc = sparse_bwd(q, kv, idx, out, dout, lse, total_q, n_kv, n_heads, d_qk, d_v, topk, sm_scale, causal,
                            dq, dkv, flags, workspace, rest, nullptr, delta, stream);
  if (rc != DSA_OK) return rc;
  // the backward's part of the workspace is free again: the sums' partials go just below Delta (the
  // pair-order scratch there is not read after the backward; the staged P tiles at its head stay)
  const size_t pbytes = align_up(dsa::sink_grad_scratch_bytes(n_heads));
  float* scratch = rest >= pbytes ? reinterpret_cast<float*>(static_cast<char*>(workspace) + rest - pbytes) : nullptr;
  return dsa::launch_sink_grad(sinks, lse, delta, total_q, n_heads, dsinks, scratch, scratch ? pbytes : 0,
                               as_stream(stream)) == 0
             ? DSA_OK
             : DSA_ERR_LAUNCH;
}

int dsa_indexer_kl_target(const void* q, const void* kv, const int32_t* idx, const float* lse, int total_q,
                          int n_kv, int n_heads, int d_qk, int topk, float sm_scale, int causal, float* target,
                          void* stream) {
  if (total_q < 0 || n_kv < 0 || n_heads < 1 || topk < 1 || !std::isfinite(sm_scale) || !(sm_scale > 0.f))
    return DSA_ERR_INVALID_ARG;
  if (d_qk != kDqk) return DSA_ERR_UNSUPPORTED;
  if (n_heads > 128) return DSA_ERR_UNSUPPORTED;
  if (total_q == 0) return DSA_OK;
  if (!q || !kv || !idx || !lse || !target || n_kv < 1) return DSA_ERR_INVALID_ARG;
  if (!aligned16(q) || !aligned16(kv)) return DSA_ERR_INVALID_ARG;
  dsa::KlTargetParams p{};
  p.q = static_cast<const dsa::bf16_t*>(q);
  p.kv = static_cast<const dsa::bf16_t*>(kv);
  p.idx = idx; p.lse = lse; p.target = target;
  p.total_q = total_q; p.n_heads = n_heads; p.n_kv = n_kv; p.topk = topk; p.causal = causal ? 1 : 0;
  p.q_stride_t = (int64_t)n_heads * kDqk; p.idx_stride = topk; p.lse_stride_t = n_heads; p.target_stride = topk;
  p.scale_log2 = sm_scale * 1.4426950408889634f;
  DSA_CHECK_DEVICE(dev);
  p.n_xcd = dev.n_xcd;
  return dsa::launch_indexer_kl_target(p, as_stream(stream));
}

static int dense_kl_params(const void* q, const void* kv, const int32_t* row_base, const int32_t* row_len, int total_q,
                    int n_kv, int n_heads, int d_qk, float sm_scale, dsa::DenseKlParams& p) {
  if (total_q < 0 || n_kv < 0 || n_heads < 1 || !std::isfinite(sm_scale) || !(sm_scale > 0.f))
    return DSA_ERR_INVALID_ARG;
  if (d_qk != kDqk) return DSA_ERR_UNSUPPORTED;
  if (n_heads > 128) return DSA_ERR_UNSUPPORTED;
  if (total_q == 0) return DSA_OK;
  if (!q || !kv || !row_base || !row_len || n_kv < 1) return DSA_ERR_INVALID_ARG;
  if (!aligned16(q) || !aligned16(kv)) return DSA_ERR_INVALID_ARG;
  p.q = static_cast<const dsa::bf16_t*>(q);
  p.kv = static_cast<const dsa::bf16_t*>(kv);
  p.row_base = row_base; p.row_len = row_len;
  p.total_q = total_q; p.n_heads = n_heads; p.n_kv = n_kv;
  p.q_stride_t = (int64_t)n_heads * kDqk;
  p.scale_log2 = sm_scale * 1.4426950408889634f;
  return DSA_OK;
}

int dsa_dense_attention_lse(const void* q, const void* kv, const int32_t* row_base, const int32_t* row_len,
                            int total_q, int n_kv, int n_heads, int d_qk, float sm_scale, float* lse, void* stream) {
  dsa::DenseKlParams p{};
  const int rc = dense_kl_params(q, kv, row_base, row_len, total_q, n_kv, n_heads, d_qk, sm_scale, p);
  if (rc != DSA_OK || total_q == 0) return rc;
  if (!lse) return DSA_ERR_INVALID_ARG;
  p.lse_out = lse;
  DSA_CHECK_DEVICE(dev);
  p.n_xcd = dev.n_xcd;
  return dsa::launch_dense_lse(p, as_stream(stream)) == 0 ? DSA_OK : DSA_ERR_LAUNCH;
}

int dsa_dense_attention_target(const void* q, const void* kv, const float* lse, const int32_t* row_base,
                               const int32_t* row_len, int total_q, int n_kv, int n_heads, int d_qk, int pitch,
                               float sm_scale, float* target, void* stream) {
  dsa::DenseKlParams p{};
  if (pitch < 1) return DSA_ERR_INVALID_ARG;
  const int rc = dense_kl_params(q, kv, row_base, row_len, total_q, n_kv, n_heads, d_qk, sm_scale, p);
  if (rc != DSA_OK || total_q == 0) return rc;
  if (!lse || !target) return DSA_ERR_INVALID_ARG;
  p.lse = lse; p.target = target; p.pitch = pitch; p.target_stride = pitch;
  DSA_CHECK_DEVICE(dev);
  p.n_xcd = dev.n_xcd;
  return dsa::launch_dense_target(p, as_stream(stream)) == 0 ? DSA_OK : DSA_ERR_LAUNCH;
}

int dsa_indexer_kl_target_from_bwd(const void* bwd_workspace, size_t bwd_workspace_bytes, const int32_t* idx,
                                   int total_q, int n_kv, int n_heads, int topk, int causal, float* target,
                                   void* stream) {
  if (total_q < 0 || n_kv < 1 || n_heads < 1 || topk < 1) return DSA_ERR_INVALID_ARG;
  if (n_heads > 128 || n_heads % 16 != 0) return DSA_ERR_UNSUPPORTED;
  if (total_q == 0) return DSA_OK;
  if (!idx || !target) return DSA_ERR_INVALID_ARG;
  const BwdLayout L = bwd_layout(total_q, n_kv, n_heads, topk);
  if (!bwd_workspace || bwd_workspace_bytes < L.total || !aligned16(bwd_workspace)) return DSA_ERR_WORKSPACE;
  dsa::KlFromPParams p{};
  p.p_stage = reinterpret_cast<const dsa::bf16_t*>(static_cast<const char*>(bwd_workspace) + L.p_stage);
  p.idx = idx; p.target = target;
  p.total_q = total_q; p.n_heads = n_heads; p.n_kv = n_kv; p.topk = topk; p.topk_pad = topk_pad(topk);
  p.causal = causal ? 1 : 0;
  p.idx_stride = topk; p.target_stride = topk;
  DSA_CHECK_DEVICE(dev);
  return dsa::launch_indexer_kl_target_from_p(p, as_stream(stream));
}

int dsa_indexer_kl_loss(const float* index_sel, const float* target, const int32_t* idx, int total_q, int n_kv,
                        int topk, int causal, float grad_scale, float* kl, float* d_index, void* stream) {
  if (total_q < 0 || n_kv < 0 || topk < 1 || !std::isfinite(grad_scale)) return DSA_ERR_INVALID_ARG;
  if (total_q == 0) return DSA_OK;
  if (!index_sel || !target || !idx || !kl || !d_index) return DSA_ERR_INVALID_ARG;
  dsa::KlLossParams p{};
  p.index_sel = index_sel; p.target = target; p.idx = idx; p.kl = kl; p.d_index = d_index;
  p.total_q = total_q; p.topk = topk; p.n_kv = n_kv; p.causal = causal ? 1 : 0;
  p.index_stride = topk; p.target_stride = topk; p.idx_stride = topk; p.d_stride = topk;
  p.grad_scale = grad_scale;
  DSA_CHECK_DEVICE(dev);
  return dsa::launch_indexer_kl(p, as_stream(stream));
}

int dsa_indexer_selected_scores(const void* q, const void* k, const float* w, const int32_t* idx, int total_q,
                                int n_k, int n_heads, int head_dim, int topk, int causal, float* scores,
                                void* stream) {
  if (total_q < 0 || n_k < 0 || n_heads < 1 || topk < 1) return DSA_ERR_INVALID_ARG;
  if (head_dim != 128 || n_heads > 64 || topk > 4096) return DSA_ERR_UNSUPPORTED;
  if (total_q == 0) return DSA_OK;
  if (!q || !k || !w || !idx || !scores || n_k < 1) return DSA_ERR_INVALID_ARG;
  if (!aligned16(q) || !aligned16(k)) return DSA_ERR_INVALID_ARG;
  dsa::IdxSelParams p{};
  p.q = static_cast<const dsa::bf16_t*>(q);
  p.k = static_cast<const dsa::bf16_t*>(k);
  p.w = w; p.idx = idx; p.scores = scores;
  p.total_q = total_q; p.n_heads = n_heads; p.n_k = n_k; p.topk = topk; p.causal = causal ? 1 : 0;
  p.q_stride_t = (int64_t)n_heads * head_dim; p.idx_stride = topk; p.scores_stride = topk;
  DSA_CHECK_DEVICE(dev);
  p.n_xcd = dev.n_xcd;
  return dsa::launch_indexer_selected_scores(p, as_stream(stream));
}

size_t dsa_indexer_scores_bwd_workspace_size(int total_q, int n_k, int topk) {
  if (total_q < 0 || n_k < 0 || topk < 1) return 0;
  return idx_bwd_layout(total_q, n_k, topk).total;
}

static size_t dense_scores_bwd_chunks(int total_q) {
  return ((size_t)total_q + dsa::kDenseQChunk - 1) / dsa::kDenseQChunk;
}

size_t dsa_dense_indexer_scores_bwd_workspace_size(int total_q, int n_k) {
  if (total_q <= 0 || n_k <= 0) return 0;
  const size_t tiles = ((size_t)n_k + dsa::kDenseDkKeys - 1) / dsa::kDenseDkKeys;
  return align_up(tiles * dense_scores_bwd_chunks(total_q) * dsa::kDenseDkKeys * 128 * sizeof(float));
}

int dsa_dense_indexer_scores_bwd(const void* q, const void* k, const float* w, const int32_t* row_base,
                                 const int32_t* row_len, int total_q, int n_k, int n_heads, int head_dim,
                                 const float* d_scores, int pitch, float* dq, float* dw, float* dk, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  if (total_q < 0 || n_k < 1 || n_heads < 1 || pitch < 1) return DSA_ERR_INVALID_ARG;
  if (head_dim != 128 || n_heads > 64) return DSA_ERR_UNSUPPORTED;
  if (!dk) return DSA_ERR_INVALID_ARG;
  if (total_q == 0) {   // no rows: dk = 0 (empty sums); dq and dw are empty
    DSA_CHECK_DEVICE(dev0);
    return dsa::launch_zero_rows(dk, n_k, head_dim, head_dim, as_stream(stream)) == 0 ? DSA_OK : DSA_ERR_LAUNCH;
  }
  if (!q || !k || !w || !row_base || !row_len || !d_scores || !dq || !dw) return DSA_ERR_INVALID_ARG;
  if (!aligned16(q) || !aligned16(k) || !aligned16(dq) || !aligned16(dk)) return DSA_ERR_INVALID_ARG;
  const size_t need = dsa_dense_indexer_scores_bwd_workspace_size(total_q, n_k);
  if (!workspace || workspace_bytes < need || !aligned16(workspace)) return DSA_ERR_WORKSPACE;
  dsa::DenseIdxBwdParams p{};
  p.q = static_cast<const dsa::bf16_t*>(q);
  p.k = static_cast<const dsa::bf16_t*>(k);
  p.w = w; p.row_base = row_base; p.row_len = row_len; p.d_scores = d_scores;
  p.dq = dq; p.dw = dw; p.dk = dk; p.dk_part = static_cast<float*>(workspace);
  p.total_q = total_q; p.n_heads = n_heads; p.n_k = n_k; p.pitch = pitch;
  p.n_tiles = (n_k + dsa::kDenseDkKeys - 1) / dsa::kDenseDkKeys;
  p.max_chunks = (int)dense_scores_bwd_chunks(total_q);
  DSA_CHECK_DEVICE(dev);
  p.n_xcd = dev.n_xcd;
  return dsa::launch_dense_scores_bwd(p, as_stream(stream)) == 0 ? DSA_OK : DSA_ERR_LAUNCH;
}

int dsa_indexer_scores_bwd(const void* q, const void* k, const float* w, const int32_t* idx, const float* d_index,
                           int total_q, int n_k, int n_heads, int head_dim, int topk, int causal, float* dq,
                           float* dw, float* dk, void* workspace, size_t workspace_bytes, void* stream) {
  if (total_q < 0 || n_k < 1 || n_heads < 1 || topk < 1) return DSA_ERR_INVALID_ARG;
  if (head_dim != 128 || n_heads > 64 || topk > 4096) return DSA_ERR_UNSUPPORTED;
  if (!dk) return DSA_ERR_INVALID_ARG;
  // no query rows: dk = 0 (empty sums); dq and dw are empty, the workspace is not needed
  if (total_q == 0) {
    DSA_CHECK_DEVICE(dev0);
    return dsa::launch_zero_rows(dk, n_k, head_dim, head_dim, as_stream(stream)) == 0 ? DSA_OK : DSA_ERR_LAUNCH;
  }
  if (!q || !k || !w || !idx || !d_index || !dq || !dw) return DSA_ERR_INVALID_ARG;
  if (!aligned16(q) || !aligned16(k) || !aligned16(dq)) return DSA_ERR_INVALID_ARG;
  const IdxBwdLayout L = idx_bwd_layout(total_q, n_k, topk);
  if (!workspace || workspace_bytes < L.total || !aligned16(workspace)) return DSA_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  dsa::IdxSelParams p{};
  p.q = static_cast<const dsa::bf16_t*>(q);
  p.k = static_cast<const dsa::bf16_t*>(k);
  p.w = w; p.idx = idx; p.d_index = d_index; p.dq = dq; p.dw = dw; p.dk = dk;
  p.g_stage = reinterpret_cast<dsa::bf16_t*>(ws + L.g_stage);
  p.g_sink_row = (int64_t)total_q * topk;
  p.pair_pos = reinterpret_cast<int64_t*>(ws + L.pair_pos);
  p.csr_offsets = reinterpret_cast<int64_t*>(ws + L.offsets);
  p.csr_counts = reinterpret_cast<int32_t*>(ws + L.counts);
  p.total_q = total_q; p.n_heads = n_heads; p.n_k = n_k; p.topk = topk; p.causal = causal ? 1 : 0;
  p.q_stride_t = (int64_t)n_heads * head_dim; p.idx_stride = topk; p.d_stride = topk;
  DSA_CHECK_DEVICE(dev);
  p.n_xcd = dev.n_xcd;
  return dsa::launch_indexer_scores_bwd(p, as_stream(stream));
}

// ---- DeepSeek-V4 compressor
static int compress_params(const void* kv, const void* gate, int64_t kv_stride, int64_t gate_stride, const void* ape,
                           const void* norm_w, const int32_t* doc_table, int n_docs, int total_tokens, int n_entries,
                           int n_items, int channels, int dim, int rate, int overlap, float eps,
                           dsa::CompressParams& p) {
  if (n_docs < 1 || total_tokens < 0 || n_entries < 0 || n_items < 0 || rate < 1 || !std::isfinite(eps) || eps < 0.f)
    return DSA_ERR_INVALID_ARG;
  if (dim != 64 && dim != 128 && dim != 256 && dim != 512) return DSA_ERR_UNSUPPORTED;
  if (channels != (overlap ? 2 * dim : dim)) return DSA_ERR_INVALID_ARG;
  if ((int64_t)n_entries * rate > total_tokens || n_items > total_tokens || n_entries > n_items)
    return DSA_ERR_INVALID_ARG;
  if (kv_stride < channels || gate_stride < channels || kv_stride % 8 || gate_stride % 8) return DSA_ERR_INVALID_ARG;
  if (!kv || !gate || !ape || !norm_w || !doc_table) return DSA_ERR_INVALID_ARG;
  if (!aligned16(kv) || !aligned16(gate) || !aligned16(ape) || !aligned16(norm_w)) return DSA_ERR_INVALID_ARG;
  p.kv = static_cast<const dsa::bf16_t*>(kv);
  p.gate = static_cast<const dsa::bf16_t*>(gate);
  p.ape = static_cast<const dsa::bf16_t*>(ape);
  p.norm_w = static_cast<const dsa::bf16_t*>(norm_w);
  p.doc_table = doc_table;
  p.n_docs = n_docs; p.total_tokens = total_tokens; p.n_entries = n_entries; p.n_items = n_items;
  p.channels = channels; p.dim = dim; p.rate = rate; p.overlap = overlap ? 1 : 0; p.eps = eps;
  p.kv_stride = kv_stride; p.gate_stride = gate_stride;
  return DSA_OK;
}

int dsa_v4_compress_fwd(const void* kv, const void* gate, int64_t kv_stride, int64_t gate_stride, const void* ape,
                        const void* norm_w, const int32_t* doc_table, int n_docs, int total_tokens, int n_entries,
                        int channels, int dim, int rate, int overlap, float eps, void* out, void* stream) {
  dsa::CompressParams p{};
  // the forward has no items of its own: n_items = n_entries passes the item checks
  const int rc = compress_params(kv, gate, kv_stride, gate_stride, ape, norm_w, doc_table, n_docs, total_tokens,
                                 n_entries, n_entries, channels, dim, rate, overlap, eps, p);
  if (rc != DSA_OK) return rc;
  if (n_entries == 0) return DSA_OK;
  if (!out || !aligned16(out)) return DSA_ERR_INVALID_ARG;
  p.out = static_cast<dsa::bf16_t*>(out);
  DSA_CHECK_DEVICE(dev);
  return dsa::launch_v4_compress_fwd(p, as_stream(stream)) == 0 ? DSA_OK : DSA_ERR_LAUNCH;
}

size_t dsa_v4_compress_bwd_workspace_size(int n_entries, int n_items, int channels, int dim, int rate) {
  if (n_entries < 0 || n_items < 0 || channels < 1 || dim < 1 || rate < 1) return 0;
  const dsa::CompressBwdGrid g = dsa::compress_bwd_grid(n_entries, n_items, channels, dim, rate);
  return align_up(sizeof(float) * (size_t)g.dnorm_floats) + align_up(sizeof(float) * (size_t)g.dape_floats) +
         align_up(sizeof(int32_t) * (size_t)g.entry_ints);
}

int dsa_v4_compress_bwd(const void* kv, const void* gate, int64_t kv_stride, int64_t gate_stride, const void* ape,
                        const void* norm_w, const int32_t* doc_table, int n_docs, int total_tokens, int n_entries,
                        int n_items, int channels, int dim, int rate, int overlap, float eps, const void* dout,
                        void* dkv, void* dgate, int64_t dkv_stride, int64_t dgate_stride, float* dape,
                        float* dnorm_w, void* workspace, size_t workspace_bytes, void* stream) {
  dsa::CompressParams p{};
  const int rc = compress_params(kv, gate, kv_stride, gate_stride, ape, norm_w, doc_table, n_docs, total_tokens,
                                 n_entries, n_items, channels, dim, rate, overlap, eps, p);
  if (rc != DSA_OK) return rc;
  if (!dape || !dnorm_w || !dkv || !dgate || (n_entries > 0 && !dout)) return DSA_ERR_INVALID_ARG;
  if (dkv_stride < channels || dgate_stride < channels || dkv_stride % 8 || dgate_stride % 8)
    return DSA_ERR_INVALID_ARG;
  if (!aligned16(dkv) || !aligned16(dgate) || (dout && !aligned16(dout))) return DSA_ERR_INVALID_ARG;
  const size_t need = dsa_v4_compress_bwd_workspace_size(n_entries, n_items, channels, dim, rate);
  if (!workspace || workspace_bytes < need || !aligned16(workspace)) return DSA_ERR_WORKSPACE;
  const dsa::CompressBwdGrid g = dsa::compress_bwd_grid(n_entries, n_items, channels, dim, rate);
  char* ws = static_cast<char*>(workspace);
  p.dout = static_cast<const dsa::bf16_t*>(dout);
  p.dkv = static_cast<dsa::bf16_t*>(dkv);
  p.dgate = static_cast<dsa::bf16_t*>(dgate);
  p.dkv_stride = dkv_stride; p.dgate_stride = dgate_stride;
  p.dnorm_part = reinterpret_cast<float*>(ws);
  const size_t dape_off = align_up(sizeof(float) * (size_t)g.dnorm_floats);
  p.dape_part = reinterpret_cast<float*>(ws + dape_off);
  p.entry_tok = reinterpret_cast<int32_t*>(ws + dape_off + align_up(sizeof(float) * (size_t)g.dape_floats));
  DSA_CHECK_DEVICE(dev);
  return dsa::launch_v4_compress_bwd(p, dape, dnorm_w, as_stream(stream)) == 0 ? DSA_OK : DSA_ERR_LAUNCH;
}


// ---- DeepSeek-V4 row transforms
static int rope_params(int64_t rows, int n_heads, int dim, int rope_dim, const float* cos, const float* sin,
                       int64_t angle_stride, int inverse, dsa::RopeParams& p) {
  if (rows < 0 || n_heads < 1 || rows % n_heads != 0 || rope_dim < 0 || rope_dim > dim || rope_dim % 8 ||
      rows / n_heads > INT32_MAX)
    return DSA_ERR_INVALID_ARG;
  if (dim != 64 && dim != 128 && dim != 256 && dim != 512) return DSA_ERR_UNSUPPORTED;
  if (rope_dim > 0 && angle_stride < rope_dim / 2) return DSA_ERR_INVALID_ARG;
  if (rows > 0 && rope_dim > 0 && (!cos || !sin)) return DSA_ERR_INVALID_ARG;   // no rows: nothing is read
  p.rows = rows; p.n_heads = n_heads; p.tokens = (int)(rows / n_heads); p.dim = dim; p.rope_dim = rope_dim;
  p.cos = cos; p.sin = sin; p.angle_stride = angle_stride; p.inverse = inverse ? 1 : 0; p.groups = 1;
  return DSA_OK;
}

int dsa_v4_norm_rope(const void* x, int64_t rows, int n_heads, int dim, int rope_dim, const float* cos,
                     const float* sin, int64_t angle_stride, int norm, float eps, int inverse, void* out,
                     void* stream) {
  dsa::RopeParams p{};
  const int rc = rope_params(rows, n_heads, dim, rope_dim, cos, sin, angle_stride, inverse, p);
  if (rc != DSA_OK) return rc;
  if (norm && (!std::isfinite(eps) || eps < 0.f)) return DSA_ERR_INVALID_ARG;
  if (rows == 0) return DSA_OK;
  if (!x || !out || !aligned16(x) || !aligned16(out)) return DSA_ERR_INVALID_ARG;
  p.x = static_cast<const dsa::bf16_t*>(x);
  p.out = static_cast<dsa::bf16_t*>(out);
  p.norm = norm ? 1 : 0; p.eps = eps;
  DSA_CHECK_DEVICE(dev);
  return dsa::launch_v4_rope(0, p, as_stream(stream)) == 0 ? DSA_OK : DSA_ERR_LAUNCH;
}

int dsa_v4_norm_rope_bwd(const void* x, const void* dout, int64_t rows, int n_heads, int dim, int rope_dim,
                         const float* cos, const float* sin, int64_t angle_stride, int norm, float eps, int inverse,
                         void* dx, void* stream) {
  dsa::RopeParams p{};
  const int rc = rope_params(rows, n_heads, dim, rope_dim, cos, sin, angle_stride, inverse, p);
  if (rc != DSA_OK) return rc;
  if (norm && (!std::isfinite(eps) || eps < 0.f)) return DSA_ERR_INVALID_ARG;
  if (rows == 0) return DSA_OK;
  if (!dout || !dx || !aligned16(dout) || !aligned16(dx) || (norm && (!x || !aligned16(x))))
    return DSA_ERR_INVALID_ARG;
  p.x = static_cast<const dsa::bf16_t*>(x);
  p.dout = static_cast<const dsa::bf16_t*>(dout);
  p.dx = static_cast<dsa::bf16_t*>(dx);
  p.norm = norm ? 1 : 0; p.eps = eps;
  DSA_CHECK_DEVICE(dev);
  return dsa::launch_v4_rope(1, p, as_stream(stream)) == 0 ? DSA_OK : DSA_ERR_LAUNCH;
}

int dsa_v4_out_rope_group(const void* o, int tokens, int n_heads, int dim, int rope_dim, int groups,
                          const float* cos, const float* sin, int64_t angle_stride, int inverse, void* og,
                          void* stream) {
  dsa::RopeParams p{};
  if (tokens < 0 || groups < 1 || n_heads % groups != 0) return DSA_ERR_INVALID_ARG;
  const int rc = rope_params((int64_t)tokens * n_heads, n_heads, dim, rope_dim, cos, sin, angle_stride, inverse, p);
  if (rc != DSA_OK) return rc;
  if (tokens == 0) return DSA_OK;
  if (!o || !og || !aligned16(o) || !aligned16(og)) return DSA_ERR_INVALID_ARG;
  p.x = static_cast<const dsa::bf16_t*>(o);
  p.out = static_cast<dsa::bf16_t*>(og);
  p.groups = groups;
  DSA_CHECK_DEVICE(dev);
  return dsa::launch_v4_rope(2, p, as_stream(stream)) == 0 ? DSA_OK : DSA_ERR_LAUNCH;
}

int dsa_v4_out_rope_group_bwd(const void* dog, int tokens, int n_heads, int dim, int rope_dim, int groups,
                              const float* cos, const float* sin, int64_t angle_stride, int inverse, void* d_o,
                              void* stream) {
  dsa::RopeParams p{};
  if (tokens < 0 || groups < 1 || n_heads % groups != 0) return DSA_ERR_INVALID_ARG;
  const int rc = rope_params((int64_t)tokens * n_heads, n_heads, dim, rope_dim, cos, sin, angle_stride, inverse, p);
  if (rc != DSA_OK) return rc;
  if (tokens == 0) return DSA_OK;
  if (!dog || !d_o || !aligned16(dog) || !aligned16(d_o)) return DSA_ERR_INVALID_ARG;
  p.dout = static_cast<const dsa::bf16_t*>(dog);
  p.dx = static_cast<dsa::bf16_t*>(d_o);
  p.groups = groups;
  DSA_CHECK_DEVICE(dev);
  return dsa::launch_v4_rope(3, p, as_stream(stream)) == 0 ? DSA_OK : DSA_ERR_LAUNCH;
}

}  // extern "C"
