// Sparse indexer KL loss (gfx950): its attention target, the KL itself and its gradient with
// respect to the index scores of the selected keys.
//
// The reference turns the loss on with dsa_indexer_loss_coeff / dsa_indexer_use_sparse_loss
// (src/mcore_bridge/config/model_config.py:204-205); megatron-core's compute_dsa_indexer_loss
// computes it from dense per-head attention scores (third-party, not vendored).  With the sparse
// loss, the target of query t over its selected keys is the head-summed attention probability,
// L1-normalised:  p[t,j] = (1/H) sum_h exp(scale * q[t,h] . kv[idx[t,j]] - lse[t,h]), and the
// loss is mean_t sum_j p (log(p + eps) - log(softmax(I_t)_j + eps)) times the coefficient.
//
//   the target itself: dsa_dense_kl.hip's attention-target kernel over the index rows (one
//       workgroup per query, S = Q . K^T per 32-key block, P = 2^(scale_log2 * S - lse2) summed
//       over heads in the lane, across its half-wave partner and across the waves through LDS).
//   kl_target_from_p_kernel   the same target as the head mean of the P tiles the sparse MLA
//       backward stages (for callers that apply the loss in the backward pass: no S recompute).
//   indexer_kl_kernel         one workgroup per query: softmax of the index scores over the valid
//       slots, the KL of the row and d(loss)/dI.
#include "dsa_common.h"
#include "dsa_kernels.h"
#include "dsa_kvtile.h"

namespace dsa {

namespace {
constexpr int kBK = kTileKeys;
}  // namespace

// One workgroup (256 threads) per query: pI = softmax of the index scores over the valid slots,
// kl[t] = sum_j p (log(p + eps) - log(pI + eps)), and d(loss)/dI[t, j] = grad_scale *
// (pI_j * sum_k r_k - r_j) with r = p * pI / (pI + eps) (0 at invalid slots).
__global__ __launch_bounds__(256) void indexer_kl_kernel(KlLossParams p) {
  __shared__ float red[8];
  const int t = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* I = p.index_sel + (int64_t)t * p.index_stride;
  const float* tg = p.target + (int64_t)t * p.target_stride;
  const int32_t* ix = p.idx + (int64_t)t * p.idx_stride;
  auto ok = [&](int j) {
    const int x = ix[j];
    return x >= 0 && x < p.n_kv && (!p.causal || x <= t);
  };
  auto block_reduce = [&](float v, bool is_max) {
    v = is_max ? wave_max(v) : wave_sum(v);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < 4; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
    return r;
  };
  float m = -INFINITY;
  for (int j = tid; j < p.topk; j += 256)
    if (ok(j)) m = fmaxf(m, I[j]);
  m = block_reduce(m, true);
  float z = 0.f;
  if (m != -INFINITY)
    for (int j = tid; j < p.topk; j += 256)
      if (ok(j)) z += expf(I[j] - m);
  z = block_reduce(z, false);
  const float lz = m + logf(z);
  constexpr float kEps = 1e-10f;
  float kl = 0.f, rs = 0.f;
  for (int j = tid; j < p.topk; j += 256) {
    if (!ok(j)) continue;
    const float pi = expf(I[j] - lz), pt = tg[j];
    kl += pt * (logf(pt + kEps) - logf(pi + kEps));
    rs += pt * pi / (pi + kEps);
  }
  kl = block_reduce(kl, false);
  rs = block_reduce(rs, false);
  if (tid == 0) p.kl[t] = kl;
  float* g = p.d_index + (int64_t)t * p.d_stride;
  for (int j = tid; j < p.topk; j += 256) {
    float v = 0.f;
    if (ok(j)) {
      const float pi = expf(I[j] - lz), pt = tg[j];
      v = p.grad_scale * (pi * rs - pt * pi / (pi + kEps));
    }
    g[j] = v;
  }
}

// The same target from the P tiles the sparse MLA backward stages (B1 recomputes P = exp(scale *
// S - lse) for every head and stores it in bf16, [t][block][head][32 keys]): target[t, j] = (1/H)
// sum_h P[t, h, j], no S recompute.  One workgroup per query; thread (c, h0) reads 8 keys of
// heads h0, h0 + 64 per block, summed over the wave's heads with lane shuffles and over the
// waves through LDS.  Blocks past the query's last valid slot were not staged: their slots are 0.
__global__ __launch_bounds__(256) void kl_target_from_p_kernel(KlFromPParams p) {
  __shared__ float part[4][32];
  __shared__ int red[4];
  const int t = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int32_t* ix = p.idx + (int64_t)t * p.idx_stride;
  int last = -1;
  for (int j = threadIdx.x; j < p.topk; j += 256) {
    const int x = ix[j];
    if (x >= 0 && x < p.n_kv && (!p.causal || x <= t)) last = j;
  }
  last = wave_max_i(last);
  if (lane == 0) red[wave] = last;
  __syncthreads();
  last = max(max(red[0], red[1]), max(red[2], red[3]));
  const int nblk = (last + kBK) / kBK;
  float* out = p.target + (int64_t)t * p.target_stride;
  const float inv_h = 1.f / (float)p.n_heads;
  const int c = threadIdx.x & 3, h0 = threadIdx.x >> 2;
  const bf16_t* base = p.p_stage + (int64_t)t * (p.topk_pad / kBK) * p.n_heads * kBK;
  for (int b = 0; b < nblk; ++b) {
    const bf16_t* tile = base + (int64_t)b * p.n_heads * kBK;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int h = h0; h < p.n_heads; h += 64) {
      const u32x4 v = gload16(tile + h * kBK + 8 * c);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[2 * e] += bf16_lo(v[e]);
        acc[2 * e + 1] += bf16_hi(v[e]);
      }
    }
#pragma unroll
    for (int o = 4; o < 64; o <<= 1)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += __shfl_xor(acc[e], o, 64);
    if (lane < 4) {
#pragma unroll
      for (int e = 0; e < 8; ++e) part[wave][8 * lane + e] = acc[e];
    }
    __syncthreads();
    if (threadIdx.x < kBK && b * kBK + (int)threadIdx.x < p.topk) {
      const int k = threadIdx.x;
      out[b * kBK + k] = (part[0][k] + part[1][k] + part[2][k] + part[3][k]) * inv_h;
    }
    __syncthreads();
  }
  for (int j = nblk * kBK + threadIdx.x; j < p.topk; j += 256) out[j] = 0.f;
}

int launch_indexer_kl_target_from_p(const KlFromPParams& p, hipStream_t stream) {
  if (p.total_q == 0) return 0;
  hipLaunchKernelGGL(kl_target_from_p_kernel, dim3(p.total_q), dim3(256), 0, stream, p);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

// The target over index rows runs the attention-target kernel of dsa_dense_kl.hip (the dense
// loss's, with index-row slices in place of key ranges).
int launch_indexer_kl_target(const KlTargetParams& p, hipStream_t stream) {
  DenseKlParams d{};
  d.q = p.q; d.kv = p.kv; d.lse = p.lse; d.target = p.target;
  d.total_q = p.total_q; d.n_heads = p.n_heads; d.n_kv = p.n_kv; d.pitch = p.topk;
  d.q_stride_t = p.q_stride_t; d.target_stride = p.target_stride;
  d.scale_log2 = p.scale_log2; d.n_xcd = p.n_xcd;
  d.idx = p.idx; d.idx_stride = p.idx_stride; d.causal = p.causal;
  return launch_sparse_target(d, stream);
}

int launch_indexer_kl(const KlLossParams& p, hipStream_t stream) {
  if (p.total_q == 0) return 0;
  hipLaunchKernelGGL(indexer_kl_kernel, dim3(p.total_q), dim3(256), 0, stream, p);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace dsa
