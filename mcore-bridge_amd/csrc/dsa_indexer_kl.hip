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
//   indexer_kl_target_kernel  one workgroup per query, the sparse forward's gather ring and Q
//       registers, S = Q . K^T per 32-key block (the forward's operands swapped, so each lane
//       holds one key and 16 heads), P = 2^(scale_log2 * S - lse2), summed over heads in the
//       lane, across its half-wave partner and across the waves through LDS.
//   kl_target_from_p_kernel   the same target as the head mean of the P tiles the sparse MLA
//       backward stages (for callers that apply the loss in the backward pass: no S recompute).
//   indexer_kl_kernel         one workgroup per query: softmax of the index scores over the valid
//       slots, the KL of the row and d(loss)/dI.
#include "dsa_common.h"
#include "dsa_kernels.h"
#include "dsa_kvtile.h"

namespace dsa {

namespace {

constexpr int kDqk = 576;
constexpr int kBK = kTileKeys;
constexpr int kStages = 3;
constexpr int kMaxTopkKl = 8192;
constexpr int kPre = 3;

struct KlSmem {
  char tile[kStages][kTileBytes];
  int32_t idx[kMaxTopkKl];
  float red[4][32];
  int rmax[4];
};

}  // namespace

template <int NW>
__global__ __launch_bounds__(NW * 64, 1) void indexer_kl_target_kernel(KlTargetParams p) {
  constexpr int G = tile_copies_per_wave<NW>();
  constexpr int kCopyEvery = kDqk / 16 / G;
  static_assert(kCopyEvery * G == kDqk / 16, "copies spread evenly over the QK MFMAs");
  __shared__ __attribute__((aligned(128))) KlSmem sm;
  const int t = xcd_remap(blockIdx.x, p.n_xcd);
  if (t >= p.total_q) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hb = lane >> 5, hl = lane & 31;
  const int head = wave * 32 + hl;
  const bool head_ok = head < p.n_heads;

  // Q fragments (the A operand of S = Q . K^T: row = head hl, dims 16 ks + 8 hb .. +7)
  u32x4 qf[kDqk / 16];
  {
    const bf16_t* qrow = p.q + (int64_t)t * p.q_stride_t + (int64_t)(head_ok ? head : 0) * kDqk + hb * 8;
#pragma unroll
    for (int ks = 0; ks < kDqk / 16; ++ks) {
      const u32x4 v = gload16(qrow + ks * 16);
      qf[ks] = head_ok ? v : u32x4{0, 0, 0, 0};
    }
  }
  // lse2 of the lane's 16 accumulator rows: head 32w + (i/4)*8 + 4*hb + i%4; dead or absent
  // heads take +inf (their probabilities are then exactly 0)
  float lse2[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int h = wave * 32 + (i >> 2) * 8 + hb * 4 + (i & 3);
    const float l = h < p.n_heads ? p.lse[(int64_t)t * p.lse_stride_t + h] : -INFINITY;
    lse2[i] = l == -INFINITY ? INFINITY : l * kLog2e;
  }

  const int nblk =
      stage_index_row<NW>(sm.idx, sm.rmax, p.idx + (int64_t)t * p.idx_stride, p.topk, p.n_kv, p.causal, t);
  float* prow = p.target + (int64_t)t * p.target_stride;
  // slots past the last valid block are zero
  for (int j = nblk * kBK + threadIdx.x; j < p.topk; j += NW * 64) prow[j] = 0.f;
  if (nblk == 0) return;

  const uint32_t qk_v = key_row(hl) * kTileVPitch + 16u * hb;
  const uint32_t qk_r = kTileVBytes + hl * 128u + 16u * (hb ^ ((hl >> 1) & 7u));
  const uint32_t tile0 = lds_addr(sm.tile[0]);
  const float inv_h = 1.f / (float)p.n_heads;
  gather_tile<NW>(tile0, p.kv, sm.idx, wave, lane);
  if (nblk > 1) gather_tile<NW>(tile0 + kTileBytes, p.kv, sm.idx + kBK, wave, lane);
  uint32_t st_cur = 0, st_next = 2 * kTileBytes;
  for (int blk = 0; blk < nblk; ++blk) {
    if (blk + 1 < nblk) wait_vmcnt<G>(); else wait_vmcnt<0>();
    __syncthreads();
    const bool gather_next = blk + 2 < nblk;
    TileSrc<NW> next_src;
    if (gather_next) next_src = tile_sources<NW>(p.kv, sm.idx + (blk + 2) * kBK, wave, lane);
    const char* next_row = gather_next ? gather_row<NW>(next_src, 0) : nullptr;
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t next_tile = tile0 + st_next;
    const uint32_t tb = tile0 + st_cur;
    st_cur = st_cur == 2 * kTileBytes ? 0 : st_cur + kTileBytes;
    st_next = st_next == 2 * kTileBytes ? 0 : st_next + kTileBytes;
    uint32_t qv = tb + qk_v, qr = tb + qk_r;
    asm volatile("" : "+v"(qv), "+v"(qr));
    const bool key_ok = sm.idx[blk * kBK + hl] >= 0;

    // S[32 heads x 32 keys] = Q . K^T (K fragments prefetched kPre MFMAs ahead)
    f32x16 s;
    {
      auto addr = [&](int ks) { return lds_ptr(ks < 32 ? (qv + 32u * ks) : (qr ^ (32u * (ks - 32)))); };
      u32x4 a[kPre];
#pragma unroll
      for (int i = 0; i < kPre; ++i) a[i] = lds_load16(addr(i));
      f32x16 sa;
#pragma unroll
      for (int ks = 0; ks < kDqk / 16; ++ks) {
        const u32x4 cur = a[ks % kPre];
        if (ks + kPre < kDqk / 16) a[ks % kPre] = lds_load16(addr(ks + kPre));
        if (ks == 0) mfma32x32x16_cV_first(sa, qf[0], cur);
        else mfma32x32x16_cV(sa, qf[ks], cur);
        if (ks % kCopyEvery == 0 && gather_next) {
          gather_issue<NW>(next_tile, next_src, next_row, wave, lane, ks / kCopyEvery);
          next_row = gather_row<NW>(next_src, ks / kCopyEvery + 1);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      s = sa;
    }
    mfma_acc_drain();
    // head sum of the probabilities of key hl: 16 heads in the lane, the other 16 of the wave
    // in lane ^ 32, the other waves through LDS
    float r = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) r += fast_exp2(__builtin_fmaf(s[i], p.scale_log2, -lse2[i]));
    r += __shfl_xor(r, 32, 64);
    if (!key_ok) r = 0.f;
    if (hb == 0) sm.red[wave][hl] = r;
    __syncthreads();
    if (wave == 0 && hb == 0 && blk * kBK + hl < p.topk) {
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) sum += sm.red[w][hl];
      prow[blk * kBK + hl] = sum * inv_h;
    }
  }
}

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

int launch_indexer_kl_target(const KlTargetParams& p, hipStream_t stream) {
  if (p.n_xcd < 1) return -1;
  if (p.topk > kMaxTopkKl) return -2;
  if (p.total_q == 0) return 0;
  const dim3 grid(xcd_grid(p.total_q, p.n_xcd));
  const int nw = p.n_heads > 64 ? 4 : (p.n_heads > 32 ? 2 : 1);
  if (nw == 4) hipLaunchKernelGGL(indexer_kl_target_kernel<4>, grid, dim3(256), 0, stream, p);
  else if (nw == 2) hipLaunchKernelGGL(indexer_kl_target_kernel<2>, grid, dim3(128), 0, stream, p);
  else hipLaunchKernelGGL(indexer_kl_target_kernel<1>, grid, dim3(64), 0, stream, p);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_indexer_kl(const KlLossParams& p, hipStream_t stream) {
  if (p.total_q == 0) return 0;
  hipLaunchKernelGGL(indexer_kl_kernel, dim3(p.total_q), dim3(256), 0, stream, p);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace dsa
