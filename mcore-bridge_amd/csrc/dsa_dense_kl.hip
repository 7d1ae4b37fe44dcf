// Dense attention statistics of the dense indexer loss (gfx950): per-head LSE over every visible
// key, then the head-mean attention probability of every visible key.
//
// The reference's default indexer loss (dsa_indexer_loss_coeff > 0 with
// dsa_indexer_use_sparse_loss = False, src/mcore_bridge/config/model_config.py:204-205; the loss
// itself is megatron-core's compute_dsa_indexer_loss, third-party) targets the head-summed dense
// causal attention of each query over EVERY key of its document:
//   lse[t,h]    = ln sum_{j < len_t} exp(scale * q[t,h] . kv[base_t + j])
//   target[t,j] = (1/H) sum_h exp(scale * q[t,h] . kv[base_t + j] - lse[t,h])     (j < len_t)
// Only the QK product is needed (no value rows), and a query's keys are one contiguous range of
// kv rows (row_base / row_len of dsa_build_rows), so neither kernel takes an index row: block b
// of query t gathers rows base_t + 32b .. +31 straight into the sparse kernels' LDS tile ring.
//
//   dense_lse_kernel     S^T = K . Q^T (lane = head, 16 keys per lane), so a head's sum over keys
//       stays in its lane.  Against a per-head reference max fixed by the first block (2^64
//       headroom, the sparse forward's scheme) each element costs one fma, one exp2, one add
//       and one max; the whole query is recomputed with its exact maximum if a score overshoots.
//       That work for block b-1 runs in the issue slots between block b's QK MFMAs.
//   attn_target_kernel   S = Q . K^T (lane = key, 16 heads per lane): exp2(scale*s - lse) summed
//       over the lane's heads, its half-wave partner's and (through LDS) the other waves'.  Block
//       b-1's exps again run between block b's MFMAs, and its cross-wave sum is stored after the
//       barrier of block b+1: one barrier per block.
// One workgroup per query, wave w = heads 32w .. 32w+31, two workgroups per CU; the tile layout
// and the copy issue (M0 from an SGPR base, copies spread over the QK MFMAs, a copy-free instance
// of the MFMA sequence for the last block) are the sparse forward's.
#include "dsa_common.h"
#include "dsa_kernels.h"
#include "dsa_kvtile.h"

namespace dsa {

namespace {

constexpr int kDqk = 576;
constexpr int kBK = kTileKeys;
// Two ring stages (block b+1 copied during block b) and two workgroups per CU: each SIMD then
// holds two waves (<= 256 registers each), so one wave's exp work, barriers and copy waits run
// under the other's MFMAs (cfg3 dense rows: LSE 10.1 -> 8.3 ms, target 9.9 -> 8.2 ms against a
// 3-stage ring at one workgroup per CU).
constexpr int kStages = 2;
constexpr int kWgPerCu = 2;
constexpr int kPre = 3;                 // LDS operand prefetch distance (MFMAs)
constexpr float kHeadroom = 64.0f;      // log2 headroom above the reference max

struct DenseSmem {
  char tile[kStages][kTileBytes];
  float red[3][4][32];   // target: per-wave head sums of the keys of the last three blocks
  int32_t ids[3][64];    // sparse target: index-row slices of blocks b, b + 1, b + 2 (32 used)
  int flag;
};

// Gather sources of one block from a slice of an index row in LDS (ids[k] = kv row of key k of the
// block; entries outside kv load row 0 and are masked by the caller).
template <int NW>
DSA_DEV TileSrc<NW> index_sources(const bf16_t* kv, const int32_t* ids, int n_kv, int wave, int lane) {
  auto row = [&](int k) {
    const int x = ids[k];
    return x >= 0 && x < n_kv ? x : 0;
  };
  TileSrc<NW> s;
  s.v = kv_row_addr(kv, row(wave + NW * (lane % (32 / NW))));
#pragma unroll
  for (int j = 0; j < 4 / NW; ++j) {
    const int key = 8 * (wave + NW * j) + (lane >> 3);
    const uint32_t c = (uint32_t)(lane & 7) ^ ((key >> 1) & 7u);
    s.rope[j] = kv_row_addr(kv, row(key)) + (64 + c) * 16;
  }
  return s;
}

// Gather sources of one block of a contiguous key range: key k of the block is kv row row0 + k
// for k < nvalid; the others (past the row's end) load row0 and are masked by the caller.
template <int NW>
DSA_DEV TileSrc<NW> range_sources(const bf16_t* kv, int row0, int nvalid, int wave, int lane) {
  TileSrc<NW> s;
  const int kv_key = wave + NW * (lane % (32 / NW));
  s.v = kv_row_addr(kv, row0 + (kv_key < nvalid ? kv_key : 0));
#pragma unroll
  for (int j = 0; j < 4 / NW; ++j) {
    const int key = 8 * (wave + NW * j) + (lane >> 3);
    const uint32_t c = (uint32_t)(lane & 7) ^ ((key >> 1) & 7u);
    s.rope[j] = kv_row_addr(kv, row0 + (key < nvalid ? key : 0)) + (64 + c) * 16;
  }
  return s;
}

// All of this wave's copies of one tile, back to back (rows read two copies ahead, the first two
// behind one explicit 5-wait-state pad: the readlane -> SGPR -> LDS DMA distance).
template <int NW>
DSA_DEV void gather_range(uint32_t tile, const TileSrc<NW>& src, int wave, int lane) {
  constexpr int n = tile_copies_per_wave<NW>();
  const char* row[2] = {gather_row<NW>(src, 0), gather_row<NW>(src, 1)};
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 4");
#pragma unroll
  for (int k = 0; k < n; ++k) {
    gather_issue<NW>(tile, src, row[k & 1], wave, lane, k);
    if (k + 2 < n) row[k & 1] = gather_row<NW>(src, k + 2);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The query's key range, clipped to the kv rows: rows row_base .. row_base + len - 1 (a row with
// row_base < 0 or outside kv is empty).
DSA_DEV void query_range(const DenseKlParams& p, int t, int& row0, int& len) {
  row0 = p.row_base[t];
  len = p.row_len[t];
  if (row0 < 0 || row0 >= p.n_kv || len < 0) len = 0;
  else len = min(len, p.n_kv - row0);
}

// Q fragments of this lane's head: dims 16 ks + 8 hb .. +7 for every 16-deep k-step (the B operand
// of S^T = K . Q^T and the A operand of S = Q . K^T alike).
DSA_DEV void load_q(const DenseKlParams& p, int t, int head, bool head_ok, int hb, u32x4 (&qf)[kDqk / 16]) {
  const bf16_t* qrow = p.q + (int64_t)t * p.q_stride_t + (int64_t)(head_ok ? head : 0) * kDqk + hb * 8;
#pragma unroll
  for (int ks = 0; ks < kDqk / 16; ++ks) {
    const u32x4 v = gload16(qrow + ks * 16);
    qf[ks] = head_ok ? v : u32x4{0, 0, 0, 0};
  }
}

// One block's QK product over the tile at LDS address tb (36 MFMAs, K fragments prefetched kPre
// MFMAs ahead).  KQ: S^T = K . Q^T (the LSE kernel), else S = Q . K^T.  With GATHER, the next
// tile's copies (this wave's share, rows read two copies ahead) are spread over the MFMAs.  step(e)
// runs in the scheduling group of MFMA e, so independent VALU work issues under the matrix pipe.
template <int NW, bool KQ, bool GATHER, class Step>
DSA_DEV f32x16 qk_block(uint32_t tb, const u32x4 (&qf)[kDqk / 16], const TileDst& nd, const TileSrc<NW>& nsrc,
                        int lane, Step&& step) {
  constexpr int QKS = kDqk / 16;
  constexpr int kCopyEvery = QKS / tile_copies_per_wave<NW>();
  const int hl = lane & 31, hb = lane >> 5;
  uint32_t qv = tb + key_row(hl) * kTileVPitch + 16u * hb;
  uint32_t qr = tb + kTileVBytes + hl * 128u + 16u * (hb ^ ((hl >> 1) & 7u));
  asm volatile("" : "+v"(qv), "+v"(qr));
  auto addr = [&](int ks) { return lds_ptr(ks < 32 ? (qv + 32u * ks) : (qr ^ (32u * (ks - 32)))); };
  const char* next_row[2] = {nullptr, nullptr};
  if constexpr (GATHER) {
    next_row[0] = gather_row<NW>(nsrc, 0);
    next_row[1] = gather_row<NW>(nsrc, 1);
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4 a[kPre];
#pragma unroll
  for (int i = 0; i < kPre; ++i) a[i] = lds_load16(addr(i));
  f32x16 s;
  static_for<0, QKS>([&](auto ksc) {
    constexpr int ks = decltype(ksc)::value;
    const u32x4 cur = a[ks % kPre];
    if constexpr (ks + kPre < QKS) a[ks % kPre] = lds_load16(addr(ks + kPre));
    if constexpr (KQ) {
      if constexpr (ks == 0) mfma32x32x16_cV_first(s, cur, qf[0]);
      else mfma32x32x16_cV(s, cur, qf[ks]);
    } else {
      if constexpr (ks == 0) mfma32x32x16_cV_first(s, qf[0], cur);
      else mfma32x32x16_cV(s, qf[ks], cur);
    }
    if constexpr (GATHER && ks % kCopyEvery == 0) {
      constexpr int k = ks / kCopyEvery;
      gather_issue_at<NW, k>(nd, nsrc, next_row[k & 1], lane);
      next_row[k & 1] = gather_row<NW>(nsrc, k + 2);
    }
    step(ksc);
    __builtin_amdgcn_sched_barrier(0);
  });
  mfma_acc_drain();
  return s;
}

}  // namespace

// ------------------------------------------------------------------------------------------
// LSE: lse[t, h] over keys row_base[t] .. + row_len[t] - 1 (-inf for an empty row).
// ------------------------------------------------------------------------------------------
template <int NW>
__global__ __launch_bounds__(NW * 64, kWgPerCu) void dense_lse_kernel(DenseKlParams p) {
  __shared__ __attribute__((aligned(128))) DenseSmem sm;
  const int t = xcd_remap(blockIdx.x, p.n_xcd);
  if (t >= p.total_q) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hb = lane >> 5, hl = lane & 31;
  const int head = wave * 32 + hl;
  const bool head_ok = head < p.n_heads;
  int row0, len;
  query_range(p, t, row0, len);
  const int nblk = (len + kBK - 1) / kBK;
  if (nblk == 0) {
    if (head_ok && hb == 0) p.lse_out[(int64_t)t * p.n_heads + head] = -INFINITY;
    return;
  }
  u32x4 qf[kDqk / 16];
  load_q(p, t, head, head_ok, hb, qf);
  wait_vmcnt0();   // Q retired before the copies: nothing compiler-visible stays in flight

  const uint32_t tile0 = lds_addr(sm.tile[0]);
  const uint32_t wsg = __builtin_amdgcn_readfirstlane(wave);
  const float c2 = p.scale_log2;
  float m_ref = 0.f, m_seen = -INFINITY, l_run = 0.f;
  for (int pass = 0; pass < 2; ++pass) {
    l_run = 0.f;
    float mx = -INFINITY;   // this lane's raw score maximum (scaled into m_seen once per pass)
    gather_range<NW>(tile0, range_sources<NW>(p.kv, row0, len, wave, lane), wave, lane);
    f32x16 sp = f32x16{};   // S^T of the previous block (masked keys at -inf)
    uint32_t st_cur = 0, st_next = kTileBytes;
    for (int blk = 0; blk < nblk; ++blk) {
      wait_vmcnt<0>();   // block blk's copies (and any earlier store)
      __syncthreads();
      const bool gather_next = blk + 1 < nblk;
      TileSrc<NW> nsrc{};
      if (gather_next) nsrc = range_sources<NW>(p.kv, row0 + (blk + 1) * kBK, len - (blk + 1) * kBK, wave, lane);
      const TileDst nd = tile_dst<NW>(tile0 + st_next, wsg);
      const uint32_t tb = tile0 + st_cur;
      st_cur ^= kTileBytes;
      st_next ^= kTileBytes;
      // block blk-1's softmax terms, one element per QK MFMA (element e = key (e/4)*8 + 4 hb + e%4)
      auto step = [&](auto ec) {
        constexpr int e = decltype(ec)::value;
        if constexpr (e < 16) {
          mx = fmaxf(mx, sp[e]);
          l_run += fast_exp2(__builtin_fmaf(sp[e], c2, -m_ref));
        }
      };
      auto nostep = [](auto) {};
      f32x16 s;
      if (blk == 0) {
        s = gather_next ? qk_block<NW, true, true>(tb, qf, nd, nsrc, lane, nostep)
                        : qk_block<NW, true, false>(tb, qf, nd, nsrc, lane, nostep);
      } else {
        s = gather_next ? qk_block<NW, true, true>(tb, qf, nd, nsrc, lane, step)
                        : qk_block<NW, true, false>(tb, qf, nd, nsrc, lane, step);
      }
      const int nvalid = len - blk * kBK;
      if (nvalid < kBK) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = (i >> 2) * 8 + hb * 4 + (i & 3);
          if (key >= nvalid) s[i] = -INFINITY;
        }
      }
      if (blk == 0 && pass == 0) {   // the reference max: block 0 holds key 0, always valid
        float bm = s[0];
#pragma unroll
        for (int i = 1; i < 16; ++i) bm = fmaxf(bm, s[i]);
        m_ref = xor32_max(bm) * c2;
      }
      sp = s;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      mx = fmaxf(mx, sp[e]);
      l_run += fast_exp2(__builtin_fmaf(sp[e], c2, -m_ref));
    }
    m_seen = xor32_max(mx) * c2;
    // did any head overshoot its reference?  (workgroup-uniform: the tile ring is shared)
    const bool over = m_seen > m_ref + kHeadroom;
    if (threadIdx.x == 0) sm.flag = 0;
    __syncthreads();
    if (__any(over) && lane == 0) sm.flag = 1;
    __syncthreads();
    if (!sm.flag) break;
    m_ref = m_seen;
  }
  const float l = xor32_sum(l_run);
  if (head_ok && hb == 0) p.lse_out[(int64_t)t * p.n_heads + head] = (m_ref + __log2f(l)) * kLn2;
}

// ------------------------------------------------------------------------------------------
// Target: target[t, j] = (1/H) sum_h exp(scale * s - lse[t,h]) over the keys of row t: IDX = false,
// the dense row (key row_base[t] + j for j < min(row_len, pitch), 0 for the other columns j <
// pitch); IDX = true, the index row (key idx[t, j], 0 at entries that are none).  The index row is
// read in 32-entry slices, each copied into a 3-slot LDS ring two blocks before its tile's gather.
// ------------------------------------------------------------------------------------------
template <int NW, bool IDX>
__global__ __launch_bounds__(NW * 64, kWgPerCu) void attn_target_kernel(DenseKlParams p) {
  __shared__ __attribute__((aligned(128))) DenseSmem sm;
  const int t = xcd_remap(blockIdx.x, p.n_xcd);
  if (t >= p.total_q) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hb = lane >> 5, hl = lane & 31;
  const int head = wave * 32 + hl;
  const bool head_ok = head < p.n_heads;
  int row0 = 0, ncols;
  const int32_t* irow = nullptr;
  auto entry_ok = [&](int x) { return x >= 0 && x < p.n_kv && (!p.causal || x <= t); };
  if constexpr (IDX) {
    // the row's blocks end with its last entry that is a key: every load issued before any is used
    irow = p.idx + (int64_t)t * p.idx_stride;
    constexpr int kBatch = 8;
    int last = -1;
    for (int j0 = threadIdx.x; j0 < p.pitch; j0 += kBatch * NW * 64) {
      int v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int j = j0 + i * NW * 64;
        v[i] = j < p.pitch ? irow[j] : -1;
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i)
        if (entry_ok(v[i])) last = j0 + i * NW * 64;
    }
    last = wave_max_i(last);
    if (lane == 0) sm.red[0][wave][0] = __builtin_bit_cast(float, last);
    __syncthreads();
    last = -1;
#pragma unroll
    for (int w = 0; w < NW; ++w) last = max(last, __builtin_bit_cast(int, sm.red[0][w][0]));
    __syncthreads();
    ncols = last + 1;
  } else {
    int len;
    query_range(p, t, row0, len);
    ncols = min(len, p.pitch);
  }
  const int nblk = __builtin_amdgcn_readfirstlane((ncols + kBK - 1) / kBK);
  float* trow = p.target + (int64_t)t * p.target_stride;
  for (int j = nblk * kBK + threadIdx.x; j < p.pitch; j += NW * 64) trow[j] = 0.f;
  if (nblk == 0) return;
  u32x4 qf[kDqk / 16];
  load_q(p, t, head, head_ok, hb, qf);
  // lse2 of the lane's 16 accumulator rows: head 32w + (i/4)*8 + 4 hb + i%4; dead heads and
  // empty rows take +inf (their probabilities are then exactly 0)
  float lse2[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int h = wave * 32 + (i >> 2) * 8 + hb * 4 + (i & 3);
    const float v = h < p.n_heads ? p.lse[(int64_t)t * p.n_heads + h] : -INFINITY;
    lse2[i] = v == -INFINITY ? INFINITY : v * kLog2e;
  }
  wait_vmcnt0();   // Q and LSE retired before the copies

  const uint32_t tile0 = lds_addr(sm.tile[0]);
  const uint32_t ids0 = lds_addr(sm.ids[0]);
  const uint32_t wsg = __builtin_amdgcn_readfirstlane(wave);
  const float c2 = p.scale_log2;
  const float inv_h = 1.f / (float)p.n_heads;
  // index-row slice of block b into ring slot b % 3 (wave 0; entries 32b .. 32b + 63, clamped)
  auto copy_ids = [&](int b) {
    if (wave == 0) async_copy4_unordered(irow + min(kBK * b + lane, p.pitch - 1), ids0 + (b % 3) * 256u);
  };
  auto sources = [&](int b) {
    if constexpr (IDX) return index_sources<NW>(p.kv, sm.ids[b % 3], p.n_kv, wave, lane);
    else return range_sources<NW>(p.kv, row0 + b * kBK, ncols - b * kBK, wave, lane);
  };
  if constexpr (IDX) {
    copy_ids(0);
    if (nblk > 1) copy_ids(1);
    wait_vmcnt0();
    __syncthreads();
  }
  gather_range<NW>(tile0, sources(0), wave, lane);
  // block b's per-wave sums (key hl of the block) go to slot b % 3 in iteration b + 1; wave 0 stores
  // the block's columns after the barrier of iteration b + 2 (every wave's sum is in), and block
  // b + 3 reuses the slot only after the barrier of iteration b + 3 (or in the tail, after the
  // last iteration's barrier): each slot access is ordered by a barrier
  auto publish = [&](int b, float r, bool key_ok) {
    r = xor32_sum(r);
    if (b * kBK + hl >= ncols || !key_ok) r = 0.f;
    if (hb == 0) sm.red[b % 3][wave][hl] = r;
  };
  auto store = [&](int b) {
    if (wave == 0 && hb == 0) {
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) sum += sm.red[b % 3][w][hl];
      if (b * kBK + hl < p.pitch) trow[b * kBK + hl] = sum * inv_h;
    }
  };
  f32x16 sp = f32x16{};   // S of the previous block
  float r = 0.f;
  bool ok_prev = true;    // IDX: key hl of the previous block is a key
  uint32_t st_cur = 0, st_next = kTileBytes;
  for (int blk = 0; blk < nblk; ++blk) {
    wait_vmcnt<0>();   // block blk's copies, block blk + 1's index slice (and wave 0's earlier stores)
    __syncthreads();
    if (blk >= 2) store(blk - 2);
    bool ok_cur = true;
    if constexpr (IDX) {
      // this block's entry of key hl, read before the slot is refilled (three iterations on)
      const int x = sm.ids[blk % 3][hl];
      ok_cur = entry_ok(x);
      asm volatile("" ::"v"(ok_cur ? 1 : 0));
      if (blk + 2 < nblk) copy_ids(blk + 2);
    }
    const bool gather_next = blk + 1 < nblk;
    TileSrc<NW> nsrc{};
    if (gather_next) nsrc = sources(blk + 1);
    const TileDst nd = tile_dst<NW>(tile0 + st_next, wsg);
    const uint32_t tb = tile0 + st_cur;
    st_cur ^= kTileBytes;
    st_next ^= kTileBytes;
    // block blk-1's probabilities of key hl, one head per QK MFMA
    auto step = [&](auto ec) {
      constexpr int e = decltype(ec)::value;
      if constexpr (e < 16) r += fast_exp2(__builtin_fmaf(sp[e], c2, -lse2[e]));
    };
    auto nostep = [](auto) {};
    f32x16 s;
    if (blk == 0) {
      s = gather_next ? qk_block<NW, false, true>(tb, qf, nd, nsrc, lane, nostep)
                      : qk_block<NW, false, false>(tb, qf, nd, nsrc, lane, nostep);
    } else {
      s = gather_next ? qk_block<NW, false, true>(tb, qf, nd, nsrc, lane, step)
                      : qk_block<NW, false, false>(tb, qf, nd, nsrc, lane, step);
      publish(blk - 1, r, ok_prev);
      r = 0.f;
    }
    sp = s;
    ok_prev = ok_cur;
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) r += fast_exp2(__builtin_fmaf(sp[e], c2, -lse2[e]));
  publish(nblk - 1, r, ok_prev);
  __syncthreads();
  if (nblk >= 2) store(nblk - 2);
  store(nblk - 1);
}

int launch_dense_lse(const DenseKlParams& p, hipStream_t stream) {
  if (p.n_xcd < 1) return -1;
  if (p.total_q == 0) return 0;
  const dim3 grid(xcd_grid(p.total_q, p.n_xcd));
  const int nw = p.n_heads > 64 ? 4 : (p.n_heads > 32 ? 2 : 1);
  if (nw == 4) hipLaunchKernelGGL(dense_lse_kernel<4>, grid, dim3(256), 0, stream, p);
  else if (nw == 2) hipLaunchKernelGGL(dense_lse_kernel<2>, grid, dim3(128), 0, stream, p);
  else hipLaunchKernelGGL(dense_lse_kernel<1>, grid, dim3(64), 0, stream, p);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

template <bool IDX>
static int launch_target(const DenseKlParams& p, hipStream_t stream) {
  if (p.n_xcd < 1) return -1;
  if (p.total_q == 0) return 0;
  const dim3 grid(xcd_grid(p.total_q, p.n_xcd));
  const int nw = p.n_heads > 64 ? 4 : (p.n_heads > 32 ? 2 : 1);
  if (nw == 4) hipLaunchKernelGGL((attn_target_kernel<4, IDX>), grid, dim3(256), 0, stream, p);
  else if (nw == 2) hipLaunchKernelGGL((attn_target_kernel<2, IDX>), grid, dim3(128), 0, stream, p);
  else hipLaunchKernelGGL((attn_target_kernel<1, IDX>), grid, dim3(64), 0, stream, p);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_dense_target(const DenseKlParams& p, hipStream_t stream) { return launch_target<false>(p, stream); }
int launch_sparse_target(const DenseKlParams& p, hipStream_t stream) { return launch_target<true>(p, stream); }

}  // namespace dsa
