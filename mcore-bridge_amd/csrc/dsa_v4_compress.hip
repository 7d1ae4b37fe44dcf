// DeepSeek-V4 compressor: softmax-gated window pooling + RMS norm, forward and backward (gfx950).
//
// The compressors of V4's compressed layers (the CSA layer's main and index compressors with
// overlapping windows, the HCA layer's without; parameters `ape`, `linear_wkv`, `linear_wgate`,
// `norm`, mapped by reference src/mcore_bridge/model/gpts/deepseek_v4.py:447-451) turn each
// complete window of `rate` tokens of a document into one compressed KV entry:
//   z[s, c] = gate[t_s, c] + ape[s, c],   p = softmax over the slots s of z,
//   P[c] = sum_s p_s kv[t_s, c],   x = bf16(P),   out = bf16(bf16(x * rsqrt(mean_c x^2 + eps)) * norm_w)
// With overlap the projections are C = 2D wide and an entry pools 2*rate slots: the previous
// window's first halves (channels [0, D), ape rows 0..rate-1) and this window's second halves
// ([D, 2D)); a document's first window has no previous one.  Without overlap C = D, rate slots.
//
// Layout: kv, gate [T, C] bf16 rows (row strides in elements), ape [rate, C] bf16, norm_w [D]
// bf16, entries [Nc, D] bf16 in document order.  doc_table: device int32 [3][n_docs + 1] --
// token offsets (cu_seqlens), entry offsets (prefix sums of len / rate) and item offsets (prefix
// sums of ceil(len / rate): the backward's work items, each complete window plus each document's
// partial tail, whose tokens get zero gradients).
//
// A group of D/8 lanes owns one entry (8 channels per lane, 16-byte loads and stores), so a wave
// holds 512/D entries.  The slots stream in chunks of 8 with an online softmax (one rescale per
// chunk; windows of <= 8 slots take none), so every kv / gate element is read from HBM once by the
// forward and once more by the backward, which recomputes the pooling (its second sweep re-reads
// the window from L2).  HBM-bound: the forward moves 2*C*2 bytes per token plus 2*D per entry.
//
// Backward (no atomics, fixed summation order, so bit-reproducible):
//   dy = dout * norm_w,  dx = r (dy - y <dy, y> / D)  (y = x r, r the rsqrt above),  dP = dx,
//   dkv[t_s] = dP p_s,  dgate[t_s] = dz_s = p_s dP (kv[t_s] - P),
//   dnorm_w = sum over entries of dout * bf16(y)   (per-workgroup partial rows, then a column sum),
//   dape[j, c] = sum of dgate[t, c] over the tokens t at window position j (uncovered gradient
//                elements are zero, so this is a strided column sum of dgate).
#include <algorithm>
#include <type_traits>

#include "dsa_common.h"
#include "dsa_kernels.h"

namespace dsa {

namespace {

constexpr int kWaves = 4;          // waves per workgroup (compressor kernels)
constexpr int kChunk = 8;          // slots per online-softmax chunk
constexpr int kChunkB = 4;         // slots per chunk of the backward's gradient sweep
constexpr int kBwdMaxWg = 1024;    // backward grid cap (rows of the dnorm partials)
constexpr int kApeMaxChunks = 256; // entry chunks of the dape column sum (rows of its partials)
constexpr int kApeTargetWg = 2048; // dape workgroups aimed for (chunks x rate x channel blocks)

// first index i in [0, n) with a[i] > x (n if none)
DSA_DEV int upper_bound_i32(const int32_t* a, int n, int x) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (a[mid] <= x) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

DSA_DEV void unpack8(const u32x4& v, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_lo(v[i]);
    f[2 * i + 1] = bf16_hi(v[i]);
  }
}

DSA_DEV u32x4 pack8(const float (&f)[8]) {
  u32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return v;
}

// sum over the LPE lanes of one entry's group (aligned power-of-two groups of the wave)
template <int LPE>
DSA_DEV float group_sum(float v) {
#pragma unroll
  for (int o = LPE / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// One entry's window: the rows, channels and ape rows of its slots.
struct Window {
  int tok;      // first token of the window
  int s_begin;  // first live slot (overlap, first window of a document: rate)
};

// The document of entry / item x from an offsets row (clamped: a malformed table cannot index
// outside it).
DSA_DEV int doc_of(const int32_t* off, int n_docs, int x) {
  return max(0, min(n_docs - 1, upper_bound_i32(off, n_docs + 1, x) - 1));
}

// Every row a window reads lies in [0, total_tokens) (false only for a malformed doc_table).
DSA_DEV bool window_in_range(const CompressParams& p, const Window& w) {
  const int lo = (p.overlap && w.s_begin == 0) ? w.tok - p.rate : w.tok;
  return lo >= 0 && w.tok + p.rate <= p.total_tokens;
}

// Slot s of a window: token row and channel offset (elements) of kv / gate, ape row.
DSA_DEV void slot_at(const CompressParams& p, const Window& w, int s, int c, int& row, int& ch, int& arow) {
  if (p.overlap) {
    if (s < p.rate) { row = w.tok - p.rate + s; ch = c; arow = s; }
    else { row = w.tok + s - p.rate; ch = p.dim + c; arow = s - p.rate; }
  } else {
    row = w.tok + s; ch = c; arow = s;
  }
}

// Partial pooling over slots [s_lo, s_hi) of a window for this lane's 8 channels (c .. c+7):
// running max m, normaliser l and numerator acc = sum_s e_s kv_s, with e_s = 2^((z_s - m) log2 e).
// Slots past s_hi in the last chunk re-load slot s_hi - 1 (an L1 hit) and take no weight, so a
// chunk has no branches.  An empty range leaves m = -inf, l = acc = 0.
DSA_DEV void pool_range(const CompressParams& p, const Window& w, int c, int s_lo, int s_hi, float (&m)[8],
                        float (&l)[8], float (&acc)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) { m[i] = -INFINITY; l[i] = 0.f; acc[i] = 0.f; }
#pragma unroll 1
  for (int s0 = s_lo; s0 < s_hi; s0 += kChunk) {
    u32x4 kr[kChunk], gr[kChunk], ar[kChunk];
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      int row, ch, arow;
      slot_at(p, w, min(s0 + i, s_hi - 1), c, row, ch, arow);
      kr[i] = gload16(p.kv + (int64_t)row * p.kv_stride + ch);
      gr[i] = gload16(p.gate + (int64_t)row * p.gate_stride + ch);
      ar[i] = gload16(p.ape + (int64_t)arow * p.channels + ch);
    }
    // z = gate + ape is formed twice (chunk max, then the exponentials) rather than held: the
    // chunk's raw rows already take 96 VGPRs
    float cm[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) cm[i] = -INFINITY;
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      float g[8], a[8];
      unpack8(gr[i], g);
      unpack8(ar[i], a);
#pragma unroll
      for (int j = 0; j < 8; ++j) cm[j] = fmaxf(cm[j], g[j] + a[j]);   // a re-loaded slot: no new max
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float mn = fmaxf(m[j], cm[j]);
      // rescale the running sums (m = -inf: they are still zero)
      const float alpha = m[j] == -INFINITY ? 0.f : fast_exp2((m[j] - mn) * kLog2e);
      l[j] *= alpha;
      acc[j] *= alpha;
      m[j] = mn;
    }
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      const bool live = s0 + i < s_hi;
      float k[8], g[8], a[8];
      unpack8(kr[i], k);
      unpack8(gr[i], g);
      unpack8(ar[i], a);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float e = live ? fast_exp2((g[j] + a[j] - m[j]) * kLog2e) : 0.f;
        l[j] += e;
        acc[j] = __builtin_fmaf(e, k[j], acc[j]);
      }
    }
  }
}

// The part of [s_begin, ns) that wave `part` of `nparts` pools (contiguous, near-equal).
DSA_DEV void split_range(int s_begin, int ns, int part, int nparts, int& lo, int& hi) {
  const int n = max(ns - s_begin, 0);
  const int q = (n + nparts - 1) / nparts;
  lo = s_begin + min(n, part * q);
  hi = s_begin + min(n, (part + 1) * q);
}

// Long windows (SPLIT > 1): the SPLIT waves of a workgroup pool contiguous parts of the same
// windows; their (m, l, acc) meet in LDS (component-major, conflict-free) and every wave leaves
// with the window's totals.  buf: [SPLIT][24][64] floats.
template <int SPLIT>
DSA_DEV void merge_parts(float (&m)[8], float (&l)[8], float (&acc)[8], float* buf, int wave, int lane) {
  if constexpr (SPLIT > 1) {
    float* mine = buf + wave * 24 * 64 + lane;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      mine[j * 64] = m[j];
      mine[(8 + j) * 64] = l[j];
      mine[(16 + j) * 64] = acc[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < SPLIT; ++w) M = fmaxf(M, buf[(w * 24 + j) * 64 + lane]);
      float L = 0.f, A = 0.f;
#pragma unroll
      for (int w = 0; w < SPLIT; ++w) {
        const float mw = buf[(w * 24 + j) * 64 + lane];
        const float sc = mw == -INFINITY ? 0.f : fast_exp2((mw - M) * kLog2e);
        L = __builtin_fmaf(buf[(w * 24 + 8 + j) * 64 + lane], sc, L);
        A = __builtin_fmaf(buf[(w * 24 + 16 + j) * 64 + lane], sc, A);
      }
      m[j] = M;
      l[j] = L;
      acc[j] = A;
    }
    __syncthreads();   // the buffer is rewritten by the next window
  }
}

// x = bf16(P); y = x * r with r = rsqrt(mean x^2 + eps) over the entry's D channels.
template <int LPE>
DSA_DEV float rms_of(const CompressParams& p, const float (&P)[8], float (&x)[8]) {
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    x[j] = (float)(bf16_t)P[j];
    ss = __builtin_fmaf(x[j], x[j], ss);
  }
  ss = group_sum<LPE>(ss);
  return rsqrtf(ss / (float)p.dim + p.eps);
}

// Waves per workgroup and entries (items) per workgroup: SPLIT == 1, four waves with their own
// entries; SPLIT > 1, SPLIT waves sharing each entry's slots.
template <int LPE, int SPLIT>
struct Shape {
  static constexpr int kEpw = 64 / LPE;
  static constexpr int kNw = SPLIT == 1 ? kWaves : SPLIT;
  static constexpr int kPerWg = SPLIT == 1 ? kWaves * kEpw : kEpw;
};

constexpr int wg_threads(int split) { return (split == 1 ? kWaves : split) * 64; }

// Window of entry / item in the forward: control flow is uniform over the workgroup (a lane
// without a live window pools an empty range and stores nothing), so the SPLIT barriers are met
// by every wave.
template <int LPE, int SPLIT>
__global__ __launch_bounds__(wg_threads(SPLIT)) void v4_compress_fwd_kernel(CompressParams p) {
  using S = Shape<LPE, SPLIT>;
  __shared__ float buf[SPLIT > 1 ? SPLIT * 24 * 64 : 1];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int e_raw = blockIdx.x * S::kPerWg + (SPLIT == 1 ? wave * S::kEpw : 0) + lane / LPE;
  const bool live = e_raw < p.n_entries;
  const int e = min(e_raw, p.n_entries - 1);
  const int c = 8 * (lane % LPE);
  const int32_t* cu = p.doc_table;
  const int32_t* coff = cu + p.n_docs + 1;
  const int d = doc_of(coff, p.n_docs, e);
  const int wi = e - coff[d];
  Window w{cu[d] + wi * p.rate, (p.overlap && wi == 0) ? p.rate : 0};
  const bool ok = window_in_range(p, w);
  const int ns = p.overlap ? 2 * p.rate : p.rate;
  int s_lo, s_hi;
  split_range(w.s_begin, ok ? ns : w.s_begin, SPLIT == 1 ? 0 : wave, SPLIT, s_lo, s_hi);
  float m[8], l[8], acc[8];
  pool_range(p, w, c, s_lo, s_hi, m, l, acc);
  merge_parts<SPLIT>(m, l, acc, buf, wave, lane);
  if (!live || (SPLIT > 1 && wave != 0)) return;
  float P[8], x[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) P[j] = ok ? acc[j] / l[j] : 0.f;
  const float r = rms_of<LPE>(p, P, x);
  float nw[8];
  unpack8(gload16(p.norm_w + c), nw);
  float o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = ok ? (float)(bf16_t)(x[j] * r) * nw[j] : 0.f;
  *reinterpret_cast<u32x4*>(p.out + (int64_t)e * p.dim + c) = pack8(o);
}

template <int LPE, int SPLIT>
__global__ __launch_bounds__(wg_threads(SPLIT)) void v4_compress_bwd_kernel(CompressParams p) {
  using S = Shape<LPE, SPLIT>;
  constexpr int NW = S::kNw;
  __shared__ float buf[SPLIT > 1 ? SPLIT * 24 * 64 : 1];
  __shared__ float red[NW][512];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int part = SPLIT == 1 ? 0 : wave;
  const int c = 8 * (lane % LPE);
  const int32_t* cu = p.doc_table;
  const int32_t* coff = cu + p.n_docs + 1;
  const int32_t* ioff = coff + p.n_docs + 1;
  const int C = p.channels;
  const int ns = p.overlap ? 2 * p.rate : p.rate;
  float nw[8];
  unpack8(gload16(p.norm_w + c), nw);
  float dnw[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const u32x4 zero4 = u32x4{0, 0, 0, 0};
#pragma unroll 1
  for (int it0 = blockIdx.x * S::kPerWg; it0 < p.n_items; it0 += gridDim.x * S::kPerWg) {
    const int it_raw = it0 + (SPLIT == 1 ? wave * S::kEpw : 0) + lane / LPE;
    const bool live = it_raw < p.n_items;
    const int it = min(it_raw, p.n_items - 1);
    const int d = doc_of(ioff, p.n_docs, it);
    const int wi = it - ioff[d];
    const int a = cu[d], len = cu[d + 1] - a;
    const int nwin = len / p.rate;
    const int tok = a + wi * p.rate;
    const bool tail = wi >= nwin;
    if (live && tail) {   // partial tail window: its tokens feed no entry (rows split over the parts)
      for (int t = max(tok, 0) + part; t < min(a + len, p.total_tokens); t += SPLIT) {
        for (int cc = c; cc < C; cc += p.dim) {
          *reinterpret_cast<u32x4*>(p.dkv + (int64_t)t * p.dkv_stride + cc) = zero4;
          *reinterpret_cast<u32x4*>(p.dgate + (int64_t)t * p.dgate_stride + cc) = zero4;
        }
      }
    }
    const int e = coff[d] + min(wi, max(nwin - 1, 0));
    Window w{tok, (p.overlap && wi == 0) ? p.rate : 0};
    const bool win = live && !tail && window_in_range(p, w);
    if (live && !tail && part == 0 && lane % LPE == 0) p.entry_tok[e] = win ? tok : -1;
    int s_lo, s_hi;
    split_range(w.s_begin, win ? ns : w.s_begin, part, SPLIT, s_lo, s_hi);
    float m[8], l[8], acc[8];
    pool_range(p, w, c, s_lo, s_hi, m, l, acc);
    merge_parts<SPLIT>(m, l, acc, buf, wave, lane);
    if (!win) continue;
    float P[8], x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) P[j] = acc[j] / l[j];
    const float r = rms_of<LPE>(p, P, x);
    float go[8], dy[8], y[8];
    unpack8(gload16(p.dout + (int64_t)e * p.dim + c), go);
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      y[j] = x[j] * r;
      if (part == 0) dnw[j] = __builtin_fmaf(go[j], (float)(bf16_t)y[j], dnw[j]);
      dy[j] = go[j] * nw[j];
      dot = __builtin_fmaf(dy[j], y[j], dot);
    }
    dot = group_sum<LPE>(dot) / (float)p.dim;
    float dP[8], inv_l[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      dP[j] = r * (dy[j] - y[j] * dot);
      inv_l[j] = 1.f / l[j];
    }
    // second sweep over this wave's slots: p_s, dkv = dP p_s, dgate = p_s dP (kv_s - P) (loads
    // clamped to the last slot as in the pooling, stores only for live slots)
#pragma unroll 1
    for (int s0 = s_lo; s0 < s_hi; s0 += kChunkB) {
      u32x4 kr[kChunkB], gr[kChunkB], ar[kChunkB];
      int64_t okv[kChunkB], og[kChunkB];
#pragma unroll
      for (int i = 0; i < kChunkB; ++i) {
        int row, ch, arow;
        slot_at(p, w, min(s0 + i, s_hi - 1), c, row, ch, arow);
        okv[i] = (int64_t)row * p.dkv_stride + ch;
        og[i] = (int64_t)row * p.dgate_stride + ch;
        kr[i] = gload16(p.kv + (int64_t)row * p.kv_stride + ch);
        gr[i] = gload16(p.gate + (int64_t)row * p.gate_stride + ch);
        ar[i] = gload16(p.ape + (int64_t)arow * C + ch);
      }
#pragma unroll
      for (int i = 0; i < kChunkB; ++i) {
        float k[8], g[8], av[8], dk[8], dz[8];
        unpack8(kr[i], k);
        unpack8(gr[i], g);
        unpack8(ar[i], av);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float pr = fast_exp2((g[j] + av[j] - m[j]) * kLog2e) * inv_l[j];
          dk[j] = dP[j] * pr;
          dz[j] = dk[j] * (k[j] - P[j]);
        }
        if (s0 + i < s_hi) {
          *reinterpret_cast<u32x4*>(p.dkv + okv[i]) = pack8(dk);
          *reinterpret_cast<u32x4*>(p.dgate + og[i]) = pack8(dz);
        }
      }
    }
    // overlap: the first halves of the document's last window feed no entry
    if (p.overlap && wi == nwin - 1) {
      for (int t = tok + part; t < tok + p.rate; t += SPLIT) {
        *reinterpret_cast<u32x4*>(p.dkv + (int64_t)t * p.dkv_stride + c) = zero4;
        *reinterpret_cast<u32x4*>(p.dgate + (int64_t)t * p.dgate_stride + c) = zero4;
      }
    }
  }
  // dnorm_w partial of this workgroup: sum over the wave's entry groups, then over its waves
#pragma unroll
  for (int j = 0; j < 8; ++j) {
#pragma unroll
    for (int o = LPE; o < 64; o <<= 1) dnw[j] += __shfl_xor(dnw[j], o, 64);
  }
  if (lane < LPE) {
#pragma unroll
    for (int j = 0; j < 8; ++j) red[wave][c + j] = dnw[j];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < p.dim; i += NW * 64) {
    float s = 0.f;
#pragma unroll
    for (int wv = 0; wv < NW; ++wv) s += red[wv][i];
    p.dnorm_part[(int64_t)blockIdx.x * p.dim + i] = s;
  }
}

// dape partial sums: workgroup (chunk, j, channel block of 512) adds the dgate rows at window
// position j of the chunk's entries (entry_tok, written by the backward kernel; -1: no window),
// lane: 8 channels, its waves taking every 4th entry.
__global__ __launch_bounds__(kWaves * 64) void v4_compress_dape_kernel(CompressParams p, int entries_per_chunk) {
  __shared__ float red[kWaves][512];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int chunk = blockIdx.x, j = blockIdx.y;
  const int c = blockIdx.z * 512 + 8 * lane;
  const int C = p.channels;
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const int e0 = chunk * entries_per_chunk;
  const int e1 = min(p.n_entries, e0 + entries_per_chunk);
  if (c < C) {
#pragma unroll 4
    for (int e = e0 + wave; e < e1; e += kWaves) {
      const int t0 = p.entry_tok[e];
      if (t0 < 0) continue;
      float g[8];
      unpack8(gload16(p.dgate + (int64_t)(t0 + j) * p.dgate_stride + c), g);
#pragma unroll
      for (int i = 0; i < 8; ++i) s[i] += g[i];
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) red[wave][8 * lane + i] = s[i];
  __syncthreads();
  for (int i = threadIdx.x; i < 512; i += kWaves * 64) {
    const int cc = blockIdx.z * 512 + i;
    if (cc < C) {
      float v = 0.f;
#pragma unroll
      for (int wv = 0; wv < kWaves; ++wv) v += red[wv][i];
      p.dape_part[((int64_t)chunk * p.rate + j) * C + cc] = v;
    }
  }
}

// out[n] = sum over rows r of part[r][n]: workgroup = 64 columns, its 16 waves split the rows.
__global__ __launch_bounds__(1024) void column_sum_kernel(const float* part, int rows, int n, float* out) {
  __shared__ float red[16][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + lane;
  float s[4] = {0.f, 0.f, 0.f, 0.f};   // four independent chains: four loads in flight per lane
  if (col < n) {
    int r = wave;
    for (; r + 48 < rows; r += 64) {
#pragma unroll
      for (int u = 0; u < 4; ++u) s[u] += part[(int64_t)(r + 16 * u) * n + col];
    }
    for (; r < rows; r += 16) s[0] += part[(int64_t)r * n + col];
  }
  red[wave][lane] = (s[0] + s[1]) + (s[2] + s[3]);
  __syncthreads();
  if (wave == 0 && col < n) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < 16; ++w) v += red[w][lane];
    out[col] = v;
  }
}

// Slots of a window and whether they are split over the waves of a workgroup (windows of 64 or
// more slots: HCA at rate 128 has few entries, T / 128, too few to fill the chip one wave each).
constexpr int kSplit = 8;
inline int split_of(int channels, int dim, int rate) {
  const int ns = channels == 2 * dim ? 2 * rate : rate;
  return ns >= 64 ? kSplit : 1;
}

template <typename F>
int by_shape(int dim, int split, F&& f) {
  auto go = [&](auto lpe) {
    return split > 1 ? f(lpe, std::integral_constant<int, kSplit>{}) : f(lpe, std::integral_constant<int, 1>{});
  };
  switch (dim) {
    case 64: return go(std::integral_constant<int, 8>{});
    case 128: return go(std::integral_constant<int, 16>{});
    case 256: return go(std::integral_constant<int, 32>{});
    case 512: return go(std::integral_constant<int, 64>{});
    default: return -2;
  }
}

}  // namespace

CompressBwdGrid compress_bwd_grid(int n_entries, int n_items, int channels, int dim, int rate) {
  CompressBwdGrid g{};
  const int per_wg = split_of(channels, dim, rate) > 1 ? 512 / dim : kWaves * (512 / dim);   // items per workgroup
  g.bwd_wg = std::max(1, std::min(kBwdMaxWg, (n_items + per_wg - 1) / per_wg));
  const int cblocks = (channels + 511) / 512;
  const int per_round = rate * cblocks;
  g.ape_chunks = std::max(1, std::min({kApeMaxChunks, (kApeTargetWg + per_round - 1) / per_round, n_entries}));
  g.entries_per_chunk = std::max(1, (n_entries + g.ape_chunks - 1) / g.ape_chunks);
  g.ape_chunks = std::max(1, (n_entries + g.entries_per_chunk - 1) / g.entries_per_chunk);
  g.dnorm_floats = (int64_t)g.bwd_wg * dim;
  g.dape_floats = (int64_t)g.ape_chunks * rate * channels;
  g.entry_ints = std::max(n_entries, 1);
  return g;
}

int launch_v4_compress_fwd(const CompressParams& p, hipStream_t stream) {
  if (p.n_entries == 0) return 0;
  return by_shape(p.dim, split_of(p.channels, p.dim, p.rate), [&](auto lpe, auto split) {
    constexpr int LPE = decltype(lpe)::value, SPLIT = decltype(split)::value;
    using S = Shape<LPE, SPLIT>;
    hipLaunchKernelGGL((v4_compress_fwd_kernel<LPE, SPLIT>), dim3((p.n_entries + S::kPerWg - 1) / S::kPerWg),
                       dim3(S::kNw * 64), 0, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -4;
  });
}

int launch_v4_compress_bwd(const CompressParams& p, float* dape, float* dnorm, hipStream_t stream) {
  const CompressBwdGrid g = compress_bwd_grid(p.n_entries, p.n_items, p.channels, p.dim, p.rate);
  if (p.n_items > 0) {
    const int rc = by_shape(p.dim, split_of(p.channels, p.dim, p.rate), [&](auto lpe, auto split) {
      constexpr int LPE = decltype(lpe)::value, SPLIT = decltype(split)::value;
      hipLaunchKernelGGL((v4_compress_bwd_kernel<LPE, SPLIT>), dim3(g.bwd_wg), dim3(Shape<LPE, SPLIT>::kNw * 64), 0,
                         stream, p);
      return hipGetLastError() == hipSuccess ? 0 : -4;
    });
    if (rc) return rc;
  }
  if (p.n_entries > 0)
    hipLaunchKernelGGL(v4_compress_dape_kernel, dim3(g.ape_chunks, p.rate, (p.channels + 511) / 512),
                       dim3(kWaves * 64), 0, stream, p, g.entries_per_chunk);
  hipLaunchKernelGGL(column_sum_kernel, dim3((p.rate * p.channels + 63) / 64), dim3(1024), 0, stream, p.dape_part,
                     p.n_entries > 0 ? g.ape_chunks : 0, p.rate * p.channels, dape);
  hipLaunchKernelGGL(column_sum_kernel, dim3((p.dim + 63) / 64), dim3(1024), 0, stream, p.dnorm_part,
                     p.n_items > 0 ? g.bwd_wg : 0, p.dim, dnorm);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace dsa
