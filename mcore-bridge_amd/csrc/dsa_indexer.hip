// K1: lightning-indexer scores, K2: per-row top-k selection (gfx950).
//
// Replaces fused_qk_topk_naive(q, k, weights, index_topk, mask) as called from
// DSAIndexer.forward_with_scores (reference src/mcore_bridge/patcher.py:358):
//   I[t, s] = sum_h w[t,h] * relu(q[t,h,:] . k[s,:])      (fp32 accumulate)
//   topk_indices[t] = the min(K, n_t) largest I[t, .] over the visible keys, ties -> lower key.
// A query row is described by (row_base, row_len): its visible keys are row_base + [0, row_len).
// Prefill with documents: row_base = document start, row_len = t - start + 1 (causal) or the
// document length; decode: row_base = cache offset, row_len = cache length.  Scores are written
// row-major with column j <-> key row_base + j, which is also the layout of the reference's
// returned index_scores when there is one document.
//
// K1: one wave = one (query, key chunk of 256..4096 keys; shorter chunks when there are few
// queries, e.g. decode, so that enough waves stream keys at once).  Q[64 heads x 128] stays in registers as the A
// operand (row = head), key rows are the B operand loaded straight from global memory (256 B
// per key, shared by the 4 waves of a workgroup through L1/L2); C[heads x 32 keys] is reduced
// over heads in registers: each lane holds 16 heads of one key, so ReLU * w and the head sum
// are lane-local plus one exchange with the lane 32 apart.
// At most 512 queries of 128-dim rows (decode) K1 runs as indexer_scores_rows_kernel (bf16) or
// indexer_scores_rows_fp8_kernel instead: one query per workgroup, key rows staged in LDS by
// contiguous LDS-direct copies.
// fp8 (OCP e4m3fn): gfx950's 32x32x64 fp8 MFMA (twice the bf16 rate per instruction), through
// the same LDS ring as bf16 when a workgroup's queries share a document;
// I = k_scale[s] * sum_h (w * q_scale)[t,h] * relu(q8 . k8) -- valid because ReLU is
// positive-homogeneous and both scales are > 0.
//
// K2: one workgroup per row, over order-preserving uint32 keys of the fp32 scores.  Rows of
// 4096 .. 65536 entries with K small against them take the sampled-threshold path
// (block_select_topk_sampled): a bound from a 2048-entry sample, one streaming pass collecting
// the ~1.5 K entries above it, the exact K-th largest selected over those candidates, and the
// selection emitted through a position bitmap.  Other rows (and rows whose bound misses): 4
// passes of 8-bit MSB-first radix select (LDS histograms, the row cached in LDS when it fits,
// else a three-pass candidate path over global memory) find the exact K-th largest value; one
// stable compaction pass (each wave ranks 64 consecutive keys per step with ballots) then emits
// every larger key plus the lowest-index ties.  Every path emits the same indices: ascending key
// order, -1 padded.  Fewer than 256 rows longer than a slice (decode) are split: a workgroup
// per (row, 16384-key slice) keeps the slice's top-K, one per row then selects from those.
#include <algorithm>
#include "dsa_common.h"
#include "dsa_kernels.h"

namespace dsa {

namespace {
// keys per workgroup work item (prefill); 4096 against 2048: cfg4's fp8 scores 4.66 -> 4.39 ms
// (half the per-workgroup setups: Q, weights and key-scale staging, each a memory round trip)
constexpr int kIdxChunkMax = 4096;
// fp8 key-block ring depth (4 KB stages): 4 against 3 measured 4.66 vs 4.89 ms at cfg4 (6: 4.70)
constexpr int kFp8Stages = 4;
constexpr int kIdxChunkMin = 256;
constexpr int kIdxWaveTarget = 8192;   // shrink the chunk until this many work items exist
constexpr int kRowsMode = 512;      // at most this many queries (128-dim rows): the rows kernels
constexpr int kMaxHi = 64;          // indexer heads handled by the register tiling
}  // namespace

// Slot of 16-byte chunk c of LDS row r is c ^ row_swz<RB>(r).  ds_read_b128 serves 16 lanes per
// cycle from gfx950's 64 banks (a 256-byte window), and the operand reads here take one chunk of
// 16 consecutive rows at a time: rows of 256 bytes all start in bank 0, so the 16 rows need 16
// distinct slots (c ^ (r & 15)); rows of 128 bytes pair up in a window, so rows r and r ^ 1 may
// share a slot but r and r + 2k may not (c ^ ((r >> 1) & 7)).  (An XOR with r & 7 leaves rows r
// and r + 8 on the same banks: 2-way conflicts, ~45 % of the LDS cycles in the counters.)
template <int RB>
DSA_DEV int row_swz(int r) {
  static_assert(RB == 256 || RB == 128, "LDS rows of 256 or 128 bytes");
  return RB == 256 ? (r & 15) : ((r >> 1) & 7);
}

// sum_e w[0][e] relu(c0[e]) + sum_e w[1][e] relu(c1[e]) for the lane's 16 + 16 accumulator rows
// (heads): one fma chain, tile 0 then tile 1 (the order of indexer_sel_kernel), ReLU by
// relu_bits: 2 VALU instructions per head (v_max_i32, v_fmac_f32) instead of ~3.5 (two v_max_f32
// per fmaxf, and a mul / fmac / add per pair of heads).
DSA_DEV float weighted_relu_sum(const float (&w)[2][16], const f32x16& c0, const f32x16& c1) {
  float acc = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc = __builtin_fmaf(w[0][e], relu_bits(c0[e]), acc);
#pragma unroll
  for (int e = 0; e < 16; ++e) acc = __builtin_fmaf(w[1][e], relu_bits(c1[e]), acc);
  return acc;
}

// bf16 scores of a workgroup whose 4 queries share a document (the same key rows): each 32-key
// block is copied into LDS once (LDS-direct, 3-stage ring) and all 4 waves take their B
// operands from there -- loaded per wave, every key row went through the L1 4 times and the
// key loads alone used the CU's whole 64 B/clk load path.  Row r of a block: 16-byte unit u at
// slot u ^ row_swz<RB>(r) (16 consecutive lanes read 16 rows at one unit: conflict-free).  The loop runs
// to the longest of the 4 rows; a wave stores only its own columns.
template <int DI>
DSA_DEV void indexer_block_lds(const IndexerParams& p, int t, int c0, int c1_wg, int c1, int base, float (&wr)[2][16],
                               const u32x4 (&qa)[2][8], char* ring) {
  constexpr int RB = DI * 2;                 // bytes per key row
  constexpr int U = RB / 16;                 // 16-byte units per row
  constexpr int CPB = 32 * RB / 1024;        // 1 KB copies per block (8 or 4)
  constexpr int CPW = CPB / 4;               // per wave
  constexpr int BLK = 32 * RB;               // bytes per staged block
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hb = lane >> 5, hl = lane & 31;
  const int wu = __builtin_amdgcn_readfirstlane(wave);
  const char* kbase = reinterpret_cast<const char*>(p.k);
  const uint32_t ring0 = lds_addr(ring);
  auto issue = [&](int blk, int k0) {        // this wave's copies of the block at key k0
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const int ci = wu * CPW + c;           // copy index within the block
      const int r = ci * (1024 / RB) + lane / U, u = lane % U;
      const int key = base + min(k0 + r, c1_wg - 1);
      async_copy16_unordered(kbase + (int64_t)key * RB + 16 * (u ^ row_swz<RB>(r)),
                             __builtin_amdgcn_readfirstlane(ring0 + (uint32_t)((blk % 3) * BLK + ci * 1024)));
    }
  };
  const int nb = (c1_wg - c0 + 31) / 32;
  issue(0, c0);
  if (nb > 1) issue(1, c0 + 32);
  for (int i = 0; i < nb; ++i) {
    if (i + 1 < nb) wait_vmcnt<CPW>(); else wait_vmcnt<0>();
    __syncthreads();
    if (i + 2 < nb) issue(i + 2, c0 + 32 * (i + 2));
    const char* row = ring + (i % 3) * BLK + hl * RB;
    u32x4 kb[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      kb[ks] = ks < DI / 16 ? lds_load16(row + 16 * ((2 * ks + hb) ^ row_swz<RB>(hl))) : u32x4{0, 0, 0, 0};
    f32x16 c0a = f32x16{}, c1a = f32x16{};
#pragma unroll
    for (int ks = 0; ks < DI / 16; ++ks) {
      c0a = mfma32x32x16(as_bf16x8(qa[0][ks]), as_bf16x8(kb[ks]), c0a);
      c1a = mfma32x32x16(as_bf16x8(qa[1][ks]), as_bf16x8(kb[ks]), c1a);
    }
    float acc = weighted_relu_sum(wr, c0a, c1a);
    acc = xor32_sum(acc);
    const int j = c0 + 32 * i + hl;
    if (hb == 0 && j < c1) p.scores[(int64_t)t * p.pitch + j] = acc;
  }
}

typedef int i32x8 __attribute__((ext_vector_type(8)));

// gfx950's fp8 MFMA: C[32x32] += A[32x64] * B[64x32] on OCP e4m3fn (format code 0 for A and B), no
// block scales.  Lane l holds 32 consecutive k of row / column l % 32; the k order inside one
// MFMA only has to agree between A and B, so both take k = 32 * (l / 32) + 0..31 of a 64-wide step.
DSA_DEV f32x16 mfma32x32x64_fp8(const i32x8& a, const i32x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

DSA_DEV i32x8 cat16(const u32x4& lo, const u32x4& hi) {
  return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

// fp8 (e4m3fn, 128-dim rows) scores of a workgroup whose 4 queries share a document: the LDS ring
// of the bf16 path with 128-byte key rows (4 KB per 32-key block, one 1 KB LDS-direct copy per
// wave), two 32x32x64 fp8 MFMAs per row tile and block, and the chunk's k_scale values staged in
// LDS once (I = k_scale[s] * sum_h (w q_scale)[t,h] relu(q8 . k8)).  Row r of a block: 16-byte unit
// u at slot u ^ row_swz<128>(r) (the operand reads of 16 consecutive keys are conflict-free).
DSA_DEV void indexer_block_lds_fp8(const IndexerParams& p, int t, int c0, int c1_wg, int c1, int base,
                                   float (&wr)[2][16], const i32x8 (&qa)[2][2], char* ring, float* ks_s) {
  constexpr int RB = 128, BLK = 32 * RB;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hb = lane >> 5, hl = lane & 31;
  const int wu = __builtin_amdgcn_readfirstlane(wave);
  const char* kbase = reinterpret_cast<const char*>(p.k);
  const uint32_t ring0 = lds_addr(ring);
  // the chunk's key scales, through compiler-visible loads retired before the first copy
  for (int j = threadIdx.x; j < c1_wg - c0; j += 256) ks_s[j] = p.k_scale[base + c0 + j];
  wait_vmcnt0();
  auto issue = [&](int blk, int k0) {        // copy wu of the block at key k0: rows 8 wu .. 8 wu + 7
    const int r = wu * 8 + (lane >> 3), u = lane & 7;
    const int key = base + min(k0 + r, c1_wg - 1);
    async_copy16_unordered(kbase + (int64_t)key * RB + 16 * (u ^ row_swz<RB>(r)),
                           __builtin_amdgcn_readfirstlane(ring0 + (uint32_t)((blk % kFp8Stages) * BLK + wu * 1024)));
  };
  const int nb = (c1_wg - c0 + 31) / 32;
#pragma unroll
  for (int b = 0; b < kFp8Stages - 1; ++b)
    if (b < nb) issue(b, c0 + 32 * b);
  for (int i = 0; i < nb; ++i) {
    if (i + kFp8Stages - 2 < nb) wait_vmcnt<kFp8Stages - 2>(); else wait_vmcnt<0>();
    __syncthreads();
    if (i + kFp8Stages - 1 < nb) issue(i + kFp8Stages - 1, c0 + 32 * (i + kFp8Stages - 1));
    const char* row = ring + (i % kFp8Stages) * BLK + hl * RB;
    i32x8 kb[2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const int u0 = 4 * st + 2 * hb;
      kb[st] = cat16(lds_load16(row + 16 * (u0 ^ row_swz<128>(hl))), lds_load16(row + 16 * ((u0 + 1) ^ row_swz<128>(hl))));
    }
    f32x16 c0a = f32x16{}, c1a = f32x16{};
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      c0a = mfma32x32x64_fp8(qa[0][st], kb[st], c0a);
      c1a = mfma32x32x64_fp8(qa[1][st], kb[st], c1a);
    }
    float acc = weighted_relu_sum(wr, c0a, c1a);
    acc = xor32_sum(acc);
    const int j = c0 + 32 * i + hl;
    if (hb == 0 && j < c1) p.scores[(int64_t)t * p.pitch + j] = acc * ks_s[j - c0];
  }
}

template <bool FP8>
__global__ __launch_bounds__(256) void indexer_scores_kernel(IndexerParams p) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  const int c0 = blockIdx.y * p.chunk;
  const int Di = p.head_dim;        // 64 or 128
  const int nks = Di / 16;          // 4 or 8 k-steps of 16
  const int hb = lane >> 5, hl = lane & 31;
  if (!FP8 || Di == 128) {
    // shared-key path: the workgroup's queries (all valid) lie in one document and the chunk
    // is not past the longest row (workgroup-uniform decisions, before any early return)
    const int t0 = blockIdx.x * 4;
    bool shared = t0 + 3 < p.total_q;
    int c1_wg = 0;
    if (shared) {
      const int b0 = p.row_base[t0];
      for (int i = 0; i < 4; ++i) {
        shared = shared && p.row_base[t0 + i] == b0;
        c1_wg = max(c1_wg, min(p.row_len[t0 + i], c0 + p.chunk));
      }
    }
    if (shared) {
      if (c0 >= c1_wg) return;
      __shared__ __attribute__((aligned(16))) char ring[3 * 32 * 256];
      const int len = p.row_len[t];
      const int c1 = min(len, c0 + p.chunk);   // this wave stores columns < c1
      const int base = p.row_base[t];
      float wr[2][16];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int h = 32 * mt + (i >> 2) * 8 + 4 * hb + (i & 3);
          float w = h < p.n_heads ? p.w[(int64_t)t * p.n_heads + h] : 0.f;
          if (FP8 && h < p.n_heads) w *= p.q_scale[(int64_t)t * p.n_heads + h];
          wr[mt][i] = w;
        }
      }
      if constexpr (FP8) {
        __shared__ float ks_s[kIdxChunkMax];
        const uint8_t* q8 = reinterpret_cast<const uint8_t*>(p.q) + (int64_t)t * p.n_heads * 128;
        i32x8 qa8[2][2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const int h = 32 * mt + hl;
#pragma unroll
          for (int st = 0; st < 2; ++st) {
            const uint8_t* src = q8 + (int64_t)(h < p.n_heads ? h : 0) * 128 + 64 * st + 32 * hb;
            const u32x4 lo = gload16(src), hi = gload16(src + 16);
            qa8[mt][st] = h < p.n_heads ? cat16(lo, hi) : i32x8{};
          }
        }
        wait_vmcnt0();
        static_assert(kFp8Stages >= 3 && kFp8Stages * 32 * 128 <= (int)sizeof(ring), "fp8 ring stages fit the ring");
        indexer_block_lds_fp8(p, t, c0, c1_wg, c1, base, wr, qa8, ring, ks_s);
        return;
      }
      const bf16_t* q = reinterpret_cast<const bf16_t*>(p.q) + (int64_t)t * p.n_heads * Di;
      u32x4 qa[2][8];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int h = 32 * mt + hl;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
          qa[mt][ks] = (h < p.n_heads && ks < nks) ? gload16(q + (int64_t)h * Di + 16 * ks + 8 * hb) : u32x4{0, 0, 0, 0};
      }
      wait_vmcnt0();   // Q and w loaded: only the ring copies are counted below
      if (Di == 128) indexer_block_lds<128>(p, t, c0, c1_wg, c1, base, wr, qa, ring);
      else indexer_block_lds<64>(p, t, c0, c1_wg, c1, base, wr, qa, ring);
      return;
    }
  }
  if (t >= p.total_q) return;
  const int len = p.row_len[t];
  if (c0 >= len) return;
  const int c1 = min(len, c0 + p.chunk);
  const int base = p.row_base[t];

  // per-lane weights for the 16 head rows of each of the 2 row tiles (heads >= n_heads -> 0)
  float wr[2][16];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int h = 32 * mt + (i >> 2) * 8 + 4 * hb + (i & 3);
      float w = h < p.n_heads ? p.w[(int64_t)t * p.n_heads + h] : 0.f;
      if (FP8 && h < p.n_heads) w *= p.q_scale[(int64_t)t * p.n_heads + h];
      wr[mt][i] = w;
    }
  }
  if (!FP8) {
    const bf16_t* q = reinterpret_cast<const bf16_t*>(p.q) + (int64_t)t * p.n_heads * Di;
    const bf16_t* k = reinterpret_cast<const bf16_t*>(p.k);
    u32x4 qa[2][8];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int h = 32 * mt + hl;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks)
        qa[mt][ks] = (h < p.n_heads && ks < nks) ? gload16(q + (int64_t)h * Di + 16 * ks + 8 * hb) : u32x4{0, 0, 0, 0};
    }
    // key block k0: lane reads key min(k0 + hl, c1 - 1) (the tail lanes re-read a valid row)
    auto load_keys = [&](int k0, u32x4 (&dst)[8]) {
      const bf16_t* krow = k + (int64_t)(base + min(k0 + hl, c1 - 1)) * Di + 8 * hb;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) dst[ks] = ks < nks ? gload16(krow + 16 * ks) : u32x4{0, 0, 0, 0};
    };
    u32x4 kn[8];
    load_keys(c0, kn);
    for (int k0 = c0; k0 < c1; k0 += 32) {
      const int j = k0 + hl;
      u32x4 kb[8];
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) kb[ks] = kn[ks];
      if (k0 + 32 < c1) load_keys(k0 + 32, kn);   // next block streams in under this one's MFMAs
      f32x16 c0a = f32x16{}, c1a = f32x16{};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        c0a = mfma32x32x16(as_bf16x8(qa[0][ks]), as_bf16x8(kb[ks]), c0a);
        c1a = mfma32x32x16(as_bf16x8(qa[1][ks]), as_bf16x8(kb[ks]), c1a);
      }
      float acc = weighted_relu_sum(wr, c0a, c1a);
      acc = xor32_sum(acc);
      if (hb == 0 && j < c1) p.scores[(int64_t)t * p.pitch + j] = acc;
    }
  } else {
    // gfx950's 32x32x64 fp8 MFMA: Di / 64 steps, lane holds 32 consecutive bytes of a row
    const uint8_t* q = reinterpret_cast<const uint8_t*>(p.q) + (int64_t)t * p.n_heads * Di;
    const uint8_t* k = reinterpret_cast<const uint8_t*>(p.k);
    const int nst = Di / 64;
    i32x8 qa[2][2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int h = 32 * mt + hl;
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const uint8_t* src = q + (int64_t)(h < p.n_heads ? h : 0) * Di + 64 * st + 32 * hb;
        qa[mt][st] = (h < p.n_heads && st < nst) ? cat16(gload16(src), gload16(src + 16)) : i32x8{};
      }
    }
    auto load_keys = [&](int k0, i32x8 (&dst)[2]) {
      const uint8_t* krow = k + (int64_t)(base + min(k0 + hl, c1 - 1)) * Di + 32 * hb;
#pragma unroll
      for (int st = 0; st < 2; ++st)
        dst[st] = st < nst ? cat16(gload16(krow + 64 * st), gload16(krow + 64 * st + 16)) : i32x8{};
    };
    i32x8 kn[2];
    load_keys(c0, kn);
    for (int k0 = c0; k0 < c1; k0 += 32) {
      const int j = k0 + hl;
      const int key = base + min(j, c1 - 1);
      i32x8 kb[2] = {kn[0], kn[1]};
      if (k0 + 32 < c1) load_keys(k0 + 32, kn);
      f32x16 c0a = f32x16{}, c1a = f32x16{};
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        if (st < nst) {
          c0a = mfma32x32x64_fp8(qa[0][st], kb[st], c0a);
          c1a = mfma32x32x64_fp8(qa[1][st], kb[st], c1a);
        }
      }
      float acc = weighted_relu_sum(wr, c0a, c1a);
      acc = xor32_sum(acc);
      if (hb == 0 && j < c1) p.scores[(int64_t)t * p.pitch + j] = acc * p.k_scale[key];
    }
  }
}

// Few long rows (decode; bf16, 128-dim rows): one query per workgroup, its 4 waves on 4 consecutive
// key chunks. The query's Q rows are staged once in LDS (chunk u of head row h at u ^ row_swz<256>(h): the
// A-operand reads of 8 consecutive heads are conflict-free) and its head weights sit in registers.
// Key rows reach LDS through contiguous LDS-direct copies, 1 KB (4 whole rows) per instruction,
// into a 2-stage ring per wave. The per-lane row loads of indexer_scores_kernel touch 32 rows of
// 32 B per instruction; at decode's few, very long rows that access pattern, not latency or
// occupancy, was what held the scan back (cfg5: ~200 us there, ~163 us here, same scores bit for
// bit). Deeper rings (3-4 stages) cost a workgroup per CU of LDS and ran slower.  The copies
// carry the non-temporal hint: each key row is read once, and keeping the stream out of the
// caches' normal replacement took the cfg5 scan from ~171 to ~151 us.
__global__ __launch_bounds__(256) void indexer_scores_rows_kernel(IndexerParams p) {
  // Q rows (chunk u of head row h at u ^ row_swz<256>(h)), head weights, and per wave a 2-stage ring of
  // 32-key blocks (chunk c of key r at c ^ row_swz<256>(r)) filled by contiguous LDS-direct copies
  __shared__ __attribute__((aligned(256))) char qs[kMaxHi * 256];
  __shared__ __attribute__((aligned(256))) char ring[4][2][32 * 256];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t = blockIdx.x;
  const int hb = lane >> 5, hl = lane & 31;
  constexpr int Di = 128, nks = Di / 16, RB = Di * 2;   // the launcher routes only 128-dim rows here
  const bf16_t* q = reinterpret_cast<const bf16_t*>(p.q) + (int64_t)t * p.n_heads * Di;
  for (int c = threadIdx.x; c < kMaxHi * 16; c += 256) {
    const int h = c >> 4, u = c & 15;
    const u32x4 v = h < p.n_heads ? gload16(q + (int64_t)h * Di + 8 * u) : u32x4{0, 0, 0, 0};
    lds_store16(qs + h * 256 + 16 * (u ^ row_swz<256>(h)), v);
  }
  float wr[2][16];   // weights of the accumulator rows: heads 32 mt + (i/4)*8 + 4 hb + i%4
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int h = 32 * mt + (i >> 2) * 8 + 4 * hb + (i & 3);
      wr[mt][i] = h < p.n_heads ? p.w[(int64_t)t * p.n_heads + h] : 0.f;
    }
  const int c0 = ((int)blockIdx.y * 4 + wave) * p.chunk;
  const int len = p.row_len[t];
  const int base = p.row_base[t];
  wait_vmcnt0();   // compiler-visible loads retired before the copies start
  __syncthreads();
  if (c0 >= len) return;
  const int c1 = min(len, c0 + p.chunk);
  const char* kbase = reinterpret_cast<const char*>(p.k);
  const uint32_t ring0 = lds_addr(ring[wave][0]);
  // copy r of a block moves keys 4r .. 4r+3 -- 1 KB contiguous in memory: lane l fills
  // slot l & 15 of key 4r + l / 16 with that key's chunk (l & 15) ^ row_swz<256>(key)
  auto gather = [&](uint32_t dst, int k0) {
    const int kk0 = lane >> 4;
    const uint32_t sl = lane & 15;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int kk = 4 * r + kk0;
      const int row = base + min(k0 + kk, c1 - 1);
      const char* src = kbase + (int64_t)row * RB + 16u * (sl ^ row_swz<256>(kk));
      async_copy16_nt(src, dst + 1024u * r);   // each key row is read once: non-temporal
    }
  };
  const uint32_t qa0 = lds_addr(qs) + hl * 256, qa1 = lds_addr(qs) + (32 + hl) * 256;
  gather(ring0, c0);
  int it = 0;
  for (int k0 = c0; k0 < c1; k0 += 32, ++it) {
    const int j = k0 + hl;
    const uint32_t tb = ring0 + (it & 1) * (32 * 256);
    if (it == 0) wait_vmcnt<0>();
    else wait_vmcnt<1>();   // issued after this block's copies: the previous block's score store
    asm volatile("" ::: "memory");
    if (k0 + 32 < c1) gather(ring0 + ((it + 1) & 1) * (32 * 256), k0 + 32);
    uint32_t a0b = qa0, a1b = qa1, kb = tb + hl * 256;
    asm volatile("" : "+v"(a0b), "+v"(a1b), "+v"(kb));
    f32x16 c0a = f32x16{}, c1a = f32x16{};
#pragma unroll
    for (int ks = 0; ks < nks; ++ks) {
      const uint32_t u = 16u * ((2 * ks + hb) ^ row_swz<256>(hl));
      const u32x4 a0 = lds_load16(lds_ptr(a0b + u)), a1 = lds_load16(lds_ptr(a1b + u));
      const u32x4 b = lds_load16(lds_ptr(kb + u));
      c0a = mfma32x32x16(as_bf16x8(a0), as_bf16x8(b), c0a);
      c1a = mfma32x32x16(as_bf16x8(a1), as_bf16x8(b), c1a);
    }
    float acc = weighted_relu_sum(wr, c0a, c1a);
    acc = xor32_sum(acc);
    if (hb == 0 && j < c1) p.scores[(int64_t)t * p.pitch + j] = acc;
  }
}

// Few long rows, fp8 (decode; e4m3fn, 128-dim rows): one query per workgroup as in
// indexer_scores_rows_kernel, with 128-byte key rows.  A 32-key block is 4 KB of rows (4
// contiguous 1 KB LDS-direct copies of 8 rows per wave, row r's 16-byte unit u at slot u ^ row_swz<128>(r))
// plus its 32 key scales (one 4-byte LDS-direct copy per lane: 256 B, lanes >= 32 repeat the
// last key), through a per-wave ring of kRowsFp8Stages blocks (kRowsFp8Stages - 1 in flight while
// one is computed; 2, 3, 4 and 6 stages and 512- or 1024-key chunks all measured within 10 % at
// cfg5: ~110 us for the 360 MB of fp8 keys and scales, 3.3 TB/s, with the L1's pending-miss
// stalls at ~40 % of the cycles; non-temporal row copies then took it to ~92 us).  The query's fp8 A fragments sit in registers
// (32 VGPRs); two 32x32x64 fp8 MFMAs per row tile and block;
// I = k_scale[s] * sum_h (w q_scale)[t,h] relu(q8 . k8).
constexpr int kRowsFp8Stages = 3;
constexpr int kRowsFp8Block = 32 * 128 + 256;   // rows + scales of one 32-key block

// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 31]
DSA_DEV void wait_vmcnt_upto31(int n) {
  switch (n) {
#define DSA_WAIT_CASE(i) case i: wait_vmcnt<i>(); break;
    DSA_WAIT_CASE(0) DSA_WAIT_CASE(1) DSA_WAIT_CASE(2) DSA_WAIT_CASE(3) DSA_WAIT_CASE(4) DSA_WAIT_CASE(5)
    DSA_WAIT_CASE(6) DSA_WAIT_CASE(7) DSA_WAIT_CASE(8) DSA_WAIT_CASE(9) DSA_WAIT_CASE(10) DSA_WAIT_CASE(11)
    DSA_WAIT_CASE(12) DSA_WAIT_CASE(13) DSA_WAIT_CASE(14) DSA_WAIT_CASE(15) DSA_WAIT_CASE(16)
    DSA_WAIT_CASE(17) DSA_WAIT_CASE(18) DSA_WAIT_CASE(19) DSA_WAIT_CASE(20) DSA_WAIT_CASE(21)
    DSA_WAIT_CASE(22) DSA_WAIT_CASE(23) DSA_WAIT_CASE(24) DSA_WAIT_CASE(25) DSA_WAIT_CASE(26)
    DSA_WAIT_CASE(27) DSA_WAIT_CASE(28) DSA_WAIT_CASE(29) DSA_WAIT_CASE(30) DSA_WAIT_CASE(31)
#undef DSA_WAIT_CASE
    default: wait_vmcnt0(); break;
  }
}

__global__ __launch_bounds__(256) void indexer_scores_rows_fp8_kernel(IndexerParams p) {
  constexpr int RB = 128, NS = kRowsFp8Stages, CPB = 5;   // copies per block: 4 row copies + scales
  __shared__ __attribute__((aligned(256))) char ring[4][NS][kRowsFp8Block];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t = blockIdx.x;
  const int hb = lane >> 5, hl = lane & 31;
  const int c0 = ((int)blockIdx.y * 4 + wave) * p.chunk;
  const int len = p.row_len[t];
  if (c0 >= len) return;   // nothing below is shared between waves: no barrier
  const int c1 = min(len, c0 + p.chunk);
  const int base = p.row_base[t];
  const char* kbase = reinterpret_cast<const char*>(p.k);
  const uint32_t ring0 = lds_addr(ring[wave][0]);
  // copy r < 4 of a block moves keys 8r .. 8r+7 -- 1 KB contiguous in memory: lane l fills slot
  // l & 7 of key 8r + l / 8 with that key's unit (l & 7) ^ row_swz<128>(key); copy 4 the key scales
  auto gather = [&](int blk) {
    const int k0 = c0 + 32 * blk;
    const uint32_t dst = ring0 + (uint32_t)(blk % NS) * kRowsFp8Block;
    const int kk0 = lane >> 3;
    const uint32_t sl = lane & 7;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int kk = 8 * r + kk0;
      const int row = base + min(k0 + kk, c1 - 1);
      async_copy16_nt(kbase + (int64_t)row * RB + 16u * (sl ^ row_swz<128>(kk)), dst + 1024u * r);   // read once
    }
    async_copy4_unordered(p.k_scale + base + min(k0 + hl, c1 - 1), dst + 4096u);
  };
  // the first blocks' copies go out before the query's loads, so the two latencies overlap
  const int nb = (c1 - c0 + 31) / 32;
#pragma unroll
  for (int i = 0; i < NS - 1; ++i)
    if (i < nb) gather(i);
  const uint8_t* q8 = reinterpret_cast<const uint8_t*>(p.q) + (int64_t)t * p.n_heads * RB;
  i32x8 qa[2][2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const int h = 32 * mt + hl;
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const uint8_t* src = q8 + (int64_t)(h < p.n_heads ? h : 0) * RB + 64 * st + 32 * hb;
      const u32x4 lo = gload16(src), hi = gload16(src + 16);
      qa[mt][st] = h < p.n_heads ? cat16(lo, hi) : i32x8{};
    }
  }
  float wr[2][16];   // (w * q_scale) of the accumulator rows: heads 32 mt + (i/4)*8 + 4 hb + i%4
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int h = 32 * mt + (i >> 2) * 8 + 4 * hb + (i & 3);
      wr[mt][i] = h < p.n_heads ? p.w[(int64_t)t * p.n_heads + h] * p.q_scale[(int64_t)t * p.n_heads + h] : 0.f;
    }
  // every load so far retired (the compiler's and the first copies): the waits below count
  // only the ring's copies and the score stores
  wait_vmcnt0();
  for (int it = 0; it < nb; ++it) {
    const int k0 = c0 + 32 * it;
    const int j = k0 + hl;
    // issued after block it's copies: the copies of min(NS - 2, nb - 1 - it) later blocks and
    // the score stores of the min(it, NS - 1) blocks before it
    wait_vmcnt_upto31(CPB * min(NS - 2, nb - 1 - it) + min(it, NS - 1));
    asm volatile("" ::: "memory");
    if (it + NS - 1 < nb) gather(it + NS - 1);
    const uint32_t tb = ring0 + (uint32_t)(it % NS) * kRowsFp8Block;
    const char* row = lds_ptr(tb + hl * RB);
    i32x8 kb[2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const int u0 = 4 * st + 2 * hb;
      kb[st] = cat16(lds_load16(row + 16 * (u0 ^ row_swz<128>(hl))), lds_load16(row + 16 * ((u0 + 1) ^ row_swz<128>(hl))));
    }
    const float ksc = *reinterpret_cast<const float*>(lds_ptr(tb + 4096u + 4u * hl));
    f32x16 c0a = f32x16{}, c1a = f32x16{};
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      c0a = mfma32x32x64_fp8(qa[0][st], kb[st], c0a);
      c1a = mfma32x32x64_fp8(qa[1][st], kb[st], c1a);
    }
    float acc = weighted_relu_sum(wr, c0a, c1a);
    acc = xor32_sum(acc);
    if (hb == 0 && j < c1) p.scores[(int64_t)t * p.pitch + j] = acc * ksc;
  }
}

// Fill the masked tail [row_len, pitch) of each score row with -inf (only when the caller
// wants the reference's dense [S, S] index_scores).
__global__ void scores_fill_masked_kernel(float* scores, int64_t pitch, const int32_t* row_len, int rows) {
  const int t = blockIdx.x;
  if (t >= rows) return;
  for (int64_t j = row_len[t] + threadIdx.x; j < pitch; j += blockDim.x) scores[(int64_t)t * pitch + j] = -INFINITY;
}

int launch_indexer_scores(const IndexerParams& p_in, hipStream_t stream) {
  IndexerParams p = p_in;
  if (p.n_heads > kMaxHi || (p.head_dim != 128 && p.head_dim != 64)) return -2;
  const int64_t max_len = p.max_row_len;
  if (p.chunk == 0) {
    p.chunk = kIdxChunkMax;
    while (p.chunk > kIdxChunkMin && (int64_t)p.total_q * ((max_len + p.chunk - 1) / p.chunk) < kIdxWaveTarget)
      p.chunk >>= 1;
  }
  const bool rows_mode = p.head_dim == 128 && p.total_q <= kRowsMode;
  if (p.chunk < 32 || p.chunk % 32 != 0) return -1;
  const dim3 grid((p.total_q + 3) / 4, (unsigned)((max_len + p.chunk - 1) / p.chunk));
  if (grid.y == 0) return 0;
  if (rows_mode) {
    const dim3 rgrid(p.total_q, (grid.y + 3) / 4);
    if (p.fp8) hipLaunchKernelGGL(indexer_scores_rows_fp8_kernel, rgrid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL(indexer_scores_rows_kernel, rgrid, dim3(256), 0, stream, p);
  } else if (p.fp8)
    hipLaunchKernelGGL(indexer_scores_kernel<true>, grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(indexer_scores_kernel<false>, grid, dim3(256), 0, stream, p);
  if (p.fill_masked)
    hipLaunchKernelGGL(scores_fill_masked_kernel, dim3(p.total_q), dim3(256), 0, stream, p.scores, p.pitch,
                       p.row_len, p.total_q);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

// ------------------------------------------------------------------------------------------
// K2: top-k
// ------------------------------------------------------------------------------------------
namespace {
constexpr int kTopkThreads = 512;
// rows up to this length are cached in LDS (64 KB); a launch sizes its cache to what its rows
// can need (the pitch, the slice or the candidates), so short rows leave LDS for more workgroups
constexpr int kCacheElems = 16384;
// histogram copies, interleaved by lane & 7 (bin b, copy c at 8 b + c): the atomics of one
// instruction that hit one bin land on 8 addresses in 8 banks instead of one
constexpr int kHistCopies = 8;

DSA_DEV uint32_t order_key(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u << 1) == 0) u = 0;  // -0.0 -> +0.0 (equal values must tie)
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

}  // namespace

// Long rows (more entries than the LDS cache holds), fp32 scores in global memory: three passes
// over the row instead of the general path's six.
//   A  histogram of the top 12 bits of every order key (4096 bins, in the unused cache): the bin
//      b* that holds the K-th largest key, and how many keys lie above it;
//   B  the keys of bin b* with their positions into an LDS candidate list, and per compaction
//      wave the number of keys above b*;
//   then the remaining 20 bits are radix-selected over the candidates alone, the compaction's
//   per-wave counts come from pass B and the candidates, and
//   C  is the compaction's emitting pass (as in block_select_topk).
// Returns false, having emitted nothing, when bin b* holds more keys than the candidate list;
// the caller then runs the general path (its own state is rebuilt from scratch).
constexpr int kLongBins = 4096;

template <class Emit>
DSA_DEV bool block_select_topk_long(const float* src, int n, int K, uint32_t* cache, int cache_cap, int* hist,
                                    int* sh, uint32_t* sel_prefix, int* sel_need, Emit&& emit) {
  constexpr int T = kTopkThreads, NW = T / 64;
  const int cap = (cache_cap - kLongBins) / 2;   // candidate slots
  if (cap < 1024 || (reinterpret_cast<uintptr_t>(src) & 15) != 0) return false;
  const uint32_t* bits = reinterpret_cast<const uint32_t*>(src);
  const uint4* b4 = reinterpret_cast<const uint4*>(src);
  int* h12 = reinterpret_cast<int*>(cache);
  uint32_t* ckey = cache + kLongBins;
  int* cpos = reinterpret_cast<int*>(cache + kLongBins + cap);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int per_w = (n + 64 * NW - 1) / (64 * NW) * 64;
  const int wa = min(n, wave * per_w), wb = min(n, wa + per_w);
  // f(j, u[4], v[4]) over this wave's range, 256 consecutive entries per call: lane l holds
  // entries j .. j+3, j = j0 + 4 l (16-byte loads, 4 calls' loads in flight); a ragged tail in
  // 4-byte loads
  auto for_wave_range = [&](auto&& f) {
    const int wb4 = wa + (wb - wa) / 256 * 256;
    int j0 = wa;
    for (; j0 + 4 * 256 <= wb4; j0 += 4 * 256) {
      uint4 x[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) x[k] = b4[(j0 + 256 * k) / 4 + lane];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t u[4] = {order_key(__builtin_bit_cast(float, x[k].x)), order_key(__builtin_bit_cast(float, x[k].y)),
                               order_key(__builtin_bit_cast(float, x[k].z)), order_key(__builtin_bit_cast(float, x[k].w))};
        const bool v[4] = {true, true, true, true};
        f(j0 + 256 * k + 4 * lane, u, v);
      }
    }
    for (; j0 < wb; j0 += 256) {
      uint32_t u[4];
      bool v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = j0 + 4 * lane + e;
        v[e] = j < wb;
        u[e] = v[e] ? order_key(__builtin_bit_cast(float, bits[j])) : 0u;
      }
      f(j0 + 4 * lane, u, v);
    }
  };

  // ---- A: 12-bit histogram
  for (int b = threadIdx.x; b < kLongBins; b += T) h12[b] = 0;
  __syncthreads();
  for_wave_range([&](int, const uint32_t (&u)[4], const bool (&v)[4]) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (v[e]) atomicAdd(&h12[u[e] >> 20], 1);
  });
  __syncthreads();
  {  // bins in descending order, 8 per thread; block scan of the per-thread totals
    const int b_hi = kLongBins - 1 - 8 * (int)threadIdx.x;
    int c[8], tot = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      c[i] = h12[b_hi - i];
      tot += c[i];
    }
    int incl = tot;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o, 64);
      if (lane >= o) incl += v;
    }
    if (lane == 63) sh[wave] = incl;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < NW; ++w)
      if (w < wave) incl += sh[w];
    const int excl = incl - tot;
    if (excl < K && K <= incl) {
      int above = excl, bin = b_hi;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (above + c[i] >= K) {
          bin = b_hi - i;
          break;
        }
        above += c[i];
      }
      *sel_prefix = (uint32_t)bin;
      *sel_need = K - above;
    }
    __syncthreads();
  }
  const uint32_t bstar = *sel_prefix;
  int need = *sel_need;
  // ---- B: candidates of bin b*, counts above it per wave (hist[0] counts the candidates)
  if (threadIdx.x == 0) hist[0] = 0;
  __syncthreads();
  int w_above = 0;
  for_wave_range([&](int j, const uint32_t (&u)[4], const bool (&v)[4]) {
    int above = 0, nin = 0;
    bool in[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t top = u[e] >> 20;
      above += (v[e] && top > bstar) ? 1 : 0;
      in[e] = v[e] && top == bstar;
      nin += in[e] ? 1 : 0;
    }
    w_above += above;
    const uint64_t m = __ballot(nin > 0);
    if (m) {   // the lanes' candidates in lane order: an exclusive scan of nin over the wave
      int incl = nin;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o, 64);
        if (lane >= o) incl += t;
      }
      int slot0 = 0;
      if (lane == 63) slot0 = atomicAdd(&hist[0], incl);
      slot0 = __shfl(slot0, 63, 64);
      int slot = slot0 + incl - nin;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (in[e]) {
          if (slot < cap) {
            ckey[slot] = u[e];
            cpos[slot] = j + e;
          }
          ++slot;
        }
    }
  });
  w_above = wave_sum_i(w_above);
  if (lane == 0) sh[wave] = w_above;
  __syncthreads();
  const int nc = hist[0];
  __syncthreads();   // every thread has read the count before hist is reused (or the fallback)
  if (nc > cap) return false;

  // ---- radix select of bits 19..0 over the candidates: digits at bits 19..12, 11..4, 7..0
  uint32_t prefix = bstar << 20, pmask = 0xFFF00000u;
  int* hcopy = hist + (threadIdx.x & (kHistCopies - 1));
  auto bin_count = [&](int b) {
    const int4 x = *reinterpret_cast<const int4*>(hist + kHistCopies * b);
    const int4 y = *reinterpret_cast<const int4*>(hist + kHistCopies * b + 4);
    return x.x + x.y + x.z + x.w + y.x + y.y + y.z + y.w;
  };
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = pass == 0 ? 12 : (pass == 1 ? 4 : 0);
    for (int b = threadIdx.x; b < 256 * kHistCopies; b += T) hist[b] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < nc; i += T) {
      const uint32_t u = ckey[i];
      if ((u & pmask) == prefix) atomicAdd(&hcopy[kHistCopies * ((u >> shift) & 255)], 1);
    }
    __syncthreads();
    if (threadIdx.x < 64) {  // one wave: suffix scan of 256 bins, 4 per lane (lane 0 = top bins)
      const int l = threadIdx.x;
      const int b0 = 255 - 4 * l;
      const int c0 = bin_count(b0), c1 = bin_count(b0 - 1), c2 = bin_count(b0 - 2), c3 = bin_count(b0 - 3);
      const int tot = c0 + c1 + c2 + c3;
      int incl = tot;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o, 64);
        if (l >= o) incl += v;
      }
      const int excl = incl - tot;
      if (excl < need && need <= incl) {
        int above = excl, bin = b0;
        const int cs[4] = {c0, c1, c2, c3};
        for (int q = 0; q < 4; ++q) {
          if (above + cs[q] >= need) { bin = b0 - q; break; }
          above += cs[q];
        }
        *sel_prefix = prefix | ((uint32_t)bin << shift);
        *sel_need = need - above;
      }
    }
    __syncthreads();
    prefix = *sel_prefix;
    need = *sel_need;
    pmask |= 255u << shift;
    __syncthreads();
  }
  const uint32_t thr = prefix;  // exact K-th largest key; `need` of the keys equal to it are taken

  // ---- per-wave counts: above b* (pass B) + candidates above thr / equal to it, by wave range
  if (threadIdx.x < 2 * NW) hist[threadIdx.x] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < nc; i += T) {
    const uint32_t u = ckey[i];
    const int w = cpos[i] / per_w;
    if (u > thr) atomicAdd(&hist[w], 1);
    else if (u == thr) atomicAdd(&hist[NW + w], 1);
  }
  __syncthreads();
  int gt_before = 0, eq_before = 0;
  for (int w = 0; w < wave; ++w) {
    gt_before += sh[w] + hist[w];
    eq_before += hist[NW + w];
  }
  // ---- C: emit, ascending position (lane-major, then the lane's 4 consecutive entries)
  int pos = gt_before + min(eq_before, need);
  int eq_run = eq_before;
  for_wave_range([&](int j, const uint32_t (&u)[4], const bool (&v)[4]) {
    bool gt[4], eq[4];
    int n_eq = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      gt[e] = v[e] && u[e] > thr;
      eq[e] = v[e] && u[e] == thr;
      n_eq += eq[e] ? 1 : 0;
    }
    int eq_incl = n_eq;   // wave scan of the per-lane tie counts
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(eq_incl, o, 64);
      if (lane >= o) eq_incl += t;
    }
    int eq_seen = eq_run + eq_incl - n_eq;   // ties before this lane's first entry
    bool take[4];
    int n_take = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      take[e] = gt[e] || (eq[e] && eq_seen < need);
      eq_seen += eq[e] ? 1 : 0;
      n_take += take[e] ? 1 : 0;
    }
    int tk_incl = n_take;   // wave scan of the per-lane take counts
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(tk_incl, o, 64);
      if (lane >= o) tk_incl += t;
    }
    int r = pos + tk_incl - n_take;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (take[e]) emit(r++, j + e, u[e]);
    pos += __shfl(tk_incl, 63, 64);
    eq_run += __shfl(eq_incl, 63, 64);
  });
  return true;
}

// Block-wide min and max of one key per thread (sh: 2 * kTopkThreads/64 ints).  One barrier; the
// caller passes another before sh is written again.
DSA_DEV void block_minmax(uint32_t vmin, uint32_t vmax, int* sh, uint32_t& omin, uint32_t& omax) {
  constexpr int NW = kTopkThreads / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    vmin = min(vmin, (uint32_t)__shfl_xor((int)vmin, o, 64));
    vmax = max(vmax, (uint32_t)__shfl_xor((int)vmax, o, 64));
  }
  if (lane == 0) {
    sh[wave] = (int)vmin;
    sh[NW + wave] = (int)vmax;
  }
  __syncthreads();
  omin = 0xFFFFFFFFu;
  omax = 0u;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    omin = min(omin, (uint32_t)sh[w]);
    omax = max(omax, (uint32_t)sh[NW + w]);
  }
}

// Exclusive scan of one int per thread over the workgroup; *total = the sum (sh: kTopkThreads/64
// ints).  One barrier; the caller passes another before sh is written again.
DSA_DEV int block_excl_scan(int v, int* sh, int* total) {
  constexpr int NW = kTopkThreads / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(incl, o, 64);
    if (lane >= o) incl += t;
  }
  if (lane == 63) sh[wave] = incl;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    before += w < wave ? sh[w] : 0;
    tot += sh[w];
  }
  *total = tot;
  return before + incl - v;
}

// True when key u lies under `prefix` in the bits at and above hi_shift (all keys when hi_shift = 32).
DSA_DEV bool under_prefix(uint32_t u, uint32_t prefix, int hi_shift) {
  return hi_shift >= 32 || (u >> hi_shift) == (prefix >> hi_shift);
}

// One histogram window of a radix select over the m keys in LDS that lie under `prefix` above
// hi_shift: bins (u >> shift) & (nb - 1), nb = 2^(hi_shift - shift) <= 2048 (hist: 2048 ints).
// Returns the bin holding the need-th largest of those keys (need >= 1 of them exist), with
// *above = their keys in higher bins and *in_bin = the bin's keys.  sel: 3 ints, written by one
// thread between two barriers and read after the second; the caller passes a barrier before
// sel[0..2], hist or sh is written again.
DSA_DEV int window_pass(const uint32_t* keys, int m, uint32_t prefix, int hi_shift, int shift, int need, int* hist,
                        int* sh, int* sel, int* above, int* in_bin) {
  constexpr int T = kTopkThreads;
  const int nb = 1 << (hi_shift - shift);
  for (int b = threadIdx.x; b < nb; b += T) hist[b] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < m; i += T) {
    const uint32_t u = keys[i];
    if (under_prefix(u, prefix, hi_shift)) atomicAdd(&hist[(u >> shift) & (uint32_t)(nb - 1)], 1);
  }
  __syncthreads();
  // bins in descending order, 4 per thread: thread t holds bins nb-1-4t .. nb-4-4t
  const int b_hi = nb - 1 - 4 * (int)threadIdx.x;
  int c[4], tot = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    c[q] = b_hi - q >= 0 ? hist[b_hi - q] : 0;
    tot += c[q];
  }
  int all;
  const int excl = block_excl_scan(tot, sh, &all);
  if (excl < need && need <= excl + tot) {
    int ab = excl;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (ab + c[q] >= need) {
        sel[0] = b_hi - q;
        sel[1] = ab;
        sel[2] = c[q];
        break;
      }
      ab += c[q];
    }
  }
  __syncthreads();
  *above = sel[1];
  *in_bin = sel[2];
  return sel[0];
}

// Exact need-th largest of the m keys in LDS (lo <= every key <= hi, need <= m): thr, and how
// many of the keys equal to it fall within the need largest.  Histogram windows of up to 11
// bits below the common prefix of lo and hi; once the chosen bin holds at most 64 keys, one
// wave ranks them directly (sel[4] must be zero on entry).  The caller passes a barrier before
// sel, hist or sh is written again.
DSA_DEV void select_exact(const uint32_t* keys, int m, int need, uint32_t lo, uint32_t hi, int* hist, int* sh,
                          int* sel, uint32_t& thr, int& need_out) {
  constexpr int T = kTopkThreads;
  int pb = lo == hi ? 32 : __clz(lo ^ hi);              // bits shared by every key
  uint32_t prefix = pb >= 32 ? lo : (pb == 0 ? 0u : lo & ~(0xFFFFFFFFu >> pb));
  while (pb < 32) {
    const int hi_shift = 32 - pb, shift = max(0, hi_shift - 11);
    int above, in_bin;
    const int bin = window_pass(keys, m, prefix, hi_shift, shift, need, hist, sh, sel, &above, &in_bin);
    prefix |= (uint32_t)bin << shift;
    need -= above;
    pb = 32 - shift;
    if (pb < 32 && in_bin <= 64) {
      // the bin's keys into hist[0..63] (slots from sel[4], zero on entry), then one wave ranks
      // them
      for (int i = threadIdx.x; i < m; i += T) {
        const uint32_t u = keys[i];
        if (under_prefix(u, prefix, 32 - pb)) hist[atomicAdd(&sel[4], 1)] = (int)u;
      }
      __syncthreads();
      if (threadIdx.x < 64) {
        const int l = threadIdx.x;
        const bool ok = l < in_bin;
        const uint32_t v = ok ? (uint32_t)hist[l] : 0u;
        int gt = 0, ge = 0;
#pragma unroll 8
        for (int j = 0; j < 64; ++j) {
          const uint32_t w = (uint32_t)__builtin_amdgcn_readlane((int)v, j);
          if (j < in_bin) {
            gt += w > v ? 1 : 0;
            ge += w >= v ? 1 : 0;
          }
        }
        if (ok && gt < need && need <= ge) {   // every such lane holds the same key
          sel[1] = (int)v;
          sel[2] = need - gt;
        }
      }
      __syncthreads();
      thr = (uint32_t)sel[1];
      need_out = sel[2];
      return;
    }
  }
  thr = prefix;
  need_out = need;
}

// Sampled-threshold selection for long rows of fp32 scores in global memory (4096 .. 65536
// entries): one streaming pass over the row instead of the cached path's LDS passes or the long
// path's three global ones.
//   1  order keys of kSampleM entries (64 evenly spaced runs of 32: one 128-byte line each) and
//      one histogram window below their common prefix give a bound that about
//      r = ceil(1.5 K M / n) + 8 of the sample reach (the lower edge of the bin holding the
//      sample's r-th largest), i.e. about 1.5 K of the row's entries;
//   2  one pass over the row: every entry at or above the bound goes to an LDS candidate list with
//      its position (wave-aggregated slots: counts bit-sliced over ballots, one LDS atomic per
//      wave and step);
//   3  if the list holds between K and `cap` entries, it contains the whole top-K: the exact K-th
//      largest key thr is selected over the candidates alone (select_exact), the selected
//      positions (keys above thr, then the lowest-positioned `need` of the keys equal to it) are
//      marked in an LDS bitmap, and each is emitted at its rank in position order (a scan of the
//      bitmap's popcounts).
// The result is the exact selection, the same as the other paths' bit for bit.  Returns false
// having emitted nothing (the caller then runs another path) for rows out of that range, K large
// against n, LDS too small, a misaligned row, or a bound that missed (fewer than K or more than
// cap entries reach it).  LDS: sampled_topk_elems(n, K) 4-byte words of the cache.
constexpr int kSampleM = 2048;
constexpr int kSampledMaxN = 65536;   // 16-bit candidate positions

DSA_HOST_DEV int sampled_topk_cap(int n, int K) { return max(kSampleM, 2 * K + 32 * ((n + kSampleM - 1) / kSampleM)); }
DSA_HOST_DEV int sampled_topk_elems(int n, int K) {
  return sampled_topk_cap(n, K) + (sampled_topk_cap(n, K) + 1) / 2 + 3 * ((n + 31) / 32);
}
DSA_HOST_DEV bool sampled_topk_eligible(int n, int K) {
  return n >= 2 * kSampleM && n <= kSampledMaxN &&
         (int)((3LL * K * kSampleM + 2LL * n - 1) / (2LL * n)) + 8 <= kSampleM / 2;
}

template <class Emit>
DSA_DEV bool block_select_topk_sampled(const float* src, int n, int K, uint32_t* cache, int cache_cap, int* hist,
                                       int* sh, uint32_t* sel_prefix, int* sel_need, Emit&& emit) {
  constexpr int T = kTopkThreads, M = kSampleM;
  static_assert(M == 4 * T, "one 16-byte sample load per thread");
  if (!sampled_topk_eligible(n, K)) return false;
  const int r = (int)((3LL * K * M + 2LL * n - 1) / (2LL * n)) + 8;
  const int cap = sampled_topk_cap(n, K);
  const int W = (n + 31) / 32;
  if (sampled_topk_elems(n, K) > cache_cap || (reinterpret_cast<uintptr_t>(src) & 15) != 0) return false;
  uint32_t* ckey = cache;                                          // [cap] keys (first the sample's)
  uint16_t* cpos = reinterpret_cast<uint16_t*>(cache + cap);       // [cap] positions
  uint32_t* take = cache + cap + (cap + 1) / 2;                    // [W] selected positions
  uint32_t* eqb = take + W;                                        // [W] candidates equal to thr
  int* wpre = reinterpret_cast<int*>(eqb + W);                     // [W] selected before each word
  // the launch's 8-int selection slots (sel_need is [1]): [0..2] window results, [3] the
  // candidate count, [4] the exact select's counter
  int* sel = reinterpret_cast<int*>(sel_prefix);
  (void)sel_need;
  const int lane = threadIdx.x & 63;
  const uint64_t lt = (1ull << lane) - 1;
  const uint4* b4 = reinterpret_cast<const uint4*>(src);
  const uint32_t* bits = reinterpret_cast<const uint32_t*>(src);
  const int n4 = n >> 2;

  if (threadIdx.x == 0) {   // (ordered before their first use by the barriers below)
    sel[3] = 0;
    sel[4] = 0;
  }
  // ---- 1: sample keys, min / max, one window -> bound (workgroup-uniform)
  uint32_t bound;
  {
    const int run = threadIdx.x >> 3, part = threadIdx.x & 7;
    const int start = (int)(((int64_t)run * (n - 32) / 63) & ~3LL);   // + 31 < n
    const uint4 sv = b4[(start >> 2) + part];
    const uint32_t s4[4] = {order_key(__builtin_bit_cast(float, sv.x)), order_key(__builtin_bit_cast(float, sv.y)),
                            order_key(__builtin_bit_cast(float, sv.z)), order_key(__builtin_bit_cast(float, sv.w))};
    *reinterpret_cast<uint4*>(ckey + 4 * threadIdx.x) = uint4{s4[0], s4[1], s4[2], s4[3]};
    for (int w = threadIdx.x; w < W; w += T) { take[w] = 0u; eqb[w] = 0u; }
    uint32_t smin, smax;
    block_minmax(min(min(s4[0], s4[1]), min(s4[2], s4[3])), max(max(s4[0], s4[1]), max(s4[2], s4[3])), sh, smin,
                 smax);
    bound = smin;
    if (smin != smax) {
      const int hi_shift = 32 - __clz(smin ^ smax), shift = max(0, hi_shift - 11);
      int above, in_bin;
      const int bin = window_pass(ckey, M, smin, hi_shift, shift, r, hist, sh, sel, &above, &in_bin);
      bound = (hi_shift >= 32 ? 0u : (smin >> hi_shift) << hi_shift) | ((uint32_t)bin << shift);
    } else {
      __syncthreads();   // (block_minmax's reads of sh before the collect writes it)
    }
  }

  // ---- 2: candidates (keys >= bound) with their positions, 16 entries per thread and step
  uint32_t cmax = 0u;
  for (int g0 = 0; g0 < n4; g0 += 4 * T) {
    uint4 x[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int g = g0 + k * T + (int)threadIdx.x;
      x[k] = g < n4 ? b4[g] : uint4{0u, 0u, 0u, 0u};   // past the row: never counted (ok below)
    }
    int c = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const bool ok = g0 + k * T + (int)threadIdx.x < n4;
      x[k] = uint4{order_key(__builtin_bit_cast(float, x[k].x)), order_key(__builtin_bit_cast(float, x[k].y)),
                   order_key(__builtin_bit_cast(float, x[k].z)), order_key(__builtin_bit_cast(float, x[k].w))};
      const uint32_t e[4] = {x[k].x, x[k].y, x[k].z, x[k].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const bool in = ok && e[q] >= bound;
        c += in ? 1 : 0;
        cmax = in ? max(cmax, e[q]) : cmax;
      }
    }
    // lane prefix of c over the wave from 5 bit-slice ballots (c <= 16)
    int pre = 0, tot = 0;
#pragma unroll
    for (int bt = 0; bt < 5; ++bt) {
      const uint64_t bm = __ballot((c >> bt) & 1);
      pre += __popcll(bm & lt) << bt;
      tot += __popcll(bm) << bt;
    }
    if (tot == 0) continue;   // wave-uniform
    int slot0 = 0;
    if (lane == 0) slot0 = atomicAdd(&sel[3], tot);
    int slot = __builtin_amdgcn_readfirstlane(slot0) + pre;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int g = g0 + k * T + (int)threadIdx.x;
      const uint32_t e[4] = {x[k].x, x[k].y, x[k].z, x[k].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (g < n4 && e[q] >= bound) {
          if (slot < cap) {
            ckey[slot] = e[q];
            cpos[slot] = (uint16_t)(4 * g + q);
          }
          ++slot;
        }
      }
    }
  }
  for (int j = 4 * n4 + (int)threadIdx.x; j < n; j += T) {   // ragged tail (< 4 entries)
    const uint32_t u = order_key(__builtin_bit_cast(float, bits[j]));
    if (u >= bound) {
      cmax = max(cmax, u);
      const int s = atomicAdd(&sel[3], 1);
      if (s < cap) { ckey[s] = u; cpos[s] = (uint16_t)j; }
    }
  }
  // the count and the candidates' maximum after one barrier (a fallback path writes neither sel
  // nor sh before its own barriers)
  {
    constexpr int NW = T / 64;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) cmax = max(cmax, (uint32_t)__shfl_xor((int)cmax, o, 64));
    if (lane == 0) sh[NW + (threadIdx.x >> 6)] = (int)cmax;
  }
  __syncthreads();
  const int nc = sel[3];
  uint32_t kmax = 0u;
#pragma unroll
  for (int w = 0; w < T / 64; ++w) kmax = max(kmax, (uint32_t)sh[T / 64 + w]);
  if (nc < K || nc > cap) return false;

  // ---- 3: exact threshold over the candidates, position bitmap, ranks, emission
  uint32_t thr;
  int need;
  select_exact(ckey, nc, K, bound, kmax, hist, sh, sel, thr, need);
  int my_eq = 0;
  for (int i = threadIdx.x; i < nc; i += T) {
    const uint32_t u = ckey[i], pos = cpos[i];
    if (u > thr) atomicOr(&take[pos >> 5], 1u << (pos & 31));
    else if (u == thr) {
      atomicOr(&eqb[pos >> 5], 1u << (pos & 31));
      ++my_eq;
    }
  }
  my_eq = wave_sum_i(my_eq);
  if (lane == 0) sh[T / 64 + (threadIdx.x >> 6)] = my_eq;
  __syncthreads();   // (also the barrier after the marks)
  int n_eq = 0;
#pragma unroll
  for (int w = 0; w < T / 64; ++w) n_eq += sh[T / 64 + w];
  const int per = (W + T - 1) / T;
  const int w0 = min(W, (int)threadIdx.x * per), w1 = min(W, w0 + per);
  if (n_eq == need) {
    for (int w = w0; w < w1; ++w) take[w] |= eqb[w];
  } else {   // keep the `need` lowest-positioned keys equal to thr
    int s = 0;
    for (int w = w0; w < w1; ++w) s += __popc(eqb[w]);
    int t_;
    int run = block_excl_scan(s, sh, &t_);
    for (int w = w0; w < w1; ++w) {
      wpre[w] = run;
      run += __popc(eqb[w]);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nc; i += T) {
      const uint32_t pos = cpos[i];
      if (ckey[i] == thr) {
        const int rk = wpre[pos >> 5] + __popc(eqb[pos >> 5] & ((1u << (pos & 31)) - 1u));
        if (rk < need) atomicOr(&take[pos >> 5], 1u << (pos & 31));
      }
    }
    __syncthreads();
  }
  {
    int s = 0;
    for (int w = w0; w < w1; ++w) s += __popc(take[w]);
    int t_;
    int run = block_excl_scan(s, sh, &t_);
    for (int w = w0; w < w1; ++w) {
      wpre[w] = run;
      run += __popc(take[w]);
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nc; i += T) {
    const uint32_t pos = cpos[i];
    const uint32_t word = take[pos >> 5], bit = 1u << (pos & 31);
    if (word & bit) emit(wpre[pos >> 5] + __popc(word & (bit - 1u)), (int)pos, ckey[i]);
  }
  return true;
}

// Exact top-k of one list of n > K entries in one workgroup: the K largest under (key desc,
// position asc), emitted as emit(rank, position, key) with rank ascending in position. Entries are
// fp32 scores mapped through order_key, or (kKeys) order keys already.
template <bool kKeys, class Emit>
DSA_DEV void block_select_topk(const void* src, int n, int K, uint32_t* cache, int cache_cap, int* hist, int* sh,
                               uint32_t* sel_prefix, int* sel_need, Emit&& emit) {
  const uint32_t* bits = static_cast<const uint32_t*>(src);
  auto conv = [](uint32_t x) -> uint32_t { return kKeys ? x : order_key(__builtin_bit_cast(float, x)); };
  const bool cached = n <= cache_cap;
  if constexpr (!kKeys) {
    if (block_select_topk_sampled(static_cast<const float*>(src), n, K, cache, cache_cap, hist, sh, sel_prefix,
                                  sel_need, emit))
      return;
    if (!cached && block_select_topk_long(static_cast<const float*>(src), n, K, cache, cache_cap, hist, sh,
                                          sel_prefix, sel_need, emit))
      return;
  }
  // long lists stay in global memory and are streamed as 16-byte vectors when aligned
  const bool vec = ((reinterpret_cast<uintptr_t>(bits) & 15) == 0);
  const uint4* sc4 = reinterpret_cast<const uint4*>(bits);
  constexpr int T = kTopkThreads;
  if (cached) {  // 16-byte loads, 4 in flight per thread: one memory round trip per 8192 entries
    int j0 = 0;
    if (vec) {
      const int n4 = n >> 2;
      uint4* c4 = reinterpret_cast<uint4*>(cache);
      int g = threadIdx.x;
      for (; g + 3 * T < n4; g += 4 * T) {
        uint4 x[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) x[k] = sc4[g + k * T];
#pragma unroll
        for (int k = 0; k < 4; ++k) c4[g + k * T] = uint4{conv(x[k].x), conv(x[k].y), conv(x[k].z), conv(x[k].w)};
      }
      for (; g < n4; g += T) {
        const uint4 x = sc4[g];
        c4[g] = uint4{conv(x.x), conv(x.y), conv(x.z), conv(x.w)};
      }
      j0 = 4 * n4;
    }
    for (int j = j0 + threadIdx.x; j < n; j += T) cache[j] = conv(bits[j]);
  }
  // (the cached and the global paths stay separate loops: a load through a pointer selected
  // between the two would be a flat load, one round trip per entry)
  // f(key) over every entry, each thread a strided subset; loads unrolled
  auto for_each_key = [&](auto&& f) {
    if (cached) {
      int j = threadIdx.x;
      for (; j + 3 * T < n; j += 4 * T) {
        uint32_t x[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) x[k] = cache[j + k * T];
#pragma unroll
        for (int k = 0; k < 4; ++k) f(x[k]);
      }
      for (; j < n; j += T) f(cache[j]);
      return;
    }
    if (!vec) {
      for (int j = threadIdx.x; j < n; j += T) f(conv(bits[j]));
      return;
    }
    const int n4 = n >> 2;
    int g = threadIdx.x;
    for (; g + 3 * T < n4; g += 4 * T) {
      uint4 x[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) x[k] = sc4[g + k * T];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        f(conv(x[k].x)); f(conv(x[k].y)); f(conv(x[k].z)); f(conv(x[k].w));
      }
    }
    for (; g < n4; g += T) {
      const uint4 x = sc4[g];
      f(conv(x.x)); f(conv(x.y)); f(conv(x.z)); f(conv(x.w));
    }
    for (int j = 4 * n4 + threadIdx.x; j < n; j += T) f(conv(bits[j]));
  };

  // ---- radix select: find the K-th largest key (prefix over the top 32 bits)
  uint32_t prefix = 0, pmask = 0;
  int need = K;  // still to take from the keys matching the current prefix
  int* hcopy = hist + (threadIdx.x & (kHistCopies - 1));
  auto bin_count = [&](int b) {
    const int4 x = *reinterpret_cast<const int4*>(hist + kHistCopies * b);
    const int4 y = *reinterpret_cast<const int4*>(hist + kHistCopies * b + 4);
    return x.x + x.y + x.z + x.w + y.x + y.y + y.z + y.w;
  };
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int b = threadIdx.x; b < 256 * kHistCopies; b += blockDim.x) hist[b] = 0;
    __syncthreads();
    for_each_key([&](uint32_t u) {
      if ((u & pmask) == prefix) atomicAdd(&hcopy[kHistCopies * ((u >> shift) & 255)], 1);
    });
    __syncthreads();
    if (threadIdx.x < 64) {  // one wave: suffix scan of 256 bins, 4 per lane (lane 0 = top bins)
      const int l = threadIdx.x;
      const int b0 = 255 - 4 * l;
      const int c0 = bin_count(b0), c1 = bin_count(b0 - 1), c2 = bin_count(b0 - 2), c3 = bin_count(b0 - 3);
      const int tot = c0 + c1 + c2 + c3;
      int incl = tot;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o, 64);
        if (l >= o) incl += v;
      }
      const int excl = incl - tot;  // keys in bins above b0
      if (excl < need && need <= incl) {
        int above = excl, bin = b0;
        const int cs[4] = {c0, c1, c2, c3};
        for (int q = 0; q < 4; ++q) {
          if (above + cs[q] >= need) { bin = b0 - q; break; }
          above += cs[q];
        }
        *sel_prefix = prefix | ((uint32_t)bin << shift);
        *sel_need = need - above;
      }
    }
    __syncthreads();
    prefix = *sel_prefix;
    need = *sel_need;
    pmask |= 255u << shift;
    __syncthreads();
  }
  const uint32_t thr = prefix;  // exact K-th largest key; take `need` of the keys equal to it

  // ---- stable compaction in ascending position order: wave w takes a contiguous range, 64
  // consecutive entries per step (conflict-free LDS reads, coalesced global ones), and ranks them
  // with ballots; the waves' offsets come from one scan of their counts
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int NW = kTopkThreads / 64;
  const int per_w = (n + 64 * NW - 1) / (64 * NW) * 64;
  const int wa = min(n, wave * per_w), wb = min(n, wa + per_w);
  const uint64_t lt_mask = (1ull << lane) - 1;
  // f(j, key, valid) over the wave's range, 64 consecutive entries per call; global loads 4 steps
  // ahead
  auto for_wave_range = [&](auto&& f) {
    if (cached) {
      for (int j0 = wa; j0 < wb; j0 += 64) {
        const int j = j0 + lane;
        f(j, j < wb ? cache[j] : 0u, j < wb);
      }
      return;
    }
    int j0 = wa;
    for (; j0 + 4 * 64 <= wb; j0 += 4 * 64) {
      uint32_t x[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) x[k] = bits[j0 + 64 * k + lane];
#pragma unroll
      for (int k = 0; k < 4; ++k) f(j0 + 64 * k + lane, conv(x[k]), true);
    }
    for (; j0 < wb; j0 += 64) {
      const int j = j0 + lane;
      f(j, j < wb ? conv(bits[j]) : 0u, j < wb);
    }
  };
  int w_gt = 0, w_eq = 0;
  for_wave_range([&](int, uint32_t u, bool v) {
    w_gt += __popcll(__ballot(v && u > thr));
    w_eq += __popcll(__ballot(v && u == thr));
  });
  if (lane == 0) { sh[wave] = w_gt; sh[NW + wave] = w_eq; }
  __syncthreads();
  int gt_before = 0, eq_before = 0;
  for (int w = 0; w < wave; ++w) { gt_before += sh[w]; eq_before += sh[NW + w]; }
  int pos = gt_before + min(eq_before, need);
  int eq_run = eq_before;
  for_wave_range([&](int j, uint32_t u, bool v) {
    const bool gt = v && u > thr, eq = v && u == thr;
    const uint64_t eqm = __ballot(eq);
    const bool take = gt || (eq && eq_run + __popcll(eqm & lt_mask) < need);
    const uint64_t tm = __ballot(take);
    if (take) emit(pos + __popcll(tm & lt_mask), j, u);
    pos += __popcll(tm);
    eq_run += __popcll(eqm);
  });
}

#define DSA_TOPK_SHARED                               \
  extern __shared__ __attribute__((aligned(16))) uint32_t cache[]; /* p.cache_elems */ \
  __shared__ __attribute__((aligned(16))) int hist[256 * kHistCopies]; \
  __shared__ int sh[2 * (kTopkThreads / 64)];         \
  __shared__ int tk_sel[8];                           \
  uint32_t& sel_prefix = reinterpret_cast<uint32_t&>(tk_sel[0]); \
  int& sel_need = tk_sel[1]

// One row in one workgroup: rows of at most K visible keys take them all, -1 padded.
DSA_DEV void topk_row(const TopkParams& p, int row, int n, uint32_t* cache, int* hist, int* sh,
                      uint32_t* sel_prefix, int* sel_need) {
  const int base = p.row_base[row];
  const int K = p.topk;
  int32_t* out = p.out_idx + (int64_t)row * K;
  if (n <= K) {  // everything visible is selected
    for (int j = threadIdx.x; j < K; j += blockDim.x) out[j] = j < n ? base + j : -1;
  } else {
    block_select_topk<false>(p.scores + (int64_t)row * p.pitch, n, K, cache, p.cache_elems, hist, sh, sel_prefix,
                             sel_need,
                             [&](int r, int j, uint32_t) { out[r] = base + j; });
  }
  if (p.out_count && threadIdx.x == 0) p.out_count[row] = min(n, K);
}

__global__ __launch_bounds__(kTopkThreads) void topk_kernel(TopkParams p) {
  DSA_TOPK_SHARED;
  const int row = blockIdx.x;
  if (row >= p.rows) return;
  topk_row(p, row, p.row_len[row], cache, hist, sh, &sel_prefix, &sel_need);
}

// Few long rows (decode): a row longer than one slice is split over blockIdx.y. Slice g keeps its
// own top-K (or all of it, when shorter -- only a row's last slice can be) as order keys and key
// ids at candidates [g K, (g+1) K) of the row; topk_merge_kernel then selects from the candidates.
// Every key of the row's top-K is in its slice's top-K (fewer than K keys of the row, hence of the
// slice, come before it), and candidate positions ascend with the key ids, so the merge's
// (key desc, position asc) order is the row's (score desc, key asc) order: the result is the
// one-workgroup selection's, bit for bit.
__global__ __launch_bounds__(kTopkThreads) void topk_slice_kernel(TopkParams p) {
  DSA_TOPK_SHARED;
  const int row = blockIdx.x, g = blockIdx.y;
  if (row >= p.rows) return;
  const int n = (int)min((int64_t)p.row_len[row], p.pitch);
  if (n <= p.slice) {  // the whole row in slice 0's workgroup
    if (g == 0) topk_row(p, row, n, cache, hist, sh, &sel_prefix, &sel_need);
    return;
  }
  const int j0 = g * p.slice;
  if (j0 >= n) return;
  const int m = min(p.slice, n - j0);
  const int K = p.topk;
  const int key0 = p.row_base[row] + j0;
  const int64_t c0 = ((int64_t)row * p.n_slices + g) * K;
  uint32_t* ck = p.cand_key + c0;
  int32_t* ci = p.cand_idx + c0;
  const float* sc = p.scores + (int64_t)row * p.pitch + j0;
  if (m <= K) {
    for (int j = threadIdx.x; j < m; j += blockDim.x) {
      ck[j] = order_key(sc[j]);
      ci[j] = key0 + j;
    }
    return;
  }
  block_select_topk<false>(sc, m, K, cache, p.cache_elems, hist, sh, &sel_prefix, &sel_need,
                           [&](int r, int j, uint32_t u) {
    ck[r] = u;
    ci[r] = key0 + j;
  });
}

__global__ __launch_bounds__(kTopkThreads) void topk_merge_kernel(TopkParams p) {
  DSA_TOPK_SHARED;
  const int row = blockIdx.x;
  if (row >= p.rows) return;
  const int n = (int)min((int64_t)p.row_len[row], p.pitch);
  if (n <= p.slice) return;  // done by topk_slice_kernel
  const int K = p.topk;
  const int full = (n - 1) / p.slice;  // slices before the last: K candidates each
  const int nc = full * K + min(K, n - full * p.slice);
  const int64_t c0 = (int64_t)row * p.n_slices * K;
  const int32_t* ci = p.cand_idx + c0;
  int32_t* out = p.out_idx + (int64_t)row * K;
  block_select_topk<true>(p.cand_key + c0, nc, K, cache, p.cache_elems, hist, sh, &sel_prefix, &sel_need,
                          [&](int r, int j, uint32_t) { out[r] = ci[j]; });
  if (p.out_count && threadIdx.x == 0) p.out_count[row] = K;
}
#undef DSA_TOPK_SHARED

// Split selection: fewer rows than this leave CUs idle in one-workgroup-per-row selection.
// 16384-key slices (the LDS-cached length) beat 8192 at cfg5 decode: 47 vs 54 us, the merge then
// taking half the candidates.
constexpr int kTopkSplitRows = 256;
constexpr int kTopkSliceMin = 16384;

int topk_slice_len(int topk) { return max(kTopkSliceMin, (topk + 3) / 4 * 16); }

size_t topk_workspace_size(int rows, int64_t pitch, int topk) {
  if (rows <= 0 || rows >= kTopkSplitRows || topk < 1) return 0;
  const int64_t slice = topk_slice_len(topk);
  if (pitch <= slice) return 0;
  const int64_t n_slices = (pitch + slice - 1) / slice;
  return (size_t)rows * n_slices * topk * (sizeof(uint32_t) + sizeof(int32_t));
}

// LDS cache entries of a launch whose rows hold up to n_max entries: the sampled path's lists
// for the longest row it can take, the rows too short for it cached whole, at least the long
// path's 12-bit histogram and 1024 candidates; otherwise rows up to kCacheElems cached whole.
int topk_cache_elems(int64_t n_max, int K) {
  const int full = (int)std::min<int64_t>(kCacheElems, (n_max + 3) / 4 * 4);
  const int n_hi = (int)std::min<int64_t>(n_max, kSampledMaxN);
  if (!sampled_topk_eligible(n_hi, K)) return full;
  int n_min = 2 * kSampleM;   // the shortest row the sampled path takes (eligibility grows with n)
  const int64_t est = (3LL * K * kSampleM + (kSampleM - 16) - 1) / (kSampleM - 16);
  if (est > n_min) n_min = (int)std::min<int64_t>(est, n_hi);
  while (n_min > 2 * kSampleM && sampled_topk_eligible(n_min - 1, K)) --n_min;
  while (!sampled_topk_eligible(n_min, K)) ++n_min;
  const int need = std::max({sampled_topk_elems(n_hi, K), (n_min + 3) / 4 * 4, kLongBins + 2 * 1024});
  return std::min(full, need);
}

int launch_topk(const TopkParams& p_in, hipStream_t stream) {
  if (p_in.rows == 0) return 0;
  TopkParams p = p_in;
  auto cache_for = [&](int64_t n) { return topk_cache_elems(n, p.topk); };
  if (p.cand_key && topk_workspace_size(p.rows, p.pitch, p.topk) > 0) {
    p.slice = topk_slice_len(p.topk);
    p.n_slices = (int)((p.pitch + p.slice - 1) / p.slice);
    // rows up to one slice run whole in the slice kernel: its cache covers min(pitch, slice)
    p.cache_elems = cache_for(std::min<int64_t>(p.pitch, p.slice));
    hipLaunchKernelGGL(topk_slice_kernel, dim3(p.rows, p.n_slices), dim3(kTopkThreads), p.cache_elems * 4, stream, p);
    // the merge selects over order keys (no sampled path): its candidates cached whole
    p.cache_elems = (int)std::min<int64_t>(kCacheElems, ((int64_t)p.n_slices * p.topk + 3) / 4 * 4);
    hipLaunchKernelGGL(topk_merge_kernel, dim3(p.rows), dim3(kTopkThreads), p.cache_elems * 4, stream, p);
  } else {
    p.cache_elems = cache_for(p.pitch);
    hipLaunchKernelGGL(topk_kernel, dim3(p.rows), dim3(kTopkThreads), p.cache_elems * 4, stream, p);
  }
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace dsa

// ------------------------------------------------------------------------------------------
// Row descriptors of packed prefill queries from cu_seqlens (documents, causal or not).
// ------------------------------------------------------------------------------------------
namespace dsa {

__global__ void build_rows_kernel(const int32_t* cu_seqlens, int n_seq, int total_q, int causal,
                                  int32_t* row_base, int32_t* row_len) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= total_q) return;
  int lo = 0, hi = n_seq;  // find document d with cu[d] <= t < cu[d+1]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (cu_seqlens[mid] <= t) lo = mid; else hi = mid;
  }
  const int start = cu_seqlens[lo], end = cu_seqlens[lo + 1];
  row_base[t] = start;
  row_len[t] = causal ? t - start + 1 : end - start;
}

// Decode rows: sequence b's one new token sits at position L_b - 1 and sees its whole cache
// rows [cu_cache[b], cu_cache[b+1]).
__global__ void build_decode_rows_kernel(const int32_t* cu_cache, int batch, int32_t* row_base, int32_t* row_len) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  row_base[b] = cu_cache[b];
  row_len[b] = cu_cache[b + 1] - cu_cache[b];
}

int launch_build_decode_rows(const int32_t* cu_cache, int batch, int32_t* row_base, int32_t* row_len,
                             hipStream_t stream) {
  if (batch == 0) return 0;
  hipLaunchKernelGGL(build_decode_rows_kernel, dim3((batch + 255) / 256), dim3(256), 0, stream, cu_cache, batch,
                     row_base, row_len);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_build_rows(const int32_t* cu_seqlens, int n_seq, int total_q, int causal, int32_t* row_base,
                      int32_t* row_len, hipStream_t stream) {
  if (total_q == 0) return 0;
  hipLaunchKernelGGL(build_rows_kernel, dim3((total_q + 255) / 256), dim3(256), 0, stream, cu_seqlens, n_seq,
                     total_q, causal, row_base, row_len);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace dsa
