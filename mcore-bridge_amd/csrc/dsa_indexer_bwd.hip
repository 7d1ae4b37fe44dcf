// Lightning-indexer scores of the selected slots and their backward (gfx950).
//
//   I[t, j] = sum_h w[t,h] relu(q[t,h] . k[idx[t,j]])          (the reference's index scores,
//             src/mcore_bridge/patcher.py:338-376 fused_qk_topk_naive, read at the top-k slots)
//   dq[t,h] = w[t,h] sum_j dI[t,j] 1[z>0] k_j,   dw[t,h] = sum_j dI[t,j] relu(z),
//   dk[s]   = sum over pairs (t, j) selecting s of sum_h dI[t,j] 1[z>0] w[t,h] q[t,h]
// with z = q[t,h] . k[idx[t,j]] (bf16 operands, fp32 accumulation).  dI comes from the sparse
// indexer KL loss (dsa_indexer_kl.hip); the reference trains the indexer with that loss
// (dsa_indexer_loss_coeff, src/mcore_bridge/config/model_config.py:204-205) through torch
// autograd, which this replaces.
//
// One workgroup (4 waves) per query; wave w takes the query's 32-key blocks w, w + 4, .., each
// gathered into a wave-private double-buffered LDS tile by asynchronous global_load_lds copies
// (so the loop has no workgroup barrier).  Per block, from the same K fragments:
//   Z   = Q . K^T     (lane = key, 16 heads per lane)   -> scores, and G = dI_j 1[z>0]
//   Z^T = K . Q^T     (lane = head, 16 keys per lane)   -> G^T and dw
//   dq^T += K^T . G^T                  (K^T by transposing LDS reads; 128 AGPR accumulators)
//   c^T  = (wQ)^T . G                  (the pair's dk row; w folded into a bf16 copy of Q, whose
//                                       transposed fragments are read once per query into 64
//                                       AccVGPRs; the four 32-dim tiles as independent chains)
// The setup issues every load (Q rows, index row, dI, pair rows, head weights) before using any:
// one memory round trip per query.  c^T goes out through the block's own LDS tile (transposed to
// 256-byte rows) to the pair's key-major row of a staging buffer; a second kernel sums every
// key's rows (no float atomics: see the sparse MLA backward for the measured atomic rate).  The
// forward (scores only) runs the Z product alone.
//
// LDS rows are 256 bytes (one key or one head, 128 bf16); 16-byte chunk c of row r sits at slot
// c ^ swz16(r), swz16(r) = 2 (r & 3) + ((r >> 2) & 1) + (r & 8).  ds_read_b128 serves 16 lanes per
// LDS cycle: the operand read (16 consecutive rows, one chunk) then meets 16 distinct slots, and
// the transposing read (4 consecutive rows x 2 chunks per 16 lanes) 8.  Adding 128 bytes to a
// chunk address is an XOR on bit 7 of the (256-byte aligned) row address.
#include "dsa_common.h"
#include "dsa_kernels.h"
#include "dsa_kvtile.h"

namespace dsa {

namespace {

constexpr int kDi = 128;
constexpr int kHi = 64;
constexpr int kRowB = kDi * 2;
constexpr int kKTile = 32 * kRowB;
constexpr int kMaxTopkIdx = 4096;
constexpr int kPreI = 3;
constexpr int kStoresPerBlock = 8;   // global stores of one block's dk rows (16 B per lane each)

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

DSA_DEV u32x2 lds_read_tr16(uint32_t a) {
  s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds_ptr(a)));
  return __builtin_bit_cast(u32x2, r);
}

DSA_DEV constexpr uint32_t swz16(uint32_t r) { return ((r & 3u) << 1) | ((r >> 2) & 1u) | (r & 8u); }

// C += A * B with A in AccVGPRs (loop-invariant operand), B and C in VGPRs; hazards as the other
// asm forms (dsa_common.h).
DSA_DEV void mfma32x32x16_aA_cV(f32x16& c, const u32x4& a, const u32x4& b) {
  asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "a"(a), "v"(b));
}
DSA_DEV void mfma32x32x16_aA_cV_first(f32x16& c, const u32x4& a, const u32x4& b) {
  asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=v"(c) : "a"(a), "v"(b));
}

struct IdxSmem {
  union {
    struct {
      char tile[4][2][kKTile];   // per-wave double-buffered K tiles
      char qw[kHi * kRowB];      // backward: bf16(w_h q_h) rows
    };
    float part[4][kHi][68];      // backward epilogue: per-wave dq partials of 64 dims
  };
  int32_t idx[kMaxTopkIdx];
  float row[kMaxTopkIdx];        // backward: dI (0 at invalid slots); forward: the scores
  int32_t pos[kMaxTopkIdx];      // backward: staging row of each pair
  float dwp[4][kHi];
  int red[4];
};
static_assert(sizeof(IdxSmem) <= 160 * 1024, "indexer backward LDS budget");

}  // namespace

template <bool kBwd>
__global__ __launch_bounds__(256, 1) void indexer_sel_kernel(IdxSelParams p) {
  __shared__ __attribute__((aligned(256))) IdxSmem sm;
  const int t = xcd_remap(blockIdx.x, p.n_xcd);
  if (t >= p.total_q) return;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hb = lane >> 5, hl = lane & 31;
  // ---- setup: every load issued before any is used (one memory round trip)
  // Q fragments (A of Z, B of Z^T): head 32 mh + hl, dims 16 ks + 8 hb .. +7
  const bf16_t* qt_row = p.q + (int64_t)t * p.q_stride_t;
  u32x4 qf[2][8];
#pragma unroll
  for (int mh = 0; mh < 2; ++mh) {
    const int head = 32 * mh + hl;
    const bool ok = head < p.n_heads;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const u32x4 v = gload16(qt_row + (ok ? head : 0) * kDi + 16 * ks + 8 * hb);
      qf[mh][ks] = ok ? v : u32x4{0, 0, 0, 0};
    }
  }
  const float* wrow = p.w + (int64_t)t * p.n_heads;
  float wz[2][16];   // forward: weights of the Z rows (heads (i/4)*8 + 4 hb + i%4 of tile mh)
  if (!kBwd) {
#pragma unroll
    for (int mh = 0; mh < 2; ++mh)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int h = 32 * mh + (i >> 2) * 8 + 4 * hb + (i & 3);
        wz[mh][i] = h < p.n_heads ? wrow[h] : 0.f;
      }
  }
  // index row and, backward, dI and the staging row of every slot
  constexpr int kPer = kMaxTopkIdx / 256;
  const int32_t* idx_row = p.idx + (int64_t)t * p.idx_stride;
  const float* drow = kBwd ? p.d_index + (int64_t)t * p.d_stride : nullptr;
  const int64_t* prow = kBwd ? p.pair_pos + (int64_t)t * p.topk : nullptr;
  int32_t iv[kPer];
  float dv[kPer];
  int64_t pv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int j = threadIdx.x + 256 * i;
    const bool in = j < p.topk;
    iv[i] = in ? idx_row[j] : -1;
    if (kBwd) {
      dv[i] = in ? drow[j] : 0.f;
      pv[i] = in ? prow[j] : -1;
    }
  }
  // backward: rows of Q and the head weights for the w-scaled copy
  u32x4 qv4[4];
  float wh4[4];
  if (kBwd) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int h = (threadIdx.x + 256 * r) >> 4, c = (threadIdx.x + 256 * r) & 15;
      const bool ok = h < p.n_heads;
      qv4[r] = gload16(qt_row + (ok ? h : 0) * kDi + 8 * c);
      wh4[r] = ok ? wrow[h] : 0.f;
    }
  }
  const int kpad_t = (p.topk + 31) / 32 * 32;
  int last = -1;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int j = threadIdx.x + 256 * i;
    if (j < kpad_t) {
      int x = iv[i];
      if (x < 0 || x >= p.n_k || (p.causal && x > t)) x = -1;
      sm.idx[j] = x;
      if (x >= 0) last = j;
      if (kBwd) {
        sm.row[j] = x >= 0 ? dv[i] : 0.f;
        sm.pos[j] = (int32_t)(x >= 0 && pv[i] >= 0 ? pv[i] : p.g_sink_row);
      }
    }
  }
  if (kBwd) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int h = (threadIdx.x + 256 * r) >> 4, c = (threadIdx.x + 256 * r) & 15;
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(wh4[r] * bf16_lo(qv4[r][e]), wh4[r] * bf16_hi(qv4[r][e]));
      lds_store16(&sm.qw[h * kRowB + 16 * (c ^ swz16(h))], o);
    }
  }
  last = wave_max_i(last);
  if (lane == 0) sm.red[wave] = last;
  wait_vmcnt0();   // every compiler-visible load retired before the asynchronous copies start
  __syncthreads();
  last = max(max(sm.red[0], sm.red[1]), max(sm.red[2], sm.red[3]));
  const int nblk = __builtin_amdgcn_readfirstlane((last + 32) / 32);
  const int kpad = nblk * 32;

  const uint32_t tiles = lds_addr(sm.tile[wave][0]);
  const uint32_t qw0 = lds_addr(sm.qw);
  // gather of block blk into the tile at LDS address buf: copy r moves keys 4r .. 4r+3, lane l
  // filling slot l & 15 of key 4r + l / 16 from that key's chunk (l & 15) ^ swz16(key)
  auto gather = [&](uint32_t buf, int blk) {
    const int kk0 = lane >> 4;
    const uint32_t sl = lane & 15;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int kk = 4 * r + kk0;
      const int row = sm.idx[blk * 32 + kk];
      const char* src = reinterpret_cast<const char*>(p.k) + (int64_t)(row >= 0 ? row : 0) * kRowB +
                        16u * (sl ^ swz16(kk));
      async_copy16_unordered(src, buf + 1024u * r);
    }
  };
  // Z operand: key hl, chunk 2 ks + hb -> (tile + zoff) ^ 32 ks
  const uint32_t zoff = hl * kRowB + 16u * (hb ^ swz16(hl));
  // transposing reads (A of dq^T / c^T): 16-lane group g, lane gi feeds row 16a + 8h + 4(g/2) +
  // gi/4 (the C-layout row order of Z^T / Z) and dims 32m + 16(g%2) + 4(gi%4); m&1 selects the
  // precomputed slot, m>>1 adds 128 bytes
  uint32_t troff[2][2][2];
  {
    const int g = lane >> 4, gi = lane & 15;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int m1 = 0; m1 < 2; ++m1) {
          const uint32_t key = 16 * a + 8 * h + 4 * (g >> 1) + (gi >> 2);
          const uint32_t cp = 2 * (g & 1) + ((gi >> 1) & 1);
          troff[a][h][m1] = key * kRowB + 16u * ((4u * m1) ^ cp ^ swz16(key)) + 8u * (gi & 1);
        }
  }

  // (wQ)^T fragments for the dk-row product, read once per query: [mt][mh][s]
  u32x4 qt[4][2][2];
  if (kBwd) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int mh = 0; mh < 2; ++mh)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const uint32_t base = qw0 + mh * kKTile, o = 128u * (mt >> 1);
          const u32x2 lo = lds_read_tr16((base + troff[s2][0][mt & 1]) ^ o);
          const u32x2 hi = lds_read_tr16((base + troff[s2][1][mt & 1]) ^ o);
          qt[mt][mh][s2] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
  }
  f32x16 dqa[4][2];
  float dwacc[2] = {0.f, 0.f};
  if (kBwd) {
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int n = 0; n < 2; ++n) dqa[m][n] = f32x16{};
  }

  if (wave < nblk) gather(tiles, wave);
  int it = 0;
  for (int blk = wave; blk < nblk; blk += 4, ++it) {
    const uint32_t tb = tiles + (it & 1) * kKTile;
    // block blk's copies were issued before the previous block's dk row stores
    if (kBwd && it > 0) wait_vmcnt<kStoresPerBlock>();
    else wait_vmcnt<0>();
    asm volatile("" ::: "memory");
    if (blk + 4 < nblk) gather(tiles + ((it + 1) & 1) * kKTile, blk + 4);

    // ---- Z (and Z^T): 8 k-steps of 16 dims, K fragments prefetched
    f32x16 z[2], zt[2];
    {
      uint32_t zb = tb + zoff;
      asm volatile("" : "+v"(zb));
      u32x4 kf[kPreI];
#pragma unroll
      for (int i = 0; i < kPreI; ++i) kf[i] = lds_load16(lds_ptr(zb ^ (32u * i)));
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const u32x4 cur = kf[ks % kPreI];
        if (ks + kPreI < 8) kf[ks % kPreI] = lds_load16(lds_ptr(zb ^ (32u * (ks + kPreI))));
        if (ks == 0) {
          mfma32x32x16_cV_first(z[0], qf[0][0], cur);
          mfma32x32x16_cV_first(z[1], qf[1][0], cur);
          if (kBwd) {
            mfma32x32x16_cV_first(zt[0], cur, qf[0][0]);
            mfma32x32x16_cV_first(zt[1], cur, qf[1][0]);
          }
        } else {
          mfma32x32x16_cV(z[0], qf[0][ks], cur);
          mfma32x32x16_cV(z[1], qf[1][ks], cur);
          if (kBwd) {
            mfma32x32x16_cV(zt[0], cur, qf[0][ks]);
            mfma32x32x16_cV(zt[1], cur, qf[1][ks]);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    auto ktr = [&](int f) {
      const uint32_t o = 128u * ((f & 3) >> 1);
      const u32x2 lo = lds_read_tr16((tb + troff[f >> 2][0][f & 1]) ^ o);
      const u32x2 hi = lds_read_tr16((tb + troff[f >> 2][1][f & 1]) ^ o);
      return u32x4{lo[0], lo[1], hi[0], hi[1]};
    };
    constexpr int kPreT = 3;
    u32x4 kt[kPreT];
    if (kBwd) {
#pragma unroll
      for (int f = 0; f < kPreT; ++f) kt[f] = ktr(f);
    }
    mfma_acc_drain();

    if (!kBwd) {
      float sc = 0.f;
#pragma unroll
      for (int mh = 0; mh < 2; ++mh)
#pragma unroll
        for (int i = 0; i < 16; ++i) sc = __builtin_fmaf(wz[mh][i], relu_bits(z[mh][i]), sc);
      sc += __shfl_xor(sc, 32, 64);
      if (hb == 0) sm.row[blk * 32 + hl] = sm.idx[blk * 32 + hl] >= 0 ? sc : -INFINITY;
      continue;
    }

    // ---- G^T (from Z^T: lane = head, rows = keys) and dw; G (from Z: lane = key, rows = heads)
    const float d_own = sm.row[blk * 32 + hl];
    float dr[16];
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(&sm.row[blk * 32 + gq * 8 + 4 * hb]);
#pragma unroll
      for (int e = 0; e < 4; ++e) dr[4 * gq + e] = v[e];
    }
    u32x4 gt[2][2], gz[2][2];
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      float dws = 0.f;
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        const float a0 = zt[n][i] > 0.f ? dr[i] : 0.f, a1 = zt[n][i + 1] > 0.f ? dr[i + 1] : 0.f;
        gt[n][i >> 3][(i & 7) >> 1] = pack_bf16x2(a0, a1);
        dws = __builtin_fmaf(dr[i], relu_bits(zt[n][i]), dws);
        dws = __builtin_fmaf(dr[i + 1], relu_bits(zt[n][i + 1]), dws);
        const float b0 = z[n][i] > 0.f ? d_own : 0.f, b1 = z[n][i + 1] > 0.f ? d_own : 0.f;
        gz[n][i >> 3][(i & 7) >> 1] = pack_bf16x2(b0, b1);
      }
      dwacc[n] += dws;
    }

    // ---- dq^T[dims x heads] += K^T . G^T (K^T fragment f = 4 a + mm, read kPreT fragments ahead;
    // the first ones before G^T is formed)
#pragma unroll
    for (int f = 0; f < 8; ++f) {
      const u32x4 cur = kt[f % kPreT];
      if (f + kPreT < 8) kt[f % kPreT] = ktr(f + kPreT);
#pragma unroll
      for (int n = 0; n < 2; ++n) mfma32x32x16_cA(dqa[f & 3][n], cur, gt[n][f >> 2]);
      __builtin_amdgcn_sched_barrier(0);
    }

    // ---- c^T[dims x keys] = (wQ)^T . G: four independent dim-tile chains, then staged as 256-byte
    // key rows in this block's tile
    {
      f32x16 c[4];
#pragma unroll
      for (int mh = 0; mh < 2; ++mh)
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
            if (mh == 0 && s == 0) mfma32x32x16_aA_cV_first(c[mt], qt[mt][mh][s], gz[mh][s]);
            else mfma32x32x16_aA_cV(c[mt], qt[mt][mh][s], gz[mh][s]);
            __builtin_amdgcn_sched_barrier(0);
          }
      mfma_acc_drain();
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const u32x2 v = u32x2{pack_bf16x2(c[mt][4 * gq], c[mt][4 * gq + 1]),
                                pack_bf16x2(c[mt][4 * gq + 2], c[mt][4 * gq + 3])};
          *reinterpret_cast<u32x2*>(const_cast<char*>(
              lds_ptr(tb + hl * kRowB + 16u * ((4u * mt + gq) ^ swz16(hl)) + 8u * hb))) = v;
        }
    }
    // ---- key rows out: copy s writes keys 4s .. 4s+3, 16 lanes per 256-byte row
    {
      const uint32_t sl = lane & 15;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int r = 4 * s + (lane >> 4);
        const u32x4 v = lds_load16(lds_ptr(tb + r * kRowB + 16u * sl));
        const int64_t grow = sm.pos[blk * 32 + r];
        *reinterpret_cast<u32x4*>(p.g_stage + grow * kDi + 8 * (sl ^ swz16(r))) = v;
      }
    }
  }

  if (!kBwd) {
    __syncthreads();
    float* out = p.scores + (int64_t)t * p.scores_stride;
    for (int j = threadIdx.x; j < p.topk; j += 256) out[j] = j < kpad ? sm.row[j] : -INFINITY;
    return;
  }

  // ---- epilogue: dw and dq summed over the four waves
  mfma_acc_drain();
#pragma unroll
  for (int n = 0; n < 2; ++n) {
    const float v = xor32_sum(dwacc[n]);
    if (hb == 0) sm.dwp[wave][32 * n + hl] = v;
  }
  __syncthreads();   // every wave is done with its tiles and the Q copy (the union is reused)
  const int h_red = threadIdx.x >> 2;          // head of this thread's sums
  const float w_red = h_red < p.n_heads ? wrow[h_red] : 0.f;
  float* dq_row = p.dq + ((int64_t)t * p.n_heads + h_red) * kDi;
#pragma unroll
  for (int ph = 0; ph < 2; ++ph) {
#pragma unroll
    for (int m2 = 0; m2 < 2; ++m2)
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const f32x16& a = dqa[2 * ph + m2][n];
          *reinterpret_cast<f32x4*>(&sm.part[wave][32 * n + hl][32 * m2 + 8 * gq + 4 * hb]) =
              f32x4{a[4 * gq], a[4 * gq + 1], a[4 * gq + 2], a[4 * gq + 3]};
        }
    __syncthreads();
    // thread -> (head threadIdx/4, 16 dims); 4 x 4 floats each
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = 16 * (threadIdx.x & 3) + 4 * q4;
      f32x4 s = *reinterpret_cast<const f32x4*>(&sm.part[0][h_red][d]);
#pragma unroll
      for (int w = 1; w < 4; ++w) s += *reinterpret_cast<const f32x4*>(&sm.part[w][h_red][d]);
      if (h_red < p.n_heads) *reinterpret_cast<f32x4*>(dq_row + 64 * ph + d) = s * w_red;
    }
    __syncthreads();
  }
  if (threadIdx.x < p.n_heads) {
    const int h = threadIdx.x;
    p.dw[(int64_t)t * p.n_heads + h] = sm.dwp[0][h] + sm.dwp[1][h] + sm.dwp[2][h] + sm.dwp[3][h];
  }
}

// dk[s] = sum of the 128-wide rows of key s's segment (fp32).  16 row lanes x 16 chunks.
__global__ __launch_bounds__(256) void idx_dk_reduce_kernel(const bf16_t* g_stage, const int64_t* offsets, int n_k,
                                                            float* dk) {
  __shared__ float red[15][kDi];
  const int s = blockIdx.x;
  if (s >= n_k) return;
  const int c = threadIdx.x & 15, r = threadIdx.x >> 4;
  const int64_t a = offsets[s], b = offsets[s + 1];
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  auto add_row = [&](const u32x4& v) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[2 * e] += bf16_lo(v[e]);
      acc[2 * e + 1] += bf16_hi(v[e]);
    }
  };
  auto load_row = [&](int64_t i) {   // each row is read once: non-temporal
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(g_stage + i * kDi + c * 8));
  };
  // rows a + r, a + r + 16, ..: four loads in flight per thread, summed in row order
  int64_t i = a + r;
  for (; i + 48 < b; i += 64) {
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = load_row(i + 16 * u);
#pragma unroll
    for (int u = 0; u < 4; ++u) add_row(v[u]);
  }
  for (; i < b; i += 16) add_row(load_row(i));
  if (r > 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[r - 1][c * 8 + e] = acc[e];
  }
  __syncthreads();
  if (r == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc[e];
#pragma unroll
      for (int k = 0; k < 15; ++k) v += red[k][c * 8 + e];
      dk[(int64_t)s * kDi + c * 8 + e] = v;
    }
  }
}

// ------------------------------------------------------------------------------------------
// Dense score backward: the gradients of I[t, j] = sum_h w relu(q[t,h] . k[row_base[t] + j]) over
// EVERY key of each row (the dense indexer loss backpropagates through the [T, pitch] scores).  A
// row's keys are one contiguous range, so neither kernel needs index rows or a pair order, and dk
// needs no staged per-pair rows:
//   dense_scores_dq_kernel  query-major (one workgroup per query, wave w takes blocks w, w + 4, ..
//       through its own double-buffered K tile and dI slot, rows swizzled by swz16): Z^T = K . Q^T (lane = head) gives
//       G^T = dI 1[z>0] and dw += dI relu(z); dq^T += K^T . G^T; dq = w * the sum over the waves.
//   dense_scores_dk_kernel  key-major: a workgroup holds 128 consecutive keys (wave w: 32, their K^T
//       fragments in registers for the whole run) and streams the queries that see them, each
//       query's Q rows, weights and dI through a double-buffered LDS slot: Z = Q . K^T (lane = key)
//       gives G = dI w 1[z>0]; dk^T += Q^T . G (Q^T by transposing LDS reads).  The queries are
//       cut into fixed chunks of kDenseQChunk (chunk c = queries 256c .. 256c + 255), one work item
//       per (key tile, chunk) that holds queries seeing the tile, so no workgroup runs a whole
//       document's queries and the items of one chunk stream the same Q rows at the same time
//       (chunk-major item order: they share them through L2); the chunks' partial dk tiles are
//       summed in chunk order by dense_dk_reduce_kernel (the same bits every run).
// Rows are monotone (row_base and row_base + row_len nondecreasing in t), so the queries that see
// a key tile are one range, found by binary search.
// ------------------------------------------------------------------------------------------
namespace {

// Row t's keys clipped to k and to the score pitch: [base, base + len).
DSA_DEV void dense_row(const DenseIdxBwdParams& p, int t, int& base, int& len) {
  base = p.row_base[t];
  len = p.row_len[t];
  if (base < 0 || base >= p.n_k || len < 0) len = 0;
  else len = min(min(len, p.n_k - base), p.pitch);
}

// Queries [lo, hi) that may see a key of key tile `tile`: lo = the first row ending past the
// tile's first key, hi = the first row starting past its last key.
DSA_DEV void dense_tile_queries(const DenseIdxBwdParams& p, int tile, int& lo, int& hi) {
  const int s0 = tile * kDenseDkKeys;
  const int s1 = min(s0 + kDenseDkKeys, p.n_k) - 1;
  int a = 0, b = p.total_q;
  while (a < b) {
    const int m = (a + b) >> 1;
    if (p.row_base[m] + p.row_len[m] > s0) b = m; else a = m + 1;
  }
  lo = a;
  b = p.total_q;
  while (a < b) {
    const int m = (a + b) >> 1;
    if (p.row_base[m] > s1) b = m; else a = m + 1;
  }
  hi = a;
}

struct DenseDqSmem {
  union {
    struct {
      char tile[4][2][kKTile];   // per-wave double-buffered K tiles
      float di[4][2][64];        // per-wave dI of the block (64 copied, 32 used)
    };
    float part[4][kHi][68];      // epilogue: per-wave dq partials of 64 dims
  };
  float dwp[4][kHi];
};

constexpr int kDkSlots = 3;        // query slots of the dk kernel's ring (rows of query i + 2 copied during i)
struct DenseDkSmem {
  char q[kDkSlots][kHi * kRowB];   // Q[t] rows (head r, 16-byte chunk c at slot c ^ swz16(r))
  float w[kDkSlots][kHi];
  float di[kDkSlots][kDenseDkKeys];  // dI[t, s - row_base[t]] of the tile's keys (masked in-register)
  float wpad[kHi];                 // target of wave 3's balancing copy (never read)
  int32_t rb[kDenseQChunk];        // row_base / row_len of the work item's queries
  int32_t rl[kDenseQChunk];
};

}  // namespace

__global__ __launch_bounds__(256, 1) void dense_scores_dq_kernel(DenseIdxBwdParams p) {
  __shared__ __attribute__((aligned(256))) DenseDqSmem sm;
  const int t = xcd_remap(blockIdx.x, p.n_xcd);
  if (t >= p.total_q) return;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hb = lane >> 5, hl = lane & 31;
  int base, len;
  dense_row(p, t, base, len);
  const int nblk = (len + 31) / 32;
  // Q fragments (B of Z^T): head 32 mh + hl, dims 16 ks + 8 hb .. +7
  const bf16_t* qt_row = p.q + (int64_t)t * p.n_heads * kDi;
  u32x4 qf[2][8];
#pragma unroll
  for (int mh = 0; mh < 2; ++mh) {
    const int head = 32 * mh + hl;
    const bool ok = head < p.n_heads;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const u32x4 v = gload16(qt_row + (ok ? head : 0) * kDi + 16 * ks + 8 * hb);
      qf[mh][ks] = ok ? v : u32x4{0, 0, 0, 0};
    }
  }
  wait_vmcnt0();   // compiler-visible loads retired before the asynchronous copies start
  const float* drow = p.d_scores + (int64_t)t * p.pitch;
  const uint32_t tiles = lds_addr(sm.tile[wave][0]);
  const uint32_t dis = lds_addr(sm.di[wave][0]);
  // block blk into slot `slot`: K rows of keys base + 32 blk + kk (past the row: its last key,
  // masked), copy r moving keys 4r .. 4r+3 (lane l: slot l & 15 of key 4r + l/16 from chunk
  // (l & 15) ^ swz16(key)); then 64 dI values from column 32 blk (clamped to the row's pitch)
  // Keys of a block past the row's end are gathered too (masked) as long as they are k rows: then
  // copy r reads 1 KB from the scalar address of key base + 32 blk + 4r plus a per-lane offset
  // (swz16(4r + lane/16) depends on r & 3 only: four offsets serve all eight copies).
  uint32_t voff[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) voff[v] = (lane >> 4) * kRowB + 16u * ((lane & 15) ^ swz16(4 * v + (lane >> 4)));
  auto gather = [&](int slot, int blk) {
    if (base + 32 * blk + 32 <= p.n_k) {
      const char* kb = reinterpret_cast<const char*>(p.k) + (int64_t)(base + 32 * blk) * kRowB;
      asm volatile("s_nop 4");   // any VALU-written SGPR of the address: 5 wait states before the DMA
#pragma unroll
      for (int r = 0; r < 8; ++r) copy_row16(tiles + slot * kKTile + 1024u * r, kb + 1024 * r, voff[r & 3]);
    } else {   // the last rows of k: clamp each key to the row
      const int kk0 = lane >> 4;
      const uint32_t sl = lane & 15;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int kk = 4 * r + kk0;
        const int j = min(32 * blk + kk, len - 1);
        const char* src = reinterpret_cast<const char*>(p.k) + (int64_t)(base + j) * kRowB + 16u * (sl ^ swz16(kk));
        async_copy16_unordered(src, tiles + slot * kKTile + 1024u * r);
      }
    }
    async_copy4_unordered(drow + min(32 * blk + lane, p.pitch - 1), dis + slot * 256u);
  };
  const uint32_t zoff = hl * kRowB + 16u * (hb ^ swz16(hl));
  uint32_t troff[2][2][2];
  {
    const int g = lane >> 4, gi = lane & 15;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int m1 = 0; m1 < 2; ++m1) {
          const uint32_t key = 16 * a + 8 * h + 4 * (g >> 1) + (gi >> 2);
          const uint32_t cp = 2 * (g & 1) + ((gi >> 1) & 1);
          troff[a][h][m1] = key * kRowB + 16u * ((4u * m1) ^ cp ^ swz16(key)) + 8u * (gi & 1);
        }
  }
  f32x16 dqa[4][2];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int n = 0; n < 2; ++n) dqa[m][n] = f32x16{};
  float dwacc[2] = {0.f, 0.f};

  if (wave < nblk) gather(0, wave);
  int it = 0;
  for (int blk = wave; blk < nblk; blk += 4, ++it) {
    const int slot = it & 1;
    const uint32_t tb = tiles + slot * kKTile;
    wait_vmcnt<0>();
    asm volatile("" ::: "memory");
    if (blk + 4 < nblk) gather(slot ^ 1, blk + 4);
    // dI of the lane's 16 keys (read before the MFMAs, used after them)
    f32x4 dv4[4];
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) dv4[gq] = *reinterpret_cast<const f32x4*>(&sm.di[wave][slot][gq * 8 + 4 * hb]);
    // ---- Z^T = K . Q^T (lane = head, rows = keys (i/4)*8 + 4 hb + i%4)
    f32x16 zt[2];
    {
      uint32_t zb = tb + zoff;
      asm volatile("" : "+v"(zb));
      u32x4 kf[kPreI];
#pragma unroll
      for (int i = 0; i < kPreI; ++i) kf[i] = lds_load16(lds_ptr(zb ^ (32u * i)));
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const u32x4 cur = kf[ks % kPreI];
        if (ks + kPreI < 8) kf[ks % kPreI] = lds_load16(lds_ptr(zb ^ (32u * (ks + kPreI))));
        if (ks == 0) {
          mfma32x32x16_cV_first(zt[0], cur, qf[0][0]);
          mfma32x32x16_cV_first(zt[1], cur, qf[1][0]);
        } else {
          mfma32x32x16_cV(zt[0], cur, qf[0][ks]);
          mfma32x32x16_cV(zt[1], cur, qf[1][ks]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    auto ktr = [&](int f) {
      const int a = f >> 2, mm = f & 3;
      const uint32_t o = 128u * (mm >> 1);
      const u32x2 lo = lds_read_tr16((tb + troff[a][0][mm & 1]) ^ o);
      const u32x2 hi = lds_read_tr16((tb + troff[a][1][mm & 1]) ^ o);
      return u32x4{lo[0], lo[1], hi[0], hi[1]};
    };
    constexpr int kPreT = 3;
    u32x4 kt[kPreT];
#pragma unroll
    for (int f = 0; f < kPreT; ++f) kt[f] = ktr(f);
    mfma_acc_drain();
    // ---- G^T = dI 1[z>0] (0 past the row) and dw
    const int nvalid = len - 32 * blk;
    float dr[16];
    if (nvalid >= 32) {
#pragma unroll
      for (int gq = 0; gq < 4; ++gq)
#pragma unroll
        for (int e = 0; e < 4; ++e) dr[4 * gq + e] = dv4[gq][e];
    } else {
#pragma unroll
      for (int gq = 0; gq < 4; ++gq)
#pragma unroll
        for (int e = 0; e < 4; ++e) dr[4 * gq + e] = gq * 8 + 4 * hb + e < nvalid ? dv4[gq][e] : 0.f;
    }
    u32x4 gt[2][2];
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      float dws = 0.f;
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        const float a0 = zt[n][i] > 0.f ? dr[i] : 0.f, a1 = zt[n][i + 1] > 0.f ? dr[i + 1] : 0.f;
        gt[n][i >> 3][(i & 7) >> 1] = pack_bf16x2(a0, a1);
        dws = __builtin_fmaf(dr[i], relu_bits(zt[n][i]), dws);
        dws = __builtin_fmaf(dr[i + 1], relu_bits(zt[n][i + 1]), dws);
      }
      dwacc[n] += dws;
    }
    // ---- dq^T[dims x heads] += K^T . G^T (K^T fragment f = 4 a + mm, read kPreT fragments ahead;
    // the first ones before G^T is formed)
#pragma unroll
    for (int f = 0; f < 8; ++f) {
      const u32x4 cur = kt[f % kPreT];
      if (f + kPreT < 8) kt[f % kPreT] = ktr(f + kPreT);
#pragma unroll
      for (int n = 0; n < 2; ++n) mfma32x32x16_cA(dqa[f & 3][n], cur, gt[n][f >> 2]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- epilogue: dw and dq summed over the four waves (the tiles' union is reused)
  mfma_acc_drain();
#pragma unroll
  for (int n = 0; n < 2; ++n) {
    const float v = xor32_sum(dwacc[n]);
    if (hb == 0) sm.dwp[wave][32 * n + hl] = v;
  }
  __syncthreads();
  const float* wrow = p.w + (int64_t)t * p.n_heads;
  const int h_red = threadIdx.x >> 2;
  const float w_red = h_red < p.n_heads ? wrow[h_red] : 0.f;
  float* dq_row = p.dq + ((int64_t)t * p.n_heads + h_red) * kDi;
#pragma unroll
  for (int ph = 0; ph < 2; ++ph) {
#pragma unroll
    for (int m2 = 0; m2 < 2; ++m2)
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const f32x16& a = dqa[2 * ph + m2][n];
          *reinterpret_cast<f32x4*>(&sm.part[wave][32 * n + hl][32 * m2 + 8 * gq + 4 * hb]) =
              f32x4{a[4 * gq], a[4 * gq + 1], a[4 * gq + 2], a[4 * gq + 3]};
        }
    __syncthreads();
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int dd = 16 * (threadIdx.x & 3) + 4 * q4;
      f32x4 sacc = *reinterpret_cast<const f32x4*>(&sm.part[0][h_red][dd]);
#pragma unroll
      for (int w = 1; w < 4; ++w) sacc += *reinterpret_cast<const f32x4*>(&sm.part[w][h_red][dd]);
      if (h_red < p.n_heads) *reinterpret_cast<f32x4*>(dq_row + 64 * ph + dd) = sacc * w_red;
    }
    __syncthreads();
  }
  if (threadIdx.x < p.n_heads) {
    const int h = threadIdx.x;
    p.dw[(int64_t)t * p.n_heads + h] = sm.dwp[0][h] + sm.dwp[1][h] + sm.dwp[2][h] + sm.dwp[3][h];
  }
}

// Work item (key tile, query chunk): chunk-major ids, so the workgroups running at once stream the
// same queries' rows.
__global__ __launch_bounds__(256, 2) void dense_scores_dk_kernel(DenseIdxBwdParams p) {
  __shared__ __attribute__((aligned(256))) DenseDkSmem sm;
  const int item = xcd_remap(blockIdx.x, p.n_xcd);
  if (item >= p.n_tiles * p.max_chunks) return;
  const int chunk = item / p.n_tiles, tile = item - chunk * p.n_tiles;
  int lo, hi;
  dense_tile_queries(p, tile, lo, hi);
  const int t_begin = max(lo, chunk * kDenseQChunk);
  const int nq = min(hi, (chunk + 1) * kDenseQChunk) - t_begin;
  if (nq <= 0) return;   // no query of this chunk sees the tile: no partial (the reduce knows)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hb = lane >> 5, hl = lane & 31;
  const int s0 = tile * kDenseDkKeys;
  const int s = s0 + 32 * wave + hl;                     // this lane's key (Z column)
  // K^T fragments (B of Z = Q . K^T): key s, dims 16 ks + 8 hb .. +7
  u32x4 kf[8];
  {
    const bf16_t* krow = p.k + (int64_t)min(s, p.n_k - 1) * kDi + 8 * hb;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) kf[ks] = gload16(krow + 16 * ks);
  }
  // the work item's row descriptors
  for (int i = threadIdx.x; i < nq; i += 256) {
    int b, l;
    dense_row(p, t_begin + i, b, l);
    sm.rb[i] = b;
    sm.rl[i] = l;
  }
  wait_vmcnt0();
  __syncthreads();
  const uint32_t qs0 = lds_addr(sm.q[0]), ws0 = lds_addr(sm.w[0]), ds0 = lds_addr(sm.di[0]);
  const uint32_t wpad0 = lds_addr(sm.wpad);
  // query i's rows into slot `slot`, five copies per wave (so every wave's waits count the same):
  // Q (16 copies of 4 head rows, 4 per wave; rows past n_heads re-read head 0, never used), the
  // tile's 128 dI columns (waves 0 and 1, 64 each; columns outside the row clamped into it and
  // masked by the caller), the weights (wave 2) and a copy of them into an unread pad (wave 3)
  // with 64 heads, copy r reads 1 KB from the scalar address of head 4r plus a per-lane offset
  // (swz16(4r + lane/16) depends on r & 3 only)
  uint32_t voff[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) voff[v] = (lane >> 4) * kRowB + 16u * ((lane & 15) ^ swz16(4 * v + (lane >> 4)));
  auto issue = [&](int slot, int i) {
    const int tq = t_begin + i;
    const bf16_t* qrow = p.q + (int64_t)tq * p.n_heads * kDi;
    if (p.n_heads == kHi) {
      const char* qb0 = reinterpret_cast<const char*>(qrow);
      asm volatile("s_nop 4");   // any VALU-written SGPR of the address: 5 wait states before the DMA
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int r = 4 * wave + r4;
        copy_row16(qs0 + slot * (kHi * kRowB) + 1024u * r, qb0 + 1024 * r, voff[r4]);
      }
    } else {
      const uint32_t sl = lane & 15;
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int r = 4 * wave + r4;
        const int h = 4 * r + (lane >> 4);
        const char* src = reinterpret_cast<const char*>(qrow + (h < p.n_heads ? h : 0) * kDi) + 16u * (sl ^ swz16(h));
        async_copy16_unordered(src, qs0 + slot * (kHi * kRowB) + 1024u * r);
      }
    }
    if (wave < 2) {
      const int j = min(max(s0 + 64 * wave + lane - sm.rb[i], 0), p.pitch - 1);
      async_copy4_unordered(p.d_scores + (int64_t)tq * p.pitch + j, ds0 + slot * 512u + 256u * wave);
    } else {
      async_copy4_unordered(p.w + (int64_t)tq * p.n_heads + min(lane, p.n_heads - 1),
                            wave == 2 ? ws0 + slot * 256u : wpad0);
    }
  };
  // Z operand (A = Q rows): head 32 n + hl, chunk 2 ks + hb; transposing reads of Q^T (A of dk^T)
  const uint32_t zoff = hl * kRowB + 16u * (hb ^ swz16(hl));
  uint32_t troff[2][2][2];
  {
    const int g = lane >> 4, gi = lane & 15;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int m1 = 0; m1 < 2; ++m1) {
          const uint32_t r = 16 * a + 8 * h + 4 * (g >> 1) + (gi >> 2);
          const uint32_t cp = 2 * (g & 1) + ((gi >> 1) & 1);
          troff[a][h][m1] = r * kRowB + 16u * ((4u * m1) ^ cp ^ swz16(r)) + 8u * (gi & 1);
        }
  }
  f32x16 dka[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) dka[m] = f32x16{};

  issue(0, 0);
  if (nq > 1) issue(1, 1);
  int slot = 0, slot2 = 2;   // query i's slot and query i + 2's
  for (int i = 0; i < nq; ++i) {
    const int base_t = sm.rb[i], len_t = sm.rl[i];
    if (i + 1 < nq) wait_vmcnt<5>(); else wait_vmcnt<0>();   // query i's five copies (i + 1's may fly)
    __syncthreads();   // query i's rows are in; every wave is done with query i - 1's slot
    if (i + 2 < nq) issue(slot2, i + 2);
    const uint32_t qb = qs0 + slot * (kHi * kRowB);
    // weights and dI of query i (read before the MFMAs, used after them)
    const bool vis = s >= base_t && s < base_t + len_t;
    const float dv = vis ? sm.di[slot][32 * wave + hl] : 0.f;
    f32x4 wv[2][4];
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) wv[n][gq] = *reinterpret_cast<const f32x4*>(&sm.w[slot][32 * n + 8 * gq + 4 * hb]);
    // ---- Z[heads x keys] = Q . K^T (lane = key s, element i = head 32 n + (i/4)*8 + 4 hb + i%4);
    // dI w of the lane's 32 (head, key) values (0 for heads past n_heads), two per MFMA
    f32x16 z[2];
    float dvw[2][16];
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      uint32_t zb = qb + n * kKTile + zoff;
      asm volatile("" : "+v"(zb));
      u32x4 qa[kPreI];
#pragma unroll
      for (int u = 0; u < kPreI; ++u) qa[u] = lds_load16(lds_ptr(zb ^ (32u * u)));
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const u32x4 cur = qa[ks % kPreI];
        if (ks + kPreI < 8) qa[ks % kPreI] = lds_load16(lds_ptr(zb ^ (32u * (ks + kPreI))));
        if (ks == 0) mfma32x32x16_cV_first(z[n], cur, kf[0]);
        else mfma32x32x16_cV(z[n], cur, kf[ks]);
#pragma unroll
        for (int e2 = 0; e2 < 2; ++e2) {
          const int i2 = 2 * ks + e2, h = 32 * n + 8 * (i2 >> 2) + 4 * hb + (i2 & 3);
          dvw[n][i2] = h < p.n_heads ? dv * wv[n][i2 >> 2][i2 & 3] : 0.f;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // Q^T fragment f of the dk^T product (f = 8 mh + 4 s2 + mt): the first kPreT are read before
    // G is formed, the others kPreT MFMAs ahead of their use
    auto qtr = [&](int f) {
      const int mh = f >> 3, s2 = (f >> 2) & 1, mt = f & 3;
      const uint32_t b = qb + mh * kKTile, o = 128u * (mt >> 1);
      const u32x2 lo2 = lds_read_tr16((b + troff[s2][0][mt & 1]) ^ o);
      const u32x2 hi2 = lds_read_tr16((b + troff[s2][1][mt & 1]) ^ o);
      return u32x4{lo2[0], lo2[1], hi2[0], hi2[1]};
    };
    constexpr int kPreT = 4;
    u32x4 qt[kPreT];
#pragma unroll
    for (int f = 0; f < kPreT; ++f) qt[f] = qtr(f);
    mfma_acc_drain();
    // ---- G = dI w 1[z>0] (0 where the query does not see key s)
    u32x4 gz[2][2];
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int i = 0; i < 16; i += 2)
        gz[n][i >> 3][(i & 7) >> 1] = pack_bf16x2(z[n][i] > 0.f ? dvw[n][i] : 0.f, z[n][i + 1] > 0.f ? dvw[n][i + 1] : 0.f);
    // ---- dk^T[dims x keys] += Q^T . G: four independent dim-tile chains
#pragma unroll
    for (int f = 0; f < 16; ++f) {
      const u32x4 cur = qt[f % kPreT];
      if (f + kPreT < 16) qt[f % kPreT] = qtr(f + kPreT);
      mfma32x32x16_cV(dka[f & 3], cur, gz[f >> 3][(f >> 2) & 1]);
      __builtin_amdgcn_sched_barrier(0);
    }
    slot = slot == kDkSlots - 1 ? 0 : slot + 1;
    slot2 = slot2 == kDkSlots - 1 ? 0 : slot2 + 1;
  }
  mfma_acc_drain();
  // ---- the partial tile: key 32 w + hl, dims 32 mt + 8 q + 4 hb .. +3
  float* part = p.dk_part + ((int64_t)tile * p.max_chunks + chunk) * (kDenseDkKeys * kDi) + (32 * wave + hl) * kDi;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<f32x4*>(part + 32 * mt + 8 * q + 4 * hb) =
          f32x4{dka[mt][4 * q], dka[mt][4 * q + 1], dka[mt][4 * q + 2], dka[mt][4 * q + 3]};
}

// dk of 32 keys (quarter blockIdx.x & 3 of key tile blockIdx.x / 4): the sum of the tile's chunks'
// partial rows, in chunk order.
__global__ __launch_bounds__(256) void dense_dk_reduce_kernel(DenseIdxBwdParams p) {
  const int tile = blockIdx.x >> 2, quarter = blockIdx.x & 3;
  int lo, hi;
  dense_tile_queries(p, tile, lo, hi);
  // chunks c0 .. c1 hold the tile's queries [lo, hi) (each of them some)
  const int c0 = lo / kDenseQChunk, c1 = hi > lo ? min((hi - 1) / kDenseQChunk, p.max_chunks - 1) : c0 - 1;
  const int s0 = tile * kDenseDkKeys;
  const f32x4* part = reinterpret_cast<const f32x4*>(p.dk_part + (int64_t)tile * p.max_chunks * (kDenseDkKeys * kDi));
  constexpr int kVec = kDenseDkKeys * kDi / 4;   // f32x4 per tile
  for (int v = quarter * (kVec / 4) + threadIdx.x; v < (quarter + 1) * (kVec / 4); v += 256) {
    const int key = v / (kDi / 4);
    if (s0 + key >= p.n_k) break;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int c = c0; c <= c1; ++c) acc += part[(int64_t)c * kVec + v];
    *reinterpret_cast<f32x4*>(p.dk + (int64_t)(s0 + key) * kDi + 4 * (v % (kDi / 4))) = acc;
  }
}

int launch_dense_scores_bwd(const DenseIdxBwdParams& p, hipStream_t stream) {
  if (p.n_xcd < 1) return -1;
  if (p.n_heads > kHi || p.n_heads < 1) return -2;
  if (p.total_q > 0)
    hipLaunchKernelGGL(dense_scores_dq_kernel, dim3(xcd_grid(p.total_q, p.n_xcd)), dim3(256), 0, stream, p);
  if (p.total_q > 0 && p.n_tiles > 0)
    hipLaunchKernelGGL(dense_scores_dk_kernel, dim3(xcd_grid(p.n_tiles * p.max_chunks, p.n_xcd)), dim3(256), 0,
                       stream, p);
  if (p.n_tiles > 0) hipLaunchKernelGGL(dense_dk_reduce_kernel, dim3(4 * p.n_tiles), dim3(256), 0, stream, p);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_indexer_selected_scores(const IdxSelParams& p, hipStream_t stream) {
  if (p.n_xcd < 1) return -1;
  if (p.topk > kMaxTopkIdx || p.n_heads > kHi) return -2;
  if (p.total_q == 0) return 0;
  hipLaunchKernelGGL(indexer_sel_kernel<false>, dim3(xcd_grid(p.total_q, p.n_xcd)), dim3(256), 0, stream, p);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_indexer_scores_bwd(const IdxSelParams& p, hipStream_t stream) {
  if (p.n_xcd < 1) return -1;
  if (p.topk > kMaxTopkIdx || p.n_heads > kHi) return -2;
  if (p.g_sink_row >= INT32_MAX) return -2;   // staging rows are kept in 32 bits
  if (p.n_k > 0) launch_pair_csr(p.idx, p.idx_stride, p.total_q, p.topk, p.n_k, p.causal, 0, p.csr_counts,
                                 p.csr_offsets, p.pair_pos, stream);
  if (p.total_q > 0)
    hipLaunchKernelGGL(indexer_sel_kernel<true>, dim3(xcd_grid(p.total_q, p.n_xcd)), dim3(256), 0, stream, p);
  if (p.n_k > 0)
    hipLaunchKernelGGL(idx_dk_reduce_kernel, dim3(p.n_k), dim3(256), 0, stream, p.g_stage, p.csr_offsets, p.n_k, p.dk);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace dsa
