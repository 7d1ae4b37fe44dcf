// K3: index-gathered sparse MLA attention forward over the shared 576-wide latent KV (gfx950).
//
// Replaces the un-fused sparse attention that Megatron's DSAttention runs on the indexer's
// top-k (called from reference src/mcore_bridge/model/modules/multi_latent_attention.py:262-270):
//   out[t,h] = sum_{j: idx[t,j] valid} softmax_j(scale * q[t,h] . kv[idx[t,j]]) * kv[idx[t,j], :512]
//   lse[t,h] = ln sum_j exp(scale * q[t,h] . kv[idx[t,j]])
//
// Work decomposition (one workgroup = one query token, up to 128 heads):
//   * wave w owns 32 heads for the scores.  Q[32 heads x 576] sits in registers for the whole
//     key loop (the B operand of S^T = K . Q^T, 144 VGPRs).
//   * the query's index row is staged once in LDS; selected KV rows are gathered 32 at a time
//     straight into LDS with global_load_lds (16 B per lane, no VGPR staging, swizzled tile of
//     dsa_kvtile.h) through a 3-stage ring.  The copies are issued through inline asm, one
//     every few QK MFMAs, and completed with an explicit s_waitcnt vmcnt(0) + barrier.
//   * QK: 36 MFMA 32x32x16 per 32-key block, A operands prefetched 3 MFMAs ahead.
//   * PV is split by latent dims: wave w accumulates O^T[128 dims x all 128 heads] in fp32
//     (256 AGPRs), so each wave reads a quarter of the V^T tile (ds_read_b64_tr_b16, the
//     hardware 16-bit transpose on the LDS read) instead of all of it.  Its B operand P^T comes
//     from every wave through LDS: each wave writes its converted S^T accumulator (the k order
//     inside each MFMA is permuted to match the S^T C layout, so no shuffle is needed), lane for
//     lane in the MFMA B layout.
//   * software pipeline: iteration j runs QK of block j, then PV of block j-1 with block j's
//     softmax interleaved between the PV MFMAs (one exp per MFMA), so the softmax VALU work
//     issues while the matrix pipe is busy.  Tiles j and j-1 are live, block j+1 is gathered
//     into the third ring slot during QK(j).
//   * softmax in the exp2 domain against a per-head reference max fixed by the first block
//     holding a valid key (2^64 headroom), so the O accumulators are never rescaled (a rescale
//     would pull the 256 AGPR accumulators through VGPRs).  A query whose scores overshoot the
//     headroom is recomputed once with its exact row max.  Row sums and overshoot maxima stay
//     per lane (one half of a head's keys) until the end of the pass: no cross-lane traffic
//     per block.
#include <mutex>

#include "dsa_common.h"
#include "dsa_kernels.h"
#include "dsa_kvtile.h"

namespace dsa {

namespace {

constexpr int kDqk = 576;
constexpr int kDv = 512;
constexpr int kBK = kTileKeys;          // keys per block (lane l%32 <-> key l%32)
constexpr int kStages = 3;
constexpr int kMaxTopk = 8192;
constexpr float kHeadroom = 64.0f;      // log2 headroom above the reference max
constexpr int kPre = 3;                 // LDS operand prefetch distance (MFMAs)

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

DSA_DEV u32x2 lds_read_tr16(const char* p) {
  s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  return __builtin_bit_cast(u32x2, r);
}

struct FwdSmem {
  union {
    struct {
      char tile[kStages][kTileBytes];
      u32x4 pbuf[2][8][64];   // P^T fragments of the last two blocks: [block & 1][2 * wave + a][lane]
      int32_t idx[kMaxTopk];
    };
    char ostage[128][kDv * 2];   // epilogue: the workgroup's 128 bf16 output rows
  };
  int red[4];
  int redo_flag;
  float inv_l[128];
};

}  // namespace

// ROPE = false: q rows of 512 (no rope part): the scores contract over the 512 latent dims only
// (32 QK MFMAs per block instead of 36) and the tiles' rope region is neither gathered nor read.
template <int NW, bool ROPE>
__global__ __launch_bounds__(NW * 64, 1) void sparse_mla_fwd_kernel(SparseFwdParams p) {
  constexpr int QKS = (ROPE ? kDqk : kDv) / 16;   // QK MFMAs (16-deep k-steps) per block
  constexpr int G = tile_copies_per_wave<NW, ROPE>();
  constexpr int kCopyEvery = QKS / G;             // QK MFMAs per gather copy
  static_assert(kCopyEvery * G == QKS, "copies spread evenly over the QK MFMAs");
  __shared__ __attribute__((aligned(128))) FwdSmem sm;

  // work item = (query t, key split); n_split > 1 only for decode, where a few queries must
  // still fill the chip: split s covers index slots [s*split_keys, (s+1)*split_keys) and writes
  // its normalised partial output and LSE to row t*n_split + s (merged by the combine kernel)
  const int n_items = p.total_q * p.n_split;
  const int item = xcd_remap(blockIdx.x, p.n_xcd);
  if (item >= n_items) return;
  const int t = item / p.n_split;
  const int split = item - t * p.n_split;
  const int64_t orow = item;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int hb = lane >> 5;          // row half of the MFMA C layout
  const int hl = lane & 31;          // head within the wave
  const int head = blockIdx.y * 128 + wave * 32 + hl;
  const bool head_ok = head < p.n_heads;

  // ---- Q fragments: lane holds q[t, head, 16*ks + 8*hb .. +7] for ks < QKS (q rows of 512 under
  // ROPE: no rope part, its fragments zero)
  u32x4 qf[QKS];
  {
    const bool q_rope = p.q_dim != kDv;
    const int qd = q_rope ? kDqk : kDv;
    const bf16_t* qrow = p.q + (int64_t)t * p.q_stride_t + (int64_t)(head_ok ? head : 0) * qd + hb * 8;
#pragma unroll
    for (int ks = 0; ks < QKS; ++ks) {
      u32x4 v = u32x4{0, 0, 0, 0};
      if (ks < kDv / 16 || q_rope) v = gload16(qrow + ks * 16);
      qf[ks] = head_ok ? v : u32x4{0, 0, 0, 0};
    }
  }

  // ---- stage the index row (invalid -> -1) and find the last valid position
  const int k_first = split * p.split_keys;
  const int n_slots = max(0, min(p.topk - k_first, p.split_keys));
  const int32_t* idx_row = p.idx + (int64_t)t * p.idx_stride + k_first;
  const int kpad = (n_slots + kBK - 1) / kBK * kBK;
  constexpr int kBatch = 8;   // index loads in flight per thread (one round trip per batch)
  int last = -1;
  for (int j0 = threadIdx.x; j0 < kpad; j0 += kBatch * NW * 64) {
    int v[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int j = j0 + i * NW * 64;
      v[i] = j < n_slots ? idx_row[j] : -1;
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int j = j0 + i * NW * 64;
      int x = v[i];
      if (x < 0 || x >= p.n_kv || (p.causal && x > t)) x = -1;
      if (j < kpad) {
        sm.idx[j] = x;
        if (x >= 0) last = j;
      }
    }
  }
  last = wave_max_i(last);
  if (lane == 0) sm.red[wave] = last;
  wait_vmcnt0();  // Q and index loads retired: nothing compiler-visible stays in flight
  __syncthreads();
#pragma unroll
  for (int w = 0; w < NW; ++w) last = max(last, sm.red[w]);
  const int nblk = __builtin_amdgcn_readfirstlane((last + kBK) / kBK);

  f32x16 o[kDv / 32];
  float m_ref = -INFINITY, m_seen = -INFINITY, l_run = 0.f;

  // QK operand addresses: lane reads key hl, chunk 2*ks + hb (see tile_off): V part at
  // qk_v + 32*ks for ks < 32, rope part at qk_r ^ (32*(ks-32)).
  const uint32_t qk_v = key_row(hl) * kTileVPitch + 16u * hb;
  const uint32_t qk_r = kTileVBytes + hl * 128u + 16u * (hb ^ ((hl >> 1) & 7u));
  // PV operand addresses (ds_read_tr): lane feeds key 16a + 8h + 4(g/2) + gi/4 (the S^T C-layout
  // key order) and dv 32m + 16(g%2) + 4(gi%4): byte pv[a][h] + 64*m.
  uint32_t pv[2][2];
  {
    const int g = lane >> 4, gi = lane & 15;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t key = 16 * a + 8 * h + 4 * (g >> 1) + (gi >> 2);
        pv[a][h] = key_row(key) * kTileVPitch + 32u * (g & 1) + 8u * (gi & 3);
      }
  }
  const uint32_t tile0 = lds_addr(sm.tile[0]);
  const uint32_t wsg = __builtin_amdgcn_readfirstlane(wave);

  // PV, split by latent dims: wave w accumulates O^T[dims DT*32*w .. +DT*32) x all NH*32 heads]
  // (o[m' * NH + n] = dim tile m', head tile n) from its own quarter of the V^T tile and the
  // P^T fragments of every wave, exchanged through LDS (lane-for-lane the MFMA B layout).  Each
  // wave then reads 512/NW dims of V^T per block instead of all 512.
  constexpr int DT = 16 / NW, NH = NW;
  const uint32_t pbuf0 = lds_addr(&sm.pbuf[0][0][0]);
  const uint32_t pv_dim0 = 64u * DT * wave;   // byte offset of this wave's first dim tile
  auto pf_addr = [&](int parity, int n, int aa) {
    return const_cast<char*>(lds_ptr(pbuf0 + (uint32_t)(((parity * 8 + 2 * n + aa) * 64 + lane) * 16)));
  };
  // O^T += V^T . P^T for one block of the tile at LDS address tp, P^T fragments of every wave in
  // slot `parity`; the two 16-key halves run one after the other, each holding its NH P^T
  // fragments while the V^T fragments stream (kPre ahead).  step(i) runs in the scheduling
  // group of PV MFMA i, so independent VALU work issues while the matrix pipe is busy.
  auto pv_block = [&](uint32_t tp, int parity, auto&& step) {
    uint32_t r00 = tp + pv[0][0] + pv_dim0, r01 = tp + pv[0][1] + pv_dim0;
    uint32_t r10 = tp + pv[1][0] + pv_dim0, r11 = tp + pv[1][1] + pv_dim0;
    asm volatile("" : "+v"(r00), "+v"(r01), "+v"(r10), "+v"(r11));
    auto vread = [&](int f) {   // V^T fragment f = DT * a + m'
      const int aa = f / DT, mm = f % DT;
      const uint32_t b0 = aa ? r10 : r00, b1 = aa ? r11 : r01;
      const u32x2 lo = lds_read_tr16(lds_ptr(b0 + 64u * mm)), hi = lds_read_tr16(lds_ptr(b1 + 64u * mm));
      return u32x4{lo[0], lo[1], hi[0], hi[1]};
    };
    constexpr int NF = 2 * DT;
    u32x4 v[kPre];
    u32x4 pfa[NH];
#pragma unroll
    for (int n = 0; n < NH; ++n) pfa[n] = lds_load16(pf_addr(parity, n, 0));
#pragma unroll
    for (int f = 0; f < kPre; ++f) v[f] = vread(f);
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      if (f == DT) {
#pragma unroll
        for (int n = 0; n < NH; ++n) pfa[n] = lds_load16(pf_addr(parity, n, 1));
      }
      const u32x4 cur = v[f % kPre];
      if (f + kPre < NF) v[f % kPre] = vread(f + kPre);
#pragma unroll
      for (int n = 0; n < NH; ++n) {
        mfma32x32x16_cA(o[(f % DT) * NH + n], cur, pfa[n]);
        step(f * NH + n);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  // Software pipeline: iteration blk multiplies S^T of block blk (QK), then runs the PV product
  // of block blk-1 with block blk's softmax interleaved between its MFMAs.  Two tiles are live
  // per iteration (blk, blk-1), so block blk+1 is gathered into the third ring slot during
  // iteration blk's QK MFMAs.  Iteration 0 multiplies tile 0 by P = 0 in place of block -1.
  // The reference max of every head is fixed by the first block holding a valid key (a
  // wave-uniform event: validity is per key, shared by all heads); row sums and the overshoot
  // maxima stay per lane (one half of a head's keys) until the end of the pass.
  bool m_set = false;
  for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
    for (int m = 0; m < kDv / 32; ++m) o[m] = f32x16{};
    mfma_acc_drain();
    l_run = 0.f;
    if (nblk > 0) gather_tile<NW, ROPE>(tile0, p.kv, sm.idx, wave, lane);
    // block -1's P^T slot holds zeros (iteration 0 multiplies tile 0 by it)
    lds_store16(pf_addr(1, wave, 0), u32x4{0, 0, 0, 0});
    lds_store16(pf_addr(1, wave, 1), u32x4{0, 0, 0, 0});
    uint32_t st_cur = 0, st_prev = 0;   // ring byte offsets of blocks blk and blk-1
    for (int blk = 0; blk < nblk; ++blk) {
      wait_vmcnt<0>();
      __syncthreads();
      const uint32_t st_next = st_cur == 2 * kTileBytes ? 0 : st_cur + kTileBytes;
      // block blk+1's gather is issued one copy per kCopyEvery QK MFMAs below
      const bool gather_next = blk + 1 < nblk;
      TileSrc<NW> next_src;
      if (gather_next) next_src = tile_sources<NW, ROPE>(p.kv, sm.idx + (blk + 1) * kBK, wave, lane);
      // source rows of the next two copies, each read two copy slots ahead of its issue (with one
      // wave the copies are one MFMA apart)
      const char* next_row[2] = {gather_next ? gather_row<NW>(next_src, 0) : nullptr,
                                 gather_next ? gather_row<NW>(next_src, 1) : nullptr};
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t next_tile = tile0 + st_next;
      // per-block absolute operand addresses (tiles are 128-byte aligned: the rope XOR below
      // only touches bits 4..6); opaque so they are not hoisted into loop-invariant VGPRs
      const uint32_t tb = tile0 + st_cur, tp = tile0 + st_prev;
      st_prev = st_cur;
      st_cur = st_next;
      uint32_t qv = tb + qk_v, qr = tb + qk_r;
      asm volatile("" : "+v"(qv), "+v"(qr));
      const uint32_t vmask = (uint32_t)__ballot(sm.idx[blk * kBK + (lane & 31)] >= 0);

      // ---- S^T[32 keys x 32 heads] = K . Q^T  (A operands prefetched).  Two instances of the
      // MFMA sequence, with and without block blk+1's gather (the last block has none), so no
      // copy sits behind a branch; each copy sets M0 with one s_add of a compile-time offset.
      f32x16 s;
      {
        auto qk_addr = [&](int ks) { return lds_ptr(ks < 32 ? (qv + 32u * ks) : (qr ^ (32u * (ks - 32)))); };
        u32x4 a[kPre];
#pragma unroll
        for (int i = 0; i < kPre; ++i) a[i] = lds_load16(qk_addr(i));
        f32x16 sa;
        const TileDst nd = tile_dst<NW>(next_tile, wsg);
        auto qk = [&](auto gather) {
          static_for<0, QKS>([&](auto ksc) {
            constexpr int ks = decltype(ksc)::value;
            const u32x4 cur = a[ks % kPre];
            if constexpr (ks + kPre < QKS) a[ks % kPre] = lds_load16(qk_addr(ks + kPre));
            if constexpr (ks == 0) mfma32x32x16_cV_first(sa, cur, qf[0]);
            else mfma32x32x16_cV(sa, cur, qf[ks]);
            if constexpr (decltype(gather)::value && ks % kCopyEvery == 0) {
              constexpr int k = ks / kCopyEvery;
              gather_issue_at<NW, k>(nd, next_src, next_row[k & 1], lane);
              next_row[k & 1] = gather_row<NW>(next_src, k + 2);
            }
            __builtin_amdgcn_sched_barrier(0);
          });
        };
        if (gather_next) qk(std::true_type{});
        else qk(std::false_type{});
        s = sa;
      }
      mfma_acc_drain();

      // ---- softmax numerator in the exp2 domain, p = 2^(scale_log2 * s - m) (scale > 0);
      // key of s[i] = (i/4)*8 + 4*hb + i%4
      if (vmask != 0xffffffffu) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = (i >> 2) * 8 + hb * 4 + (i & 3);
          if (!((vmask >> key) & 1u)) s[i] = -INFINITY;
        }
      }
      if (!m_set && vmask != 0u) {   // both row halves of a head take the same reference
        float bm = s[0];
#pragma unroll
        for (int i = 1; i < 16; ++i) bm = fmaxf(bm, s[i]);
        m_ref = xor32_max(bm) * p.scale_log2;
        m_set = true;
      }
      const float m_use = m_set ? m_ref : 0.f;
      float bm0 = 0.f, bm1 = 0.f, rs = 0.f, p_even = 0.f;
      u32x4 pb_new[2];
      // no clamp: an exponent above kHeadroom means m_seen > m_ref + kHeadroom, and the whole
      // row is then recomputed against its true maximum (inf/NaN here is discarded)
      auto softmax_step = [&](int i) {
        if (i == 0)
          bm0 = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
        if (i == 1)
          bm1 = fmaxf(fmaxf(fmaxf(s[8], s[9]), fmaxf(s[10], s[11])), fmaxf(fmaxf(s[12], s[13]), fmaxf(s[14], s[15])));
        if (i == 2) m_seen = fmaxf(m_seen, fmaxf(bm0, bm1) * p.scale_log2);
        if (i >= 4 && i < 20) {   // one exp per PV MFMA
          const int e = i - 4;
          const float pe = fast_exp2(__builtin_fmaf(s[e], p.scale_log2, -m_use));
          rs += pe;
          if (e & 1) pb_new[e >> 3][(e & 7) >> 1] = pack_bf16x2(p_even, pe);
          else p_even = pe;
        }
        if (i == 21) {   // publish block blk's P^T fragments (read after the next barrier)
          lds_store16(pf_addr(blk & 1, wave, 0), pb_new[0]);
          lds_store16(pf_addr(blk & 1, wave, 1), pb_new[1]);
        }
      };
      pv_block(tp, (blk + 1) & 1, softmax_step);   // block blk-1's P^T slot
      l_run += rs;
    }
    if (nblk > 0) {
      __syncthreads();   // the last block's P^T fragments of every wave
      pv_block(tile0 + st_prev, (nblk - 1) & 1, [](int) {});
    }
    // ---- did any head overshoot its reference?  (workgroup-uniform decision)
    const bool over = m_seen > m_ref + kHeadroom;
    if (threadIdx.x == 0) sm.redo_flag = 0;
    __syncthreads();
    if (__any(over) && lane == 0) sm.redo_flag = 1;
    __syncthreads();
    if (!sm.redo_flag) break;
    m_ref = xor32_max(m_seen);
  }
  l_run = xor32_sum(l_run);
  // ---- per-head attention sink (a logit with no value): the row's normaliser gains
  // exp(sink), O is scaled by 1 / (keys' sum + sink term), the LSE includes it.  Everything is
  // taken relative to mf = max(key reference, sink) so neither term overflows.
  float o_scale = l_run > 0.f ? 1.f / l_run : 0.f;
  float lse_out = -INFINITY;
  {
    const float ms = m_set ? m_ref : -INFINITY;
    if (p.sinks != nullptr) {
      const float s2 = head_ok ? p.sinks[head] * kLog2e : -INFINITY;
      const float mf = fmaxf(ms, s2);
      if (mf != -INFINITY) {
        const float rel = ms == -INFINITY ? 0.f : fast_exp2(ms - mf);   // keys' sum rescaled to mf
        const float l_tot = l_run * rel + fast_exp2(s2 - mf);
        o_scale = rel / l_tot;
        lse_out = (mf + __log2f(l_tot)) * kLn2;
      }
    } else if (l_run > 0.f) {
      lse_out = ((ms == -INFINITY ? 0.f : ms) + __log2f(l_run)) * kLn2;
    }
  }

  // ---- epilogue: normalise, store O (bf16) and LSE (natural log).  The output rows go
  // through LDS (the tile ring, P^T slots and index row are dead: every wave passed the
  // barriers above): wave w writes its dims of every head row, chunk c of row r at c ^ (r & 7),
  // then stores its own 32 rows, one whole 1 KB row (16 B per lane) per store instruction.
  // Stored straight from the accumulator layout, each store would write 32 rows 16 bytes
  // apart: 8x the L2 requests.
  mfma_acc_drain();
  if (hb == 0) sm.inv_l[wave * 32 + hl] = o_scale;
  __syncthreads();
  {
#pragma unroll
    for (int n = 0; n < NH; ++n) {
      const float inv_l = sm.inv_l[32 * n + hl];
      char* mine = sm.ostage[32 * n + hl];
#pragma unroll
      for (int mm = 0; mm < DT; ++mm) {
        const f32x16& acc = o[mm * NH + n];
        const int m = DT * wave + mm;   // dim tile: dims 32m .. 32m+31
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          u32x2 v;
          v[0] = pack_bf16x2(acc[4 * q4 + 0] * inv_l, acc[4 * q4 + 1] * inv_l);
          v[1] = pack_bf16x2(acc[4 * q4 + 2] * inv_l, acc[4 * q4 + 3] * inv_l);
          *reinterpret_cast<u32x2*>(mine + 16 * ((4 * m + q4) ^ (hl & 7)) + 8 * hb) = v;
        }
      }
    }
    __syncthreads();
    const char* slab = sm.ostage[wave * 32];
    const int h0w = blockIdx.y * 128 + wave * 32;
    const int rows = min(32, p.n_heads - h0w);
    bf16_t* obase = p.out + orow * p.out_stride_t + (int64_t)h0w * kDv;
    for (int r = 0; r < rows; ++r)
      *reinterpret_cast<u32x4*>(obase + (int64_t)r * kDv + 8 * lane) =
          lds_load16(slab + r * (kDv * 2) + 16 * (lane ^ (r & 7)));
  }
  if (head_ok && hb == 0) p.lse[orow * p.lse_stride_t + head] = lse_out;
}

// Decode split merge: out[b,h] = sum_s e^{lse_s} O_s / sum_s e^{lse_s} over the n_split
// normalised partials of (b, h); lse[b,h] = ln sum_s e^{lse_s}.  One wave per (b, h), 8 dv per lane.
__global__ __launch_bounds__(256) void decode_combine_kernel(const bf16_t* part_o, const float* part_lse,
                                                             int batch, int n_heads, int n_split,
                                                             bf16_t* out, float* lse) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= batch * n_heads) return;
  const int lane = threadIdx.x & 63;
  const int b = r / n_heads, h = r - b * n_heads;
  const int64_t prow0 = (int64_t)b * n_split * n_heads + h;   // partial row of split 0
  float m = -INFINITY;
  for (int s = 0; s < n_split; ++s) m = fmaxf(m, part_lse[prow0 + (int64_t)s * n_heads]);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float den = 0.f;
  if (m != -INFINITY) {
    for (int s = 0; s < n_split; ++s) {
      const int64_t prow = prow0 + (int64_t)s * n_heads;
      const float wgt = fast_exp2((part_lse[prow] - m) * kLog2e);
      den += wgt;
      const u32x4 v = gload16(part_o + prow * kDv + 8 * lane);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[2 * e] += wgt * bf16_lo(v[e]);
        acc[2 * e + 1] += wgt * bf16_hi(v[e]);
      }
    }
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(acc[2 * e] * inv, acc[2 * e + 1] * inv);
  *reinterpret_cast<u32x4*>(out + (int64_t)r * kDv + 8 * lane) = o;
  if (lane == 0) lse[r] = den > 0.f ? m + __log2f(den) * kLn2 : -INFINITY;
}

int launch_sparse_mla_fwd(const SparseFwdParams& p, hipStream_t stream) {
  if (p.n_xcd < 1) return -1;
  if (p.split_keys > kMaxTopk || p.n_split < 1 || (p.n_split > 1 && p.split_keys % kBK != 0)) return -2;
  if ((int64_t)(p.n_split - 1) * p.split_keys >= p.topk) return -1;   // every split owns >= 1 slot
  if (p.sinks != nullptr && p.n_split != 1) return -2;                  // a sink joins each row once
  const dim3 grid(xcd_grid(p.total_q * p.n_split, p.n_xcd), (p.n_heads + 127) / 128);
  const int nw = p.n_heads > 64 ? 4 : (p.n_heads > 32 ? 2 : 1);
  if (p.q_dim == kDv) {   // 512-wide q: the rope-free instantiation
    if (nw == 4)
      hipLaunchKernelGGL((sparse_mla_fwd_kernel<4, false>), grid, dim3(256), 0, stream, p);
    else if (nw == 2)
      hipLaunchKernelGGL((sparse_mla_fwd_kernel<2, false>), grid, dim3(128), 0, stream, p);
    else
      hipLaunchKernelGGL((sparse_mla_fwd_kernel<1, false>), grid, dim3(64), 0, stream, p);
  } else if (nw == 4) {
    hipLaunchKernelGGL((sparse_mla_fwd_kernel<4, true>), grid, dim3(256), 0, stream, p);
  } else if (nw == 2) {
    hipLaunchKernelGGL((sparse_mla_fwd_kernel<2, true>), grid, dim3(128), 0, stream, p);
  } else {
    hipLaunchKernelGGL((sparse_mla_fwd_kernel<1, true>), grid, dim3(64), 0, stream, p);
  }
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

// Static device scratch of the allocation-free decode entry point: the split partials live here
// instead of in a caller workspace.  Every GPU the library runs on holds its own copy until the
// process ends; in host code `decode_scratch` names a host-side stand-in, so kernels get the
// device address that hipGetSymbolAddress returns, looked up once per device.
namespace {
__device__ __align__(256) char decode_scratch[kDecodeScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

int decode_scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -5;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(decode_scratch)) != hipSuccess || !ptr) return -4;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

int launch_decode_combine(const bf16_t* part_o, const float* part_lse, int batch, int n_heads, int n_split,
                          bf16_t* out, float* lse, hipStream_t stream) {
  const int rows = batch * n_heads;
  if (rows == 0) return 0;
  hipLaunchKernelGGL(decode_combine_kernel, dim3((rows + 3) / 4), dim3(256), 0, stream, part_o, part_lse, batch,
                     n_heads, n_split, out, lse);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace dsa
