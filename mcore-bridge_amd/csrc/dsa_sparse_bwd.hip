// K4: sparse MLA attention backward (gfx950), deterministic, no floating-point atomics.
//
// Reference: torch autograd through Megatron's un-fused sparse attention (DSAttention, called
// from src/mcore_bridge/model/modules/multi_latent_attention.py:262-270); the reference defines no
// custom backward.  Closed form (P = exp(scale*S - lse), Delta = rowsum(dO * O)):
//   dS = P * (dO . V^T - Delta),   dQ = scale * dS . K,
//   dKV[s] = sum_{(t,h) selecting s} scale * dS[t,h,s] * q[t,h,:576] + P[t,h,s] * dO[t,h,:512].
//
// Why five stages.  One query carries 128 heads x (576 + 512) bf16 of Q/dO (278 KB).  The
// products that recompute S and dP contract over d (Q/dO must be d-contiguous per lane), the dKV
// product contracts over heads (Q/dO head-contiguous per lane), and dQ needs a 128 x 576 fp32
// accumulator (295 KB): together far beyond one CU's 512 KB of registers + 160 KB of LDS.  The
// dKV reduction over queries is a scatter of 576 floats per selected pair; MI355X executes fp32
// atomics at ~0.33 T/s device-wide (one per L2 channel per clock, measured), which would cost
// ~50 ms at S = 16k, so the scatter is done as bf16 partial rows grouped by key and reduced in a
// streaming pass instead.
//   B1 bwd_sp_kernel   per query: recompute S, P, dP (shared K/V operand reads), Delta fused;
//                      stage P and scale*dS (bf16, [t][h][j]).
//   B2 bwd_dq_kernel   per query: dQ^T += K^T . dS^T over the gathered rows (K^T via transposing
//                      LDS reads, dS^T tile copied into LDS next to the KV tile).
//   B3 bwd_g_kernel    per query: G^T[576 x keys] = Q^T . dS + dO^T . P contracted over all
//                      heads (Q^T / dO^T held in registers), written as bf16 rows at the pair's
//                      key-major position.
//   B4 csr_*           key-major order of the selected pairs: count, scan, position.
//   B5 bwd_dkv_reduce  per key: fp32 sum of its contiguous G rows -> dKV.
// The G rows (1152 B per selected pair, far more than the caches hold) are written and read with
// non-temporal stores and loads, so they stream through L2 without displacing the operands B3
// and B5 re-read; B2 and B3 read the staged P / dS tiles (read once each) with non-temporal
// LDS-direct copies.  B1 writes those tiles with ordinary 16-byte stores: non-temporal stores
// that cover a fraction of a cache line each ran B1 ~3x slower.
// B1-B3 stream their per-block operands into LDS through 3-stage rings of asynchronous
// global_load_lds copies (see dsa_kvtile.h) completed by explicit s_waitcnt vmcnt + barrier.
// vmcnt counts every vector-memory instruction of the wave in issue order, so each wave issues
// a fixed number of copies and stores per block and the waits count them exactly.
// B1, B2 and B3 have instantiations without the rope part (ROPE = false) for 512-wide q rows
// (the DeepSeek-V4 sink attention): S contracts over the 512 latent dims only, dQ has 512
// columns, the KV tiles' rope region is neither gathered nor read, and the bf16 G rows carry the
// 512 latent dims only (1024 bytes; B5 writes dKV's rope columns as zeros).
#include <algorithm>
#include <type_traits>

#include "dsa_common.h"
#include "dsa_kernels.h"
#include "dsa_bwd_g.h"
#include "dsa_kvtile.h"

namespace dsa {

namespace {

// lo = keys k .. k+3 and hi = keys k+8 .. k+11 in the lower half-wave (lane l < 32), keys
// k+4 .. k+7 and k+12 .. k+15 in the upper half (lane l + 32, same head).  One
// v_permlane32_swap per dword trades the lower half's hi for the upper half's lo, after which
// the lower lane holds keys k .. k+7 and the upper lane k+8 .. k+15: one 16-byte store each.
DSA_DEV u32x4 swap_key_halves(u32x2 lo, u32x2 hi) {
  u32x4 r;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const auto sw = __builtin_amdgcn_permlane32_swap(lo[c], hi[c], false, false);
    // sw[0] = lo with lanes 32..63 taken from hi's lanes 0..31; sw[1] = hi with lanes 0..31
    // taken from lo's lanes 32..63
    r[c] = sw[0];
    r[2 + c] = sw[1];
  }
  return r;
}

}  // namespace

// ------------------------------------------------------------------------------------------
// B1: recompute P and dS; stage them.  One workgroup per query, wave = 32 heads.
// ------------------------------------------------------------------------------------------
struct SpSmem {
  union {
    char tile[kStages][kTileBytes];
    char ostage[4][32][kDv * 2];   // setup: O rows of each wave's 32 heads (for Delta)
  };
  int32_t idx[kMaxTopkBwd];
  float lse[4][64];                // setup: LSE of each lane's head
  int red[4];
};

template <int NW, bool ROPE>
__global__ __launch_bounds__(NW * 64, 1) void bwd_sp_kernel(SparseBwdParams p) {
  constexpr int QKS = (ROPE ? kDqk : kDv) / 16;   // S k-steps per block (no rope part: 32)
  constexpr int G = tile_copies_per_wave<NW, ROPE>();
  constexpr int S = 4;  // staging stores per wave per block (2 x P, 2 x dS)
  constexpr int kCopyEvery = QKS / G;   // S/dP steps per gather copy
  static_assert(kCopyEvery * G == QKS, "copies spread evenly over the k-steps");
  __shared__ __attribute__((aligned(128))) SpSmem sm;
  const int t = xcd_remap(blockIdx.x, p.n_xcd);
  if (t >= p.total_q) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hb = lane >> 5, hl = lane & 31;
  const int head = blockIdx.y * 128 + wave * 32 + hl;
  const bool head_ok = head < p.n_heads;
  const bool wave_stores = blockIdx.y * 128 + wave * 32 < p.n_heads;  // wave-uniform
  const int hsafe = head_ok ? head : 0;

  static_assert(NW <= 4, "O staging holds 4 waves");
  // Setup, one memory round trip: the O rows of this wave's 32 heads stream into LDS
  // (asynchronous, no registers; row i = head 32w + i, 16-byte chunk c at c ^ (i & 7)) while
  // Q and dO load into their fragments and the index row into LDS.
  {
    const uint32_t ob = __builtin_amdgcn_readfirstlane(lds_addr(sm.ostage[wave]));
    const char* o_t = reinterpret_cast<const char*>(p.out + (int64_t)t * p.out_stride_t);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int h = blockIdx.y * 128 + wave * 32 + i;
      const int hs = h < p.n_heads ? h : 0;   // rows past n_heads re-read head 0 (unused)
      async_copy16_unordered(o_t + (int64_t)hs * (kDv * 2) + 16 * (lane ^ (i & 7)), ob + 1024u * i);
    }
  }
  // Q (576, or 512 without ROPE) and dO (512) fragments, d-contiguous: lane holds [16*ks + 8*hb, +8).
  u32x4 qf[QKS], df[kDv / 16];
  // (q rows of 512 under ROPE: no rope part, its fragments zero)
  const bool q_rope = p.q_dim != kDv;
  const bf16_t* qrow = p.q + (int64_t)t * p.q_stride_t + (int64_t)hsafe * (q_rope ? kDqk : kDv) + hb * 8;
  const bf16_t* drow = p.dout + (int64_t)t * p.dout_stride_t + (int64_t)hsafe * kDv + hb * 8;
#pragma unroll
  for (int ks = 0; ks < QKS; ++ks) {
    u32x4 v = u32x4{0, 0, 0, 0};
    if (ks < kDv / 16 || q_rope) v = gload16(qrow + ks * 16);
    qf[ks] = head_ok ? v : u32x4{0, 0, 0, 0};
  }
#pragma unroll
  for (int ks = 0; ks < kDv / 16; ++ks) {
    const u32x4 v = gload16(drow + ks * 16);
    df[ks] = head_ok ? v : u32x4{0, 0, 0, 0};
  }
  // LSE of this lane's head, also through LDS (a register load would be waited for at once)
  async_copy4_unordered(p.lse + (int64_t)t * p.lse_stride_t + hsafe,
                        __builtin_amdgcn_readfirstlane(lds_addr(sm.lse[wave])));
  // (waits for every load above, the O copies included, then a barrier)
  const int nblk = stage_index_row<NW>(sm.idx, sm.red, p.idx + (int64_t)t * p.idx_stride, p.topk, p.n_kv,
                                       p.causal, t + p.q_offset);
  // Delta = rowsum(dO * O) of this lane's head: chunks 2*ks + hb of O row hl from LDS
  float delta = 0.f;
  {
    const char* orow_s = sm.ostage[wave][hl];
#pragma unroll
    for (int ks = 0; ks < kDv / 16; ++ks) {
      const u32x4 o = lds_load16(orow_s + 16 * ((2 * ks + hb) ^ (hl & 7)));
      const u32x4 v = df[ks];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        delta += bf16_lo(v[e]) * bf16_lo(o[e]) + bf16_hi(v[e]) * bf16_hi(o[e]);
    }
  }
  delta = xor32_sum(delta);
  if (p.delta_out != nullptr && head_ok && hb == 0) p.delta_out[(int64_t)t * p.n_heads + head] = delta;
  const float delta_s = delta * p.scale;
  const float lse = head_ok ? sm.lse[wave][lane] : -INFINITY;
  const float lse2 = lse * kLog2e;
  const bool row_live = lse != -INFINITY;
  __syncthreads();   // O staging dead: the union now holds the KV tile ring

  // staged tiles: element (t, head, slot 32*b + k) at ((t * NB + b) * H + head) * 32 + k
  // (NB = topk_pad / 32): each block's [H heads x 32 keys] tile is contiguous; after the half
  // swap (swap_key_halves) lane writes keys 16*pr + 8*hb .. +7 of each block, pr = 0, 1
  const int64_t stage_off = ((int64_t)t * (p.topk_pad / kBK) * p.n_heads + hsafe) * kBK + hb * 8;
  const int64_t stage_blk = (int64_t)p.n_heads * kBK;   // elements per staged block tile
  bf16_t* ps_row = p.p_stage + stage_off;
  bf16_t* ds_row = p.ds_stage + stage_off;
  const uint32_t qk_v = key_row(hl) * kTileVPitch + 16u * hb;
  const uint32_t qk_r = kTileVBytes + hl * 128u + 16u * (hb ^ ((hl >> 1) & 7u));
  const uint32_t tile0 = lds_addr(sm.tile[0]);
  const uint32_t wsg = __builtin_amdgcn_readfirstlane(wave);

  if (nblk > 0) gather_tile<NW, ROPE>(tile0, p.kv, sm.idx, wave, lane);
  if (nblk > 1) gather_tile<NW, ROPE>(tile0 + kTileBytes, p.kv, sm.idx + kBK, wave, lane);
  uint32_t st_cur = 0, st_next = 2 * kTileBytes;   // ring byte offsets of blocks blk, blk+2
  u32x4 pw[2], dw[2];   // previous block's values, stored right after the next block's barrier
  for (int blk = 0; blk < nblk; ++blk) {
    // issue order per block: [wait][barrier], then between the S/dP MFMAs the copies of block
    // blk+2 (k-steps 0, 4, .., 32) and the P/dS stores of block blk-1 (k-steps 1, 9, 17, 25,
    // all before the last copy).  Block blk needs copies(blk) done; issued after them are
    // block blk-1's copies(blk+1) and, from blk = 2 on (block 0 stores nothing), its stores of
    // block blk-2.
    if (blk == 0) {
      if (nblk > 1) wait_vmcnt<G>(); else wait_vmcnt<0>();
    } else if (blk == 1 || !wave_stores) {
      wait_vmcnt<G>();
    } else {
      wait_vmcnt<G + S>();
    }
    __syncthreads();
    const bool store_prev = blk > 0 && head_ok;   // wave_stores => the wave issues all S stores
    const int64_t store_j = (blk - 1) * stage_blk;
    // block blk+2's gather, one copy per kCopyEvery S/dP steps below.  Issued every iteration:
    // the last two re-gather block nblk-1 into the ring slot no block reads any more (so no copy
    // sits behind a branch); they are retired before the kernel ends.
    const TileSrc<NW> next_src = tile_sources<NW, ROPE>(p.kv, sm.idx + min(blk + 2, nblk - 1) * kBK, wave, lane);
    // source row of the next copy, read one copy slot ahead of its issue
    const char* next_row = gather_row<NW>(next_src, 0);
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t next_tile = tile0 + st_next;
    const TileDst nd = tile_dst<NW>(next_tile, wsg);
    const uint32_t tb = tile0 + st_cur;   // 128-byte aligned: the rope XOR stays in its row
    st_cur = st_cur == 2 * kTileBytes ? 0 : st_cur + kTileBytes;
    st_next = st_next == 2 * kTileBytes ? 0 : st_next + kTileBytes;
    uint32_t qv = tb + qk_v, qr = tb + qk_r;
    asm volatile("" : "+v"(qv), "+v"(qr));
    const uint32_t vmask = (uint32_t)__ballot(sm.idx[blk * kBK + (lane & 31)] >= 0);

    // S^T = K . Q^T and dP^T = V . dO^T share the A operand (V = K[:, :512]); the dO^T
    // fragments and the dP accumulator stay in AccVGPRs (Q + dO = 272 registers per lane).
    f32x16 s = f32x16{}, dp;
    {
      auto addr = [&](int ks) { return lds_ptr(ks < 32 ? (qv + 32u * ks) : (qr ^ (32u * (ks - 32)))); };
      u32x4 a[kPre];
#pragma unroll
      for (int i = 0; i < kPre; ++i) a[i] = lds_load16(addr(i));
#pragma unroll
      for (int ks = 0; ks < QKS; ++ks) {
        const u32x4 cur = a[ks % kPre];
        if (ks + kPre < QKS) a[ks % kPre] = lds_load16(addr(ks + kPre));
        s = mfma32x32x16(as_bf16x8(cur), as_bf16x8(qf[ks]), s);
        if (ks == 0) mfma32x32x16_acc_first(dp, cur, df[0]);
        else if (ks < kDv / 16) mfma32x32x16_acc(dp, cur, df[ks]);
        if (ks % kCopyEvery == 0) {
          gather_issue_dst<NW>(nd, next_src, next_row, lane, ks / kCopyEvery);
          next_row = gather_row<NW>(next_src, ks / kCopyEvery + 1);
        }
        if (ks % 8 == 1 && ks < 32 && store_prev) {
          const int q = ks / 8;   // 0..3: P then dS of key half pr = q / 2
          if (q & 1) *reinterpret_cast<u32x4*>(ds_row + store_j + 16 * (q >> 1)) = dw[q >> 1];
          else *reinterpret_cast<u32x4*>(ps_row + store_j + 16 * (q >> 1)) = pw[q >> 1];
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    mfma_acc_drain();
    // P = 2^(scale_log2 * s - lse2) and scale * dS = P * (scale * dP - scale * Delta); key of
    // element i = (i/4)*8 + 4*hb + i%4.  Partial blocks / dead heads take the masked path.
    float pv[16];
    if (vmask == 0xffffffffu && __all(row_live)) {
#pragma unroll
      for (int i = 0; i < 16; ++i) pv[i] = fast_exp2(__builtin_fmaf(s[i], p.scale_log2, -lse2));
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = (i >> 2) * 8 + hb * 4 + (i & 3);
        const bool ok = row_live && ((vmask >> key) & 1u);
        pv[i] = ok ? fast_exp2(__builtin_fmaf(s[i], p.scale_log2, -lse2)) : 0.f;
      }
    }
    u32x2 pk[4], dk[4];   // keys 8*q4 + 4*hb .. +3
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      float dv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) dv[e] = pv[4 * q4 + e] * __builtin_fmaf(dp[4 * q4 + e], p.scale, -delta_s);
      pk[q4] = u32x2{pack_bf16x2(pv[4 * q4], pv[4 * q4 + 1]), pack_bf16x2(pv[4 * q4 + 2], pv[4 * q4 + 3])};
      dk[q4] = u32x2{pack_bf16x2(dv[0], dv[1]), pack_bf16x2(dv[2], dv[3])};
    }
#pragma unroll
    for (int pr = 0; pr < 2; ++pr) {
      pw[pr] = swap_key_halves(pk[2 * pr], pk[2 * pr + 1]);
      dw[pr] = swap_key_halves(dk[2 * pr], dk[2 * pr + 1]);
    }
  }
  if (nblk > 0 && head_ok) {
    const int64_t j = (nblk - 1) * stage_blk;
#pragma unroll
    for (int pr = 0; pr < 2; ++pr) {
      *reinterpret_cast<u32x4*>(ps_row + j + 16 * pr) = pw[pr];
      *reinterpret_cast<u32x4*>(ds_row + j + 16 * pr) = dw[pr];
    }
  }
  wait_vmcnt0();   // the last re-gathers have landed in LDS before the workgroup ends
}

// ------------------------------------------------------------------------------------------
// B2: dQ^T[576 x 32*NW heads] = K^T . (scale*dS)^T over the query's gathered rows, with
// 16x16x32 MFMAs.  Wave w owns 576/NW latent dims (DT tiles of 16) for every head of the
// workgroup (HT tiles of 16): per 32-key block it reads DT K^T fragments (transposing reads of
// the KV tile) and HT dS^T fragments, each K^T fragment feeding HT MFMAs and each dS^T fragment
// DT.  (Split by heads instead, every wave would read the whole K^T tile for 36 MFMAs: four
// times the LDS reads.)
// ------------------------------------------------------------------------------------------
constexpr int kDsTileBytes = 128 * 64;  // [128 heads][32 keys] bf16
constexpr int kDqPitch = kDqk * 2 + 16;  // LDS pitch of a staged bf16 dQ row

struct DqSmem {
  union {
    struct {
      char tile[kStages][kTileBytes];
      char ds[kStages][kDsTileBytes];   // 16-byte chunk q of head row h at q ^ ((h >> 1) & 3)
    } ring;
    char out[64][kDqPitch];             // epilogue: bf16 dQ rows of 64 heads
  };
  int32_t idx[kMaxTopkBwd];
  int red[8];
};

template <int NW, bool ROPE>
__global__ __launch_bounds__(NW * 64, 1) void bwd_dq_kernel(SparseBwdParams p) {
  constexpr int DQ = ROPE ? kDqk : kDv;                        // dq row width
  constexpr int HR = 32 * NW;                                  // head rows of the workgroup
  constexpr int HT = HR / 16;                                  // head tiles
  constexpr int DT = DQ / 16 / NW;                             // dim tiles per wave
  constexpr int TC = tile_copies_per_wave<NW, ROPE>();
  constexpr int G = TC + HR / 16 / NW;
  static_assert(HR / 16 / NW == 2, "two dS copies per wave per block");
  static_assert(DT * NW * 16 == DQ && DT >= TC, "dims split evenly; one tile copy per dim step");
  __shared__ __attribute__((aligned(128))) DqSmem sm;
  const int t = xcd_remap(blockIdx.x, p.n_xcd);
  if (t >= p.total_q) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, gi = lane & 15;
  const int h0 = blockIdx.y * 128;
  const int nblk = stage_index_row<NW>(sm.idx, sm.red, p.idx + (int64_t)t * p.idx_stride, p.topk, p.n_kv,
                                       p.causal, t + p.q_offset);
  // dS rows of this workgroup's heads; rows past n_heads re-read row 0 (never stored).
  const int hrows = min(HR, p.n_heads - h0);
  // staged dS tile of block b: [H heads][32 keys] contiguous at ((t * NB + b) * H) * 32
  const char* ds_base = reinterpret_cast<const char*>(p.ds_stage + ((int64_t)t * (p.topk_pad / kBK) * p.n_heads + h0) * kBK);
  const int64_t ds_blk = (int64_t)p.n_heads * kBK * 2;   // bytes per staged block tile
  // copy k (0 <= k < 2) of this wave's share of block blk's dS rows
  auto copy_ds_part = [&](char* dst, int blk, int k) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(dst));
    const int w = __builtin_amdgcn_readfirstlane(wave);
    const int i = w + k * NW;
    const int h = 16 * i + (lane >> 2);
    const int q = (lane & 3) ^ ((h >> 1) & 3);
    const int hs = h < hrows ? h : 0;
    async_copy16_nt(ds_base + blk * ds_blk + hs * (kBK * 2) + q * 16, base + i * 1024u);
  };
  auto copy_ds = [&](char* dst, int blk) {
#pragma unroll
    for (int k = 0; k < HR / 16 / NW; ++k) copy_ds_part(dst, blk, k);
  };

  // A operand (K^T, dims x keys) of dim tile D: lane (g, gi) gets dim 16D + gi, keys 8g .. 8g+7
  // as two transposing reads of 4 keys (rows 8g + gi/4 and 8g + 4 + gi/4, 4 dims from
  // 16D + 4(gi%4)).  V dims (D < 32): tile row key_row(key) (keys 8g + j sit 2 rows apart:
  // conflict-free), byte kv[h] + 32D; rope dims: kr[h] ^ (32(D - 32)).
  uint32_t kv[2], kr[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t key = 8 * g + 4 * h + (gi >> 2);
    kv[h] = key_row(key) * kTileVPitch + 8u * (gi & 3);
    kr[h] = kTileVBytes + key * 128u + 8u * (gi & 1) + 16u * (((gi & 3) >> 1) ^ ((key >> 1) & 7u));
  }
  // B operand (dS^T, keys x heads) of head tile j: head row 16j + gi, keys 8g .. 8g+7
  const uint32_t ds_lane = gi * 64u + 16u * (g ^ ((gi >> 1) & 3));
  const int d0 = __builtin_amdgcn_readfirstlane(wave) * DT;   // first dim tile of this wave
  const uint32_t tile0 = lds_addr(sm.ring.tile[0]);

  // dQ^T accumulators: DT x HT tiles of 16 x 16, 288 registers per lane -- more than either
  // register file: tiles 0..63 (row-major) are pinned in AccVGPRs, the rest in VGPRs
  // (AGPR/VGPR-constrained MFMAs; left to itself the compiler moves tiles between the files
  // around the MFMAs).
  constexpr int kTilesA = 64;
  f32x4 acc[DT][HT];
#pragma unroll
  for (int i = 0; i < DT; ++i)
#pragma unroll
    for (int j = 0; j < HT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  mfma_acc_drain();   // zero writes of the accumulators before their first MFMA read

  if (nblk > 0) {
    gather_tile<NW, ROPE>(tile0, p.kv, sm.idx, wave, lane);
    copy_ds(sm.ring.ds[0], 0);
  }
  if (nblk > 1) {
    gather_tile<NW, ROPE>(tile0 + kTileBytes, p.kv, sm.idx + kBK, wave, lane);
    copy_ds(sm.ring.ds[1], 1);
  }
  int st = 0;   // ring stage of block blk
  for (int blk = 0; blk < nblk; ++blk) {
    if (blk + 1 < nblk) wait_vmcnt<G>(); else wait_vmcnt<0>();
    __syncthreads();
    // block blk+2's copies, one tile copy per dim step below, the dS copies at steps 1 and 3
    const bool copy_next = blk + 2 < nblk;
    const int st_next = st == 0 ? 2 : st - 1;   // (blk + 2) % 3
    TileSrc<NW> next_src;
    if (copy_next) next_src = tile_sources<NW, ROPE>(p.kv, sm.idx + (blk + 2) * kBK, wave, lane);
    // source row of the next tile copy, read one copy slot ahead of its issue
    const char* next_row = copy_next ? gather_row<NW>(next_src, 0) : nullptr;
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t next_tile = tile0 + st_next * kTileBytes;
    char* const next_ds = sm.ring.ds[st_next];
    const uint32_t tb = tile0 + st * kTileBytes;   // 128-byte aligned: the rope XOR stays in its row
    const char* dsl = sm.ring.ds[st] + ds_lane;
    st = st == 2 ? 0 : st + 1;
    uint32_t v0 = tb + kv[0], v1 = tb + kv[1], r0 = tb + kr[0], r1 = tb + kr[1];
    asm volatile("" : "+v"(v0), "+v"(v1), "+v"(r0), "+v"(r1));
    u32x4 b[HT];
#pragma unroll
    for (int j = 0; j < HT; ++j) b[j] = lds_load16(dsl + 1024 * j);
    auto ld = [&](int i) {
      const int D = d0 + i;   // wave-uniform
      const uint32_t x0 = D < 32 ? v0 + 32u * D : r0 ^ (32u * (D - 32));
      const uint32_t x1 = D < 32 ? v1 + 32u * D : r1 ^ (32u * (D - 32));
      const u32x2 lo = lds_read_tr16(lds_ptr(x0)), hi = lds_read_tr16(lds_ptr(x1));
      return u32x4{lo[0], lo[1], hi[0], hi[1]};
    };
    u32x4 a[kPre];
#pragma unroll
    for (int i = 0; i < kPre; ++i) a[i] = ld(i);
#pragma unroll
    for (int i = 0; i < DT; ++i) {
      const u32x4 cur = a[i % kPre];
      if (i + kPre < DT) a[i % kPre] = ld(i + kPre);
#pragma unroll
      for (int j = 0; j < HT; ++j) {
        if (i * HT + j < kTilesA) mfma16x16x32_cA(acc[i][j], cur, b[j]);
        else mfma16x16x32_cV(acc[i][j], cur, b[j]);
      }
      if (copy_next) {
        if (i < TC) {
          gather_issue<NW>(next_tile, next_src, next_row, wave, lane, i);
          next_row = gather_row<NW>(next_src, i + 1);
        }
        if (i == 1 || i == 3) copy_ds_part(next_ds, blk + 2, i >> 1);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  mfma_acc_drain();
  // ---- epilogue: dQ rows through LDS (64 heads at a time), then coalesced 16-byte stores.
  // Lane holds head 16j + gi, dims 16(d0 + i) + 4g .. +3 of tile (i, j).
  bf16_t* dq_t = p.dq + (int64_t)t * p.dq_stride_t;
#pragma unroll
  for (int half = 0; half < (HT + 3) / 4; ++half) {
    __syncthreads();   // ring (or the previous half) no longer read
#pragma unroll
    for (int j = 4 * half; j < HT && j < 4 * half + 4; ++j) {
      char* row = sm.out[16 * (j - 4 * half) + gi];
#pragma unroll
      for (int i = 0; i < DT; ++i)
        *reinterpret_cast<u32x2*>(row + 2 * (16 * (d0 + i) + 4 * g)) =
            u32x2{pack_bf16x2(acc[i][j][0], acc[i][j][1]), pack_bf16x2(acc[i][j][2], acc[i][j][3])};
    }
    __syncthreads();
    const int rows = min(64, hrows - 64 * half);
    const int qc = (p.q_dim != kDv ? kDqk : kDv) / 8;   // 16-byte chunks of a dq row (512: no rope part)
    for (int c = threadIdx.x; c < rows * qc; c += NW * 64) {
      const int r = c / qc, q = c - r * qc;
      *reinterpret_cast<u32x4*>(dq_t + (int64_t)(h0 + 64 * half + r) * (8 * qc) + 8 * q) =
          lds_load16(sm.out[r] + 16 * q);
    }
  }
}

// B2 for 64 < n_heads <= 128: 8 waves, two per SIMD.  Waves 0-3 issue the block gathers (the
// 4-wave copy split of the KV and dS tiles) and own 5 dim tiles each (dims 80w ..), waves 4-7
// own 4 dim tiles each and only multiply, so a copy-issuing wave stalled on its copies leaves
// its SIMD to its partner (with one wave per SIMD those stalls cost ~30% of the block).  Every
// wave covers all 8 head tiles: K^T fragments are read once per workgroup.  Per SIMD: 72
// MFMAs per block.  Accumulators: 5 x 8 tiles of 16 x 16; at two waves per SIMD each register
// file holds 128 per wave, so dim tiles 0-3 are pinned in AccVGPRs and the 5th in VGPRs.
// Without ROPE (512-wide dq rows) every wave owns 4 dim tiles: 64 MFMAs per SIMD per block.
template <bool ROPE>
__global__ __launch_bounds__(512, 1) void bwd_dq8_kernel(SparseBwdParams p) {
  constexpr int NW = 8, NWC = 4;                 // waves; copy-issuing waves
  constexpr int HT = 8;                          // head tiles (128 heads)
  constexpr int DTMAX = ROPE ? 5 : 4;            // dim tiles of a copy-issuing wave
  constexpr int DTP = 4;                         // dim tiles of the other waves
  static_assert(NWC * DTMAX + (NW - NWC) * DTP == (ROPE ? kDqk : kDv) / 16, "dims split over the waves");
  constexpr int TC = tile_copies_per_wave<NWC, ROPE>();
  constexpr int G = TC + 2;                      // copies per copy-issuing wave per block
  static_assert(TC <= 2 * HT - 6, "tile copies before the dS copy slots");
  __shared__ __attribute__((aligned(128))) DqSmem sm;
  const int t = xcd_remap(blockIdx.x, p.n_xcd);
  if (t >= p.total_q) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wu = __builtin_amdgcn_readfirstlane(wave);
  const bool copier = wu < NWC;
  const int g = lane >> 4, gi = lane & 15;
  const int nblk = stage_index_row<NW>(sm.idx, sm.red, p.idx + (int64_t)t * p.idx_stride, p.topk, p.n_kv,
                                       p.causal, t + p.q_offset);
  const int hrows = min(128, p.n_heads);
  const char* ds_base = reinterpret_cast<const char*>(p.ds_stage + (int64_t)t * (p.topk_pad / kBK) * p.n_heads * kBK);
  const int64_t ds_blk = (int64_t)p.n_heads * kBK * 2;   // bytes per staged block tile
  // dS copy k (0, 1) of copy-issuing wave w: head rows 16 * (w + 4k) .. +15 (rows past n_heads
  // re-read row 0; never stored)
  auto copy_ds_part = [&](char* dst, int blk, int k) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(dst));
    const int i = wu + k * NWC;
    const int h = 16 * i + (lane >> 2);
    const int q = (lane & 3) ^ ((h >> 1) & 3);
    const int hs = h < hrows ? h : 0;
    async_copy16_nt(ds_base + blk * ds_blk + hs * (kBK * 2) + q * 16, base + i * 1024u);
  };
  // operand addresses as in bwd_dq_kernel
  uint32_t kv[2], kr[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t key = 8 * g + 4 * h + (gi >> 2);
    kv[h] = key_row(key) * kTileVPitch + 8u * (gi & 3);
    kr[h] = kTileVBytes + key * 128u + 8u * (gi & 1) + 16u * (((gi & 3) >> 1) ^ ((key >> 1) & 7u));
  }
  const uint32_t ds_lane = gi * 64u + 16u * (g ^ ((gi >> 1) & 3));
  const int d0 = copier ? DTMAX * wu : DTMAX * NWC + DTP * (wu - NWC);   // first dim tile
  const int nd = copier ? DTMAX : DTP;
  const uint32_t tile0 = lds_addr(sm.ring.tile[0]);

  f32x4 acc[DTMAX][HT];
#pragma unroll
  for (int i = 0; i < DTMAX; ++i)
#pragma unroll
    for (int j = 0; j < HT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  mfma_acc_drain();   // zero writes of the accumulators before their first MFMA read

  if (copier) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      if (b < nblk) {
        gather_tile<NWC, ROPE>(tile0 + b * kTileBytes, p.kv, sm.idx + b * kBK, wu, lane);
        copy_ds_part(sm.ring.ds[b], b, 0);
        copy_ds_part(sm.ring.ds[b], b, 1);
      }
    }
  }
  // block loop, specialised for the two wave roles (dim tiles ND; copies or not)
  auto block_loop = [&](auto nd_c, auto copier_c) {
    constexpr int ND = decltype(nd_c)::value;
    constexpr bool CP = decltype(copier_c)::value;
    int st = 0;   // ring stage of block blk
    for (int blk = 0; blk < nblk; ++blk) {
      if (CP) {
        if (blk + 1 < nblk) wait_vmcnt<G>(); else wait_vmcnt<0>();
      }
      __syncthreads();
      // block blk+2's copies (copy-issuing waves): tile copy k at half head step k, the dS
      // copies at half steps 10 and 12; each copy's source row is read two copy slots ahead
      // (the readlanes' SGPRs need 5 wait states before the copy reads them).
      // Issued every iteration: the last two re-copy block nblk-1 into the ring slot no block
      // reads any more (so no copy sits behind a branch); retired before the epilogue.
      const int src_blk = min(blk + 2, nblk - 1);
      const int st_next = st == 0 ? 2 : st - 1;   // (blk + 2) % 3
      TileSrc<NWC> next_src;
      if (CP) next_src = tile_sources<NWC, ROPE>(p.kv, sm.idx + src_blk * kBK, wu, lane);
      const char* next_row[2] = {CP ? gather_row<NWC>(next_src, 0) : nullptr, CP ? gather_row<NWC>(next_src, 1) : nullptr};
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t next_tile = tile0 + st_next * kTileBytes;
      char* const next_ds = sm.ring.ds[st_next];
      const uint32_t tb = tile0 + st * kTileBytes;
      const char* dsl = sm.ring.ds[st] + ds_lane;
      st = st == 2 ? 0 : st + 1;
      uint32_t v0 = tb + kv[0], v1 = tb + kv[1], r0 = tb + kr[0], r1 = tb + kr[1];
      asm volatile("" : "+v"(v0), "+v"(v1), "+v"(r0), "+v"(r1));
      auto ld = [&](int i) {
        const int D = d0 + i;   // wave-uniform
        const uint32_t x0 = D < 32 ? v0 + 32u * D : r0 ^ (32u * (D - 32));
        const uint32_t x1 = D < 32 ? v1 + 32u * D : r1 ^ (32u * (D - 32));
        const u32x2 lo = lds_read_tr16(lds_ptr(x0)), hi = lds_read_tr16(lds_ptr(x1));
        return u32x4{lo[0], lo[1], hi[0], hi[1]};
      };
      auto copy_slot = [&](int h) {
        if (!CP) return;
        if (h < TC) {
          gather_issue<NWC>(next_tile, next_src, next_row[h & 1], wu, lane, h);
          next_row[h & 1] = gather_row<NWC>(next_src, h + 2);
        }
        if (h == 10 || h == 12) copy_ds_part(next_ds, src_blk, (h - 10) >> 1);
      };
      // the wave's K^T fragments stay in registers; dS^T fragments stream in two head tiles ahead
      u32x4 a[ND];
#pragma unroll
      for (int i = 0; i < ND; ++i) a[i] = ld(i);
      u32x4 bq[2] = {lds_load16(dsl), lds_load16(dsl + 1024)};
#pragma unroll
      for (int j = 0; j < HT; ++j) {
        const u32x4 bj = bq[j & 1];
#pragma unroll
        for (int i = 0; i < ND; ++i) {
          if (i < 4) mfma16x16x32_cA(acc[i][j], a[i], bj);   // 128 registers in AccVGPRs
          else mfma16x16x32_cV(acc[i][j], a[i], bj);          // the 5th dim tile in VGPRs
          if (i == 1) {
            copy_slot(2 * j);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        copy_slot(2 * j + 1);
        if (j + 2 < HT) bq[j & 1] = lds_load16(dsl + 1024 * (j + 2));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  if (copier) block_loop(std::integral_constant<int, DTMAX>{}, std::true_type{});
  else block_loop(std::integral_constant<int, DTP>{}, std::false_type{});
  wait_vmcnt0();   // the last re-copies have landed before the epilogue reuses the ring
  mfma_acc_drain();
  // ---- epilogue: dQ rows through LDS (64 heads at a time), then coalesced 16-byte stores.
  bf16_t* dq_t = p.dq + (int64_t)t * p.dq_stride_t;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    __syncthreads();   // ring (or the previous half) no longer read
#pragma unroll
    for (int j = 4 * half; j < 4 * half + 4; ++j) {
      char* row = sm.out[16 * (j - 4 * half) + gi];
#pragma unroll
      for (int i = 0; i < DTMAX; ++i)
        if (i < nd)
          *reinterpret_cast<u32x2*>(row + 2 * (16 * (d0 + i) + 4 * g)) =
              u32x2{pack_bf16x2(acc[i][j][0], acc[i][j][1]), pack_bf16x2(acc[i][j][2], acc[i][j][3])};
    }
    __syncthreads();
    const int rows = min(64, hrows - 64 * half);
    const int qc = (p.q_dim != kDv ? kDqk : kDv) / 8;   // 16-byte chunks of a dq row (512: no rope part)
    for (int c = threadIdx.x; c < rows * qc; c += NW * 64) {
      const int r = c / qc, q = c - r * qc;
      *reinterpret_cast<u32x4*>(dq_t + (int64_t)(64 * half + r) * (8 * qc) + 8 * q) = lds_load16(sm.out[r] + 16 * q);
    }
  }
}

// B4: key-major order of the selected (query, slot) pairs, ascending in query inside every
// key's segment, so that B5 adds each key's G rows in one fixed order and dKV is the same bit
// for bit from run to run.  The query rows are cut into csr_groups() contiguous runs, run b
// taken by workgroup b, and the keys into LDS tiles of kCsrLdsKeys:
//   csr_hist_kernel     cnt[b][k] = pairs of run b that select key k
//   csr_colscan_kernel  per key: cnt[b][k] <- pairs of the runs before b; cnt[nb][k] = total
//   csr_scan_kernel     offsets = exclusive scan of the totals
//   csr_fill_kernel     run b hands out key k's slots from offsets[k] + cnt[b][k] on, one row
//                       at a time in row order (a barrier between rows)
// Integer counts make every step exact.  A top-k row holds a key at most once; a row that
// repeats one gives it consecutive slots in either order, and those G rows are equal (same
// logits, same P and dS), so the sum is still the same.
// ------------------------------------------------------------------------------------------
constexpr int kCsrLdsKeys = 16384;
constexpr int kCsrThreads = 1024;
constexpr int kCsrPer = kMaxTopkBwd / kCsrThreads;   // index slots per thread and row
DSA_DEV bool csr_pair_ok(int v, int t, int n_kv, int causal) { return v >= 0 && v < n_kv && (!causal || v <= t); }

// rows [t0, t1) of this workgroup's run
DSA_DEV void csr_run(int total_q, int& t0, int& t1) {
  const int per = (total_q + gridDim.x - 1) / gridDim.x;
  t0 = min(total_q, (int)blockIdx.x * per);
  t1 = min(total_q, t0 + per);
}

__global__ __launch_bounds__(kCsrThreads) void csr_hist_kernel(const int32_t* idx, int64_t idx_stride, int total_q,
                                                              int topk, int n_kv, int causal, int t_offset, int32_t* cnt) {
  __shared__ int32_t hist[kCsrLdsKeys];
  int t0, t1;
  csr_run(total_q, t0, t1);
  for (int k0 = 0; k0 < n_kv; k0 += kCsrLdsKeys) {
    const int nk = min(kCsrLdsKeys, n_kv - k0);
    for (int k = threadIdx.x; k < nk; k += kCsrThreads) hist[k] = 0;
    __syncthreads();
    for (int t = t0; t < t1; ++t)
      for (int j = threadIdx.x; j < topk; j += kCsrThreads) {
        const int v = idx[(int64_t)t * idx_stride + j];
        if (csr_pair_ok(v, t + t_offset, n_kv, causal) && v >= k0 && v - k0 < nk) atomicAdd(hist + (v - k0), 1);
      }
    __syncthreads();
    for (int k = threadIdx.x; k < nk; k += kCsrThreads) cnt[(int64_t)blockIdx.x * n_kv + k0 + k] = hist[k];
    __syncthreads();   // the next tile clears hist
  }
}

// One thread per key walks the runs in order (8 loads in flight per step).
__global__ __launch_bounds__(256) void csr_colscan_kernel(int32_t* cnt, int n_runs, int n_kv) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= n_kv) return;
  int32_t run = 0;
  int b = 0;
  for (; b + 8 <= n_runs; b += 8) {
    int32_t c[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) c[u] = cnt[(int64_t)(b + u) * n_kv + k];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      cnt[(int64_t)(b + u) * n_kv + k] = run;
      run += c[u];
    }
  }
  for (; b < n_runs; ++b) {
    const int32_t c = cnt[(int64_t)b * n_kv + k];
    cnt[(int64_t)b * n_kv + k] = run;
    run += c;
  }
  cnt[(int64_t)n_runs * n_kv + k] = run;
}

// Single-workgroup exclusive scan of totals[n] -> offsets[n + 1] (int64).
__global__ __launch_bounds__(1024) void csr_scan_kernel(const int32_t* totals, int n, int64_t* offsets) {
  __shared__ int64_t part[1024];
  const int tid = threadIdx.x;
  const int per = (n + 1023) / 1024;
  const int a = min(n, tid * per), b = min(n, a + per);
  int64_t s = 0;
  for (int i = a; i < b; ++i) s += totals[i];
  part[tid] = s;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int64_t v = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int64_t run = tid > 0 ? part[tid - 1] : 0;
  for (int i = a; i < b; ++i) {
    offsets[i] = run;
    run += totals[i];
  }
  if (tid == 1023) offsets[n] = part[1023];
}

__global__ __launch_bounds__(kCsrThreads) void csr_fill_kernel(const int32_t* idx, int64_t idx_stride, int total_q,
                                                              int topk, int n_kv, int causal, int t_offset,
                                                              const int64_t* offsets,
                                                              const int32_t* cnt, int64_t* pair_pos) {
  __shared__ int32_t next[kCsrLdsKeys];   // next free slot of each key of the tile
  int t0, t1;
  csr_run(total_q, t0, t1);
  auto load_row = [&](int t, int32_t (&v)[kCsrPer]) {
#pragma unroll
    for (int i = 0; i < kCsrPer; ++i) {
      const int j = (int)threadIdx.x + kCsrThreads * i;
      v[i] = t < t1 && j < topk ? idx[(int64_t)t * idx_stride + j] : -1;
    }
  };
  for (int k0 = 0; k0 < n_kv; k0 += kCsrLdsKeys) {
    const int nk = min(kCsrLdsKeys, n_kv - k0);
    for (int k = threadIdx.x; k < nk; k += kCsrThreads)   // < 2^31: checked by the launchers
      next[k] = (int32_t)(offsets[k0 + k] + cnt[(int64_t)blockIdx.x * n_kv + k0 + k]);
    __syncthreads();
    int32_t cur[kCsrPer], nxt[kCsrPer];
    load_row(t0, cur);
    for (int t = t0; t < t1; ++t) {
      load_row(t + 1, nxt);   // the next row's indices under this row's slot claims
#pragma unroll
      for (int i = 0; i < kCsrPer; ++i) {
        const int j = (int)threadIdx.x + kCsrThreads * i;
        if (j < topk) {
          const int v = cur[i];
          int64_t* dst = pair_pos + (int64_t)t * topk + j;
          if (!csr_pair_ok(v, t + t_offset, n_kv, causal)) {
            if (k0 == 0) *dst = -1;
          } else if (v >= k0 && v - k0 < nk) {
            *dst = atomicAdd(next + (v - k0), 1);
          }
        }
      }
      __syncthreads();   // every slot of row t before any of row t + 1
#pragma unroll
      for (int i = 0; i < kCsrPer; ++i) cur[i] = nxt[i];
    }
  }
}

// ------------------------------------------------------------------------------------------
// B5: dKV[s] = sum of G rows in s's segment (fp32), or dKV[s] += that sum for the later query
// chunks of a chunked backward.  One workgroup (4 * W / 8 threads) per key: 4 row lanes x W / 8
// chunks of 8 dims.  W = 576, or 512 for the G rows of 512-wide q rows (dKV's rope columns are
// then zero).
// ------------------------------------------------------------------------------------------
template <int W>
__global__ __launch_bounds__(W / 2) void bwd_dkv_reduce_kernel(const bf16_t* g_stage, const int64_t* offsets,
                                                               int n_kv, float* dkv, int64_t dkv_stride,
                                                               int accumulate) {
  __shared__ float red[3][W];
  const int s = blockIdx.x;
  if (s >= n_kv) return;
  constexpr int kChunks = W / 8;
  const int c = threadIdx.x % kChunks, r = threadIdx.x / kChunks;
  const int64_t a = offsets[s], b = offsets[s + 1];
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  auto add_row = [&](const u32x4& v) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[2 * e] += bf16_lo(v[e]);
      acc[2 * e + 1] += bf16_hi(v[e]);
    }
  };
  auto load_row = [&](int64_t i) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(g_stage + i * W + c * 8));
  };
  // rows a + r, a + r + 4, ..: four loads in flight per thread, summed in row order (a loop of
  // one load and its adds kept a single 16-byte load per thread in flight)
  int64_t i = a + r;
  for (; i + 12 < b; i += 16) {
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = load_row(i + 4 * u);
#pragma unroll
    for (int u = 0; u < 4; ++u) add_row(v[u]);
  }
  for (; i < b; i += 4) add_row(load_row(i));
  if (r > 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[r - 1][c * 8 + e] = acc[e];
  }
  __syncthreads();
  if (r == 0) {
    float* out = dkv + (int64_t)s * dkv_stride + c * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = acc[e] + red[0][c * 8 + e] + red[1][c * 8 + e] + red[2][c * 8 + e];
      out[e] = accumulate ? out[e] + v : v;
    }
  }
  if constexpr (W < kDqk) {
    if (!accumulate && (int)threadIdx.x < kDqk - W) dkv[(int64_t)s * dkv_stride + W + threadIdx.x] = 0.f;
  }
}

// B5 over int8 G rows (format: dsa_kernels.h): the same per-key sums in a fixed order, each value
// dequantised exactly ((u - 128) * s is a 16-bit product, so the fma is exact).  Latent part:
// one wave per row, lane l dims 8l..8l+7 (8 bytes, group l / 4), wave w rows a + w, a + w + 4, ..
// (eight in flight), so each 128-byte line is read by one wave (rows cut across waves mid-line
// were fetched twice).  Rope part (the 128-byte tail line: 8 bytes of slot j = rope dims
// 512 + 8j.., group 16 + j / 4): thread t takes slot t % 8 of rows a + t / 8, a + t / 8 + 32, ..
// Then the four waves' latent sums, and the 32 rope partials of each slot, are added in a fixed
// order.
__global__ __launch_bounds__(256) void bwd_dkv_reduce_i8_kernel(const char* g_rows, const int64_t* offsets,
                                                                int n_kv, float* dkv, int64_t dkv_stride,
                                                                int accumulate) {
  __shared__ float red[3][512];
  __shared__ float rred[32][64];
  const int s = blockIdx.x;
  if (s >= n_kv) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int grp = lane >> 2;
  const int scale_off = 512 + 16 * (grp / 3) + 8 + 2 * (grp % 3);
  const int rj = tid & 7, rgrp = 16 + (rj >> 2);
  const int rscale_off = 512 + 16 * (rgrp / 3) + 8 + 2 * (rgrp % 3);
  const int64_t a = offsets[s], b = offsets[s + 1];
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0}, racc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  struct Part { u32x2 v; uint32_t sb; };
  auto add8 = [](float (&dst)[8], const Part& x) {
    const float sc = __builtin_bit_cast(float, x.sb << 16), nb = -128.f * sc;
#pragma unroll
    for (int e = 0; e < 8; ++e) dst[e] += fmaf((float)((x.v[e >> 2] >> (8 * (e & 3))) & 0xffu), sc, nb);
  };
  auto latent = [&](int64_t i) {
    const char* row = g_rows + i * kGRowBytesI8;
    return Part{__builtin_nontemporal_load(reinterpret_cast<const u32x2*>(row + 8 * lane)),
                *reinterpret_cast<const uint16_t*>(row + scale_off)};
  };
  auto ropepart = [&](int64_t i) {
    const char* row = g_rows + i * kGRowBytesI8;
    return Part{*reinterpret_cast<const u32x2*>(row + 512 + 16 * rj), *reinterpret_cast<const uint16_t*>(row + rscale_off)};
  };
  // Chunks of 32 rows: wave w takes the latent parts of rows c+w, c+w+4, ..., thread t the rope
  // slot t%8 of row c+t/8.  Both parts of a chunk are loaded together, so the rope loads find the
  // tail lines the scale loads have just brought into the L2 (a second pass over the key's rows
  // would fetch every tail line twice).  Each thread still adds its rows in ascending order.
  int64_t c = a;
  for (; c + 31 < b; c += 32) {
    Part v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = latent(c + w + 4 * u);
    const Part rp = ropepart(c + (tid >> 3));
#pragma unroll
    for (int u = 0; u < 8; ++u) add8(acc, v[u]);
    add8(racc, rp);
  }
  for (int64_t i = c + w; i < b; i += 4) add8(acc, latent(i));
  for (int64_t r = c + (tid >> 3); r < b; r += 32) add8(racc, ropepart(r));
  if (w > 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[w - 1][8 * lane + e] = acc[e];
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) rred[tid >> 3][8 * rj + e] = racc[e];
  __syncthreads();
  float* out = dkv + (int64_t)s * dkv_stride;
  if (w == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = 8 * lane + e;
      const float v = acc[e] + red[0][d] + red[1][d] + red[2][d];
      out[d] = accumulate ? out[d] + v : v;
    }
  } else if (w == 1) {   // rope dim 512 + lane: the 32 row-offset partials in order
    float v = 0.f;
#pragma unroll 8
    for (int k = 0; k < 32; ++k) v += rred[k][lane];
    out[512 + lane] = accumulate ? out[512 + lane] + v : v;
  }
}

// Key gradients of a backward with no query rows: every key's sum is empty.  A fill kernel
// rather than a memset, so a captured graph holds no memset node.
__global__ __launch_bounds__(256) void zero_rows_kernel(float* rows, int n_rows, int64_t stride, int width) {
  const int r = blockIdx.x;
  if (r >= n_rows) return;
  for (int c = threadIdx.x; c < width; c += 256) rows[(int64_t)r * stride + c] = 0.f;
}

// d sinks: one workgroup per head, a fixed-order sum over the query rows (strided per thread, then
// a wave and a cross-wave reduction), so the result is the same from run to run (short batches
// and callers without scratch; longer ones take the two-level form below).
__global__ __launch_bounds__(256) void sink_grad_kernel(const float* sinks, const float* lse, const float* delta,
                                                        int total_q, int n_heads, float* dsinks) {
  const int h = blockIdx.x;
  __shared__ float part[4];
  const float sk = sinks[h];
  float acc = 0.f;
  for (int t = threadIdx.x; t < total_q; t += 256) {
    const float l = lse[(int64_t)t * n_heads + h];
    if (l != -INFINITY) acc += expf(sk - l) * delta[(int64_t)t * n_heads + h];
  }
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) dsinks[h] = 0.f - ((part[0] + part[1]) + (part[2] + part[3]));
}

// Long batches: the same sums in two fixed-order levels over coalesced rows.  Workgroup (chunk,
// 64-head tile): lane = head, its 4 waves take every 4th row of the chunk; then one workgroup per
// head tile adds the chunks' partials, its 16 waves every 16th chunk, and the waves in order.
constexpr int kSinkChunks = 256;
__global__ __launch_bounds__(256) void sink_grad_partial_kernel(const float* sinks, const float* lse,
                                                                const float* delta, int total_q, int n_heads,
                                                                int rows_per_chunk, float* part) {
  __shared__ float red[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = blockIdx.y * 64 + lane;
  const int t0 = blockIdx.x * rows_per_chunk, t1 = min(total_q, t0 + rows_per_chunk);
  float acc = 0.f;
  if (h < n_heads) {
    const float sk = sinks[h];
#pragma unroll 4
    for (int t = t0 + wave; t < t1; t += 4) {
      const float l = lse[(int64_t)t * n_heads + h];
      if (l != -INFINITY) acc += expf(sk - l) * delta[(int64_t)t * n_heads + h];
    }
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && h < n_heads)
    part[(int64_t)blockIdx.x * n_heads + h] = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
}

__global__ __launch_bounds__(1024) void sink_grad_final_kernel(const float* part, int chunks, int n_heads,
                                                               float* dsinks) {
  __shared__ float red[16][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = blockIdx.x * 64 + lane;
  float acc = 0.f;
  if (h < n_heads) {
#pragma unroll 4
    for (int c = wave; c < chunks; c += 16) acc += part[(int64_t)c * n_heads + h];
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && h < n_heads) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < 16; ++w) s += red[w][lane];
    dsinks[h] = 0.f - s;
  }
}

size_t sink_grad_scratch_bytes(int n_heads) { return sizeof(float) * (size_t)kSinkChunks * (size_t)n_heads; }

int launch_sink_grad(const float* sinks, const float* lse, const float* delta, int total_q, int n_heads,
                     float* dsinks, float* scratch, size_t scratch_bytes, hipStream_t stream) {
  if (n_heads < 1) return 0;
  if (scratch != nullptr && scratch_bytes >= sink_grad_scratch_bytes(n_heads) && total_q >= 4 * kSinkChunks) {
    const int rows = (total_q + kSinkChunks - 1) / kSinkChunks;
    const int chunks = (total_q + rows - 1) / rows;
    const int tiles = (n_heads + 63) / 64;
    hipLaunchKernelGGL(sink_grad_partial_kernel, dim3(chunks, tiles), dim3(256), 0, stream, sinks, lse, delta,
                       total_q, n_heads, rows, scratch);
    hipLaunchKernelGGL(sink_grad_final_kernel, dim3(tiles), dim3(1024), 0, stream, scratch, chunks, n_heads, dsinks);
  } else {
    hipLaunchKernelGGL(sink_grad_kernel, dim3(n_heads), dim3(256), 0, stream, sinks, lse, delta, total_q, n_heads,
                       dsinks);
  }
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_zero_rows(float* rows, int n_rows, int64_t stride, int width, hipStream_t stream) {
  if (n_rows <= 0 || width <= 0) return 0;
  hipLaunchKernelGGL(zero_rows_kernel, dim3(n_rows), dim3(256), 0, stream, rows, n_rows, stride, width);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

void launch_pair_csr(const int32_t* idx, int64_t idx_stride, int total_q, int topk, int n_kv, int causal,
                     int t_offset, int32_t* csr_counts, int64_t* csr_offsets, int64_t* pair_pos, hipStream_t stream) {
  const int nr = csr_groups(total_q, n_kv);
  hipLaunchKernelGGL(csr_hist_kernel, dim3(nr), dim3(kCsrThreads), 0, stream, idx, idx_stride, total_q, topk, n_kv,
                     causal, t_offset, csr_counts);
  hipLaunchKernelGGL(csr_colscan_kernel, dim3((n_kv + 255) / 256), dim3(256), 0, stream, csr_counts, nr, n_kv);
  hipLaunchKernelGGL(csr_scan_kernel, dim3(1), dim3(1024), 0, stream, csr_counts + (int64_t)nr * n_kv, n_kv,
                     csr_offsets);
  hipLaunchKernelGGL(csr_fill_kernel, dim3(nr), dim3(kCsrThreads), 0, stream, idx, idx_stride, total_q, topk, n_kv,
                     causal, t_offset, csr_offsets, csr_counts, pair_pos);
}

int launch_sparse_mla_bwd(const SparseBwdParams& p, hipStream_t stream, hipEvent_t const* ev) {
  if (p.n_xcd < 1) return -1;
  if (p.topk > kMaxTopkBwd) return -2;
  if (p.g_sink_row >= INT32_MAX) return -2;   // B3 keeps G row numbers in 32 bits
  bool marks_ok = true;   // a failed event record is reported like a failed launch
  auto mark = [&](int i) {
    if (ev && hipEventRecord(ev[i], stream) != hipSuccess) marks_ok = false;
  };
  mark(0);
  const int nw = p.n_heads > 64 ? 4 : (p.n_heads > 32 ? 2 : 1);
  const dim3 grid(xcd_grid(p.total_q, p.n_xcd), (p.n_heads + 127) / 128);
  // B4 first: it only depends on idx.
  launch_pair_csr(p.idx, p.idx_stride, p.total_q, p.topk, p.n_kv, p.causal, p.q_offset, p.csr_counts,
                  p.csr_offsets, p.pair_pos, stream);
  mark(1);
  // B1, B2: 512-wide q rows (no rope part) take the instantiations without the rope k-steps
  auto launch_sp_dq = [&](auto rope_c) {
    constexpr bool R = decltype(rope_c)::value;
    if (nw == 4) {
      hipLaunchKernelGGL((bwd_sp_kernel<4, R>), grid, dim3(256), 0, stream, p);
      mark(2);
      if (grid.y == 1) hipLaunchKernelGGL((bwd_dq8_kernel<R>), grid, dim3(512), 0, stream, p);
      else hipLaunchKernelGGL((bwd_dq_kernel<4, R>), grid, dim3(256), 0, stream, p);
    } else if (nw == 2) {
      hipLaunchKernelGGL((bwd_sp_kernel<2, R>), grid, dim3(128), 0, stream, p);
      mark(2);
      hipLaunchKernelGGL((bwd_dq_kernel<2, R>), grid, dim3(128), 0, stream, p);
    } else {
      hipLaunchKernelGGL((bwd_sp_kernel<1, R>), grid, dim3(64), 0, stream, p);
      mark(2);
      hipLaunchKernelGGL((bwd_dq_kernel<1, R>), grid, dim3(64), 0, stream, p);
    }
  };
  if (p.q_dim == kDv) launch_sp_dq(std::false_type{});
  else launch_sp_dq(std::true_type{});
  mark(3);
  const int nks = p.n_heads / 16;
  const dim3 ggrid(xcd_grid(p.total_q, p.n_xcd));
  // bf16 G rows of 512-wide q rows are 1024 bytes (no rope part); int8 rows keep their format
  const bool g512 = !p.g_int8 && p.q_dim == kDv;
  auto launch_g = [&](auto rope_c) {
    constexpr bool R = decltype(rope_c)::value;
    if (nks > 4)
      hipLaunchKernelGGL((bwd_g_kernel<8, false, R>), ggrid, dim3(256), 0, stream, p);
    else if (nks > 2)
      hipLaunchKernelGGL((bwd_g_kernel<4, false, R>), ggrid, dim3(256), 0, stream, p);
    else if (nks > 1)
      hipLaunchKernelGGL((bwd_g_kernel<2, false, R>), ggrid, dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL((bwd_g_kernel<1, false, R>), ggrid, dim3(256), 0, stream, p);
  };
  if (p.g_int8) launch_bwd_g_i8(p, stream);
  else if (g512) launch_g(std::false_type{});
  else launch_g(std::true_type{});
  mark(4);
  const bf16_t* g_rows = reinterpret_cast<const bf16_t*>(p.g_stage);
  if (p.g_int8)
    hipLaunchKernelGGL(bwd_dkv_reduce_i8_kernel, dim3(p.n_kv), dim3(256), 0, stream, p.g_stage, p.csr_offsets,
                       p.n_kv, p.dkv, p.dkv_stride, p.dkv_accumulate);
  else if (g512)
    hipLaunchKernelGGL(bwd_dkv_reduce_kernel<kDv>, dim3(p.n_kv), dim3(kDv / 2), 0, stream, g_rows, p.csr_offsets,
                       p.n_kv, p.dkv, p.dkv_stride, p.dkv_accumulate);
  else
    hipLaunchKernelGGL(bwd_dkv_reduce_kernel<kDqk>, dim3(p.n_kv), dim3(kDqk / 2), 0, stream, g_rows, p.csr_offsets,
                       p.n_kv, p.dkv, p.dkv_stride, p.dkv_accumulate);
  mark(5);
  return hipGetLastError() == hipSuccess && marks_ok ? 0 : -4;
}

}  // namespace dsa
