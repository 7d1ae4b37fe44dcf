// B3 of the sparse MLA backward (bwd_g_kernel) and the constants every backward kernel shares.
// dsa_sparse_bwd.hip instantiates B3 for bf16 G rows; dsa_sparse_bwd_i8.hip instantiates it for
// int8 G rows, in a file compiled with MFMA accumulators in VGPRs (-mllvm -amdgpu-mfma-vgpr-form)
// because that variant reads every accumulator with VALU instructions.
#pragma once

#include <type_traits>

#include "dsa_common.h"
#include "dsa_kernels.h"
#include "dsa_kvtile.h"

namespace dsa {

constexpr int kDqk = 576;
// 16 zero bytes in global memory: the LDS-direct source of the rope chunks of 512-wide q rows
static __device__ __attribute__((aligned(16))) const uint32_t kZero16[4] = {0u, 0u, 0u, 0u};
constexpr int kDv = 512;
constexpr int kBK = kTileKeys;
constexpr int kStages = 3;
constexpr int kMaxTopkBwd = 4096;
constexpr int kPre = 3;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

DSA_DEV u32x2 lds_read_tr16(const char* p) {
  s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  return __builtin_bit_cast(u32x2, r);
}

// ------------------------------------------------------------------------------------------
// B3: per-pair dKV partial rows G = (scale*dS)^T Q + P^T dO, contracted over all heads.
// Wave w owns output row tiles (32 latent dims each): Q part {4w..4w+3} (+16+w for w < 2),
// dO part {4w..4w+3}.
// Setup: Q[t] and dO[t] (contiguous [H x 576] / [H x 512] bf16) are copied straight into LDS
// with asynchronous LDS-direct loads, 16 heads per round through a 3-round ring (two rounds in
// flight while one is read), and the Q^T / dO^T operand fragments are taken from it with
// transposing reads.  Chunk c of head row r sits at chunk c ^ (2 * (r & 3)), which puts the four
// rows of every transposing read on distinct banks.
// Each block's G tile [32 keys x 576] goes through LDS in fp32, written straight from the
// accumulators, so that every row is written to its key-major position with contiguous 16-byte
// lane stores: wave w stores the latent part of rows 8w..8w+7 (one 1 KB row per instruction) and
// the rope part of the same rows (one instruction), 9 stores per wave, converted to bf16 and
// issued between the next block's MFMAs.  Written straight from the MFMA layout, every store
// instruction would touch 32 rows 16 bytes each.
// With int8 G rows (block_loop_i8) a tile is quantised straight from its accumulators instead
// and only the 640-byte rows pass through LDS (double-buffered, no G-tile barrier): a fifth of the
// fp32 tile's LDS traffic.
// ------------------------------------------------------------------------------------------
constexpr int kGHeads = 128;                        // B3 handles up to 128 heads (n_heads % 16 == 0)
constexpr int kGKs = kGHeads / 16;                  // head k-steps
constexpr int kStageTile = kGHeads * 64;            // one staged [128 heads][32 keys] bf16 tile
constexpr int kQRound = 16 * kDqk * 2;              // Q bytes of one setup round (16 heads)
constexpr int kORound = 16 * kDv * 2;               // dO bytes of one setup round
constexpr int kRoundBytes = kQRound + kORound;
constexpr int kRoundCopies = kRoundBytes / 1024;    // 1 KB LDS-direct copies per round (34)
constexpr int kSetupStages = 3;
constexpr int kGTilePitch = kDqk * 4 + 16;          // LDS pitch of an fp32 G tile row (bank spread)
constexpr int kGStores = 9;                         // stores per wave per block: 8 rows + rope
constexpr int kGQPitch = kGRowBytesI8 + 16;         // LDS pitch of an int8 G row (16 rows of a
                                                    //   16-byte write on distinct banks)
static_assert(2 * kBK * kGQPitch <= kBK * kGTilePitch, "int8 G tiles fit the fp32 tile's space");

struct GSmem {
  union {
    char ring[kSetupStages][kRoundBytes];           // setup: Q / dO rows of 16 heads per round
    struct {
      char st[kStages][2][kStageTile];              // [dS | P] tiles; 16-byte chunk c of head row h
                                                    //   at chunk c ^ (2 * ((h >> 1) & 1))
      union {
        char gtile[kBK * kGTilePitch];              // bf16 rows: fp32 G tile of the last finished
                                                    //   block; 16-byte chunk j of a row at
                                                    //   j ^ ((j >> 3) & 1)
        char gq[2][kBK][kGQPitch];                  // int8 rows: the G rows of blocks b and b - 1
      };                                            //   (buffer b & 1) in their HBM format
    } loop;
  };
  int32_t pos[kMaxTopkBwd];                         // G row of every index slot (sink if unselected)
  int32_t idx[kMaxTopkBwd];
  int red[4];
};
static_assert(sizeof(GSmem) <= 160 * 1024, "B3 LDS budget");

// ---- int8 G rows (format: dsa_kernels.h), quantised straight from the MFMA accumulators ----
// A finished 32 x 32 tile (32 keys x one 32-dim group) holds key l % 32, dims 8*q4 + 4*(l / 32)
// .. +3 (q4 = 0..3) in lane l, so each key's group is split over lanes l and l + 32.
// max(|x|, |y|, |z|) in one v_max3_f32 with |.| source modifiers.  G values are finite, so the
// NaN quieting that fmaxf adds in IEEE mode (a max of each input with itself) is not needed.
DSA_DEV float absmax3(float x, float y, float z) {
  float r;
  asm("v_max3_f32 %0, |%1|, |%2|, |%3|" : "=v"(r) : "v"(x), "v"(y), "v"(z));
  return r;
}
// Largest |x| of accumulator values o .. o+7 as a bit pattern (for |x| >= 0 the integer order of
// the bits is the float order).
DSA_DEV uint32_t absmax_bits8(const f32x16& a, int o) {
  const float x = absmax3(a[o], a[o + 1], a[o + 2]);
  const float y = absmax3(x, a[o + 3], a[o + 4]);
  const float z = absmax3(y, a[o + 5], a[o + 6]);
  return __builtin_bit_cast(uint32_t, absmax3(z, a[o + 7], a[o + 7]));
}
// bf16 bits of a group scale: max / 127 rounded up, so every |g / s| <= 127.
DSA_DEV uint32_t i8_scale_bits(uint32_t max_bits) {
  const float f = __builtin_bit_cast(float, max_bits) * (1.0f / 127.0f);
  return (__builtin_bit_cast(uint32_t, f) + 0xffffu) >> 16;
}
// Accumulator values o .. o+3 as offset-binary bytes rint(x * inv) + 128 (byte k = value o + k).
// Adding 1.5 * 2^23 + 128 in the fma rounds x * inv to the nearest integer (ties to even) in the
// low mantissa bits, whose low byte is then the code (1..255 for |x * inv| <= 127); v_perm_b32
// gathers the low bytes.
DSA_DEV uint32_t i8_pack4(const f32x16& a, int o, float inv) {
  constexpr float kRound = 12582912.0f + 128.0f;
  auto c = [&](int i) { return __builtin_bit_cast(uint32_t, fmaf(a[o + i], inv, kRound)); };
  // selector byte k picks byte sel of {src1 bytes 0..3, src0 bytes 4..7}; 0x0c gives zero
  const uint32_t lo = __builtin_amdgcn_perm(c(1), c(0), 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm(c(3), c(2), 0x0c0c0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// Chunk slot of fp32 G-tile chunk j (4 dims): consecutive-lane reads of 32-byte pieces and
// same-column writes of 32 rows are both conflict-free.
DSA_DEV int gtile_slot(int j) { return j ^ ((j >> 3) & 1); }

// KS = head k-steps run per block (a power of two >= n_heads / 16; steps past n_heads multiply
// zero Q^T / dO^T fragments).  ROPE = false (512-wide q rows, bf16 G rows only): the G rows are
// 1024 bytes (no rope part, whose sums would be zero), every wave runs 4 output tiles and 8
// stores per block.
template <int KS, bool I8, bool ROPE = true>
__global__ __launch_bounds__(256, 1) void bwd_g_kernel(SparseBwdParams p) {
  static_assert(ROPE || !I8, "int8 G rows keep the 576-dim format");
  constexpr int NW = 4;
  constexpr int G = 2 * kGHeads / 16 / NW;          // 4 copies per wave per block
  constexpr int NGS = ROPE ? kGStores : kGStores - 1;   // G-tile stores per wave per block
  constexpr int GW = ROPE ? kDqk : kDv;              // bf16 elements per G row
  __shared__ __attribute__((aligned(16))) GSmem sm;
  const int t = xcd_remap(blockIdx.x, p.n_xcd);
  if (t >= p.total_q) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hb = lane >> 5;
  const int g = lane >> 4, gi = lane & 15;
  const int nks = p.n_heads / 16;
  const int wu = __builtin_amdgcn_readfirstlane(wave);
  // ---- setup copies: round r = heads 16r..16r+15 into ring[r % 3]; copy j (1 KB of LDS) is
  // Q bytes 1024j of the round for j < 18, dO bytes 1024(j - 18) after; wave w issues copies
  // w, w + 4, ... (9 for waves 0-1, 8 for waves 2-3)
  const bool q_rope = p.q_dim != kDv;   // 512: q rows without the rope part (copied as zeros)
  const int qd = q_rope ? kDqk : kDv;
  const char* q_t = reinterpret_cast<const char*>(p.q + (int64_t)t * p.q_stride_t);
  const char* o_t = reinterpret_cast<const char*>(p.dout + (int64_t)t * p.dout_stride_t);
  const uint32_t ring0 = lds_addr(sm.ring[0]);
  auto issue_round = [&](int r) {
    const uint32_t dst = ring0 + (uint32_t)(r % kSetupStages) * kRoundBytes;
#pragma unroll
    for (int i = 0; i < (kRoundCopies + NW - 1) / NW; ++i) {
      const int j = NW * i + wu;
      if (j < kRoundCopies) {
        const char* src;
        if (j < kQRound / 1024) {   // 16-byte chunk c of the round's Q rows (72 per row)
          const int c = j * 64 + lane, row = c / (kDqk / 8), slot = c - row * (kDqk / 8);
          const int sc = slot ^ (2 * (row & 3));   // source chunk (rope chunks 64..71 stay in 64..71)
          src = q_t + (int64_t)(16 * r + row) * (2 * qd) + 16 * sc;
          if (sc >= kDv / 8 && !q_rope) src = reinterpret_cast<const char*>(kZero16);   // q rows of 512
        } else {                    // chunk c of the round's dO rows (64 per row)
          const int c = (j - kQRound / 1024) * 64 + lane, row = c >> 6, slot = c & 63;
          src = o_t + (int64_t)(16 * r + row) * (kDv * 2) + 16 * (slot ^ (2 * (row & 3)));
        }
        async_copy16_unordered(src, __builtin_amdgcn_readfirstlane(dst + 1024u * j));
      }
    }
  };
  issue_round(0);
  if (nks > 1) issue_round(1);

  // ---- index row and G rows of every slot, all loads in flight together (and with the copies)
  int nblk;
  {
    const int32_t* idx_row = p.idx + (int64_t)t * p.idx_stride;
    const int64_t* pos_row = p.pair_pos + (int64_t)t * p.topk;
    const int kpad = (p.topk + kBK - 1) / kBK * kBK;
    constexpr int kPer = kMaxTopkBwd / (NW * 64);
    int32_t iv[kPer];
    int64_t pv[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int j = threadIdx.x + NW * 64 * i;
      iv[i] = j < p.topk ? idx_row[j] : -1;
      pv[i] = j < p.topk ? pos_row[j] : -1;
    }
    int last = -1;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int j = threadIdx.x + NW * 64 * i;
      if (j < kpad) {
        int v = iv[i];
        if (v < 0 || v >= p.n_kv || (p.causal && v > t + p.q_offset)) v = -1;
        sm.idx[j] = v;
        if (v >= 0) last = j;
        sm.pos[j] = (int32_t)(pv[i] < 0 ? p.g_sink_row : pv[i]);   // < 2^31: checked by the launcher
      }
    }
    last = wave_max_i(last);
    if (lane == 0) sm.red[wave] = last;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < NW; ++w) last = max(last, sm.red[w]);
    nblk = __builtin_amdgcn_readfirstlane((last + kBK) / kBK);
  }
  if (nblk == 0) {
    wait_vmcnt0();   // no copy outlives the workgroup
    return;
  }
  auto qtile = [&](int i) { return i < 4 ? 4 * wave + i : 16 + wave; };

  // ---- Q^T and dO^T fragments (A operand: row = latent dim, k = 8 heads)
  u32x4 qa[5][KS], va[4][KS];
  const int tr_h = 8 * (g >> 1) + (gi >> 2);        // head row this lane feeds into ds_read_tr
  const int tr_c = 16 * (g & 1) + 4 * (gi & 3);     // latent column this lane feeds
  const int tr_sw = 2 * (gi >> 2);                  // chunk swizzle of rows tr_h and tr_h + 4
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
    for (int i = 0; i < 5; ++i) qa[i][ks] = u32x4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) va[i][ks] = u32x4{0, 0, 0, 0};
  }
  const int nq = ROPE && wave < 2 ? 5 : 4;
  // byte address of (row tr_h + dr, latent column tr_c of tile mt) in a round part of row pitch rp
  auto tr_at = [&](uint32_t part, int rp, int mt, int dr) {
    const int cb = 64 * mt + 2 * tr_c;
    return lds_ptr(part + (tr_h + dr) * rp + 16 * ((cb >> 4) ^ tr_sw) + (cb & 15));
  };
  // round ks: ready once this wave's copies of it are done (only round ks + 1 may still be in
  // flight) and every wave has passed the barrier; the barrier also retires the reads of round
  // ks - 1, whose buffer round ks + 2 then refills
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if (ks >= nks) break;
    if (ks + 1 < nks) {
      if (wu < kRoundCopies % NW) wait_vmcnt<(kRoundCopies + NW - 1) / NW>();
      else wait_vmcnt<kRoundCopies / NW>();
    } else {
      wait_vmcnt0();
    }
    __syncthreads();
    if (ks + 2 < nks) issue_round(ks + 2);
    const uint32_t qb = ring0 + (uint32_t)(ks % kSetupStages) * kRoundBytes, ob = qb + kQRound;
#pragma unroll
    for (int i = 0; i < 5; ++i) {
      if (i < nq) {
        const u32x2 lo = lds_read_tr16(tr_at(qb, kDqk * 2, qtile(i), 0)), hi = lds_read_tr16(tr_at(qb, kDqk * 2, qtile(i), 4));
        qa[i][ks] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x2 lo = lds_read_tr16(tr_at(ob, kDv * 2, 4 * wave + i, 0)), hi = lds_read_tr16(tr_at(ob, kDv * 2, 4 * wave + i, 4));
      va[i][ks] = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
  }
  __syncthreads();  // ring dead (every copy waited for): the union now holds the [dS | P] ring
  if constexpr (I8) {
    // tail bytes of the int8 G tiles that no quantised value lands on: the two zero bytes of every
    // slot and the scale bytes of slots 6-7 (groups 18-23 do not exist); the first block's
    // barrier orders these writes before every scale write and store read
    for (int e = threadIdx.x; e < 2 * kBK * 8; e += NW * 64) {
      char* s = sm.loop.gq[e / (kBK * 8)][(e >> 3) % kBK] + 512 + 16 * (e & 7);
      if ((e & 7) < 6) *reinterpret_cast<uint32_t*>(s + 12) = 0u;
      else *reinterpret_cast<u32x2*>(s + 8) = u32x2{0u, 0u};
    }
  }

  // ---- key blocks: [dS | P] tiles (rows = heads, 32 keys each) through a 3-stage copy ring
  // staged tiles of block b: [H heads][32 keys] bf16, contiguous (see B1)
  const char* dsb = reinterpret_cast<const char*>(p.ds_stage + (int64_t)t * p.n_heads * p.topk_pad);
  const char* psb = reinterpret_cast<const char*>(p.p_stage + (int64_t)t * p.n_heads * p.topk_pad);
  const int64_t st_blk = (int64_t)p.n_heads * kBK * 2;   // bytes per staged block tile
  // copy c (0..3) of this wave's share of block blk's [dS | P] rows: rows 16*(w + (c/2)*NW) ..,
  // dS for even c, P for odd c.  Head rows past n_heads re-read row 0 (valid memory; their
  // k-steps multiply zeros).
  auto stage_part = [&](int s, int blk, int c) {
    const uint32_t b = __builtin_amdgcn_readfirstlane(lds_addr(sm.loop.st[s][c & 1]));
    const int i = wu + (c >> 1) * NW;
    const int h = 16 * i + (lane >> 2);
    const int hs = h < p.n_heads ? h : 0;
    const int chunk = (lane & 3) ^ (2 * ((h >> 1) & 1));   // LDS chunk lane&3 <- global chunk
    const int64_t off = blk * st_blk + hs * (kBK * 2) + chunk * 16;
    async_copy16_nt(((c & 1) ? psb : dsb) + off, b + i * 1024u);
  };
  auto stage = [&](int s, int blk) {
#pragma unroll
    for (int c = 0; c < G; ++c) stage_part(s, blk, c);
  };
  // B operand address of this lane inside a tile: head row 16*ks + tr_h, bytes 2*tr_c .. +8
  const uint32_t b_off = tr_h * 64 + 16 * (((2 * tr_c) >> 4) ^ (2 * ((tr_h >> 1) & 1))) + ((2 * tr_c) & 15);
  // G tile row of this lane's accumulators: key lane % 32.  Chunk 8*qtile + 2*q4 + hb of tile
  // 4w + i sits at slot (8*(4w + i) + 2*q4) + (hb ^ (i & 1)), of the rope tile 16 + w at
  // (8*(16 + w) + 2*q4) + (hb ^ (w & 1)): per-lane bases plus immediates.
  const uint32_t gtile = lds_addr(sm.loop.gtile);
  const uint32_t gt_w = gtile + (lane & 31) * kGTilePitch;
  const uint32_t pk_even = gt_w + 512 * wave + 16 * hb, pk_odd = gt_w + 512 * wave + 16 * (hb ^ 1);
  const uint32_t pk_rope = gt_w + 16 * (8 * (16 + wave)) + 16 * (hb ^ (wave & 1));
  // stores of a finished G tile by this wave: latent dims 8*lane .. +7 of rows 8w + i (i < 8),
  // then the rope dims 512 + 8 * (lane % 8) .. +7 of row 8w + lane / 8
  const int rope_row = 8 * wave + (lane >> 3);
  // store i of a finished tile: its 8 fp32 values are read from LDS one k-step ahead
  // (store_load), converted and stored later (store_issue) -- no exposed LDS latency.
  struct StoreData { f32x4 a, b; };
  auto store_load = [&](int i) {
    const int row = i < 8 ? 8 * wave + i : rope_row;
    const int j = i < 8 ? 2 * lane : 128 + 2 * (lane & 7);   // first of the two 4-dim chunks
    const char* r = lds_ptr(gtile + row * kGTilePitch);
    return StoreData{*reinterpret_cast<const f32x4*>(r + 16 * gtile_slot(j)),
                     *reinterpret_cast<const f32x4*>(r + 16 * gtile_slot(j + 1))};
  };
  auto store_issue = [&](const int32_t (&rpos)[8], int32_t rope_pos, int i, const StoreData& v) {
    const u32x4 o{pack_bf16x2(v.a[0], v.a[1]), pack_bf16x2(v.a[2], v.a[3]), pack_bf16x2(v.b[0], v.b[1]),
                  pack_bf16x2(v.b[2], v.b[3])};
    bf16_t* g = reinterpret_cast<bf16_t*>(p.g_stage);
    if (i < 8)
      __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(g + (int64_t)rpos[i] * GW + 8 * lane));
    else
      __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(g + (int64_t)rope_pos * GW + 8 * (64 + (lane & 7))));
  };
  // k-step of copy c (c < G) and of store i (i < NGS); stores follow copies in a step
  constexpr auto copy_ks = [](int c) { return c * KS / G; };
  constexpr auto store_ks = [](int i) { return i * KS / NGS; };
  constexpr int kStoresAfterLastCopy = [] {
    int n = 0;
    for (int i = 0; i < NGS; ++i) n += (i * KS / NGS) >= ((G - 1) * KS / G);
    return n;
  }();

  auto block_loop = [&](auto nq_c) {
    constexpr int NQ = decltype(nq_c)::value;
    stage(0, 0);
    if (nblk > 1) stage(1, 1);
    for (int blk = 0; blk < nblk; ++blk) {
      // issue order of block blk: [wait][barrier] then, between its MFMAs, copies(blk+2) and
      // stores(blk-1) (stores after copies within a k-step), then [barrier][G(blk) -> LDS].
      // Block blk needs copies(blk) done; issued after them: block 0 nothing of its own, block 1
      // the copies(3) + stores(0), block b >= 3 the trailing stores(b-3) of block b-2 plus block
      // b-1's copies(b+1) + stores(b-2).
      if (blk + 1 >= nblk) wait_vmcnt<0>();
      else if (blk <= 1) wait_vmcnt<G>();
      else if (blk == 2) wait_vmcnt<G + NGS>();
      else wait_vmcnt<G + NGS + kStoresAfterLastCopy>();
      __syncthreads();
      const bool copy_next = blk + 2 < nblk;
      const bool store_prev = blk > 0;
      // G rows of the previous block's tile: this wave's 8 latent rows (wave-uniform) and the
      // rope row of this lane
      int32_t rpos[8], rope_pos = 0;
      StoreData sv[NGS];
      if (store_prev) {
#pragma unroll
        for (int i = 0; i < 8; ++i) rpos[i] = __builtin_amdgcn_readfirstlane(sm.pos[(blk - 1) * kBK + 8 * wave + i]);
        rope_pos = sm.pos[(blk - 1) * kBK + rope_row];
#pragma unroll
        for (int i = 0; i < NGS; ++i)
          if (store_ks(i) == 0) sv[i] = store_load(i);
      }
      const char* sd = sm.loop.st[blk % kStages][0] + b_off;
      const char* sp = sm.loop.st[blk % kStages][1] + b_off;
      f32x16 acc[NQ];
#pragma unroll
      for (int i = 0; i < NQ; ++i) acc[i] = f32x16{};
      auto load_b = [&](int ks, u32x4& bs, u32x4& bp) {
        const u32x2 s_lo = lds_read_tr16(sd + ks * 1024), s_hi = lds_read_tr16(sd + ks * 1024 + 4 * 64);
        const u32x2 p_lo = lds_read_tr16(sp + ks * 1024), p_hi = lds_read_tr16(sp + ks * 1024 + 4 * 64);
        bs = u32x4{s_lo[0], s_lo[1], s_hi[0], s_hi[1]};
        bp = u32x4{p_lo[0], p_lo[1], p_hi[0], p_hi[1]};
      };
      u32x4 bs, bp;
      load_b(0, bs, bp);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        u32x4 bs_n, bp_n;
        if (ks + 1 < KS) load_b(ks + 1, bs_n, bp_n);   // next k-step's operands under these MFMAs
        if (copy_next) {
#pragma unroll
          for (int c = 0; c < G; ++c)
            if (copy_ks(c) == ks) stage_part((blk + 2) % kStages, blk + 2, c);
        }
        if (store_prev) {
#pragma unroll
          for (int i = 0; i < NGS; ++i) {
            if (store_ks(i) == ks + 1) sv[i] = store_load(i);   // next step's data
            if (store_ks(i) == ks) store_issue(rpos, rope_pos, i, sv[i]);
          }
        }
        // Q-part products of all tiles first, then the dO-part ones: dependent MFMAs on one
        // accumulator are NQ instructions apart instead of back to back
#pragma unroll
        for (int i = 0; i < NQ; ++i) acc[i] = mfma32x32x16(as_bf16x8(qa[i][ks]), as_bf16x8(bs), acc[i]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = mfma32x32x16(as_bf16x8(va[i][ks]), as_bf16x8(bp), acc[i]);
        if (ks + 1 < KS) { bs = bs_n; bp = bp_n; }
      }
      // G tile -> LDS (fp32, straight from the accumulators) once every wave has read the
      // previous tile: lane holds key lane % 32, dims 32*qtile(i) + 8*q4 + 4*hb .. +3
      __syncthreads();
#pragma unroll
      for (int i = 0; i < NQ; ++i) {
        const uint32_t base = i < 4 ? ((i & 1) ? pk_odd : pk_even) + 128 * i : pk_rope;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          *reinterpret_cast<f32x4*>(const_cast<char*>(lds_ptr(base + 32 * q4))) =
              f32x4{acc[i][4 * q4], acc[i][4 * q4 + 1], acc[i][4 * q4 + 2], acc[i][4 * q4 + 3]};
      }
    }
    // the last block's G tile
    __syncthreads();
    {
      int32_t rpos[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) rpos[i] = __builtin_amdgcn_readfirstlane(sm.pos[(nblk - 1) * kBK + 8 * wave + i]);
      const int32_t rope_pos = sm.pos[(nblk - 1) * kBK + rope_row];
#pragma unroll
      for (int i = 0; i < NGS; ++i) store_issue(rpos, rope_pos, i, store_load(i));
    }
  };
  // ---- int8 G rows.  Each wave runs its output tiles one after another (a tile's MFMAs, Q part
  // then dO part per head k-step as above, form one accumulation chain) and quantises tile
  // tq - 1 straight from its accumulators while tile tq's MFMAs run.  The codes and scales go to
  // LDS buffer blk & 1 in the rows' HBM format, from which block blk + 1 stores whole rows; with
  // two buffers no barrier separates a tile from the stores of the previous one.  The side work
  // of a block is spread over its KS * NQ k-step slots: tile 0's B operands, copies(blk + 2),
  // the 5 stores of block blk - 1 (each read from LDS one store ahead) and five quantisation
  // pieces per tile.
  auto block_loop_i8 = [&](auto nq_c) {
    constexpr int NQ = decltype(nq_c)::value;
    constexpr int S = KS * NQ;                                   // side-work slots per block
    constexpr auto copy_slot = [](int c) { return c * S / G; };
    constexpr int NS = 5;                                        // stores per wave per block
    constexpr auto st_slot = [](int i) { return i * S / NS; };
    constexpr auto piece_ks = [](int piece) { return (piece + 1) * KS / 6; };
    // stores of a block issued after its last copy (a slot issues its copies first)
    constexpr int kAfter = [] {
      int n = 0;
      for (int i = 0; i < NS; ++i) n += (i * S / NS) >= ((G - 1) * S / G);
      return n;
    }();
    const int key = lane & 31;
    // store i of a finished tile: the latent bytes of rows 8w + 2i and 8w + 2i + 1 (i < 4; lanes
    // 32 * h .. 32 * h + 31 take row 8w + 2i + h, 16 bytes each), then tail slot lane % 8 of row
    // 8w + lane / 8
    auto st_read = [&](const char* gb, int i) {
      if (i < 4) return *reinterpret_cast<const u32x4*>(gb + (8 * wave + 2 * i + hb) * kGQPitch + 16 * key);
      return *reinterpret_cast<const u32x4*>(gb + rope_row * kGQPitch + 512 + 16 * (lane & 7));
    };
    auto st_issue = [&](const int32_t (&rpos)[8], int32_t rope_pos, int i, const u32x4& v) {
      if (i < 4) {
        const int32_t r = hb ? rpos[2 * i + 1] : rpos[2 * i];
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p.g_stage + (int64_t)r * kGRowBytesI8 + 16 * key));
      } else {
        __builtin_nontemporal_store(
            v, reinterpret_cast<u32x4*>(p.g_stage + (int64_t)rope_pos * kGRowBytesI8 + 512 + 16 * (lane & 7)));
      }
    };
    stage(0, 0);
    if (nblk > 1) stage(1, 1);
    for (int blk = 0; blk < nblk; ++blk) {
      // issue order as in the bf16 loop: block blk needs copies(blk); issued after them are block
      // blk - 2's last kAfter stores, block blk - 1's copies(blk + 1) and its NS stores
      if (blk + 1 >= nblk) wait_vmcnt<0>();
      else if (blk <= 1) wait_vmcnt<G>();
      else if (blk == 2) wait_vmcnt<G + NS>();
      else wait_vmcnt<G + NS + kAfter>();
      __syncthreads();
      const bool copy_next = blk + 2 < nblk;
      const bool store_prev = blk > 0;
      char* const gcur = sm.loop.gq[blk & 1][0];
      const char* const gprev = sm.loop.gq[(blk & 1) ^ 1][0];
      int32_t rpos[8], rope_pos = 0;
      u32x4 sdat = u32x4{0u, 0u, 0u, 0u};
      if (store_prev) {
#pragma unroll
        for (int i = 0; i < 8; ++i) rpos[i] = __builtin_amdgcn_readfirstlane(sm.pos[(blk - 1) * kBK + 8 * wave + i]);
        rope_pos = sm.pos[(blk - 1) * kBK + rope_row];
        sdat = st_read(gprev, 0);
      }
      const char* sd = sm.loop.st[blk % kStages][0] + b_off;
      const char* sp = sm.loop.st[blk % kStages][1] + b_off;
      u32x4 bs[KS], bp[KS];
      auto load_b = [&](int ks) {
        const u32x2 s_lo = lds_read_tr16(sd + ks * 1024), s_hi = lds_read_tr16(sd + ks * 1024 + 4 * 64);
        const u32x2 p_lo = lds_read_tr16(sp + ks * 1024), p_hi = lds_read_tr16(sp + ks * 1024 + 4 * 64);
        bs[ks] = u32x4{s_lo[0], s_lo[1], s_hi[0], s_hi[1]};
        bp[ks] = u32x4{p_lo[0], p_lo[1], p_hi[0], p_hi[1]};
      };
      load_b(0);
      if (KS > 1) load_b(1);
      // quantisation of a finished tile, in five pieces: |g| max of values 0-7, then of 8-15 and
      // the partner lane's (the group's scale and its reciprocal), codes of values 0-7, codes of
      // 8-15, then the codes (after a permlane32 swap lane k holds the group's bytes 0-15, lane
      // k + 32 bytes 16-31) and the scale into the LDS row of key k
      uint32_t qm = 0, qsb = 0, qdw[4] = {0u, 0u, 0u, 0u};
      float qinv = 0.f;
      auto quant = [&](const f32x16& a, int tq, int piece) {
        char* row = gcur + key * kGQPitch;
        const int gq = tq < 4 ? 4 * wave + tq : 16 + wave;
        if (piece == 0) {
          // absmax3's inline asm reads the accumulators (VGPRs in the int8 build) where the
          // compiler does not count the MFMA result's wait states: give them here
          mfma_acc_drain();
          qm = absmax_bits8(a, 0);
        } else if (piece == 1) {
          const uint32_t m = max(qm, absmax_bits8(a, 8));
          const auto sw = __builtin_amdgcn_permlane32_swap(m, m, false, false);
          qsb = i8_scale_bits(max((uint32_t)sw[0], (uint32_t)sw[1]));
          qinv = qsb ? __builtin_amdgcn_rcpf(__builtin_bit_cast(float, qsb << 16)) : 0.f;
        } else if (piece == 2) {
          qdw[0] = i8_pack4(a, 0, qinv);
          qdw[1] = i8_pack4(a, 4, qinv);
        } else if (piece == 3) {
          qdw[2] = i8_pack4(a, 8, qinv);
          qdw[3] = i8_pack4(a, 12, qinv);
        } else {
          const auto s0 = __builtin_amdgcn_permlane32_swap(qdw[0], qdw[2], false, false);
          const auto s1 = __builtin_amdgcn_permlane32_swap(qdw[1], qdw[3], false, false);
          if (tq < 4) {   // latent group gq: bytes 32*gq + 16*hb ..
            *reinterpret_cast<u32x4*>(row + 32 * gq + 16 * hb) = u32x4{s0[0], s0[1], s1[0], s1[1]};
          } else {        // rope dims 32w + 16*hb .. +15: tail slots 4w + 2*hb and 4w + 2*hb + 1
            *reinterpret_cast<u32x2*>(row + 512 + 16 * (4 * wave + 2 * hb)) = u32x2{s0[0], s0[1]};
            *reinterpret_cast<u32x2*>(row + 512 + 16 * (4 * wave + 2 * hb + 1)) = u32x2{s1[0], s1[1]};
          }
          *reinterpret_cast<uint16_t*>(row + 512 + 16 * (gq / 3) + 8 + 2 * (gq % 3)) = (uint16_t)qsb;
        }
      };
      f32x16 prev = f32x16{};
#pragma unroll
      for (int tq = 0; tq < NQ; ++tq) {
        f32x16 acc = f32x16{};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          acc = mfma32x32x16(as_bf16x8(qa[tq][ks]), as_bf16x8(bs[ks]), acc);
          if (tq < 4) acc = mfma32x32x16(as_bf16x8(va[tq][ks]), as_bf16x8(bp[ks]), acc);
          const int s = tq * KS + ks;
          if (tq == 0 && ks + 2 < KS) load_b(ks + 2);
          if (copy_next) {
#pragma unroll
            for (int c = 0; c < G; ++c)
              if (copy_slot(c) == s) stage_part((blk + 2) % kStages, blk + 2, c);
          }
          if (store_prev) {
#pragma unroll
            for (int i = 0; i < NS; ++i) {
              if (st_slot(i) == s) {
                st_issue(rpos, rope_pos, i, sdat);
                if (i + 1 < NS) sdat = st_read(gprev, i + 1);
              }
            }
          }
          if (tq > 0) {
#pragma unroll
            for (int piece = 0; piece < 5; ++piece)
              if (piece_ks(piece) == ks) quant(prev, tq - 1, piece);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        prev = acc;
      }
#pragma unroll
      for (int piece = 0; piece < 5; ++piece) quant(prev, NQ - 1, piece);
    }
    // the last block's rows
    __syncthreads();
    {
      const char* gb = sm.loop.gq[(nblk - 1) & 1][0];
      int32_t rpos[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) rpos[i] = __builtin_amdgcn_readfirstlane(sm.pos[(nblk - 1) * kBK + 8 * wave + i]);
      const int32_t rope_pos = sm.pos[(nblk - 1) * kBK + rope_row];
#pragma unroll
      for (int i = 0; i < NS; ++i) st_issue(rpos, rope_pos, i, st_read(gb, i));
    }
  };
  if constexpr (I8) {
    if (nq == 5) block_loop_i8(std::integral_constant<int, 5>{});
    else block_loop_i8(std::integral_constant<int, 4>{});
  } else if constexpr (ROPE) {
    if (nq == 5) block_loop(std::integral_constant<int, 5>{});
    else block_loop(std::integral_constant<int, 4>{});
  } else {
    block_loop(std::integral_constant<int, 4>{});
  }
}

}  // namespace dsa
