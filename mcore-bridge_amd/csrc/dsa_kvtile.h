// LDS tile of 32 gathered latent KV rows (576 bf16 each) and its gather, shared by the sparse
// MLA forward and backward kernels (gfx950).
//
// Layout (37,376 B per tile; tiles are 128-byte aligned):
//   V region    32 rows x 1040 B: latent dims 0..511 of one key in natural order + 16 B pad.
//               Key k of the block lives in row key_row(k) = (k & ~7) | ((k & 3) << 1) | ((k >> 2) & 1).
//   rope region [32 keys][8 chunks of 16 B] (dims 512..575); chunk c of key k sits at slot
//               c ^ ((k >> 1) & 7).
// LDS serves 8 lanes of a ds_read_b128 (16 lanes of a ds_read_b64_tr_b16) per clock from 32
// four-byte banks (measured on MI355X).  The 1040-byte pitch puts 8 consecutive rows on 8
// different 16-byte bank groups, so the QK operand read (8 consecutive lanes = 8 consecutive
// keys, one 16-byte chunk each) is conflict free; key_row() places the 4 consecutive keys of
// one 16-lane group of a transposing PV / dQ read on rows 2 apart (4 x 32 B, distinct banks).
// Every V operand address is a per-lane base plus an immediate offset -- no per-access XOR.
//
// Gather: one wave instruction (global_load_lds_dwordx4, 64 lanes x 16 B) fills one V row:
// the KV row address is wave-uniform (two readlanes into an SGPR pair) and lane i copies
// chunk i to row base + 16*i.  4 more instructions fill the rope region (8 keys x 8 chunks
// each).  36 instructions per tile, split evenly over 1, 2 or 4 waves.  The copies are issued
// through inline asm: the caller completes them with s_waitcnt vmcnt + a barrier.
#pragma once
#include "dsa_common.h"

namespace dsa {

constexpr int kTileKeys = 32;
constexpr int kTileVPitch = 1040;
constexpr int kTileVBytes = 32 * kTileVPitch;               // 33,280
constexpr int kTileRopeBytes = 32 * 128;
constexpr int kTileBytes = kTileVBytes + kTileRopeBytes;    // 37,376 = 292 * 128
constexpr int kTileInstr = 36;
constexpr int kLatent = 576;

// V row of block key k (0..31).
DSA_DEV constexpr uint32_t key_row(uint32_t k) { return (k & ~7u) | ((k & 3u) << 1) | ((k >> 2) & 1u); }

// Byte offset of (key k, 16-byte chunk c) inside a tile (c in 0..71).
DSA_DEV uint32_t tile_off(uint32_t k, uint32_t c) {
  return c < 64 ? key_row(k) * kTileVPitch + 16u * c : kTileVBytes + k * 128u + 16u * ((c - 64) ^ ((k >> 1) & 7u));
}

// Copies issued per wave per tile.  ROPE = false: 512-wide score rows (q without a rope part),
// which never read the rope region, so only the 32 V rows are gathered.
template <int NW, bool ROPE = true>
constexpr int tile_copies_per_wave() {
  static_assert(NW == 1 || NW == 2 || NW == 4, "1, 2 or 4 waves");
  return (ROPE ? kTileInstr : kTileKeys) / NW;
}

// Per-lane gather sources of one wave for one block, from the block's 32 KV row ids in LDS
// (idx_blk[k], -1 = no key: row 0 is loaded and the caller masks it).
//   v     lane j < 32/NW: KV row address of key w + NW*j (its V copy is copy j)
//   rope  [j]: this lane's 16 source bytes of rope group w + NW*j (keys 8*group + lane/8)
template <int NW>
struct TileSrc {
  const char* v;
  const char* rope[4 / NW];
};

DSA_DEV const char* kv_row_addr(const bf16_t* kv, int row) {
  return reinterpret_cast<const char*>(kv) + (int64_t)(row >= 0 ? row : 0) * (kLatent * 2);
}

template <int NW, bool ROPE = true>
DSA_DEV TileSrc<NW> tile_sources(const bf16_t* kv, const int32_t* idx_blk, int wave, int lane) {
  TileSrc<NW> s;
  s.v = kv_row_addr(kv, idx_blk[wave + NW * (lane % (32 / NW))]);
  if constexpr (ROPE) {
#pragma unroll
    for (int j = 0; j < 4 / NW; ++j) {
      const int key = 8 * (wave + NW * j) + (lane >> 3);
      const uint32_t c = (uint32_t)(lane & 7) ^ ((key >> 1) & 7u);
      s.rope[j] = kv_row_addr(kv, idx_blk[key]) + (64 + c) * 16;
    }
  }
  return s;
}

// global_load_lds_dwordx4 with a scalar 64-bit row address and a per-lane byte offset.  M0 is
// written right before the LDS DMA, which reads it one wait state later (s_nop 0).  The row
// address comes from v_readlane, a VALU write of the SGPRs the DMA reads: that needs 5 wait
// states, which the compiler cannot see inside the asm -- callers read a row (gather_row) at
// least one copy slot before issuing it, in an earlier scheduling group (tests/test_codegen.py
// checks the distance in the generated code).
DSA_DEV void copy_row16(uint32_t lds_wave_base, const char* row, uint32_t lane_off) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_wave_base), "v"(lane_off), "s"(row)
               : "memory", "m0");
}

// Scalar source row of copy k of this wave's share of a tile gather (V copies, k < 32/NW: two
// readlanes; rope copies use per-lane addresses and need none).
template <int NW>
DSA_DEV const char* gather_row(const TileSrc<NW>& src, int k) {
  if (k >= 32 / NW) return nullptr;
  const uint64_t a = (uint64_t)src.v;
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)a, k);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(a >> 32), k);
  return reinterpret_cast<const char*>(((uint64_t)hi << 32) | lo);
}

// Copy k (0 <= k < tile_copies_per_wave<NW>()) of this wave's share of a tile gather into the
// tile at LDS byte address `tile`; `row` = gather_row(src, k), read earlier.  Copies
// 0 .. 32/NW-1 fill the V rows of keys w + NW*k (row key_row(w + NW*k) = key_row(NW*k) + 2w),
// the rest fill rope groups.
template <int NW>
DSA_DEV void gather_issue(uint32_t tile, const TileSrc<NW>& src, const char* row, int wave, int lane, int k) {
  const uint32_t w = (uint32_t)__builtin_amdgcn_readfirstlane(wave);
  if (k < 32 / NW) {
    copy_row16(tile + (key_row(NW * k) + 2 * w) * kTileVPitch, row, (uint32_t)lane * 16u);
  } else {
    const int j = k - 32 / NW;
    async_copy16_unordered(src.rope[j], tile + kTileVBytes + (w + NW * j) * 1024u);
  }
}

// LDS byte addresses of this wave's share of one tile (wave-uniform): v = the V row of key w
// (key_row(w) = 2w), rope = its first rope group.  Computed once per tile, so each copy sets M0
// with a single s_add_u32 of a compile-time offset.
struct TileDst {
  uint32_t v, rope;
};
template <int NW>
DSA_DEV TileDst tile_dst(uint32_t tile, uint32_t wsg) {
  return TileDst{tile + 2u * wsg * kTileVPitch, tile + kTileVBytes + wsg * 1024u};
}

// copy_row16 with M0 = base + OFF (one SALU instruction; the LDS DMA reads M0 one wait state
// later: s_nop 0).
template <uint32_t OFF>
DSA_DEV void copy_row16_at(uint32_t base, const char* row, uint32_t lane_off) {
  asm volatile("s_add_u32 m0, %0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, %3" ::"s"(base), "i"(OFF),
               "v"(lane_off), "s"(row)
               : "memory", "m0", "scc");
}
template <uint32_t OFF>
DSA_DEV void copy16_at(const void* gsrc, uint32_t base) {
  asm volatile("s_add_u32 m0, %0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, off" ::"s"(base), "i"(OFF), "v"(gsrc)
               : "memory", "m0", "scc");
}

// gather_issue with the wave's TileDst: M0 = an SGPR base plus a constant once k is one (the
// callers' unrolled loops), no per-copy readfirstlane.
template <int NW>
DSA_DEV void gather_issue_dst(const TileDst& d, const TileSrc<NW>& src, const char* row, int lane, int k) {
  if (k < 32 / NW) {
    copy_row16(d.v + key_row(NW * k) * kTileVPitch, row, (uint32_t)lane * 16u);
  } else {
    const int j = k - 32 / NW;
    async_copy16_unordered(src.rope[j], d.rope + NW * j * 1024u);
  }
}

// gather_issue for a compile-time copy index K with the wave's TileDst.
template <int NW, int K>
DSA_DEV void gather_issue_at(const TileDst& d, const TileSrc<NW>& src, const char* row, int lane) {
  if constexpr (K < 32 / NW) {
    copy_row16_at<key_row(NW * K) * kTileVPitch>(d.v, row, (uint32_t)lane * 16u);
  } else {
    constexpr int j = K - 32 / NW;
    copy16_at<NW * j * 1024u>(src.rope[j], d.rope);
  }
}

// The whole gather of one tile (all of this wave's copies back to back; rows read two copies
// ahead, the first two behind one explicit 5-wait-state pad).
template <int NW, bool ROPE = true>
DSA_DEV void gather_tile(uint32_t tile, const bf16_t* kv, const int32_t* idx_blk, int wave, int lane) {
  constexpr int n = tile_copies_per_wave<NW, ROPE>();
  const TileSrc<NW> src = tile_sources<NW, ROPE>(kv, idx_blk, wave, lane);
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

// Stage the query's index row in LDS (invalid -> -1); returns the number of 32-key blocks up
// to the last valid entry (workgroup-uniform).  Also retires every outstanding load.
template <int NW>
DSA_DEV int stage_index_row(int32_t* idx_s, int* red, const int32_t* idx_row, int topk, int n_kv, int causal,
                            int t) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kpad = (topk + kTileKeys - 1) / kTileKeys * kTileKeys;
  constexpr int kBatch = 8;   // loads in flight per thread (one memory round trip per batch)
  int last = -1;
  for (int j0 = threadIdx.x; j0 < kpad; j0 += kBatch * NW * 64) {
    int v[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int j = j0 + i * NW * 64;
      v[i] = j < topk ? idx_row[j] : -1;
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int j = j0 + i * NW * 64;
      int x = v[i];
      if (x < 0 || x >= n_kv || (causal && x > t)) x = -1;
      if (j < kpad) {
        idx_s[j] = x;
        if (x >= 0) last = j;
      }
    }
  }
  last = wave_max_i(last);
  if (lane == 0) red[wave] = last;
  wait_vmcnt0();
  __syncthreads();
#pragma unroll
  for (int w = 0; w < NW; ++w) last = max(last, red[w]);
  return __builtin_amdgcn_readfirstlane((last + kTileKeys) / kTileKeys);
}

}  // namespace dsa
