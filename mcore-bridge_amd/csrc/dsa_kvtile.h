// LDS tile of 32 gathered latent KV rows (576 bf16 each) and its gather, shared by the sparse
// MLA forward and backward kernels (gfx950).
//
// Layout (36 KB per tile):
//   V region    [32 rows][64 chunks of 16 B]  (latent dims 0..511), 1 KB per row.  Chunk c of
//               row r sits at slot c ^ swz(r), swz(r) = (4r + r/4) & 63.
//   rope region [32 rows][8 chunks of 16 B]   (dims 512..575).  Chunk c of row r sits at slot
//               c ^ ((r >> 1) & 7).
// The swizzles make both access patterns of the kernels bank-conflict free: 16 lanes reading
// the same chunk of 16 consecutive rows (QK operand, ds_read_b128), and 32 lanes reading 4
// rows x 4 neighbouring chunks in 8-byte halves (ds_read_b64_tr_b16 operands of PV / dQ).
//
// Gather: one wave instruction (global_load_lds_dwordx4, 64 lanes x 16 B) fills one V row --
// the row id is wave-uniform (readlane), the address is SGPR base + per-lane offset and the
// 64 lanes read one contiguous 1 KB row in swizzled order; 4 more instructions fill the rope
// region (8 rows x 8 chunks each).  36 instructions per tile, split evenly over 1, 2 or 4
// waves.  The copies are issued through inline asm (see async_copy16_unordered): the caller
// completes them with s_waitcnt vmcnt + a barrier.
#pragma once
#include "dsa_common.h"

namespace dsa {

constexpr int kTileKeys = 32;
constexpr int kTileVBytes = 32 * 1024;
constexpr int kTileRopeBytes = 32 * 128;
constexpr int kTileBytes = kTileVBytes + kTileRopeBytes;   // 36864
constexpr int kTileInstr = 36;
constexpr int kLatent = 576;

DSA_DEV uint32_t kv_swz(uint32_t r) { return ((4u * r) + (r >> 2)) & 63u; }

// Byte offset of (row r, chunk c) inside a tile (c in 0..71).
DSA_DEV uint32_t tile_off(uint32_t r, uint32_t c) {
  return c < 64 ? r * 1024u + 16u * (c ^ kv_swz(r)) : kTileVBytes + r * 128u + 16u * ((c - 64) ^ ((r >> 1) & 7u));
}

// global_load_lds_dwordx4 with a scalar 64-bit base and a per-lane 32-bit byte offset.
DSA_DEV void async_copy16_sv(const void* sbase, uint32_t voff, uint32_t lds_wave_base) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_wave_base), "v"(voff), "s"(sbase)
               : "memory", "m0");
}

// Copies issued per wave per tile.
template <int NW>
constexpr int tile_copies_per_wave() {
  static_assert(NW == 1 || NW == 2 || NW == 4, "1, 2 or 4 waves");
  return kTileInstr / NW;
}

// Gather the 32 rows whose ids lane l%32 holds in `row_of_lane` (-1 = none: row 0 is loaded
// and the caller masks it) into `tile`.
template <int NW>
DSA_DEV void gather_tile(char* tile, int row_of_lane, const bf16_t* kv, int wave, int lane) {
  const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(tile));
  const int w = __builtin_amdgcn_readfirstlane(wave);
  const char* kvb = reinterpret_cast<const char*>(kv);
#pragma unroll
  for (int k = 0; k < 32 / NW; ++k) {
    const int r = w + k * NW;
    const int row = __builtin_amdgcn_readlane(row_of_lane, r);
    const char* src = kvb + (int64_t)(row >= 0 ? row : 0) * (kLatent * 2);
    async_copy16_sv(src, (uint32_t)(lane ^ kv_swz(r)) * 16u, base + r * 1024u);
  }
#pragma unroll
  for (int j = 0; j < 4; j += NW) {
    const int jj = j + w;
    if (NW == 4 || jj < 4) {
      const int r = 8 * jj + (lane >> 3);
      const int row = __shfl(row_of_lane, r, 64);
      const uint32_t c = (uint32_t)(lane & 7) ^ ((r >> 1) & 7u);
      const char* src = kvb + (int64_t)(row >= 0 ? row : 0) * (kLatent * 2) + (64 + c) * 16;
      async_copy16_unordered(src, base + kTileVBytes + jj * 1024u);
    }
  }
}

}  // namespace dsa
