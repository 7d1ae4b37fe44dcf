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
//                      LDS reads, dS^T straight from the staging buffer).
//   B3 bwd_g_kernel    per query: G^T[576 x keys] = Q^T . dS + dO^T . P contracted over all 128
//                      heads (Q^T / dO^T held in registers), written as bf16 rows at the pair's
//                      key-major position.
//   B4 csr_*           key-major order of the selected pairs: count, scan, position.
//   B5 bwd_dkv_reduce  per key: fp32 sum of its contiguous G rows -> dKV.
#include "dsa_common.h"
#include "dsa_kernels.h"

namespace dsa {

namespace {

constexpr int kDqk = 576;
constexpr int kDv = 512;
constexpr int kChunks = kDqk / 8;
constexpr int kPitch = kChunks + 1;
constexpr int kBK = 32;
constexpr int kGatherInstr = (kBK * kPitch + 63) / 64;
constexpr int kBufBytes = kGatherInstr * 1024;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

DSA_DEV u32x2 lds_read_tr16(const char* p) {
  s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  return __builtin_bit_cast(u32x2, r);
}

DSA_DEV void gather_block(char* buf, const bf16_t* kv, int64_t kv_stride, int row_id_lane,
                          int wave, int nwaves, int lane) {
  for (int n = wave; n < kGatherInstr; n += nwaves) {
    const int p = n * 64 + lane;
    const int r = p / kPitch;
    const int c = p - r * kPitch;
    const int row = __shfl(row_id_lane, r & 31, 64);
    const bf16_t* src = kv;
    if (r < kBK && row >= 0 && c < kChunks) src = kv + (int64_t)row * kv_stride + c * 8;
    async_copy16(src, buf + n * 1024);
  }
}

// Number of 32-key blocks of a query row: up to its last valid index (same rule as the forward).
DSA_DEV int count_blocks(const int32_t* idx_row, int topk, int n_kv, int causal, int t, int lane) {
  int last = -1;
  for (int j = lane; j < topk; j += 64) {
    const int v = idx_row[j];
    if (v >= 0 && v < n_kv && (!causal || v <= t)) last = j;
  }
  last = wave_max_i(last);
  return (last + kBK) / kBK;
}

DSA_DEV int load_idx(const int32_t* idx_row, int blk, int nblk, int topk, int n_kv, int lane) {
  const int j = blk * kBK + (lane & 31);
  if (blk >= nblk || j >= topk) return -1;
  const int v = idx_row[j];
  return (v >= 0 && v < n_kv) ? v : -1;
}

}  // namespace

// ------------------------------------------------------------------------------------------
// B1: recompute P and dS; stage them.  One workgroup per query, wave = 32 heads.
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256, 1) void bwd_sp_kernel(SparseBwdParams p) {
  __shared__ __attribute__((aligned(16))) char smem[2 * kBufBytes];
  const int t = xcd_remap(blockIdx.x, p.total_q);
  if (t >= p.total_q) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int hb = lane >> 5, hl = lane & 31;
  const int head = blockIdx.y * 128 + wave * 32 + hl;
  const bool head_ok = head < p.n_heads;
  const int hsafe = head_ok ? head : 0;
  const int32_t* idx_row = p.idx + (int64_t)t * p.idx_stride;
  const int nblk = count_blocks(idx_row, p.topk, p.n_kv, p.causal, t, lane);

  // Q (576) and dO (512) fragments, d-contiguous: lane holds [16*ks + 8*hb, +8).
  u32x4 qf[kDqk / 16], df[kDv / 16];
  const bf16_t* qrow = p.q + (int64_t)t * p.q_stride_t + (int64_t)hsafe * kDqk + hb * 8;
  const bf16_t* drow = p.dout + (int64_t)t * p.dout_stride_t + (int64_t)hsafe * kDv + hb * 8;
  const bf16_t* orow = p.out + (int64_t)t * p.out_stride_t + (int64_t)hsafe * kDv + hb * 8;
#pragma unroll
  for (int ks = 0; ks < kDqk / 16; ++ks) {
    const u32x4 v = gload16(qrow + ks * 16);
    qf[ks] = head_ok ? v : u32x4{0, 0, 0, 0};
  }
  float delta = 0.f;
#pragma unroll
  for (int ks = 0; ks < kDv / 16; ++ks) {
    const u32x4 v = gload16(drow + ks * 16);
    const u32x4 o = gload16(orow + ks * 16);
    df[ks] = head_ok ? v : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      delta += bf16_lo(v[e]) * bf16_lo(o[e]) + bf16_hi(v[e]) * bf16_hi(o[e]);
  }
  delta = xor32_sum(delta);
  const float lse = head_ok ? p.lse[(int64_t)t * p.lse_stride_t + head] : -INFINITY;
  const float lse2 = lse * kLog2e;
  const bool row_live = lse != -INFINITY;

  const int64_t stage_off = ((int64_t)t * p.n_heads + hsafe) * p.topk_pad;
  bf16_t* ps_row = p.p_stage + stage_off;
  bf16_t* ds_row = p.ds_stage + stage_off;

  int idx_cur = load_idx(idx_row, 0, nblk, p.topk, p.n_kv, lane);
  int idx_nxt = load_idx(idx_row, 1, nblk, p.topk, p.n_kv, lane);
  if (nblk > 0) gather_block(smem, p.kv, p.kv_stride, idx_cur, wave, nwaves, lane);

  for (int blk = 0; blk < nblk; ++blk) {
    wait_vmcnt0();
    __syncthreads();
    if (blk + 1 < nblk)
      gather_block(smem + ((blk + 1) & 1) * kBufBytes, p.kv, p.kv_stride, idx_nxt, wave, nwaves, lane);
    const int idx_nn = load_idx(idx_row, blk + 2, nblk, p.topk, p.n_kv, lane);
    const char* buf = smem + (blk & 1) * kBufBytes;
    const bool kvalid = idx_cur >= 0 && (!p.causal || idx_cur <= t);
    const uint32_t vmask = (uint32_t)__ballot(kvalid);

    // S^T = K . Q^T and dP^T = V . dO^T share the A operand (V = K[:, :512]).
    f32x16 s = f32x16{}, dp = f32x16{};
    const char* a0 = buf + (hl * kPitch + hb) * 16;
#pragma unroll
    for (int ks = 0; ks < kDqk / 16; ++ks) {
      const bf16x8 a = as_bf16x8(lds_load16(a0 + ks * 32));
      s = mfma32x32x16(a, as_bf16x8(qf[ks]), s);
      if (ks < kDv / 16) dp = mfma32x32x16(a, as_bf16x8(df[ks]), dp);
      if ((ks & 3) == 3) __builtin_amdgcn_sched_barrier(0);
    }
    // P and scale * dS; key of element i = (i/4)*8 + 4*hb + i%4
    u32x2 pw[4], dw[4];
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      float pv[4], dv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 4 * q4 + e;
        const int key = q4 * 8 + hb * 4 + e;
        const bool ok = row_live && ((vmask >> key) & 1u);
        const float pp = ok ? fast_exp2(s[i] * p.scale_log2 - lse2) : 0.f;
        pv[e] = pp;
        dv[e] = p.scale * pp * (dp[i] - delta);
      }
      pw[q4] = u32x2{pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3])};
      dw[q4] = u32x2{pack_bf16x2(dv[0], dv[1]), pack_bf16x2(dv[2], dv[3])};
    }
    if (head_ok) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int j = blk * kBK + q4 * 8 + hb * 4;
        *reinterpret_cast<u32x2*>(ps_row + j) = pw[q4];
        *reinterpret_cast<u32x2*>(ds_row + j) = dw[q4];
      }
    }
    idx_cur = idx_nxt;
    idx_nxt = idx_nn;
  }
}

// ------------------------------------------------------------------------------------------
// B2: dQ^T[576 x 32 heads] = K^T . (scale*dS)^T per wave, over the query's gathered rows.
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256, 1) void bwd_dq_kernel(SparseBwdParams p) {
  __shared__ __attribute__((aligned(16))) char smem[2 * kBufBytes];
  const int t = xcd_remap(blockIdx.x, p.total_q);
  if (t >= p.total_q) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int hb = lane >> 5, hl = lane & 31;
  const int head = blockIdx.y * 128 + wave * 32 + hl;
  const bool head_ok = head < p.n_heads;
  const int hsafe = head_ok ? head : 0;
  const int32_t* idx_row = p.idx + (int64_t)t * p.idx_stride;
  const int nblk = count_blocks(idx_row, p.topk, p.n_kv, p.causal, t, lane);
  const bf16_t* ds_row = p.ds_stage + ((int64_t)t * p.n_heads + hsafe) * p.topk_pad + hb * 8;

  const int g = lane >> 4, gi = lane & 15;
  const int tr_key = 8 * (g >> 1) + (gi >> 2);     // natural key order: k-slot 8*hb + e
  const int tr_col = 16 * (g & 1) + 4 * (gi & 3);

  f32x16 acc[kDqk / 32];
#pragma unroll
  for (int m = 0; m < kDqk / 32; ++m) acc[m] = f32x16{};

  int idx_cur = load_idx(idx_row, 0, nblk, p.topk, p.n_kv, lane);
  int idx_nxt = load_idx(idx_row, 1, nblk, p.topk, p.n_kv, lane);
  if (nblk > 0) gather_block(smem, p.kv, p.kv_stride, idx_cur, wave, nwaves, lane);
  u32x4 dsv[2] = {u32x4{0, 0, 0, 0}, u32x4{0, 0, 0, 0}};
  if (nblk > 0) {
    dsv[0] = gload16(ds_row);
    dsv[1] = gload16(ds_row + 16);
  }

  for (int blk = 0; blk < nblk; ++blk) {
    wait_vmcnt0();
    __syncthreads();
    if (blk + 1 < nblk)
      gather_block(smem + ((blk + 1) & 1) * kBufBytes, p.kv, p.kv_stride, idx_nxt, wave, nwaves, lane);
    const int idx_nn = load_idx(idx_row, blk + 2, nblk, p.topk, p.n_kv, lane);
    u32x4 dsn[2] = {u32x4{0, 0, 0, 0}, u32x4{0, 0, 0, 0}};
    if (blk + 1 < nblk) {
      dsn[0] = gload16(ds_row + (blk + 1) * kBK);
      dsn[1] = gload16(ds_row + (blk + 1) * kBK + 16);
    }
    const char* buf = smem + (blk & 1) * kBufBytes;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const char* r0 = buf + ((16 * a + tr_key) * kPitch) * 16 + tr_col * 2;
      const char* r1 = r0 + 4 * kPitch * 16;
      const bf16x8 b = as_bf16x8(head_ok ? dsv[a] : u32x4{0, 0, 0, 0});
#pragma unroll
      for (int m = 0; m < kDqk / 32; ++m) {
        const u32x2 lo = lds_read_tr16(r0 + m * 64);
        const u32x2 hi = lds_read_tr16(r1 + m * 64);
        acc[m] = mfma32x32x16(as_bf16x8(u32x4{lo[0], lo[1], hi[0], hi[1]}), b, acc[m]);
        if ((m & 3) == 3) __builtin_amdgcn_sched_barrier(0);
      }
    }
    dsv[0] = dsn[0];
    dsv[1] = dsn[1];
    idx_cur = idx_nxt;
    idx_nxt = idx_nn;
  }
  if (!head_ok) return;
  bf16_t* dqrow = p.dq + (int64_t)t * p.dq_stride_t + (int64_t)head * kDqk;
#pragma unroll
  for (int m = 0; m < kDqk / 32; ++m) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = 32 * m + 8 * q4 + 4 * hb;
      *reinterpret_cast<u32x2*>(dqrow + d) =
          u32x2{pack_bf16x2(acc[m][4 * q4], acc[m][4 * q4 + 1]), pack_bf16x2(acc[m][4 * q4 + 2], acc[m][4 * q4 + 3])};
    }
  }
}

// ------------------------------------------------------------------------------------------
// B3: per-pair dKV partial rows G = (scale*dS)^T Q + P^T dO, contracted over all heads.
// Wave w owns output row tiles (32 latent dims each): Q part tiles kQT[w], dO part tiles kVT[w].
// ------------------------------------------------------------------------------------------
namespace {
constexpr int kHeads = 128;                         // B3 handles up to 128 heads (n_heads % 16 == 0)
constexpr int kKs = kHeads / 16;                    // up to 8 head k-steps
constexpr int kStagePitch = kBK * 2 + 16;           // bytes per head row of a staged 32-key tile (+pad)
constexpr int kTileBytes = kHeads * kStagePitch;    // one staged [128 heads][32 keys] bf16 tile
constexpr int kRowPitch = kDqk * 2 + 16;            // bytes per staged head row of Q / dO
}  // namespace

__global__ __launch_bounds__(256, 1) void bwd_g_kernel(SparseBwdParams p) {
  // LDS: staged Q / dO rows for the transposed register load (16 heads at a time), then the
  // double-buffered [dS | P] tiles of each key block.
  __shared__ __attribute__((aligned(16))) char smem[2 * kTileBytes + 16 * kRowPitch];
  const int t = xcd_remap(blockIdx.x, p.total_q);
  if (t >= p.total_q) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hb = lane >> 5;
  const int g = lane >> 4, gi = lane & 15;
  const int32_t* idx_row = p.idx + (int64_t)t * p.idx_stride;
  const int nblk = count_blocks(idx_row, p.topk, p.n_kv, p.causal, t, lane);
  if (nblk == 0) return;

  // tiles owned by this wave: Q part {4w..4w+3} (+16+w for w < 2), dO part {4w..4w+3}
  const int nq = wave < 2 ? 5 : 4;
  auto qtile = [&](int i) { return i < 4 ? 4 * wave + i : 16 + wave; };

  // ---- load Q^T and dO^T fragments (A operand: lane row = latent dim, k = 8 heads) via LDS
  u32x4 qa[5][kKs], va[4][kKs];
  char* rows = smem + 2 * kTileBytes;
  const int nks = p.n_heads / 16;
  const int tr_h = 8 * (g >> 1) + (gi >> 2);        // head row this lane feeds into ds_read_tr
  const int tr_c = 16 * (g & 1) + 4 * (gi & 3);     // latent column this lane feeds
  for (int ks = 0; ks < kKs; ++ks) {
    if (ks >= nks) {
#pragma unroll
      for (int i = 0; i < 5; ++i) qa[i][ks] = u32x4{0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < 4; ++i) va[i][ks] = u32x4{0, 0, 0, 0};
      continue;
    }
    for (int part = 0; part < 2; ++part) {
      const bf16_t* src = part == 0 ? p.q + (int64_t)t * p.q_stride_t : p.dout + (int64_t)t * p.dout_stride_t;
      const int width = part == 0 ? kDqk : kDv;
      __syncthreads();
      for (int c = threadIdx.x; c < 16 * (width / 8); c += blockDim.x) {
        const int r = c / (width / 8), cc = c - r * (width / 8);
        lds_store16(rows + r * kRowPitch + cc * 16, gload16(src + (int64_t)(16 * ks + r) * width + cc * 8));
      }
      __syncthreads();
      if (part == 0) {
#pragma unroll
        for (int i = 0; i < 5; ++i) {
          if (i < nq) {
            const char* r0 = rows + tr_h * kRowPitch + (32 * qtile(i) + tr_c) * 2;
            const u32x2 lo = lds_read_tr16(r0), hi = lds_read_tr16(r0 + 4 * kRowPitch);
            qa[i][ks] = u32x4{lo[0], lo[1], hi[0], hi[1]};
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const char* r0 = rows + tr_h * kRowPitch + (32 * (4 * wave + i) + tr_c) * 2;
          const u32x2 lo = lds_read_tr16(r0), hi = lds_read_tr16(r0 + 4 * kRowPitch);
          va[i][ks] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
      }
    }
  }

  // ---- key blocks: stage [dS | P] tiles (rows = heads, 32 keys each) with LDS-direct copies
  const int64_t st_base = (int64_t)t * p.n_heads * p.topk_pad;
  auto stage = [&](int blk, char* dst) {
    // 2 tiles x 128 rows x 64 B = 256 x 64 B pieces; lane c copies piece c (4 x 16 B each)
    for (int c = threadIdx.x; c < 2 * p.n_heads * 4; c += blockDim.x) {
      const int tile = c / (p.n_heads * 4), r = (c / 4) % p.n_heads, q = c & 3;
      const bf16_t* src = (tile == 0 ? p.ds_stage : p.p_stage) + st_base + (int64_t)r * p.topk_pad + blk * kBK + q * 8;
      lds_store16(dst + tile * kTileBytes + r * kStagePitch + q * 16, gload16(src));
    }
  };
  const int64_t* pos_row = p.pair_pos + (int64_t)t * p.topk;
  for (int blk = 0; blk < nblk; ++blk) {
    __syncthreads();
    stage(blk, smem);
    __syncthreads();
    f32x16 acc[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) acc[i] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < kKs; ++ks) {
      if (ks >= nks) break;
      // B operands: dS / P [k = 8 heads][n = key]; lane key = lane % 32
      const char* b0 = smem + (16 * ks + tr_h) * kStagePitch + tr_c * 2;
      const u32x2 s_lo = lds_read_tr16(b0), s_hi = lds_read_tr16(b0 + 4 * kStagePitch);
      const u32x2 p_lo = lds_read_tr16(b0 + kTileBytes), p_hi = lds_read_tr16(b0 + kTileBytes + 4 * kStagePitch);
      const bf16x8 bs = as_bf16x8(u32x4{s_lo[0], s_lo[1], s_hi[0], s_hi[1]});
      const bf16x8 bp = as_bf16x8(u32x4{p_lo[0], p_lo[1], p_hi[0], p_hi[1]});
#pragma unroll
      for (int i = 0; i < 5; ++i) {
        if (i < nq) acc[i] = mfma32x32x16(as_bf16x8(qa[i][ks]), bs, acc[i]);
        if (i < 4) acc[i] = mfma32x32x16(as_bf16x8(va[i][ks]), bp, acc[i]);
      }
    }
    // write G rows (bf16) for the valid keys of this block; lane key = lane % 32
    const int j = blk * kBK + (lane & 31);
    const int64_t pos = j < p.topk ? pos_row[j] : -1;
    if (pos >= 0) {
      bf16_t* grow = p.g_stage + pos * kDqk;
#pragma unroll
      for (int i = 0; i < 5; ++i) {
        if (i < nq) {
          const int d0 = 32 * qtile(i);
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const int d = d0 + 8 * q4 + 4 * hb;
            *reinterpret_cast<u32x2*>(grow + d) =
                u32x2{pack_bf16x2(acc[i][4 * q4], acc[i][4 * q4 + 1]), pack_bf16x2(acc[i][4 * q4 + 2], acc[i][4 * q4 + 3])};
          }
        }
      }
    }
  }
}

// Zero fill (a kernel, not hipMemsetAsync, so the sequence stays safe under graph capture).
__global__ void zero_i32_kernel(int32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// ------------------------------------------------------------------------------------------
// B4: key-major order of the selected (query, slot) pairs.
// ------------------------------------------------------------------------------------------
__global__ void csr_count_kernel(const int32_t* idx, int64_t idx_stride, int total_q, int topk, int n_kv,
                                 int causal, int32_t* counts) {
  const int64_t n = (int64_t)total_q * topk;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int t = (int)(e / topk), j = (int)(e - (int64_t)t * topk);
    const int v = idx[(int64_t)t * idx_stride + j];
    if (v >= 0 && v < n_kv && (!causal || v <= t)) atomicAdd(counts + v, 1);
  }
}

// Single-workgroup exclusive scan of counts[n] -> offsets[n+1] (int64), cursor[] zeroed.
__global__ __launch_bounds__(1024) void csr_scan_kernel(const int32_t* counts, int n, int64_t* offsets, int32_t* cursor) {
  __shared__ int64_t part[1024];
  const int tid = threadIdx.x;
  const int per = (n + 1023) / 1024;
  const int a = min(n, tid * per), b = min(n, a + per);
  int64_t s = 0;
  for (int i = a; i < b; ++i) s += counts[i];
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
    run += counts[i];
    cursor[i] = 0;
  }
  if (tid == 1023) offsets[n] = part[1023];
}

// Position of every pair inside its key's segment (one integer atomic per pair claims a slot).
// Slot order inside a segment follows scheduling, and B5 sums a segment in slot order, so dKV
// can differ in the last fp32 bits between runs (bounded by a test).
__global__ void csr_fill_kernel(const int32_t* idx, int64_t idx_stride, int total_q, int topk, int n_kv,
                                int causal, const int64_t* offsets, int32_t* cursor, int64_t* pair_pos) {
  const int64_t n = (int64_t)total_q * topk;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int t = (int)(e / topk), j = (int)(e - (int64_t)t * topk);
    const int v = idx[(int64_t)t * idx_stride + j];
    int64_t pos = -1;
    if (v >= 0 && v < n_kv && (!causal || v <= t)) pos = offsets[v] + atomicAdd(cursor + v, 1);
    pair_pos[e] = pos;
  }
}

// ------------------------------------------------------------------------------------------
// B5: dKV[s] = sum of G rows in s's segment (fp32).  One workgroup (288 threads) per key:
// 4 row lanes x 72 chunks of 8 dims.
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(288) void bwd_dkv_reduce_kernel(const bf16_t* g_stage, const int64_t* offsets,
                                                             int n_kv, float* dkv, int64_t dkv_stride) {
  __shared__ float red[3][kDqk];
  const int s = blockIdx.x;
  if (s >= n_kv) return;
  const int c = threadIdx.x % kChunks, r = threadIdx.x / kChunks;
  const int64_t a = offsets[s], b = offsets[s + 1];
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t i = a + r; i < b; i += 4) {
    const u32x4 v = gload16(g_stage + i * kDqk + c * 8);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[2 * e] += bf16_lo(v[e]);
      acc[2 * e + 1] += bf16_hi(v[e]);
    }
  }
  if (r > 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[r - 1][c * 8 + e] = acc[e];
  }
  __syncthreads();
  if (r == 0) {
    float* out = dkv + (int64_t)s * dkv_stride + c * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = acc[e] + red[0][c * 8 + e] + red[1][c * 8 + e] + red[2][c * 8 + e];
  }
}

int launch_sparse_mla_bwd(const SparseBwdParams& p, hipStream_t stream) {
  const int nwaves = p.n_heads >= 128 ? 4 : (p.n_heads + 31) / 32;
  const dim3 grid(((p.total_q + 7) / 8) * 8, (p.n_heads + 127) / 128);
  // B4 first: it only depends on idx.
  hipLaunchKernelGGL(zero_i32_kernel, dim3((p.n_kv + 255) / 256), dim3(256), 0, stream, p.csr_counts, p.n_kv);
  const int64_t pairs = (int64_t)p.total_q * p.topk;
  const int nb = (int)std::min<int64_t>((pairs + 255) / 256, 65536);
  hipLaunchKernelGGL(csr_count_kernel, dim3(nb), dim3(256), 0, stream, p.idx, p.idx_stride, p.total_q, p.topk,
                     p.n_kv, p.causal, p.csr_counts);
  hipLaunchKernelGGL(csr_scan_kernel, dim3(1), dim3(1024), 0, stream, p.csr_counts, p.n_kv, p.csr_offsets, p.csr_counts);
  hipLaunchKernelGGL(csr_fill_kernel, dim3(nb), dim3(256), 0, stream, p.idx, p.idx_stride, p.total_q, p.topk,
                     p.n_kv, p.causal, p.csr_offsets, p.csr_counts, p.pair_pos);
  hipLaunchKernelGGL(bwd_sp_kernel, grid, dim3(64 * nwaves), 0, stream, p);
  hipLaunchKernelGGL(bwd_dq_kernel, grid, dim3(64 * nwaves), 0, stream, p);
  hipLaunchKernelGGL(bwd_g_kernel, dim3(((p.total_q + 7) / 8) * 8), dim3(256), 0, stream, p);
  hipLaunchKernelGGL(bwd_dkv_reduce_kernel, dim3(p.n_kv), dim3(288), 0, stream, p.g_stage, p.csr_offsets, p.n_kv,
                     p.dkv, p.dkv_stride);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace dsa
