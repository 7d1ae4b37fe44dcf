// K3: index-gathered sparse MLA attention forward over the shared 576-wide latent KV (gfx950).
//
// Replaces the un-fused sparse attention that Megatron's DSAttention runs on the indexer's
// top-k (called from reference src/mcore_bridge/model/modules/multi_latent_attention.py:262-270):
//   out[t,h] = sum_{j: idx[t,j] valid} softmax_j(scale * q[t,h] . kv[idx[t,j]]) * kv[idx[t,j], :512]
//   lse[t,h] = ln sum_j exp(scale * q[t,h] . kv[idx[t,j]])
//
// Work decomposition (one workgroup = one query token, up to 128 heads):
//   * wave w owns 32 heads.  Q[32 heads x 576] sits in registers for the whole key loop (the B
//     operand of S^T = K . Q^T, 144 VGPRs), the output accumulator O^T[512 x 32 heads] in fp32
//     (256 registers, AGPR-backed).  Keeping O transposed puts all accumulators of one lane on a
//     single head, so the online-softmax rescale needs no cross-lane traffic.
//   * selected KV rows are gathered 32 at a time straight into LDS with global_load_lds (16 B per
//     lane, no VGPR staging), double buffered: row pitch 73 x 16 B (one pad chunk) makes the
//     32-row column reads of the QK product bank-conflict free.
//   * QK: 36 MFMA 32x32x16 per 32-key block; PV: O^T += V^T . P^T, where the V^T operand comes
//     from ds_read_b64_tr_b16 (hardware 16-bit transpose on the LDS read) and P^T is the S^T
//     accumulator converted to bf16 in place (the k order inside each MFMA is permuted to
//     match the S^T C layout, so no shuffle is needed).
//   * softmax in the exp2 domain against a per-head reference max fixed by the first valid
//     block (2^64 headroom), so the O accumulators are never rescaled (a rescale would pull the
//     256 AGPR accumulators through VGPRs).  A query whose scores overshoot the headroom is
//     recomputed once with its exact row max.
#include "dsa_common.h"
#include "dsa_kernels.h"

namespace dsa {

namespace {

constexpr int kDqk = 576;
constexpr int kDv = 512;
constexpr int kChunks = kDqk / 8;       // 72 16-byte chunks per latent row
constexpr int kPitch = kChunks + 1;     // LDS row pitch in chunks (pad = bank-conflict free)
constexpr int kBK = 32;                 // keys per block (lane l%32 holds the index of key l%32)
constexpr int kGatherInstr = (kBK * kPitch + 63) / 64;   // 37 wave-instructions per block
constexpr int kBufBytes = kGatherInstr * 1024;
constexpr float kHeadroom = 64.0f;      // log2 headroom above the reference max

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

DSA_DEV u32x2 lds_read_tr16(const char* p) {
  s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  return __builtin_bit_cast(u32x2, r);
}

// Issue the LDS-direct gather of one 32-key block.  Slot p (16 B) of the buffer holds
// row p / 73, chunk p % 73 (chunk 72 is the pad; slots past the last row are filler).
// Wave-instruction n covers slots 64n..64n+63.
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

}  // namespace

__global__ __launch_bounds__(256, 1) void sparse_mla_fwd_kernel(SparseFwdParams p) {
  __shared__ __attribute__((aligned(16))) char smem[2 * kBufBytes];

  const int t = xcd_remap(blockIdx.x, p.total_q);
  if (t >= p.total_q) return;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int hb = lane >> 5;          // row half of the MFMA C layout
  const int hl = lane & 31;          // head within the wave
  const int head = blockIdx.y * 128 + wave * 32 + hl;
  const bool head_ok = head < p.n_heads;
  const int32_t* idx_row = p.idx + (int64_t)t * p.idx_stride;

  // ---- number of key blocks: up to the last valid index of the row
  int last = -1;
  for (int j = lane; j < p.topk; j += 64) {
    const int v = idx_row[j];
    if (v >= 0 && v < p.n_kv && (!p.causal || v <= t)) last = j;
  }
  last = wave_max_i(last);
  const int nblk = (last + kBK) / kBK;

  // ---- Q fragments: lane holds q[t, head, 16*ks + 8*hb .. +7] for ks = 0..35
  u32x4 qf[kDqk / 16];
  {
    const bf16_t* qrow = p.q + (int64_t)t * p.q_stride_t + (int64_t)(head_ok ? head : 0) * kDqk + hb * 8;
#pragma unroll
    for (int ks = 0; ks < kDqk / 16; ++ks) {
      u32x4 v = gload16(qrow + ks * 16);
      qf[ks] = head_ok ? v : u32x4{0, 0, 0, 0};
    }
  }

  f32x16 o[kDv / 32];
  // Softmax reference: m_ref (log2 units of scale*s) is the max of the first block that has a
  // valid key for this head; later blocks are taken relative to it with 2^kHeadroom of
  // headroom, so O never needs rescaling.  If any score overshoots the headroom the whole query
  // is recomputed once with the exact row max (m_seen), which cannot overshoot.
  float m_ref = -INFINITY;
  float m_seen = -INFINITY;
  float l_run = 0.f;
  __shared__ int redo_flag;

  const int g = lane >> 4;  // 16-lane group (ds_read_tr operand rows)
  const int gi = lane & 15;
  const int tr_key = 4 * (g >> 1) + (gi >> 2);       // key row this lane feeds into ds_read_tr
  const int tr_dv = 16 * (g & 1) + 4 * (gi & 3);     // dv column this lane feeds into ds_read_tr

  auto load_idx = [&](int blk) -> int {
    const int j = blk * kBK + (lane & 31);
    if (blk >= nblk || j >= p.topk) return -1;
    const int v = idx_row[j];
    return (v >= 0 && v < p.n_kv) ? v : -1;
  };

  for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
    for (int m = 0; m < kDv / 32; ++m) o[m] = f32x16{};
    l_run = 0.f;
    int idx_cur = load_idx(0);
    int idx_nxt = load_idx(1);
    if (nblk > 0) gather_block(smem, p.kv, p.kv_stride, idx_cur, wave, nwaves, lane);

    for (int blk = 0; blk < nblk; ++blk) {
      wait_vmcnt0();
      __syncthreads();
      if (blk + 1 < nblk)
        gather_block(smem + ((blk + 1) & 1) * kBufBytes, p.kv, p.kv_stride, idx_nxt, wave, nwaves, lane);
      const int idx_nn = load_idx(blk + 2);
      const char* buf = smem + (blk & 1) * kBufBytes;

      const bool kvalid = idx_cur >= 0 && (!p.causal || idx_cur <= t);
      const uint32_t vmask = (uint32_t)__ballot(kvalid);

      // ---- S^T[32 keys x 32 heads] = K . Q^T
      f32x16 s = f32x16{};
      {
        const char* a0 = buf + (hl * kPitch + hb) * 16;
#pragma unroll
        for (int ks = 0; ks < kDqk / 16; ++ks) {
          s = mfma32x32x16(as_bf16x8(lds_load16(a0 + ks * 32)), as_bf16x8(qf[ks]), s);
          if ((ks & 3) == 3) __builtin_amdgcn_sched_barrier(0);
        }
      }

      // ---- softmax numerator; key of s[i] = (i/4)*8 + 4*hb + i%4
#pragma unroll
      for (int i = 0; i < 16; ++i) s[i] *= p.scale_log2;
      if (vmask != 0xffffffffu) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = (i >> 2) * 8 + hb * 4 + (i & 3);
          if (!((vmask >> key) & 1u)) s[i] = -INFINITY;
        }
      }
      float bmax = s[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) bmax = fmaxf(bmax, s[i]);
      bmax = xor32_max(bmax);
      m_seen = fmaxf(m_seen, bmax);
      if (m_ref == -INFINITY) m_ref = bmax;          // O and l are still zero for this head
      const float m_use = (m_ref == -INFINITY) ? 0.f : m_ref;
      float rs = 0.f;
      u32x4 pb[2];
#pragma unroll
      for (int a = 0; a < 2; ++a) {
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const float p0 = fast_exp2(fminf(s[a * 8 + e] - m_use, kHeadroom));
          const float p1 = fast_exp2(fminf(s[a * 8 + e + 1] - m_use, kHeadroom));
          rs += p0 + p1;
          pb[a][e >> 1] = pack_bf16x2(p0, p1);
        }
      }
      l_run += xor32_sum(rs);

      // ---- O^T[512 x 32 heads] += V^T . P^T   (V^T via transposing LDS reads)
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int kb = 16 * a + tr_key;
        const char* r0 = buf + (kb * kPitch) * 16 + tr_dv * 2;
        const char* r1 = r0 + 8 * kPitch * 16;
        const bf16x8 b = as_bf16x8(pb[a]);
#pragma unroll
        for (int m = 0; m < kDv / 32; ++m) {
          const u32x2 lo = lds_read_tr16(r0 + m * 64);
          const u32x2 hi = lds_read_tr16(r1 + m * 64);
          const u32x4 av = {lo[0], lo[1], hi[0], hi[1]};
          o[m] = mfma32x32x16(as_bf16x8(av), b, o[m]);
          if ((m & 3) == 3) __builtin_amdgcn_sched_barrier(0);
        }
      }
      idx_cur = idx_nxt;
      idx_nxt = idx_nn;
    }
    // ---- did any head overshoot its reference?  (workgroup-uniform decision)
    const bool over = m_seen > m_ref + kHeadroom;
    if (threadIdx.x == 0) redo_flag = 0;
    __syncthreads();
    if (__any(over) && lane == 0) redo_flag = 1;
    __syncthreads();
    if (!redo_flag) break;
    m_ref = m_seen;
  }

  // ---- epilogue: normalise, store O (bf16) and LSE (natural log)
  if (!head_ok) return;
  const float inv_l = l_run > 0.f ? 1.f / l_run : 0.f;
  bf16_t* orow = p.out + (int64_t)t * p.out_stride_t + (int64_t)head * kDv;
#pragma unroll
  for (int m = 0; m < kDv / 32; ++m) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int dv = 32 * m + 8 * q4 + 4 * hb;
      u32x2 v;
      v[0] = pack_bf16x2(o[m][4 * q4 + 0] * inv_l, o[m][4 * q4 + 1] * inv_l);
      v[1] = pack_bf16x2(o[m][4 * q4 + 2] * inv_l, o[m][4 * q4 + 3] * inv_l);
      *reinterpret_cast<u32x2*>(orow + dv) = v;
    }
  }
  if (hb == 0) {
    const float m_use = (m_ref == -INFINITY) ? 0.f : m_ref;
    p.lse[(int64_t)t * p.lse_stride_t + head] = l_run > 0.f ? (m_use + __log2f(l_run)) * kLn2 : -INFINITY;
  }
}

int launch_sparse_mla_fwd(const SparseFwdParams& p, hipStream_t stream) {
  const int nwaves = p.n_heads >= 128 ? 4 : (p.n_heads + 31) / 32;
  dim3 grid(((p.total_q + 7) / 8) * 8, (p.n_heads + 127) / 128);
  hipLaunchKernelGGL(sparse_mla_fwd_kernel, grid, dim3(64 * nwaves), 0, stream, p);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace dsa
