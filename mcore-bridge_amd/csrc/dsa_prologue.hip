// K0: lightning-indexer prologue (gfx950) -- everything between the indexer's three
// projections and the scores, fused into one pass over the projected rows.
//
// Replaces the tail of DSAIndexer.forward_before_topk (reference src/mcore_bridge/patcher.py:
// 268-300) with its RoPE helper _apply_rope (patcher.py:304-324) and the patched
// _apply_rotary_pos_emb_bshd (src/mcore_bridge/model/modules/transformer_layer.py:240-278):
//   k      = LayerNorm(k_lin) with bias                        (patcher.py:281-282)
//   x_pe   = RoPE(first Di - 64 dims), x_nope passes through    (patcher.py:307-324)
//            optional de-interleave of x_pe (dsa_indexer_rotary_interleaved), half-split or
//            interleaved rotate_half (config.rotary_interleaved), cos/sin * mscale rounded to
//            bf16, every product and the sum rounded to bf16 as the reference's bf16 ops do
//   q, k   = rotate_activation = normalised 128-point Walsh-Hadamard transform (:292-293)
//   w      = weights * Hi^-0.5 * Di^-0.5, two bf16 roundings    (patcher.py:299-300)
// and optionally quantises q and k to OCP e4m3fn with one absmax scale per 128-dim row (the
// fp8 input layout of the indexer scores kernel).  The three projections are plain GEMMs and
// stay with hipBLASLt.
//
// One workgroup per token; 16 lanes per 128-dim row (the token's q rows and its k row), 4 rows
// per wave.  The token's cos/sin are computed once into LDS; each row is read once, transformed
// in registers (Hadamard butterflies and RoPE partners move between lanes by DPP) and written
// once: the kernel is bound by HBM (2 bytes in, 2 or 1 out per dim).
#include "dsa_common.h"
#include "dsa_kernels.h"

namespace dsa {

namespace {

constexpr int kDi = 128;    // indexer head dim
constexpr int kRot = 64;    // RoPE dims (the first kDi - kRot dims of the row)

DSA_DEV float round_bf16(float x) { return (float)(bf16_t)x; }

// element i (0..127) of the row held as (x0, x1) = dims (2l, 2l+1) by lane l
DSA_DEV float fetch(float x0, float x1, int i) {
  const float a = __shfl(x0, i >> 1, 64), b = __shfl(x1, i >> 1, 64);
  return (i & 1) ? b : a;
}

// e4m3fn byte of a value already clamped to [-448, 448] (hardware RNE conversion)
DSA_DEV uint32_t pack_e4m3x2(float a, float b) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}

}  // namespace

// ---- forward: 16-lane row groups.  Lane L = lane & 15 of group g = lane >> 4 holds dims
// 4L..4L+3 (h = 0: the RoPE dims) and 64 + 4L..+3 (h = 1) of one 128-dim row, so a wave
// transforms 4 rows at once.  Dim index bits 0-1 and 6 are in-lane, bits 2-5 are the lane bits:
// the Hadamard's four cross-lane butterfly stages and the half-split RoPE partner (lane ^ 8)
// are DPP operations inside 16-lane rows, at VALU rate and with no trip through the LDS crossbar
// (the previous one-row-per-wave layout needed 16 dependent ds_bpermute per row).  After the
// transform lane L holds chunk hadamard_chunk(L) of the output row (dims 4C.., 64 + 4C..).
// (all rows and banks enabled and every source lane inside the row: no lane keeps an old value)
template <int CTRL>
DSA_DEV float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
constexpr int kDppXor1 = 0xB1;         // quad_perm [1, 0, 3, 2]: lane i <- i ^ 1
constexpr int kDppXor2 = 0x4E;         // quad_perm [2, 3, 0, 1]: lane i <- i ^ 2
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror: lane i <- 7 - i in its half row of 8 (i ^ 7)
constexpr int kDppRor8 = 0x128;        // row_ror:8: lane i <- (i + 8) mod 16 in its row (i ^ 8)

// Sum / max over the 16 lanes of a group: butterflies on lane masks 7, 1, 2, 8 (together they
// span the 4 lane bits; each is one DPP move, which the compiler folds into the add / max).  A
// pair of lanes computes a + b and b + a, so every lane ends with the same value.
DSA_DEV float group_sum(float v) {
  v += dpp_mov<kDppHalfMirror>(v);
  v += dpp_mov<kDppXor1>(v);
  v += dpp_mov<kDppXor2>(v);
  return v + dpp_mov<kDppRor8>(v);
}
// Largest of non-negative values (|x|): their bit patterns order as unsigned integers, so each
// step is one v_max_u32 with a DPP source (a float max would first quiet NaNs with an extra
// v_max per step).
template <int CTRL>
DSA_DEV uint32_t dpp_mov_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}
DSA_DEV float group_max_nonneg(float x) {
  uint32_t v = __builtin_bit_cast(uint32_t, x);
  v = max(v, dpp_mov_u<kDppHalfMirror>(v));
  v = max(v, dpp_mov_u<kDppXor1>(v));
  v = max(v, dpp_mov_u<kDppXor2>(v));
  return __builtin_bit_cast(float, max(v, dpp_mov_u<kDppRor8>(v)));
}

// The Hadamard's 16-point transform over the lane bits as four butterfly stages on lane masks
// 7, 1, 2, 8 (pivot bits 2, 0, 1, 3), each one v_fmac_f32 per value with the partner's value
// as a DPP source: x <- x + c * x[partner], c = -1 on the lane whose pivot bit is set.  That
// lane holds the negated butterfly difference (x[partner] - x rounds to the exact negation), so
// lane L ends with sigma(L) * (H16 y)[hadamard_chunk(L)] where sigma = hadamard_sign(L): the
// caller scales by sigma and stores lane L's values at chunk hadamard_chunk(L).  (Masks 4 and
// 8 as XORs would need two DPP moves each; 7 and 8 need one.)  The leading s_nop covers the
// DPP-read hazards of the asm block (VALU write -> DPP read of the same VGPR: 2 wait states;
// EXEC write -> DPP: 5); inside the block each value is re-read 8 instructions after its
// write, and the trailing s_nop gives a DPP read of the block's results after it its 2 wait
// states.  Every lane of the wave executes it (no divergence at the call sites).
DSA_DEV void hadamard_lanes(float (&v)[2][4], int L) {
  const float c0 = (L & 4) ? -1.f : 1.f, c1 = (L & 1) ? -1.f : 1.f;
  const float c2 = (L & 2) ? -1.f : 1.f, c3 = (L & 8) ? -1.f : 1.f;
#define DSA_FMAC_DPP(ctrl, c)                                                     \
  "v_fmac_f32_dpp %0, %0, " c " " ctrl " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t" \
  "v_fmac_f32_dpp %1, %1, " c " " ctrl " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t" \
  "v_fmac_f32_dpp %2, %2, " c " " ctrl " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t" \
  "v_fmac_f32_dpp %3, %3, " c " " ctrl " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t" \
  "v_fmac_f32_dpp %4, %4, " c " " ctrl " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t" \
  "v_fmac_f32_dpp %5, %5, " c " " ctrl " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t" \
  "v_fmac_f32_dpp %6, %6, " c " " ctrl " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t" \
  "v_fmac_f32_dpp %7, %7, " c " " ctrl " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
  asm("s_nop 4\n\t"
      DSA_FMAC_DPP("row_half_mirror", "%8")
      DSA_FMAC_DPP("quad_perm:[1,0,3,2]", "%9")
      DSA_FMAC_DPP("quad_perm:[2,3,0,1]", "%10")
      DSA_FMAC_DPP("row_ror:8", "%11")
      "s_nop 1"
      : "+v"(v[0][0]), "+v"(v[0][1]), "+v"(v[0][2]), "+v"(v[0][3]),
        "+v"(v[1][0]), "+v"(v[1][1]), "+v"(v[1][2]), "+v"(v[1][3])
      : "v"(c0), "v"(c1), "v"(c2), "v"(c3));
#undef DSA_FMAC_DPP
}
// chunk of the natural-order transform that lane L holds after hadamard_lanes: L with bit 2
// flipped where bits 0 and 1 differ
DSA_DEV int hadamard_chunk(int L) { return L ^ (((L ^ (L >> 1)) & 1) << 2); }
// its sign: the signed permutation of the mask-7 stage (-1 on lanes 5, 6, 13, 14) times the
// parity of L (one negation per pivot bit set)
DSA_DEV float hadamard_sign(int L) {
  const int neg = (((L ^ (L >> 1)) & (L >> 2)) ^ __builtin_popcount(L)) & 1;
  return neg ? -1.f : 1.f;
}

// RoPE on the h = 0 values (bf16-exact inputs; u = the row or its de-interleave), then the
// normalised natural-order Walsh-Hadamard transform over all 128 dims (fp32; the caller rounds
// to bf16); lane L ends with output dims 4C..4C+3 and 64 + 4C..+3, C = hadamard_chunk(L).
// cs, sn: the token's bf16 cos / sin * mscale of this lane's RoPE dims 4L..4L+3.
DSA_DEV void rope_hadamard_group(float (&v)[2][4], const float (&cs)[4], const float (&sn)[4], int lane,
                                 int deinterleave, int rotary_interleaved) {
  const int L = lane & 15;
  float u[4];
  if (deinterleave) {
    // u(j) = x[2j] (j < 32), x[2(j - 32) + 1] (j >= 32): the 4 values of lane L come from the
    // even (L < 8) or odd (L >= 8) halves of the two words of lanes 2 (L & 7) and 2 (L & 7) + 1
    const int w0 = (int)pack_bf16x2(v[0][0], v[0][1]), w1 = (int)pack_bf16x2(v[0][2], v[0][3]);
    const int src = 4 * ((lane & 48) + 2 * (L & 7));
    const uint32_t a0 = __builtin_amdgcn_ds_bpermute(src, w0), a1 = __builtin_amdgcn_ds_bpermute(src, w1);
    const uint32_t b0 = __builtin_amdgcn_ds_bpermute(src + 4, w0), b1 = __builtin_amdgcn_ds_bpermute(src + 4, w1);
    const bool odd = L >= 8;
    u[0] = odd ? bf16_hi(a0) : bf16_lo(a0);
    u[1] = odd ? bf16_hi(a1) : bf16_lo(a1);
    u[2] = odd ? bf16_hi(b0) : bf16_lo(b0);
    u[3] = odd ? bf16_hi(b1) : bf16_lo(b1);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) u[e] = v[0][e];
  }
  // rotate_half partner u(jr) and the sign of dim j = 4L + e
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float ur, sg;
    if (rotary_interleaved) {
      ur = u[e ^ 1];
      sg = (e & 1) ? 1.f : -1.f;
    } else {
      ur = dpp_mov<kDppRor8>(u[e]);   // lane L ^ 8: dim j + 32 or j - 32
      sg = L < 8 ? -1.f : 1.f;
    }
    v[0][e] = round_bf16(round_bf16(u[e] * cs[e]) + round_bf16(sg * ur * sn[e]));
  }
  // Hadamard: in-lane bits 0, 1 and 6, then lane bits 0-3
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float a = v[h][0] + v[h][1], b = v[h][0] - v[h][1];
    const float c = v[h][2] + v[h][3], d = v[h][2] - v[h][3];
    v[h][0] = a + c;
    v[h][1] = b + d;
    v[h][2] = a - c;
    v[h][3] = b - d;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float a = v[0][e] + v[1][e], b = v[0][e] - v[1][e];
    v[0][e] = a;
    v[1][e] = b;
  }
  hadamard_lanes(v, L);
  const float norm = hadamard_sign(L) * 0.08838834764831845f;   // +-128^-0.5
  // v * norm + 0: an exact zero (a zero row, a cancelled sum) leaves as +0 on the lanes with
  // norm < 0 too, as in the natural-order transform
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 4; ++e) v[h][e] = fmaf(v[h][e], norm, 0.f);
}

// One row of a group (fp32 values, rounded to bf16 here): bf16, or e4m3fn of the bf16 values
// + the row's absmax scale (scale = amax / 448, 1 for a
// zero row; x / scale clamped to +-448, RNE).  Every lane of the wave takes part (group
// reductions); only lanes of a valid row store.  The lane's values are output chunk C (dims
// 4C..4C+3 and 64 + 4C..+3).
DSA_DEV void store_group_row(float (&v)[2][4], void* out, float* scale_out, int64_t row, bool valid, int L,
                             int C, int fp8) {
  if (!fp8) {   // the packing conversion is the bf16 rounding (RNE)
    if (!valid) return;
    uint32_t* dst = reinterpret_cast<uint32_t*>(reinterpret_cast<bf16_t*>(out) + row * kDi);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      dst[32 * h + 2 * C] = pack_bf16x2(v[h][0], v[h][1]);
      dst[32 * h + 2 * C + 1] = pack_bf16x2(v[h][2], v[h][3]);
    }
    return;
  }
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
      const uint32_t w = pack_bf16x2(v[h][e], v[h][e + 1]);
      v[h][e] = bf16_lo(w);
      v[h][e + 1] = bf16_hi(w);
    }
  float m = 0.f;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 4; ++e) m = fmaxf(m, fabsf(v[h][e]));
  const float amax = group_max_nonneg(m);
  if (!valid) return;
  // scale = RN(amax / 448) and rcp = RN(1 / scale) without IEEE division sequences: amax times
  // RN(1/448) plus one exact-remainder correction is the correctly rounded quotient, and one fma
  // Newton step from v_rcp_f32 (within 1 ulp) the correctly rounded reciprocal.  Both hold for
  // every positive bf16 amax >= 2^-100 (checked exhaustively on the host with exact arithmetic,
  // reciprocal seeds up to 1 ulp off); smaller rows take the division.
  float scale, rcp;
  if (amax >= 0x1p-100f) {
    constexpr float kInv448 = 1.f / 448.f;
    const float s0 = amax * kInv448;
    scale = fmaf(fmaf(-s0, 448.f, amax), kInv448, s0);
    const float y0 = __builtin_amdgcn_rcpf(scale);
    rcp = fmaf(fmaf(-scale, y0, 1.f), y0, y0);
  } else {
    scale = amax > 0.f ? amax / 448.f : 1.f;
    rcp = 1.f / scale;
  }
  // x / scale correctly rounded from the correctly rounded reciprocal plus one exact-remainder
  // correction (Markstein): the remainder x - q0 * scale is exact in an fma, and
  // q0 + rem * (1 / scale) rounds to the nearest quotient -- for |x| >= 2^-100 and normal
  // quotients; below that the remainder underflows and the result may be an ulp off.
  uint32_t* dst = reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(out) + row * kDi);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float q[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float q0 = v[h][e] * rcp;
      const float qc = fmaf(fmaf(-q0, scale, v[h][e]), rcp, q0);
      q[e] = fminf(fmaxf(qc, -448.f), 448.f);
    }
    const uint32_t lo = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
    dst[16 * h + C] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], (int)lo, true);
  }
  if (L == 0) scale_out[row] = scale;
}

// One workgroup per token: every wave issues the loads of its rows, then wave 0 computes the
// token's 64 cos/sin values into LDS and scales the head weights; the token's n_heads q rows
// and its k row (row n_heads, LayerNorm first) are taken 4 at a time, wave w taking row quads
// w, w + 4, ..
__global__ __launch_bounds__(256) void indexer_prologue_kernel(PrologueParams p) {
  __shared__ __attribute__((aligned(16))) float cs_s[kRot], sn_s[kRot];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 4, L = lane & 15;
  const int t = blockIdx.x;
  // all loads of this wave's rows first: 4 words per lane and row (dims 4L.., 64 + 4L..)
  constexpr int kMaxQuads = (64 + 1 + 15) / 16;   // row quads per wave
  const int n_rows = p.n_heads + 1, n_quads = (n_rows + 3) / 4;
  uint32_t w[kMaxQuads][4];
#pragma unroll
  for (int i = 0; i < kMaxQuads; ++i) {
    const int quad = wave + 4 * i, r = 4 * quad + g;
#pragma unroll
    for (int k = 0; k < 4; ++k) w[i][k] = 0;
    if (quad < n_quads && r < n_rows) {
      const bf16_t* src = r == p.n_heads ? p.k_lin + (int64_t)t * p.k_stride_t
                                         : p.q_lin + (int64_t)t * p.q_stride_t + (int64_t)r * kDi;
      const uint32_t* s32 = reinterpret_cast<const uint32_t*>(src);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        w[i][2 * h] = s32[32 * h + 2 * L];
        w[i][2 * h + 1] = s32[32 * h + 2 * L + 1];
      }
    }
  }
  if (wave == 0) {   // under the row loads: the token's cos / sin and head weights
    const float f = p.freqs[(int64_t)t * p.freqs_stride_t + lane];
    cs_s[lane] = round_bf16(cosf(f) * p.mscale);
    sn_s[lane] = round_bf16(sinf(f) * p.mscale);
    if (lane < p.n_heads) {   // head weights: w * Hi^-0.5, then * Di^-0.5, each rounded to bf16
      const float w = (float)p.w_lin[(int64_t)t * p.w_stride_t + lane];
      p.w_out[(int64_t)t * p.n_heads + lane] = round_bf16(round_bf16(w * p.w_scale_heads) * p.w_scale_softmax);
    }
  }
  __syncthreads();
  float cs[4], sn[4];
  {
    const f32x4 c4 = *reinterpret_cast<const f32x4*>(cs_s + 4 * L), s4 = *reinterpret_cast<const f32x4*>(sn_s + 4 * L);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      cs[e] = c4[e];
      sn[e] = s4[e];
    }
  }
#pragma unroll
  for (int i = 0; i < kMaxQuads; ++i) {
    const int quad = wave + 4 * i;
    if (quad >= n_quads) break;
    const int r = 4 * quad + g;
    const bool valid = r < n_rows, is_k = r == p.n_heads;
    float v[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      v[h][0] = bf16_lo(w[i][2 * h]);
      v[h][1] = bf16_hi(w[i][2 * h]);
      v[h][2] = bf16_lo(w[i][2 * h + 1]);
      v[h][3] = bf16_hi(w[i][2 * h + 1]);
    }
    if (quad == p.n_heads / 4) {
      // the quad with the k row: k_norm (fp32 LayerNorm over the row, output rounded to bf16),
      // computed by every group, kept by the k row's
      float s = 0.f;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) s += v[h][e];
      const float mean = group_sum(s) * (1.f / kDi);
      float d[2][4], s2 = 0.f;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          d[h][e] = v[h][e] - mean;
          s2 += d[h][e] * d[h][e];
        }
      const float rstd = 1.f / sqrtf(group_sum(s2) * (1.f / kDi) + p.eps);
      if (is_k) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int dim = 64 * h + 4 * L + e;
            v[h][e] = round_bf16(d[h][e] * rstd * p.ln_w[dim] + p.ln_b[dim]);
          }
      }
    }
    rope_hadamard_group(v, cs, sn, lane, p.deinterleave, p.rotary_interleaved);
    const int C = hadamard_chunk(L);
    if (is_k) store_group_row(v, p.k_out, p.k_scale, t, valid, L, C, p.out_fp8);
    else store_group_row(v, p.q_out, p.q_scale, (int64_t)t * p.n_heads + r, valid, L, C, p.out_fp8);
  }
}

// Backward of the prologue (the bf16 roundings of the forward pass the gradient through, as the
// chain rule of the exact operations): per row, dy = H dz / sqrt(128) (the normalised Hadamard
// matrix is symmetric and orthogonal), then the transpose of the RoPE rotation, du_j =
// dy_j cs_j + sg_{jr(j)} dy_{jr(j)} sn_{jr(j)} (jr = the rotate_half partner, an involution), then
// the transpose of the de-interleave; the k row continues through the LayerNorm backward
// (per-token dgamma, dbeta rows, summed over tokens by a second kernel), and dw_lin =
// dw * w_scale_heads * w_scale_softmax.
DSA_DEV void rope_hadamard_bwd(float& x0, float& x1, const float* cs, const float* sn, int lane, int deinterleave,
                               int rotary_interleaved) {
  const float a = x0 + x1, b = x0 - x1;
  x0 = a;
  x1 = b;
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const float p0 = __shfl_xor(x0, m, 64), p1 = __shfl_xor(x1, m, 64);
    const bool hi = lane & m;
    x0 = hi ? p0 - x0 : x0 + p0;
    x1 = hi ? p1 - x1 : x1 + p1;
  }
  constexpr float kNorm = 0.08838834764831845f;   // 128^-0.5
  x0 *= kNorm;
  x1 *= kNorm;
  // du_j for j = 2l, 2l+1 (lanes 0..31 hold the RoPE dims)
  float du[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int j = (2 * lane + e) & (kRot - 1);
    const int jr = rotary_interleaved ? (j ^ 1) : ((j + kRot / 2) & (kRot - 1));
    const float sgr = rotary_interleaved ? ((jr & 1) ? 1.f : -1.f) : (jr < kRot / 2 ? -1.f : 1.f);
    du[e] = fetch(x0, x1, j) * cs[j] + sgr * fetch(x0, x1, jr) * sn[jr];
  }
  // dx[i] = du[src^-1(i)]: with de-interleave, dx[2l] = du[l] and dx[2l+1] = du[32 + l]
  const float g0 = deinterleave ? fetch(du[0], du[1], lane & 31) : du[0];
  const float g1 = deinterleave ? fetch(du[0], du[1], 32 + (lane & 31)) : du[1];
  if (lane < kRot / 2) {
    x0 = g0;
    x1 = g1;
  }
}

__global__ __launch_bounds__(256) void indexer_prologue_bwd_kernel(PrologueBwdParams p) {
  __shared__ float cs[kRot], sn[kRot];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x;
  if (wave == 0) {
    const float f = p.freqs[(int64_t)t * p.freqs_stride_t + lane];
    cs[lane] = round_bf16(cosf(f) * p.mscale);
    sn[lane] = round_bf16(sinf(f) * p.mscale);
  }
  __syncthreads();
  constexpr int kRowsPerWave = (64 + 1 + 3) / 4;
  float2 g[kRowsPerWave];
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const int r = wave + 4 * i;
    g[i] = float2{0.f, 0.f};
    if (r <= p.n_heads) {
      const float* src = r == p.n_heads ? p.dk + (int64_t)t * kDi : p.dq + ((int64_t)t * p.n_heads + r) * kDi;
      g[i] = *reinterpret_cast<const float2*>(src + 2 * lane);
    }
  }
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const int r = wave + 4 * i;
    if (r > p.n_heads) break;
    float x0 = g[i].x, x1 = g[i].y;
    rope_hadamard_bwd(x0, x1, cs, sn, lane, p.deinterleave, p.rotary_interleaved);
    if (r < p.n_heads) {
      bf16_t* dst = p.dq_lin + (int64_t)t * p.dq_lin_stride_t + (int64_t)r * kDi;
      *reinterpret_cast<uint32_t*>(dst + 2 * lane) = pack_bf16x2(x0, x1);
      continue;
    }
    // k row: LayerNorm backward (statistics recomputed in fp32 as in the forward)
    const uint32_t kv = *reinterpret_cast<const uint32_t*>(p.k_lin + (int64_t)t * p.k_stride_t + 2 * lane);
    const float k0 = bf16_lo(kv), k1 = bf16_hi(kv);
    const float mean = wave_sum(k0 + k1) * (1.f / kDi);
    const float d0 = k0 - mean, d1 = k1 - mean;
    const float rstd = 1.f / sqrtf(wave_sum(d0 * d0 + d1 * d1) * (1.f / kDi) + p.eps);
    const float h0 = d0 * rstd, h1 = d1 * rstd;
    float* part = p.dln_part + (int64_t)t * 2 * kDi;
    *reinterpret_cast<float2*>(part + 2 * lane) = float2{x0 * h0, x1 * h1};
    *reinterpret_cast<float2*>(part + kDi + 2 * lane) = float2{x0, x1};
    const float e0 = x0 * p.ln_w[2 * lane], e1 = x1 * p.ln_w[2 * lane + 1];
    const float me = wave_sum(e0 + e1) * (1.f / kDi);
    const float mh = wave_sum(e0 * h0 + e1 * h1) * (1.f / kDi);
    const float o0 = rstd * (e0 - me - h0 * mh), o1 = rstd * (e1 - me - h1 * mh);
    *reinterpret_cast<uint32_t*>(p.dk_lin + (int64_t)t * p.dk_lin_stride_t + 2 * lane) = pack_bf16x2(o0, o1);
    if (lane < p.n_heads) {
      const float dwv = p.dw[(int64_t)t * p.n_heads + lane];
      p.dw_lin[(int64_t)t * p.dw_lin_stride_t + lane] = (bf16_t)(dwv * p.w_scale_heads * p.w_scale_softmax);
    }
  }
}

// dgamma, dbeta = column sums of the per-token rows [T, 256]: kColParts workgroups sum strided
// row sets, one workgroup adds their partials (fixed order: deterministic).
constexpr int kColParts = 64;
__global__ __launch_bounds__(256) void ln_col_partial_kernel(const float* part, int rows, float* out) {
  float s = 0.f;
  for (int r = blockIdx.x; r < rows; r += kColParts) s += part[(int64_t)r * 256 + threadIdx.x];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}
__global__ __launch_bounds__(256) void ln_col_final_kernel(const float* part2, float* dw, float* db) {
  float s = 0.f;
  for (int b = 0; b < kColParts; ++b) s += part2[b * 256 + threadIdx.x];
  if (threadIdx.x < kDi) dw[threadIdx.x] = s;
  else db[threadIdx.x - kDi] = s;
}

int launch_indexer_prologue_bwd(const PrologueBwdParams& p, hipStream_t stream) {
  if (p.total_q > 0)
    hipLaunchKernelGGL(indexer_prologue_bwd_kernel, dim3(p.total_q), dim3(256), 0, stream, p);
  float* part2 = p.dln_part + (int64_t)p.total_q * 2 * kDi;
  hipLaunchKernelGGL(ln_col_partial_kernel, dim3(kColParts), dim3(256), 0, stream, p.dln_part, p.total_q, part2);
  hipLaunchKernelGGL(ln_col_final_kernel, dim3(1), dim3(256), 0, stream, part2, p.dln_w, p.dln_b);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_indexer_prologue(const PrologueParams& p, hipStream_t stream) {
  if (p.total_q == 0) return 0;
  hipLaunchKernelGGL(indexer_prologue_kernel, dim3(p.total_q), dim3(256), 0, stream, p);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace dsa
