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
// One workgroup per token, one wave per 128-dim row (the token's q rows and its k row); lane l
// holds dims 2l, 2l+1.  The token's cos/sin are computed once into LDS; each row is read once,
// transformed in registers (RoPE operands and Hadamard butterflies move between lanes) and
// written once: the kernel is bound by HBM (2 bytes in, 2 or 1 out per dim).
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

// Transform of one 128-dim row held as (x0, x1) = dims (2l, 2l+1) of lane l: RoPE on dims
// [0, 64) with the token's bf16 cos/sin from LDS, then the Hadamard rotation; returns the
// bf16-rounded result in (x0, x1).
DSA_DEV void rope_hadamard(float& x0, float& x1, const float* cs, const float* sn, int lane, int deinterleave,
                           int rotary_interleaved) {
  // output j takes u(j) and the rotate_half partner sign * u(jr), u = x or its de-interleave
  // (u(j) = x[2j], u(32 + j) = x[2j + 1]); every lane runs the shuffles, lanes 0..31 own
  // outputs 2l, 2l+1
  float y[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int j = (2 * lane + e) & (kRot - 1);
    const int jr = rotary_interleaved ? (j ^ 1) : ((j + kRot / 2) & (kRot - 1));
    const float sg = rotary_interleaved ? ((j & 1) ? 1.f : -1.f) : (j < kRot / 2 ? -1.f : 1.f);
    const int sj = deinterleave ? (j < kRot / 2 ? 2 * j : 2 * (j - kRot / 2) + 1) : j;
    const int sr = deinterleave ? (jr < kRot / 2 ? 2 * jr : 2 * (jr - kRot / 2) + 1) : jr;
    const float u = fetch(x0, x1, sj), ur = sg * fetch(x0, x1, sr);
    y[e] = round_bf16(round_bf16(u * cs[j]) + round_bf16(ur * sn[j]));
  }
  if (lane < kRot / 2) {
    x0 = y[0];
    x1 = y[1];
  }
  // normalised Walsh-Hadamard transform, natural order: stride 1 inside the lane, strides
  // 2..64 between lanes l and l ^ (stride / 2)
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
  x0 = round_bf16(x0 * kNorm);
  x1 = round_bf16(x1 * kNorm);
}

// bf16 pair, or e4m3fn pair + the row's absmax scale (scale = amax / 448, 1 for a zero row;
// x / scale clamped to +-448, RNE)
DSA_DEV void store_row(float x0, float x1, void* out, float* scale_out, int64_t row, int lane, int fp8) {
  if (!fp8) {
    bf16_t* dst = reinterpret_cast<bf16_t*>(out) + row * kDi;
    *reinterpret_cast<uint32_t*>(dst + 2 * lane) = pack_bf16x2(x0, x1);
  } else {
    const float amax = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
    const float scale = amax > 0.f ? amax / 448.f : 1.f;
    const float q0 = fminf(fmaxf(x0 / scale, -448.f), 448.f), q1 = fminf(fmaxf(x1 / scale, -448.f), 448.f);
    uint8_t* dst = reinterpret_cast<uint8_t*>(out) + row * kDi;
    *reinterpret_cast<uint16_t*>(dst + 2 * lane) = (uint16_t)pack_e4m3x2(q0, q1);
    if (lane == 0) scale_out[row] = scale;
  }
}

// One workgroup per token: its 64 cos/sin values are computed once (wave 0) into LDS, then the
// four waves share the token's n_heads q rows and its k row (LayerNorm first; that wave also
// scales the head weights).
__global__ __launch_bounds__(256) void indexer_prologue_kernel(PrologueParams p) {
  __shared__ float cs[kRot], sn[kRot];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x;
  if (wave == 0) {
    const float f = p.freqs[(int64_t)t * p.freqs_stride_t + lane];
    cs[lane] = round_bf16(cosf(f) * p.mscale);
    sn[lane] = round_bf16(sinf(f) * p.mscale);
  }
  __syncthreads();
  // rows r = 0 .. n_heads: q head r, or (r = n_heads) the k row; wave w takes r = w, w + 4, ..
  // (at most kRowsPerWave), all of its loads issued before the first row is transformed
  constexpr int kRowsPerWave = (64 + 1 + 3) / 4;
  uint32_t pr[kRowsPerWave];
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const int r = wave + 4 * i;
    pr[i] = 0;
    if (r <= p.n_heads) {
      const bf16_t* src = r == p.n_heads ? p.k_lin + (int64_t)t * p.k_stride_t
                                         : p.q_lin + (int64_t)t * p.q_stride_t + (int64_t)r * kDi;
      pr[i] = *reinterpret_cast<const uint32_t*>(src + 2 * lane);
    }
  }
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const int r = wave + 4 * i;
    if (r > p.n_heads) break;
    const bool is_k = r == p.n_heads;
    float x0 = bf16_lo(pr[i]), x1 = bf16_hi(pr[i]);
    if (is_k) {
      // k_norm: fp32 LayerNorm over the row, output rounded to bf16
      const float mean = wave_sum(x0 + x1) * (1.f / kDi);
      const float d0 = x0 - mean, d1 = x1 - mean;
      const float rstd = 1.f / sqrtf(wave_sum(d0 * d0 + d1 * d1) * (1.f / kDi) + p.eps);
      x0 = round_bf16(d0 * rstd * p.ln_w[2 * lane] + p.ln_b[2 * lane]);
      x1 = round_bf16(d1 * rstd * p.ln_w[2 * lane + 1] + p.ln_b[2 * lane + 1]);
      // head weights: w * Hi^-0.5, then * Di^-0.5, each rounded to bf16
      if (lane < p.n_heads) {
        const float w = (float)p.w_lin[(int64_t)t * p.w_stride_t + lane];
        p.w_out[(int64_t)t * p.n_heads + lane] = round_bf16(round_bf16(w * p.w_scale_heads) * p.w_scale_softmax);
      }
    }
    rope_hadamard(x0, x1, cs, sn, lane, p.deinterleave, p.rotary_interleaved);
    if (is_k) store_row(x0, x1, p.k_out, p.k_scale, t, lane, p.out_fp8);
    else store_row(x0, x1, p.q_out, p.q_scale, (int64_t)t * p.n_heads + r, lane, p.out_fp8);
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
