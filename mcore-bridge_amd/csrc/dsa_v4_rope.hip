// DeepSeek-V4 per-head row transforms around the sparse attention (gfx950), one HBM pass each.
//
// Reference layer: src/mcore_bridge/model/gpts/deepseek_v4.py:61-328 (DSv4HybridSelfAttention).
//   q path (:114-142): q = RoPE(RMSNorm_noweight(q_up(q_res)))   per (token, head) row
//   output (:287-318): o = RoPE^-1(o); grouped output projection over o viewed as [T, G, H*D/G]
// RoPE is the interleaved form on the last `rope_dim` dims of a row: pairs (2i, 2i+1) rotate by
// angle i of the row's token, out = (a c - b s, b c + a s), c / s the token's cos / sin (already
// multiplied by the attention mscale; the inverse rotation negates s).
//
// norm_rope (rows of D dims, token t = row / n_heads):
//   forward  y = bf16(x * rsqrt(mean x^2 + eps))   (norm = 0: y = x), out = bf16(RoPE(y))
//   backward dy = RoPE^T(dout) on the rope dims (dout elsewhere),
//            dx = r (dy - yf <dy, yf> / D)  with yf = x r        (norm = 0: dx = dy)
// out_rope_group (rows of D dims of o [T, H, D]):
//   forward  og[g, t, (h % HG) * D + d] = RoPE^{+-1}(o[t, h])[d],  g = h / HG, HG = H / G: the
//            rotation and the layout the grouped projection multiplies, in one pass
//   backward do[t, h] = RoPE^T(dog[g, t, (h % HG) * D ..])
// Lanes: D/8 per row, 8 dims (16 bytes) each; rope lanes read 4 cos and 4 sin values.  The
// rotations are evaluated without contraction (a*c and b*s rounded, then the difference), as the
// torch composition rounds them.
#include "dsa_common.h"
#include "dsa_kernels.h"

namespace dsa {

namespace {

constexpr int kWaves = 4;

DSA_DEV void unpack8(const u32x4& v, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_lo(v[i]);
    f[2 * i + 1] = bf16_hi(v[i]);
  }
}

DSA_DEV u32x4 pack8(const float (&f)[8]) {
  u32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return v;
}

template <int LPE>
DSA_DEV float group_sum(float v) {
#pragma unroll
  for (int o = LPE / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Rotate the 4 pairs of f by angles (c[i], s[i]): f[2i], f[2i+1] = a c - b s, b c + a s.
DSA_DEV void rotate4(float (&f)[8], const float (&c)[4], const float (&s)[4]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = f[2 * i], b = f[2 * i + 1];
    f[2 * i] = a * c[i] - b * s[i];
    f[2 * i + 1] = b * c[i] + a * s[i];
  }
}

// Transposed rotation (the gradient of rotate4): ga, gb -> ga c + gb s, gb c - ga s.
DSA_DEV void rotate4_t(float (&f)[8], const float (&c)[4], const float (&s)[4]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float ga = f[2 * i], gb = f[2 * i + 1];
    f[2 * i] = ga * c[i] + gb * s[i];
    f[2 * i + 1] = gb * c[i] - ga * s[i];
  }
}

// The 4 angles of this lane's rope dims (pairs (c - rope0)/2 .. +3) of token t; sgn = -1 for the
// inverse rotation.
DSA_DEV void load_angles(const RopeParams& p, int t, int c, float sgn, float (&cs)[4], float (&sn)[4]) {
  const int i0 = (c - (p.dim - p.rope_dim)) >> 1;
  const float* cr = p.cos + (int64_t)t * p.angle_stride + i0;
  const float* sr = p.sin + (int64_t)t * p.angle_stride + i0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    cs[i] = cr[i];
    sn[i] = sgn * sr[i];
  }
}

template <int LPE>
__global__ __launch_bounds__(kWaves * 64) void v4_norm_rope_fwd_kernel(RopeParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = ((int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6)) * (64 / LPE) + lane / LPE;
  if (row >= p.rows) return;
  const int c = 8 * (lane % LPE);
  const int t = (int)(row / p.n_heads);
  float f[8];
  unpack8(gload16(p.x + row * p.dim + c), f);
  if (p.norm) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(f[j], f[j], ss);
    const float r = rsqrtf(group_sum<LPE>(ss) / (float)p.dim + p.eps);
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = (float)(bf16_t)(f[j] * r);
  }
  if (c >= p.dim - p.rope_dim) {
    float cs[4], sn[4];
    load_angles(p, t, c, p.inverse ? -1.f : 1.f, cs, sn);
    rotate4(f, cs, sn);
  }
  *reinterpret_cast<u32x4*>(p.out + row * p.dim + c) = pack8(f);
}

template <int LPE>
__global__ __launch_bounds__(kWaves * 64) void v4_norm_rope_bwd_kernel(RopeParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = ((int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6)) * (64 / LPE) + lane / LPE;
  if (row >= p.rows) return;
  const int c = 8 * (lane % LPE);
  const int t = (int)(row / p.n_heads);
  float g[8];
  unpack8(gload16(p.dout + row * p.dim + c), g);
  if (c >= p.dim - p.rope_dim) {
    float cs[4], sn[4];
    load_angles(p, t, c, p.inverse ? -1.f : 1.f, cs, sn);
    rotate4_t(g, cs, sn);
  }
  if (p.norm) {
    float x[8];
    unpack8(gload16(p.x + row * p.dim + c), x);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(x[j], x[j], ss);
    const float r = rsqrtf(group_sum<LPE>(ss) / (float)p.dim + p.eps);
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      x[j] *= r;   // yf
      dot = __builtin_fmaf(g[j], x[j], dot);
    }
    dot = group_sum<LPE>(dot) / (float)p.dim;
#pragma unroll
    for (int j = 0; j < 8; ++j) g[j] = r * (g[j] - x[j] * dot);
  }
  *reinterpret_cast<u32x4*>(p.dx + row * p.dim + c) = pack8(g);
}

// Offset of row (t, h)'s dims in the grouped layout [G, T, HG * D].
DSA_DEV int64_t grouped_off(const RopeParams& p, int t, int h) {
  const int hg = p.n_heads / p.groups;
  const int g = h / hg;
  return (((int64_t)g * p.tokens + t) * hg + (h - g * hg)) * p.dim;
}

template <int LPE>
__global__ __launch_bounds__(kWaves * 64) void v4_out_rope_group_fwd_kernel(RopeParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = ((int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6)) * (64 / LPE) + lane / LPE;
  if (row >= p.rows) return;
  const int c = 8 * (lane % LPE);
  const int t = (int)(row / p.n_heads), h = (int)(row - (int64_t)t * p.n_heads);
  u32x4 v = gload16(p.x + row * p.dim + c);
  if (c >= p.dim - p.rope_dim) {
    float f[8], cs[4], sn[4];
    unpack8(v, f);
    load_angles(p, t, c, p.inverse ? -1.f : 1.f, cs, sn);
    rotate4(f, cs, sn);
    v = pack8(f);
  }
  *reinterpret_cast<u32x4*>(p.out + grouped_off(p, t, h) + c) = v;
}

template <int LPE>
__global__ __launch_bounds__(kWaves * 64) void v4_out_rope_group_bwd_kernel(RopeParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = ((int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6)) * (64 / LPE) + lane / LPE;
  if (row >= p.rows) return;
  const int c = 8 * (lane % LPE);
  const int t = (int)(row / p.n_heads), h = (int)(row - (int64_t)t * p.n_heads);
  u32x4 v = gload16(p.dout + grouped_off(p, t, h) + c);
  if (c >= p.dim - p.rope_dim) {
    float f[8], cs[4], sn[4];
    unpack8(v, f);
    load_angles(p, t, c, p.inverse ? -1.f : 1.f, cs, sn);
    rotate4_t(f, cs, sn);
    v = pack8(f);
  }
  *reinterpret_cast<u32x4*>(p.dx + row * p.dim + c) = v;
}

template <int LPE>
int launch_lpe(int which, const RopeParams& p, hipStream_t stream) {
  const int64_t per_wg = (int64_t)kWaves * (64 / LPE);
  const dim3 grid((unsigned)((p.rows + per_wg - 1) / per_wg)), block(kWaves * 64);
  switch (which) {
    case 0: hipLaunchKernelGGL(v4_norm_rope_fwd_kernel<LPE>, grid, block, 0, stream, p); break;
    case 1: hipLaunchKernelGGL(v4_norm_rope_bwd_kernel<LPE>, grid, block, 0, stream, p); break;
    case 2: hipLaunchKernelGGL(v4_out_rope_group_fwd_kernel<LPE>, grid, block, 0, stream, p); break;
    default: hipLaunchKernelGGL(v4_out_rope_group_bwd_kernel<LPE>, grid, block, 0, stream, p); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace

int launch_v4_rope(int which, const RopeParams& p, hipStream_t stream) {
  if (p.rows == 0) return 0;
  switch (p.dim) {
    case 64: return launch_lpe<8>(which, p, stream);
    case 128: return launch_lpe<16>(which, p, stream);
    case 256: return launch_lpe<32>(which, p, stream);
    case 512: return launch_lpe<64>(which, p, stream);
    default: return -2;
  }
}

}  // namespace dsa
