// Shared device helpers for the gfx950 DSA kernels (CDNA4, wave64).
//
// MFMA operand layouts used throughout (checked on the device through the parity tests in
// tests/test_gpu_parity.py, and by construction below):
//   v_mfma_f32_32x32x16_bf16  C[32x32] += A[32x16] * B[16x32]
//     A: lane l holds A[row = l%32][k = (l/32)*8 + 0..7]
//     B: lane l holds B[k = (l/32)*8 + 0..7][col = l%32]
//     C: lane l holds C[row = (i/4)*8 + (l/32)*4 + i%4][col = l%32], i = 0..15
//   v_mfma_f32_16x16x32_bf16  C[16x16] += A[16x32] * B[32x16]
//     A: lane l holds A[row = l%16][k = (l/16)*8 + 0..7]
//     B: lane l holds B[k = (l/16)*8 + 0..7][col = l%16]
//     C: lane l holds C[row = (l/16)*4 + i][col = l%16], i = 0..3
// The order of the k index inside one MFMA is free as long as A and B agree; the kernels
// use that freedom to feed the C layout of one product straight into the next one.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

typedef __bf16 bf16_t;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define DSA_DEV __device__ __forceinline__
#define DSA_HOST_DEV __host__ __device__ __forceinline__

namespace dsa {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

DSA_DEV f32x16 mfma32x32x16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
DSA_DEV f32x4 mfma16x16x32(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// C += A * B with B and C in AccVGPRs.  gfx950 MFMAs read any operand from AccVGPRs, but the
// compiler only ever feeds A/B from VGPRs (spilled fragments then cost 4 v_accvgpr_read per
// MFMA); these forms let a kernel keep a loop-invariant B operand set in AccVGPRs.  Hazards the
// compiler cannot see inside the asm are covered here and by the caller:
//   - s_nop 1 before the MFMA: 2 wait states after a VALU write of A or an AccVGPR write of B/C;
//   - the caller issues mfma_acc_drain() before any VALU reads C (8-pass XDL result: 11 wait
//     states needed, 16 given).
DSA_DEV void mfma32x32x16_acc_first(f32x16& c, const u32x4& a, const u32x4& b) {
  asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=a"(c) : "v"(a), "a"(b));
}
DSA_DEV void mfma32x32x16_acc(f32x16& c, const u32x4& a, const u32x4& b) {
  asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "a"(b));
}
// C += A * B with C pinned in AccVGPRs ("a") or VGPRs ("v") and A, B in VGPRs -- for kernels
// whose accumulators exceed 256 registers, where the compiler would shuttle tiles between the
// two files around every MFMA.  Same hazard contract as above.
DSA_DEV void mfma32x32x16_cA(f32x16& c, const u32x4& a, const u32x4& b) {
  asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
DSA_DEV void mfma32x32x16_cV(f32x16& c, const u32x4& a, const u32x4& b) {
  asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
}
DSA_DEV void mfma32x32x16_cV_first(f32x16& c, const u32x4& a, const u32x4& b) {
  asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=v"(c) : "v"(a), "v"(b));
}
// 16x16x32 forms (4-pass XDL; the same hazard contract).
DSA_DEV void mfma16x16x32_cA(f32x4& c, const u32x4& a, const u32x4& b) {
  asm("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
DSA_DEV void mfma16x16x32_cV(f32x4& c, const u32x4& a, const u32x4& b) {
  asm("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
}
DSA_DEV void mfma_acc_drain() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 15");
  __builtin_amdgcn_sched_barrier(0);
}

DSA_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// f(std::integral_constant<int, i>) for i = B .. E-1: a loop whose index is a compile-time
// constant in the body (template arguments such as a copy's LDS offset).
template <int B, int E, class F>
DSA_DEV void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// 16-byte LDS / global access helpers.
DSA_DEV u32x4 lds_load16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
DSA_DEV void lds_store16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }
DSA_DEV u32x4 gload16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

DSA_DEV bf16x8 as_bf16x8(const u32x4& v) { return __builtin_bit_cast(bf16x8, v); }
DSA_DEV u32x4 as_u32x4(const bf16x8& v) { return __builtin_bit_cast(u32x4, v); }

// Pack two floats into one dword of two bf16 (round to nearest even): one v_cvt_pk_bf16_f32.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
DSA_DEV uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}

DSA_DEV float bf16_lo(uint32_t v) { return __builtin_bit_cast(float, v << 16); }
DSA_DEV float bf16_hi(uint32_t v) { return __builtin_bit_cast(float, v & 0xffff0000u); }
// max(x, 0) as an integer max of the bit pattern: one v_max_i32 (negative values and -0 give +0;
// a NaN with the sign bit clear passes through).  fmaxf(x, 0) costs two v_max_f32 in IEEE mode
// (a NaN-quieting max of x with itself first).
DSA_DEV float relu_bits(float x) { return __builtin_bit_cast(float, max(__builtin_bit_cast(int, x), 0)); }

// 8x8 transpose of 16-bit elements held as 8 rows x 4 dwords (row r = 8 consecutive
// elements of one source row).  Output operand t (t = 0..7) gathers element t of each row:
//   out[t].dword[n] = (row[2n].elem[t], row[2n+1].elem[t]).
// v_perm_b32 selector 0x05040100 keeps the low halves, 0x07060302 the high halves.
DSA_DEV void transpose8x8_b16(const u32x4 (&row)[8], u32x4 (&out)[8]) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const uint32_t a = row[2 * n][m];
      const uint32_t b = row[2 * n + 1][m];
      out[2 * m][n] = __builtin_amdgcn_perm(b, a, 0x05040100u);
      out[2 * m + 1][n] = __builtin_amdgcn_perm(b, a, 0x07060302u);
    }
  }
}

// One output operand of the transpose above (lets the caller interleave with MFMAs).
DSA_DEV u32x4 transpose8x8_b16_col(const u32x4 (&row)[8], int t) {
  const int m = t >> 1;
  const uint32_t sel = (t & 1) ? 0x07060302u : 0x05040100u;
  u32x4 o;
#pragma unroll
  for (int n = 0; n < 4; ++n) o[n] = __builtin_amdgcn_perm(row[2 * n + 1][m], row[2 * n][m], sel);
  return o;
}

// wave64 reductions (xor butterflies through ds_swizzle/dpp chosen by the compiler)
DSA_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
DSA_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
DSA_DEV int wave_max_i(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
  return v;
}
DSA_DEV int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Combine a per-lane value with the lane 32 apart (same MFMA column, other row half).
DSA_DEV float xor32_max(float v) { return fmaxf(v, __shfl_xor(v, 32, 64)); }
DSA_DEV float xor32_sum(float v) { return v + __shfl_xor(v, 32, 64); }

// Asynchronous 16-byte global -> LDS copy (gfx950 global_load_lds_dwordx4).  Lane i of the
// wave writes 16 bytes at lds_wave_base + 16*i; lds_wave_base must be wave-uniform.
DSA_DEV void async_copy16(const void* gsrc, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(const_cast<void*>(gsrc),
                                   (__attribute__((address_space(3))) void*)lds_wave_base, 16, 0, 0);
}

// Generic pointer to the LDS byte address `a` (inverse of lds_addr).
DSA_DEV const char* lds_ptr(uint32_t a) {
  return (const char*)(const __attribute__((address_space(3))) char*)(uintptr_t)a;
}

// LDS byte address of a pointer into __shared__ memory.
DSA_DEV uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// The same copy issued through inline asm (M0 = wave-uniform LDS base).  The compiler does not
// model it, so it neither serialises later LDS reads against it nor waits for it: the caller
// owns completion (s_waitcnt vmcnt(N) + barrier) -- that is what lets a multi-stage gather ring
// overlap the MFMA work on earlier stages.  M0 is written right before the LDS DMA, which reads
// it one wait state later (s_nop 0).
DSA_DEV void async_copy16_unordered(const void* gsrc, uint32_t lds_wave_base) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_wave_base), "v"(gsrc)
               : "memory", "m0");
}

// The same copy with the non-temporal cache policy (nt): streamed data that is read once.
DSA_DEV void async_copy16_nt(const void* gsrc, uint32_t lds_wave_base) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off nt" ::"s"(lds_wave_base), "v"(gsrc)
               : "memory", "m0");
}

// 4-byte variant (global_load_lds_dword): lane i writes 4 bytes at lds_wave_base + 4*i.
DSA_DEV void async_copy4_unordered(const void* gsrc, uint32_t lds_wave_base) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(lds_wave_base), "v"(gsrc)
               : "memory", "m0");
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt[3:0] | expcnt=7 | lgkmcnt=15 | vmcnt[5:4] << 14).
template <int N>
DSA_DEV void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | 0x70 | 0xF00 | ((N >> 4) << 14));
}

// s_waitcnt vmcnt(0): all of this wave's vector-memory loads (including LDS-direct ones) done.
DSA_DEV void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// XCD-aware remap of a 1-D grid.  Consecutive workgroup ids are dispatched round-robin over the
// device's n_xcd XCDs (8 on a whole MI355X, fewer on a partition); work items are handed out in
// chunks of kXcdChunk consecutive items, chunk c to XCD c % n_xcd.  The ~32 workgroups an XCD runs
// at once then work on neighbouring items (neighbouring query tokens share most of their selected
// KV rows, which stay in that XCD's L2), and every XCD draws items from the whole range: with one
// contiguous share per XCD, the XCDs holding document starts (short causal rows) ran out of work
// early.  The grid must come from xcd_grid() with the same n_xcd; a grid of fewer than
// n_xcd * kXcdChunk workgroups gives each XCD one contiguous run.  With n_xcd = 1 the map is the
// identity.
constexpr int kXcdChunk = 64;
DSA_DEV int xcd_remap(int bid, int n_xcd) {
  const int per = (int)gridDim.x / n_xcd;
  const int c = per < kXcdChunk ? per : kXcdChunk;
  const int j = bid / n_xcd, x = bid - j * n_xcd, jc = j / c;
  return (jc * n_xcd + x) * c + (j - jc * c);
}
// Grid size for xcd_remap over n work items (items >= n exit at once).
inline int xcd_grid(int n, int n_xcd) {
  const int full = n_xcd * kXcdChunk;
  return n >= full ? (n + full - 1) / full * full : (n + n_xcd - 1) / n_xcd * n_xcd;
}

}  // namespace dsa
