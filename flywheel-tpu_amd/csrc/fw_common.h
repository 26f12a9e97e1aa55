// Shared device/host helpers of the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include "../../include/flywheel_hip.h"

namespace fw {

// ---------------------------------------------------------------- errors
int set_error(int code, const char *fmt, ...);
int check_launch(const char *what);

#define FW_REQUIRE(cond, code, ...)                \
  do {                                             \
    if (!(cond)) return ::fw::set_error(code, __VA_ARGS__); \
  } while (0)

// ---------------------------------------------------------------- vector types
typedef short bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Two f32 -> packed bf16 pair (round to nearest even; v_cvt_pk_bf16_f32).
// One v_cvt_pk_bf16_f32 (round to nearest even): written as a two-lane vector
// conversion, since two scalar conversions are sometimes selected as two
// half-used converts and a v_perm_b32 that merges them.
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  typedef float f32x2v_t __attribute__((ext_vector_type(2)));
  const f32x2v_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Columns i .. i + 3 (i a multiple of 4) of a RoPE table held as f32 or bf16,
// one vector load.
template <bool F32>
__device__ __forceinline__ void rope_load4(const void *t, size_t i, float (&v)[4]) {
  if constexpr (F32) {
    const f32x4_t x = *(const f32x4_t *)((const float *)t + i);
    v[0] = x[0]; v[1] = x[1]; v[2] = x[2]; v[3] = x[3];
  } else {
    const u32x2_t x = *(const u32x2_t *)((const uint16_t *)t + i);
    v[0] = bf16_lo(x[0]); v[1] = bf16_hi(x[0]); v[2] = bf16_lo(x[1]); v[3] = bf16_hi(x[1]);
  }
}

__device__ __forceinline__ uint16_t to_bf16(float a) {
  __bf16 r = (__bf16)a;
  return __builtin_bit_cast(uint16_t, r);
}

// Two fp8 codes (byte 0,1 or 2,3 of w) -> packed bf16 pair.  Exact: every
// e4m3 / e5m2 value is representable in bf16.
template <int KV>
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t w, bool hi) {
  if constexpr (KV == FW_FP8_E4M3) {
    return hi ? __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true))
              : __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
  } else {
    return hi ? __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, true))
              : __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, false));
  }
}

// Select 16-bit halves of two words: (lo of a, lo of b) or (hi of a, hi of b).
__device__ __forceinline__ uint32_t perm_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t perm_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Branch-free tanh: 1 - 2 / (e^{2x} + 1), from the hardware exp2 and rcp.
// Saturates to +-1 for large |x|; absolute error ~1e-7 (the softcap scales it).
__device__ __forceinline__ float fast_tanh(float x) {
  const float t = __builtin_amdgcn_exp2f(x * (2.0f * 1.4426950408889634f));
  return 1.0f - 2.0f * __builtin_amdgcn_rcpf(t + 1.0f);
}

// softcap_log2 * tanh(x) for the scores of a wave (sc: an array of floats or
// of float vectors, read and written through sc[i][e] / sc[e]).  By the
// largest |x| of the wave (a wave-uniform choice):
//   <= kTanhPoly3Bound: x (d0 + d1 x^2), minimax on [-0.12, 0.12];
//   <= kTanhPolyBound:  x (c0 + c1 x^2 + c2 x^4), minimax on [-0.3, 0.3];
//   else fast_tanh (two transcendentals).
// Both polynomials stay below 2.5e-7 abs error with float32 evaluation (the
// Taylor polynomial through x^7 has 4.3e-7 on [-0.3, 0.3]).  With ANCHOR the
// result is softcap_log2 * tanh(x) - anchor (the last multiply becomes an FMA).
constexpr float kTanhPolyBound = 0.3f;
constexpr float kTanhC0 = 0.999995887f, kTanhC1 = -0.332973301f, kTanhC2 = 0.125218078f;
constexpr float kTanhPoly3Bound = 0.12f;
constexpr float kTanhD0 = 0.999990642f, kTanhD1 = -0.330870956f;
template <bool ANCHOR>
__device__ __forceinline__ float tanh_poly3_scaled(float x, float d0, float d1, float anchor) {
  const float p = fmaf(x * x, d1, d0);
  return ANCHOR ? fmaf(x, p, -anchor) : x * p;
}
template <bool ANCHOR>
__device__ __forceinline__ float tanh_poly_scaled(float x, float c0, float c1, float c2,
                                                  float anchor) {
  const float x2 = x * x;
  float p = fmaf(x2, c2, c1);
  p = fmaf(x2, p, c0);
  return ANCHOR ? fmaf(x, p, -anchor) : x * p;
}
template <int N, int M, bool ANCHOR = false, typename Acc>
__device__ __forceinline__ void softcap_scores(Acc &sc, float softcap_log2, float anchor = 0.f) {
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i)
#pragma unroll
    for (int e = 0; e < M; ++e) amax = fmaxf(amax, fabsf(sc[i][e]));
  if (__any(amax > kTanhPolyBound)) {
#pragma unroll
    for (int i = 0; i < N; ++i)
#pragma unroll
      for (int e = 0; e < M; ++e)
        sc[i][e] = ANCHOR ? fmaf(fast_tanh(sc[i][e]), softcap_log2, -anchor)
                          : fast_tanh(sc[i][e]) * softcap_log2;
  } else if (__any(amax > kTanhPoly3Bound)) {
    const float c0 = softcap_log2 * kTanhC0, c1 = softcap_log2 * kTanhC1;
    const float c2 = softcap_log2 * kTanhC2;
#pragma unroll
    for (int i = 0; i < N; ++i)
#pragma unroll
      for (int e = 0; e < M; ++e)
        sc[i][e] = tanh_poly_scaled<ANCHOR>(sc[i][e], c0, c1, c2, anchor);
  } else {
    const float d0 = softcap_log2 * kTanhD0, d1 = softcap_log2 * kTanhD1;
#pragma unroll
    for (int i = 0; i < N; ++i)
#pragma unroll
      for (int e = 0; e < M; ++e)
        sc[i][e] = tanh_poly3_scaled<ANCHOR>(sc[i][e], d0, d1, anchor);
  }
}

// acc *= s on an MFMA accumulator kept in AGPRs: each register is read,
// scaled and written back in place.  Written as plain VALU code, the rescale
// makes the compiler keep a VGPR copy of every accumulator live across the
// loop around it (an AGPR read per register per iteration).  Callers run it
// where every MFMA that wrote acc has long completed; the s_nop covers the
// next MFMA's read of the rewritten AGPRs.
template <typename Vec>
__device__ __forceinline__ void scale_in_agprs(Vec &acc, float s) {
  constexpr int N = sizeof(Vec) / sizeof(float);
#pragma unroll
  for (int e = 0; e < N; ++e) {
    float t;
    asm volatile(
        "v_accvgpr_read_b32 %1, %0\n\t"
        "v_mul_f32 %1, %1, %2\n\t"
        "v_accvgpr_write_b32 %0, %1"
        : "+a"(acc[e]), "=&v"(t)
        : "v"(s));
  }
  asm volatile("s_nop 4" ::: "memory");
}

// 64 lanes x 16 bytes from base + voff[lane] into LDS at lds_addr + 16 * lane
// (global_load_lds_dwordx4).  Issued from asm so the compiler does not add a
// wait for it before every later LDS read: the kernel waits for its own
// copies (s_waitcnt vmcnt) before the barrier that publishes the buffer.
__device__ __forceinline__ void lds_dma16(const uint8_t *base, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :: "s"(lds_addr), "v"(voff), "s"(base) : "memory", "m0");
}
// 4 bytes per active lane from base + voff[lane] into LDS at lds_addr + 4 *
// lane (global_load_lds_dword).
__device__ __forceinline__ void lds_dma4(const uint8_t *base, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2"
               :: "s"(lds_addr), "v"(voff), "s"(base) : "memory", "m0");
}
// The same copy with the non-temporal hint, for data read once.
__device__ __forceinline__ void lds_dma16_nt(const uint8_t *base, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt"
               :: "s"(lds_addr), "v"(voff), "s"(base) : "memory", "m0");
}
// Two copies into LDS at lds_addr and lds_addr + 1024 under one M0 value: the
// second instruction's immediate offset (1024) moves both its LDS and its
// global address, so its base is passed 1024 lower (the sum is the address
// voff2 names; nothing is read below base).
__device__ __forceinline__ void lds_dma16x2(const uint8_t *base, uint32_t voff1, uint32_t voff2,
                                            uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %3\n\t"
               "global_load_lds_dwordx4 %2, %4 offset:1024"
               :: "s"(lds_addr), "v"(voff1), "v"(voff2), "s"(base), "s"(base - 1024)
               : "memory", "m0");
}

__device__ __forceinline__ float wave_max_xor(float v, int mask) {
  return fmaxf(v, __shfl_xor(v, mask, 64));
}

// ---------------------------------------------------------------- MFMA
__device__ __forceinline__ f32x4_t mfma16(const bf16x8_t &a, const bf16x8_t &b, const f32x4_t &c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16_t mfma32(const bf16x8_t &a, const bf16x8_t &b, const f32x16_t &c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
// ---- ragged append of new K/V token rows into the merged paged pool
// (fw_append_ragged; also fused into fw_prefill's launch).  Token i belongs
// to the request r with cu[r] <= i < cu[r + 1] (or T / B tokens per request
// without cu) and lands at position lens[r] + (i - cu[r]) of that request.
struct AppendArgs {
  uint8_t *cache;
  const uint8_t *k, *v;  // (T, Hk, head_bytes) rows
  const int32_t *cu, *lens, *table, *num_active;
  int B, T, Hk, head_bytes, CH, P, num_pages, max_pages;
};
constexpr int kAppendTokensPerBlock = 16;  // 256 threads: 16 lanes a token
inline int append_blocks(int T) { return (T + kAppendTokensPerBlock - 1) / kAppendTokensPerBlock; }

// Chunk c (16 bytes) of a merged token row: head row hr = c / chunks_per_head
// is K (even) or V (odd) of KV head hr / 2; head rows past 2 * Hk (an fp8
// pool's pad head) are zero.
__device__ __forceinline__ u32x4_t merged_chunk(const uint8_t *k_row, const uint8_t *v_row, int c,
                                                int chunks_per_head, int nheads_k) {
  const int hr = c / chunks_per_head;
  const int off = (c % chunks_per_head) * 16;
  const int kvh = hr >> 1;
  if (kvh >= nheads_k) return u32x4_t{0u, 0u, 0u, 0u};
  const uint8_t *src = (hr & 1 ? v_row : k_row) + (size_t)kvh * chunks_per_head * 16 + off;
  return *(const u32x4_t *)src;
}

// Workgroup `blk` (256 threads) writes tokens 16 blk .. 16 blk + 15.  Rows past
// the last active request, positions past the table and page ids outside
// [0, num_pages) write nothing.
__device__ __forceinline__ void append_token_rows(const AppendArgs &a, int blk) {
  const int i = blk * kAppendTokensPerBlock + (int)(threadIdx.x >> 4);
  const int lane = threadIdx.x & 15;
  if (i >= a.T) return;
  const int nact = a.num_active ? min(max(*a.num_active, 0), a.B) : a.B;
  int r, first;
  if (a.cu) {
    if (i >= a.cu[nact]) return;  // rows past the last active request are padding
    int lo = 0, hi = nact;  // cu[lo] <= i < cu[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (a.cu[mid] <= i) lo = mid; else hi = mid;
    }
    r = lo;
    first = a.cu[r];
    if (i < first) return;
  } else {  // T / B tokens per request
    const int per = a.T / a.B;
    r = i / per;
    first = r * per;
    if (r >= nact) return;
  }
  const int pos = a.lens[r] + (i - first);
  if (pos < 0 || pos / a.P >= a.max_pages) return;
  const int page = a.table[(size_t)r * a.max_pages + pos / a.P];
  if (page < 0 || page >= a.num_pages) return;
  const size_t row_bytes = (size_t)a.CH * a.head_bytes;
  uint8_t *dst = a.cache + ((size_t)page * a.P + pos % a.P) * row_bytes;
  const uint8_t *k_row = a.k + (size_t)i * a.Hk * a.head_bytes;
  const uint8_t *v_row = a.v + (size_t)i * a.Hk * a.head_bytes;
  const int cph = a.head_bytes / 16;
  const int nchunks = a.CH * cph;
  // eight loads in flight before their stores (the compiler cannot reorder a
  // load past a store that may alias it)
  for (int c0 = lane; c0 < nchunks; c0 += 8 * 16) {
    u32x4_t x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = c0 + 16 * j;
      x[j] = c < nchunks ? merged_chunk(k_row, v_row, c, cph, a.Hk) : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = c0 + 16 * j;
      if (c < nchunks) *(u32x4_t *)(dst + (size_t)c * 16) = x[j];
    }
  }
}

// Compute units of the current device (cached per device).
static inline int device_cus() {
  static int cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
      v = 256;
    cus[dev] = v;
  }
  return cus[dev];
}
inline size_t align_up(size_t a, size_t b) { return (a + b - 1) / b * b; }

inline int dtype_bytes(int kv_dtype) { return kv_dtype == FW_BF16 ? 2 : 1; }
inline int merged_heads(int nheads_k, int kv_dtype) {
  int per_word = kv_dtype == FW_BF16 ? 1 : 2;
  return 2 * ((nheads_k + per_word - 1) / per_word * per_word);
}

}  // namespace fw
