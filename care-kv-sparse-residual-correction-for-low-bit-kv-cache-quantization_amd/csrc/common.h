// Device helpers shared by the CARE-KV kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "carekv.h"

namespace carekv {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kPage = 16;  // page_size supported by the kernels
constexpr int kGroup = 32; // quant group, K channel group
constexpr int kVtb = 4;    // V token block

__device__ __forceinline__ float h2f(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return (float)v;
}
__device__ __forceinline__ uint16_t f2h(float f) {  // round to nearest even
  _Float16 v = (_Float16)f;
  uint16_t h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}
__device__ __forceinline__ _Float16 bits2half(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return v;
}
__device__ __forceinline__ uint16_t half2bits(_Float16 v) {
  uint16_t h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}

// MFMA f32 16x16x16 f16.  Operand layout (wave64):
//   A[row=l%16][k=4*(l/16)+i], B[k=4*(l/16)+i][col=l%16],
//   C[row=4*(l/16)+i][col=l%16], i = 0..3.
__device__ __forceinline__ float4_t mfma16(half4_t a, half4_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// Sign-extended BITS-bit field k of a little-endian bit string held in
// 32-bit words (field k starts at bit BITS*k).
template <int BITS>
__device__ __forceinline__ int get_code(const uint32_t* w, int k) {
  const int bit = BITS * k;
  const int wi = bit >> 5, sh = bit & 31;
  uint32_t v;
  if (sh + BITS <= 32) {
    v = w[wi] >> sh;
  } else {
    v = (uint32_t)((((uint64_t)w[wi + 1] << 32) | w[wi]) >> sh);
  }
  v &= (1u << BITS) - 1u;
  const int half_range = 1 << (BITS - 1);
  return (int)(v ^ (uint32_t)half_range) - half_range;  // two's complement BITS-bit
}

// Exact dequantised value half(code * s) (quantizer.py:67-82: float product,
// one rounding to fp16).  code*s is exact in fp32, so the fp16 multiply
// (single RNE rounding) gives the same bits.
__device__ __forceinline__ _Float16 dq(int code, _Float16 s) { return (_Float16)code * s; }

// Wave reductions over the 64 lanes (xor butterflies).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Load N bytes (N in {4,6,8,12,16,24,32,48,64}) at p into 32-bit words; p is
// aligned to the largest power of two dividing both the row size and N.
template <int N>
__device__ __forceinline__ void load_bytes(uint32_t* w, const int8_t* p) {
  if constexpr (N % 16 == 0) {
#pragma unroll
    for (int i = 0; i < N / 16; ++i) {
      uint4 v = *reinterpret_cast<const uint4*>(p + 16 * i);
      w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
  } else if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) w[i] = *reinterpret_cast<const uint32_t*>(p + 4 * i);
  } else {
    static_assert(N % 2 == 0, "even byte count");
#pragma unroll
    for (int i = 0; i < (N + 3) / 4; ++i) w[i] = 0;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      uint32_t v = *reinterpret_cast<const uint16_t*>(p + 2 * i);
      w[i >> 1] |= v << (16 * (i & 1));
    }
  }
}

template <int N>
__device__ __forceinline__ void store_bytes(int8_t* p, const uint32_t* w) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) *reinterpret_cast<uint32_t*>(p + 4 * i) = w[i];
  } else {
    static_assert(N % 2 == 0, "even byte count");
#pragma unroll
    for (int i = 0; i < N / 2; ++i)
      *reinterpret_cast<uint16_t*>(p + 2 * i) = (uint16_t)(w[i >> 1] >> (16 * (i & 1)));
  }
}

__host__ __device__ constexpr int row_bytes(int D, int bits) { return D * bits / 8; }

// Code-buffer page of the row whose metadata pages start at pg_base
// (= (kv head * n_seq + seq) * max_pages): pg_base itself, or on a view with
// a code-page map (carekv_arena::code_pages > 0) the row's code pages moved
// back by its offset, so that page p of the row is code page
// code_base + p.
__device__ __forceinline__ long code_base(const carekv_arena& A, long pg_base) {
  if (A.code_pages <= 0) return pg_base;
  const long r = pg_base / A.max_pages;  // kv head * n_seq + seq
  return r * A.code_pages - A.code_page_off[r % A.n_seq];
}
// One past the last page of the row the code-page map holds.
__device__ __forceinline__ int code_page_limit(const carekv_arena& A, long pg_base) {
  const long r = pg_base / A.max_pages;
  return A.code_page_off[r % A.n_seq] + A.code_pages;
}
// Whether the code-page map (if any) holds metadata page pg.
__device__ __forceinline__ bool code_pg_in(const carekv_arena& A, long pg) {
  if (A.code_pages <= 0) return true;
  const long r = pg / A.max_pages;
  const long t = pg - r * A.max_pages - A.code_page_off[r % A.n_seq];
  return t >= 0 && t < A.code_pages;
}
// Code-buffer page of metadata page pg.
__device__ __forceinline__ long code_pg(const carekv_arena& A, long pg) {
  if (A.code_pages <= 0) return pg;
  const long r = pg / A.max_pages;
  return code_base(A, r * A.max_pages) + (pg - r * A.max_pages);
}

// Wait for this wave's outstanding LDS operations; also a compiler barrier
// for memory so LDS writes by other lanes are read after they landed.
__device__ __forceinline__ void lds_sync_wave() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

}  // namespace carekv
